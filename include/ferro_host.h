/*
 * ferro_host.h — load-time host routines of the ferrolm MI355X library:
 * synthetic weights and the int8/int4 quantizer. They run on the CPU, once
 * per model, like the reference's Model::random / Model::quantize; their
 * output is the weight format the device path consumes (ferro_gpu.h).
 * Same error conventions as ferro_gpu.h (0 ok, negative FG_E_* code).
 */
#ifndef FERRO_HOST_H
#define FERRO_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model::random's weight draw (src/model.rs:156-163): values N(0, std)
 * from the reference's xorshift64* + Box-Muller generator (src/rng.rs),
 * rounded to bf16 (RNE, src/safetensors.rs:171-178). Rows are drawn in
 * blocks of 64, block b from Rng::new(fh_stream_seed(seed, tensor, b)),
 * so the result does not depend on the thread count. */
int fh_random_bf16(uint64_t seed, uint64_t tensor, int64_t rows, int64_t cols, float std,
                   uint16_t* out);
uint64_t fh_stream_seed(uint64_t seed, uint64_t tensor, uint64_t block);

/* QMatrix::quantize (src/quant.rs:78-143): symmetric group-32 int8/int4
 * with the reference's clip search, importance weighting and code layout.
 * kind 1 = int8, 2 = int4. w is rows x cols f32 row-major; importance
 * (cols floats) may be NULL. q receives rows*cols (int8) or rows*cols/2
 * (int4) bytes, s rows*cols/32 floats. */
int fh_quantize(int32_t kind, int32_t rows, int32_t cols, const float* w,
                const float* importance, uint8_t* q, float* s);

/* AWQ channel statistics (src/awq.rs:128-142): mean |x| and mean x^2 of
 * each of the k input channels over the m calibration rows (cal, m x k),
 * summed in f64 in row order. */
int fh_awq_stats(const float* cal, int32_t m, int32_t k, float* abs_mean, float* sq_mean);

/* AWQ scales for one alpha (src/awq.rs:144-150): max(a, 1e-5)^alpha,
 * normalised so that max * min = 1, floored at 1e-4. */
int fh_awq_scales(const float* abs_mean, int32_t k, float alpha, float* s);

#ifdef __cplusplus
}
#endif
#endif
