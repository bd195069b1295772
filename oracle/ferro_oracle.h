/*
 * CPU oracle for the ferrolm speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * CPU algorithm (Rust, the src directory of /root/reference) used as the parity checker
 * for the HIP path and as the timed CPU baseline. Only tests/, the smoke()
 * entry point and bench.py's cpu_baseline leg may load it; the product
 * library (ferrolm_amd) never does.
 *
 * Every function follows one reference function; the file:line is given at
 * each definition in ferro_oracle.c. Floating-point operations are written
 * in the reference's order with explicit fmaf() where Rust uses mul_add or
 * an FMA intrinsic, and the file is compiled with -ffp-contract=off, so
 * the results are the reference's bits wherever the libm calls agree
 * (glibc cosf/sinf/powf/log/cos/sqrt, as Rust std uses on Linux).
 */
#ifndef FERRO_ORACLE_H
#define FERRO_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_BF16 = 0, OR_INT8 = 1, OR_INT4 = 2 };
enum { OR_LOGITS_NONE = 0, OR_LOGITS_LAST = 1, OR_LOGITS_ALL = 2 };

/* src/config.rs:21-39 (the fields the forward pass reads). */
typedef struct {
    int32_t vocab, hidden, intermediate, layers, heads, kv_heads, head_dim;
    float rms_eps, rope_theta;
    int32_t rope_llama3; /* 0: RopeScaling::None, 1: Llama3 */
    float rope_factor, rope_low_freq, rope_high_freq;
    int32_t rope_orig_max_pos;
    int32_t max_position;
    int32_t tie_embeddings;
    int32_t qkv_bias;
} or_config;

/* A weight matrix as the caller holds it: bf16 row-major (Matrix::new,
 * src/kernels.rs:53) or a QMatrix (codes + scales in the reference's panel
 * order, src/quant.rs:66-76). */
typedef struct {
    int32_t kind, rows, cols, _pad;
    const uint16_t* bf16;
    const uint8_t* q;
    const float* s;
} or_matrix_desc;

/* src/model.rs:28-38 */
typedef struct {
    const float* attn_norm;
    or_matrix_desc wqkv;
    const float* bqkv;
    or_matrix_desc wo;
    const float* mlp_norm;
    or_matrix_desc w_gate_up;
    or_matrix_desc w_down;
} or_layer_desc;

/* src/model.rs:84-89 */
typedef struct {
    const uint32_t* tokens;
    int32_t n, pos;
    const uint32_t* blocks;
    int32_t n_blocks, logits;
} or_chunk;

typedef struct or_model or_model;
typedef struct or_kv or_kv;

/* ---- scalar helpers (exported for unit tests) ---- */
uint64_t or_rng_new(uint64_t seed);
uint64_t or_rng_next(uint64_t* state);
double or_rng_uniform(uint64_t* state);
double or_rng_normal(uint64_t* state);
uint16_t or_f32_to_bf16(float x);
float or_bf16_to_f32(uint16_t x);
float or_exp(float x);
float or_dot(const float* a, const float* b, int32_t n);
void or_rms_norm(const float* x, const float* w, int32_t dim, int32_t rows, float eps, float* out);
void or_silu_mul(const float* gate_up, int32_t inter, int32_t rows, float* out);
/* sampler::distribution (src/sampler.rs:54-90): the (token, probability)
 * pairs in the reference's order; returns their count (tok/p hold vocab). */
int32_t or_distribution(const float* logits, int32_t vocab, float temperature, float top_p, int32_t top_k,
                        uint32_t* tok_out, float* p_out);
/* sampler::draw (src/sampler.rs:93-103) */
uint32_t or_draw(const uint32_t* tok, const float* p, int32_t n, uint64_t* rng);
uint32_t or_argmax(const float* v, int32_t n);
void or_set_threads(int32_t n);
/* The CPU baseline's fast path: the reference's AVX-512 register tiles for
 * the matmuls and eight-wide attention scores, on a spinning pool of
 * `threads` threads (0: all cores), bit-identical to the portable loops.
 * on = 0 returns to the portable loops. 0, or -1 when the CPU lacks
 * AVX-512 F/BW (the portable loops stay). */
int32_t or_set_fast(int32_t on, int32_t threads);

/* QMatrix::quantize (src/quant.rs:82-143): codes/scales in the reference's
 * panel layout. q must hold rows*cols (int8) or rows*cols/2 (int4) bytes,
 * s rows*(cols/32) floats. */
int32_t or_quantize(int32_t kind, int32_t rows, int32_t cols, const float* w,
                    const float* importance, uint8_t* q, float* s);
/* QMatrix::row_f32 (src/quant.rs:164-168) over the whole matrix. */
void or_dequantize(int32_t kind, int32_t rows, int32_t cols, const uint8_t* q,
                   const float* s, float* out);

/* kernels::matmul (src/kernels.rs:249-275) for a single matrix. */
int32_t or_matmul(const or_matrix_desc* w, const float* x, int32_t m,
                  const float* bias, float* y);

/* ---- model, cache, forward ---- */
or_model* or_model_create(const or_config* cfg, const or_layer_desc* layers,
                          const uint16_t* embed, const float* norm,
                          const uint16_t* lm_head);
/* Model::truncated (src/model.rs:237-241): shares the base's weights. */
or_model* or_model_truncated(const or_model* base, int32_t layers);
void or_model_destroy(or_model* m);

or_kv* or_kv_create(int32_t layers, int32_t kv_heads, int32_t head_dim,
                    int32_t block_size, int32_t blocks);
void or_kv_destroy(or_kv* kv);
/* Copies of one layer's K and V arrays ([block][kv_head][16][hd]). */
int32_t or_kv_read(const or_kv* kv, int32_t layer, float* k_out, float* v_out);
int32_t or_kv_write_layer(or_kv* kv, int32_t layer, const float* k, const float* v);

/* Model::forward (src/model.rs:269-362). Returns the number of logits rows
 * written to logits_out (rows x vocab), or -1 on a shape error.
 * hidden_out, if not NULL, receives the residual stream after the
 * embedding and after each layer: (layers+1) x rows x hidden. */
int32_t or_forward(const or_model* m, or_kv* kv, const or_chunk* chunks,
                   int32_t n_chunks, float* logits_out, float* hidden_out);

/* The same forward, also writing Model::record's four projection inputs
 * (src/model.rs:312,323,329,333) of every row: per layer, [rows x hidden
 * (q/k/v input)][rows x heads*head_dim (attention output)][rows x hidden
 * (gate/up input)][rows x intermediate (down input)]. proj_out may be NULL. */
int32_t or_forward_taps(const or_model* m, or_kv* kv, const or_chunk* chunks,
                        int32_t n_chunks, float* logits_out, float* hidden_out,
                        float* proj_out);

/* AWQ (src/awq.rs:128-217): channel statistics, the scales for one alpha,
 * and the alpha search with the final quantization (see ferro_oracle.c). */
void or_awq_stats(const float* cal, int32_t m, int32_t k, float* abs_mean, float* sq_mean);
void or_awq_scales(const float* abs_mean, int32_t k, float alpha, float* s);
int32_t or_awq_search(int32_t kind, int32_t rows, int32_t k, const float* w, int32_t m,
                      const float* cal, float* scales_out, float* alpha_out, double* errs,
                      uint8_t* q, float* s);

/* Greedy generation with the reference engine's speculative loop for one
 * sequence (Engine::schedule/execute/propose, src/engine.rs:395-717,
 * greedy branches, ignore_eos). draft may be NULL (k = 0: plain decode).
 * Writes up to max_tokens ids to out; per-step accepted counts to
 * accepted_out (may be NULL, capacity max_tokens). Returns tokens written,
 * or -1 on error. stats[0] = proposed, stats[1] = accepted, stats[2] = spec
 * steps. */
int32_t or_generate(const or_model* target, const or_model* draft,
                    const uint32_t* prompt, int32_t n_prompt, int32_t max_tokens,
                    int32_t k, int32_t kv_blocks, int32_t max_batch_tokens,
                    uint32_t* out, int32_t* accepted_out, int64_t* stats);

/* One verify step of the reference (target forward over [last, d1..dk] at
 * pos, Logits::All, greedy accept, src/engine.rs:563-616) on an existing
 * cache. Writes the emitted ids to out (<= k+1) and returns their count;
 * *accepted receives the accepted-proposal count. */
int32_t or_verify(const or_model* target, or_kv* kv, const uint32_t* blocks,
                  int32_t n_blocks, int32_t pos, uint32_t last,
                  const uint32_t* drafts, int32_t k, uint32_t* out,
                  int32_t* accepted, float* logits_out);

/* One greedy speculative step of the reference engine for one sequence
 * from an existing state (Engine::propose + the verify pass + accept,
 * src/engine.rs:499-717): tokens[0..len) is the sequence, *computed ==
 * len - 1, *draft_computed <= len - 1; both caches must already hold the
 * positions below those counters and the block tables must cover len + k
 * (target) and len + k - 1 (draft) slots. Writes the emitted ids to out
 * (<= k+1), updates the counters as the reference does and returns the
 * emitted count (or -1). */
int32_t or_spec_step(const or_model* target, or_kv* tkv, const or_model* draft, or_kv* dkv,
                     const uint32_t* tokens, int32_t len, int32_t* computed, int32_t* draft_computed,
                     const uint32_t* blocks, int32_t n_blocks, const uint32_t* draft_blocks,
                     int32_t n_draft_blocks, int32_t k, uint32_t* out, int32_t* accepted);

#ifdef __cplusplus
}
#endif
#endif
