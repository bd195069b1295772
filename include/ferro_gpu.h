/*
 * ferro_gpu.h — C ABI of the MI355X (gfx950) speculative-decoding verify
 * path for ferrolm.
 *
 * The reference has no FFI: its seam is the internal Rust call
 * `Model::forward(&self, pool, cache: &mut KvCache, chunks: &[Chunk]) ->
 * Vec<f32>` (src/model.rs:269) and the engine's accept loop
 * (src/engine.rs:563-616). Each entry point below replaces one reference
 * interface, named at its declaration, so a Rust caller binds it with a
 * thin `extern "C"` block that mirrors this header.
 *
 * Conventions
 *  - Every function returns 0 on success and a negative FG_E_* code on
 *    failure; fg_last_error() gives the message (thread-local). Nothing
 *    aborts or unwinds across the ABI: the reference's shape `assert!`s
 *    (src/model.rs:284-287, src/kernels.rs:251-252, src/quant.rs:83-86)
 *    become FG_E_SHAPE returns.
 *  - Host pointers are borrowed for the duration of the call only.
 *  - One host thread per context. Work is queued on the context's HIP
 *    stream; calls that return results to host memory synchronise it.
 *  - Token ids are uint32, positions and counts int32, weights in the
 *    reference's formats (see fg_matrix).
 */
#ifndef FERRO_GPU_H
#define FERRO_GPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FG_OK 0
#define FG_E_ARG -1      /* null pointer or out-of-range argument */
#define FG_E_SHAPE -2    /* shapes do not fit (reference: assert! panic) */
#define FG_E_DEVICE -3   /* HIP runtime error */
#define FG_E_NOMEM -4    /* device allocation failed */

enum { FG_BF16 = 0, FG_INT8 = 1, FG_INT4 = 2 };
enum { FG_LOGITS_NONE = 0, FG_LOGITS_LAST = 1, FG_LOGITS_ALL = 2 }; /* src/model.rs:74-79 */

typedef struct fg_ctx fg_ctx;
typedef struct fg_model fg_model;
typedef struct fg_kv fg_kv;
typedef struct fg_mat fg_mat;

/* Model hyperparameters: the fields of Config (src/config.rs:21-39) the
 * forward pass reads. */
typedef struct {
    int32_t vocab, hidden, intermediate, layers, heads, kv_heads, head_dim;
    float rms_eps, rope_theta;
    int32_t rope_llama3; /* RopeScaling::Llama3 when nonzero */
    float rope_factor, rope_low_freq, rope_high_freq;
    int32_t rope_orig_max_pos;
    int32_t max_position;
    int32_t tie_embeddings;
    int32_t qkv_bias;
} fg_config;

/* One weight matrix as the reference holds it (rows x cols, y = x W^T):
 *  - FG_BF16: `bf16` row-major bf16 bit patterns (the data given to
 *    Matrix::new, src/kernels.rs:53);
 *  - FG_INT8 / FG_INT4: a QMatrix (src/quant.rs:64-76): `q` codes per
 *    32-row panel and input position (int8: one signed byte per row; int4:
 *    byte i = row i low nibble | row i+16 high nibble, each offset by 8),
 *    `s` f32 scales [panel][group of 32][32 rows].
 * The library repacks on upload into its own device layout. */
typedef struct {
    int32_t format, rows, cols, _pad;
    const uint16_t* bf16;
    const uint8_t* q;
    const float* s;
} fg_matrix;

/* One transformer layer (Layer, src/model.rs:28-38): q/k/v and gate/up
 * stacked, norms already carrying any AWQ fold (src/awq.rs:109-122). */
typedef struct {
    const float* attn_norm;
    fg_matrix wqkv;
    const float* bqkv; /* NULL unless qkv_bias */
    fg_matrix wo;
    const float* mlp_norm;
    fg_matrix w_gate_up;
    fg_matrix w_down;
} fg_layer;

/* Chunk (src/model.rs:84-89): `n` tokens at positions pos..pos+n-1 of a
 * sequence whose cache blocks are `blocks`. */
typedef struct {
    const uint32_t* tokens;
    int32_t n, pos;
    const uint32_t* blocks;
    int32_t n_blocks, logits;
} fg_chunk;

/* One sequence of a speculative step (state of Seq, src/engine.rs:150-168
 * that Engine::execute/propose read, src/engine.rs:499-717). */
typedef struct {
    const uint32_t* tail;   /* tokens[draft_computed..]: the draft's round-0 input */
    int32_t n_tail;         /* >= 1 */
    int32_t draft_pos;      /* draft_computed */
    int32_t pos;            /* computed == tokens.len() - 1 */
    const uint32_t* blocks; /* target block table (>= pos + k + 1 slots) */
    int32_t n_blocks;
    const uint32_t* draft_blocks; /* draft block table (>= pos + k slots) */
    int32_t n_draft_blocks;
} fg_spec_seq;

/* The sampling fields of SamplingParams (src/sampler.rs:8-19, :34-38):
 * temperature <= 0 is greedy; otherwise logits are divided by
 * max(temperature, 1e-5), cut to the top_k largest (0: no limit, the whole
 * vocabulary; negative values are refused with FG_E_ARG) and to the
 * shortest prefix whose probability reaches top_p (1 keeps all). */
typedef struct {
    float temperature;
    float top_p;
    int32_t top_k;
    int32_t reserved;
} fg_sampling;

/* ---- context ---------------------------------------------------------- */
/* Engine::new's device side: binds `device`, creates the stream and
 * workspace. No reference counterpart beyond Pool::new (src/pool.rs:45). */
int fg_ctx_create(int device, fg_ctx** out);
void fg_ctx_destroy(fg_ctx* ctx);
const char* fg_last_error(void);
/* Blocks until all work queued on the context has finished. */
int fg_ctx_sync(fg_ctx* ctx);

/* ---- weights ---------------------------------------------------------- */
/* The shape checks of Config::parse (src/config.rs:70-74: heads divisible by
 * kv_heads, head_dim and hidden multiples of 16) plus the device's own limits:
 * head_dim one of 16, 32, 64, 128 (the attention kernel instances), GQA group
 * at most 32 (64 below head_dim 64), hidden / intermediate / heads*head_dim /
 * vocab multiples of 32. Host-only: 0 or FG_E_SHAPE with fg_last_error().
 * fg_model_upload runs it first. */
int fg_config_check(const fg_config* cfg);
/* Model::load/random + Model::quantize output handed to the device
 * (src/model.rs:92-219). embed is vocab x hidden bf16 row-major; lm_head
 * NULL when tied (src/model.rs:263-265). */
int fg_model_upload(fg_ctx* ctx, const fg_config* cfg, const fg_layer* layers,
                    const uint16_t* embed, const float* norm,
                    const uint16_t* lm_head, fg_model** out);
/* Model::truncated (src/model.rs:237-241): the first `layers` layers of
 * `base`, sharing its device weights. `base` must outlive the result. */
int fg_model_truncated(fg_ctx* ctx, const fg_model* base, int32_t layers,
                       fg_model** out);
void fg_model_destroy(fg_model* m);
/* Device bytes of the model's weights in the reference's accounting
 * (Model::weight_bytes, src/model.rs:221-229). */
int64_t fg_model_weight_bytes(const fg_model* m);

/* ---- paged KV cache --------------------------------------------------- */
/* KvCache::new (src/kv.rs:33-44): f32 keys and values for every layer in
 * the reference layout [layer][block][kv_head][block_size][head_dim].
 * block_size must be 16 (FG_E_ARG) and head_dim 16, 32, 64 or 128
 * (FG_E_SHAPE). */
int fg_kv_create(fg_ctx* ctx, int32_t layers, int32_t kv_heads,
                 int32_t head_dim, int32_t block_size, int32_t blocks,
                 fg_kv** out);
void fg_kv_destroy(fg_kv* kv);
/* KvCache::layer (src/kv.rs:58-61): copies one layer's K and V to host
 * (each blocks*block_size*kv_heads*head_dim floats). For tests. */
int fg_kv_read(fg_ctx* ctx, const fg_kv* kv, int32_t layer, float* k_out,
               float* v_out);
/* Overwrites one layer's K and V from host. For tests and baselines. */
int fg_kv_write(fg_ctx* ctx, fg_kv* kv, int32_t layer, const float* k,
                const float* v);

/* ---- forward ---------------------------------------------------------- */
/* Model::forward (src/model.rs:269-362): runs the chunks through the
 * model, writes their keys/values into `kv` and produces the requested
 * logits rows in chunk order. logits_out (rows x vocab, may be NULL)
 * receives the logits; argmax_out (rows, may be NULL) their greedy token,
 * sampler::argmax (src/sampler.rs:42-51): first index of the maximum.
 * *rows_out (may be NULL) receives the row count. hidden_out, if not NULL,
 * receives the residual stream after the embedding and after each layer,
 * (layers+1) x tokens x hidden — the per-layer tap for parity tests. */
int fg_forward(fg_ctx* ctx, const fg_model* m, fg_kv* kv,
               const fg_chunk* chunks, int32_t n_chunks, float* logits_out,
               uint32_t* argmax_out, int32_t* rows_out, float* hidden_out);

/* The capture of Model::calibrate (src/awq.rs:38-62): Model::forward with
 * Model::record's taps (src/model.rs:312-333). Runs the chunks like
 * fg_forward (no logits rows, whatever their mode) and writes the f32
 * inputs of every layer's four projections, tokens in chunk order, layer
 * after layer: [qkv: tokens x hidden = rms_norm(x, attn_norm)]
 * [o: tokens x heads*head_dim = attention output]
 * [gate_up: tokens x hidden = rms_norm(x, mlp_norm)]
 * [down: tokens x intermediate = silu(gate) * up]. Model::record's
 * reservoir sampling runs on the host over these rows. Allocates a device
 * buffer of the output's size for the call (FG_E_NOMEM when it cannot). */
int fg_forward_capture(fg_ctx* ctx, const fg_model* m, fg_kv* kv,
                       const fg_chunk* chunks, int32_t n_chunks,
                       float* inputs_out);

/* ---- speculative step ------------------------------------------------- */
/* One greedy speculative step for n_seqs sequences, entirely on device:
 * Engine::propose's k draft rounds (src/engine.rs:658-717), the target's
 * verify pass over [last, d1..dk] (src/engine.rs:512-542, Logits::All),
 * greedy accept-prefix + bonus token (src/engine.rs:563-610). Only the
 * emitted ids cross to the host: out_tokens[s*(k+1) + j], j <
 * out_count[s]; out_accepted[s] = accepted proposals. The caller's
 * rollback is the reference's (src/engine.rs:613-615):
 * computed = pos + 1 + accepted, draft_computed = min(pos + k, pos + 1 +
 * accepted). Draft proposals never leave the device. */
int fg_spec_step(fg_ctx* ctx, const fg_model* target, fg_kv* target_kv,
                 const fg_model* draft, fg_kv* draft_kv,
                 const fg_spec_seq* seqs, int32_t n_seqs, int32_t k,
                 uint32_t* out_tokens, int32_t* out_count,
                 int32_t* out_accepted);

/* fg_spec_step whose verify pass also carries other sequences' chunks:
 * prefill chunks and plain decode rows (FG_LOGITS_NONE or FG_LOGITS_LAST,
 * host tokens), after the verify rows of the same target forward, as
 * Engine::execute runs one target pass over every plan of an engine step
 * (src/engine.rs:511-542). The chunks do not touch the draft (its cache
 * catches up in the first draft round, as in Engine::propose). Outputs as
 * fg_spec_step, plus chunk_argmax_out[i]: sampler::argmax of the i-th
 * FG_LOGITS_LAST chunk row (chunks with n > 0, in order). Greedy only
 * (sampled steps make two calls). A step with chunks launches directly,
 * without the step graphs. */
int fg_spec_step_mixed(fg_ctx* ctx, const fg_model* target, fg_kv* target_kv,
                       const fg_model* draft, fg_kv* draft_kv,
                       const fg_spec_seq* seqs, int32_t n_seqs, int32_t k,
                       const fg_chunk* chunks, int32_t n_chunks,
                       uint32_t* out_tokens, int32_t* out_count,
                       int32_t* out_accepted, uint32_t* chunk_argmax_out);

/* fg_spec_step under per-sequence sampling (Engine::propose and
 * Engine::execute with !params.greedy(), src/engine.rs:575-610, 691-700):
 * each draft round draws its proposal from sampler::distribution of the
 * draft's logits; proposal j is accepted when its draft probability q is
 * positive and a uniform draw is below min(1, p/q) under the target's
 * distribution p of verify row j; the first rejection emits a draw from
 * max(0, p - q) in token order (from p when that is empty) and ends the
 * step; k acceptances add a draw from the target's last row. rng[s] is the
 * state of sequence s's Rng (src/rng.rs:5-16; Rng::new(seed) =
 * seed * 0x9E3779B97F4A7C15 | 1), advanced on the device in the
 * reference's order and written back. Sequences with temperature <= 0 are
 * verified greedily as in fg_spec_step and draw nothing. */
int fg_spec_step_sampled(fg_ctx* ctx, const fg_model* target, fg_kv* target_kv,
                         const fg_model* draft, fg_kv* draft_kv,
                         const fg_spec_seq* seqs, int32_t n_seqs, int32_t k,
                         const fg_sampling* params, uint64_t* rng,
                         uint32_t* out_tokens, int32_t* out_count,
                         int32_t* out_accepted);

/* fg_forward whose selected rows are sampled on the device
 * (sampler::sample, src/sampler.rs:105-111; the engine's step of a prompt's
 * last chunk, src/engine.rs:549-560): params[r] and rng[r] (advanced in
 * place) belong to selected row r, tokens_out[r] receives its token. */
int fg_forward_sampled(fg_ctx* ctx, const fg_model* m, fg_kv* kv,
                       const fg_chunk* chunks, int32_t n_chunks,
                       const fg_sampling* params, uint64_t* rng,
                       uint32_t* tokens_out, int32_t* rows_out);

/* Device time in microseconds of the last fg_spec_step's phases, measured
 * with HIP events on the context stream: [0] draft rounds, [1] verify
 * (target forward + argmax + accept), [2] whole step. */
int fg_last_step_times(const fg_ctx* ctx, float* us3);

/* Per-launch device timing of the GEMV kernels (no reference counterpart:
 * the reference only has wall clocks, src/engine.rs:375,382). While on,
 * every GEMV launch on the context's stream is bracketed by HIP events;
 * fg_profile_read() synchronises, folds the finished launches into one
 * record per kernel class and returns up to `cap` records:
 * cls[i] = format*4 + (GEMV by passes of 4 rows: 1, 2 or more -> 0, 1, 2;
 * the GEMM of more than 16 rows, including its split-K finish -> 3),
 * launches[i], us[i] (summed device time), bytes[i] (summed algorithmic
 * bytes: codes + scales + activations in + outputs, per launch), flops[i]
 * (summed algorithmic flops, 2 x rows x n x k per launch).
 * Returns the record count (or a negative error). reset != 0 clears. */
int fg_profile(fg_ctx* ctx, int32_t on);
/* In-kernel timeline of the GEMV, attention, merge and split output-projection
 * launches (no reference counterpart; a measurement aid). Only a library built
 * with stamps records (python -m ferrolm_amd.build --stamps, which writes
 * libferro_gpu_stamps.so): each such launch takes the next slot in launch order,
 * starting at 0 in every fg_forward and speculative step (a step replayed from
 * a graph keeps the slots of its capture), and thread 0 of each of its first
 * 1024 workgroups stores its s_memrealtime ticks (100 MHz) at entry and at exit.
 * fg_stamps_reset synchronises and clears every slot. fg_stamps_read
 * synchronises, copies `slots` (at most 1024) slots of 1024 workgroups x
 * {entry, exit} ticks (0: no record) into ticks, and the slots' kernel labels,
 * one per line, into labels (label_cap bytes, NUL-terminated); it returns the
 * number of labelled slots. Both return FG_E_ARG in a library built without
 * stamps. */
int fg_stamps_reset(fg_ctx* ctx);
int fg_stamps_read(fg_ctx* ctx, int32_t slots, uint64_t* ticks, char* labels, int32_t label_cap);
int fg_profile_read(fg_ctx* ctx, int32_t cap, int32_t* cls, int64_t* launches,
                    double* us, double* bytes, double* flops, int32_t reset);

/* ---- single matrix (kernels::matmul, src/kernels.rs:249-275) ----------- */
int fg_mat_upload(fg_ctx* ctx, const fg_matrix* w, fg_mat** out);
void fg_mat_destroy(fg_mat* m);
/* y (m x rows) = x (m x cols) W^T (+ bias), host buffers. */
int fg_matmul(fg_ctx* ctx, const fg_mat* w, const float* x, int32_t m,
              const float* bias, float* y);
/* The same product on device-resident buffers (x_dev, y_dev device
 * pointers), queued on the context stream without synchronising; used to
 * time the GEMV kernels. */
int fg_matmul_device(fg_ctx* ctx, const fg_mat* w, const float* x_dev,
                     int32_t m, float* y_dev);
/* fg_matmul_device without allocating: no counterpart in the reference; for
 * callers that cannot allocate device memory (HIP graph capture, tight
 * serving loops). The same kernels, with the activation pieces in a static
 * 2 MiB device array (one per GPU, kept until the process ends) instead of
 * the context workspace. At most 15 rows (FG_E_SHAPE beyond), and the
 * pieces of m rows must fit the array: ceil(m / 4) x k-blocks x 1040 bytes,
 * k-blocks = ceil(cols / 32) rounded up to 4 (FG_E_SHAPE beyond). Calls
 * that overlap on one GPU share the array and race. Queued on the context
 * stream without synchronising. */
int fg_matmul_device_noalloc(fg_ctx* ctx, const fg_mat* w, const float* x_dev,
                             int32_t m, float* y_dev);

/* ---- load-time quantization on the device ------------------------------ */
/* QMatrix::quantize (src/quant.rs:78-143) on the device, bit for bit the
 * reference's codes and scales: fh_quantize's contract (ferro_host.h), host
 * buffers in and out. kind FG_INT8 or FG_INT4; rows and cols multiples of
 * 32 (else FG_E_SHAPE); importance (cols floats) may be NULL. */
int fg_quantize(fg_ctx* ctx, int32_t kind, int32_t rows, int32_t cols, const float* w,
                const float* importance, uint8_t* q, float* s);

/* What the AWQ search chose for one projection (awq::Choice,
 * src/awq.rs:24-31, without the layer name). */
typedef struct {
    float alpha;
    int32_t _pad;
    double error_plain, error_awq;
} fg_awq_choice;

/* awq::search + apply (src/awq.rs:152-217) on the device: for alpha in
 * 0, 0.1, ..., 1 the scales (mean |x|)^alpha of the m calibration rows
 * cal (m x k), the weights w (rows x k f32) quantized with their columns
 * times the scales, and the mean squared error of that projection of the
 * scaled rows against the unquantized (bf16) one; the first minimum wins.
 * Writes the chosen scales (k floats, to be folded into the producer of the
 * projection's input), the choice, and the quantized matrix (QMatrix codes
 * q and scales s, as fg_quantize). The errors and codes equal the
 * reference's bit for bit. */
int fg_awq_search(fg_ctx* ctx, int32_t kind, int32_t rows, int32_t k, const float* w,
                  int32_t m, const float* cal, float* scales, fg_awq_choice* choice,
                  uint8_t* q, float* s);

#ifdef __cplusplus
}
#endif
#endif
