// Internal declarations shared by the device kernels (kernels.hip) and the
// host side of the C ABI (api.hip). Not part of the public interface.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fg {

// ---------------------------------------------------------------------------
// Device weight layout (repacked at upload from the reference's formats).
//
// A matrix of N output rows x K inputs is cut into n-tiles of 16 rows and
// k-blocks of 32 inputs (one quantization group). K is padded with zeros to
// a multiple of 128 (4 k-blocks, a "chunk"). One n-tile x k-block is exactly
// one MFMA B-operand: lane l (0..63) holds row n = l % 16, inputs
// 8*(l/16) .. +7.
//
//   BF16: [tile][kb][lane][8 x bf16]            16 B per lane per k-block
//   INT8: [tile][kb/2][lane][2 kb x 8 x int8]   16 B per lane per 2 k-blocks
//   INT4: [tile][kb/4][lane][4 kb x 4 B]        16 B per lane per 4 k-blocks
//         each 4-byte word holds 8 codes as two's-complement nibbles; input
//         slot s of the lane sits in nibble (s < 4 ? 2s : 2(s-4)+1), so
//         (w << 4) & 0xF0F0F0F0 and w & 0xF0F0F0F0 are the slots as int8
//         holding 16 x code.
//   scales (INT8/INT4): [tile][kb/4][16 rows][4 kb] f32; INT4 scales are
//         stored divided by 16 (exact) to undo the 16 x code above.
// Each (tile, chunk) is contiguous, so a wave's 16-byte loads cover 1 KB of
// consecutive memory.
//
// Row order: the stacked gate/up matrix is stored interleaved in blocks of
// il rows (DMat::il), [gate il*c .. +il-1, up il*c .. +il-1] for c = 0.., so
// one 2*il-row output group holds the gate and up values of il intermediate
// channels. il is 32 when the down projection takes int8 pieces (their scale
// spans a whole k-block) and 16 for bf16 pieces.
// ---------------------------------------------------------------------------
enum { BF16 = 0, INT8 = 1, INT4 = 2 };
// Activation operand formats ("pieces", below): BF16 and INT8 for the GEMV
// consumers, MM for the GEMM consumers (16 rows or more).
enum { MM = 3 };

struct DMat {
    int kind = 0;
    int rows = 0, cols = 0;   // N, K (unpadded)
    int n_tiles = 0, kb = 0;  // rows/16, padded K/32 (multiple of 4)
    int il = 0;               // gate/up interleave block (0: not interleaved)
    void* w = nullptr;        // packed codes / bf16
    float* s = nullptr;       // packed scales (quantized kinds)
    size_t w_bytes = 0, s_bytes = 0;
    int64_t ref_bytes = 0;    // bytes in the reference's accounting
};

// Activation operand ("pieces"). Rows of x are taken four at a time (a
// "pass"); each row is split into four pieces so that one MFMA A-operand
// row holds one (row, piece) pair: lane l holds pair c = l % 16 (row
// 4*pass + c/4, piece c%4) at inputs 8*(l/16) .. +7 of the k-block.
//   INT8 consumers: pieces are int8 with one power-of-two scale per (row,
//     k-block): x = s * (a0 + a1/128 + a2/128^2 + a3/128^3) to 2^-29 of the
//     block's largest |x|. Layout [kb][pass][lane][8 x int8] plus scales
//     [kb][pass*4 + row-in-pass] f32.
//   BF16 consumers: x = p0 + p1 + p2 + p3 with each piece a bf16, exact to
//     f32. Layout [kb][pass][lane][8 x bf16].
//   MM (GEMM) consumers: x = hi + lo, two bf16 pieces (16 significant bits),
//     in the MFMA A-operand layout of 16 distinct rows: [kb][rt][h][lane]
//     [8 x bf16] for row tile rt = row / 16 (ceil(passes / 4) of them), h = 0
//     hi / 1 lo; lane l holds row 16 rt + l % 16, inputs 8 (l / 16) .. +7.
//     Rows past the last pass are never written (a GEMM output row depends on
//     its own input row only, and rows >= m are discarded).
struct Pieces {
    void* a = nullptr;
    float* xs = nullptr;
    int kb = 0, passes = 0;
};

// GEMV epilogues.
enum Epi {
    EPI_STORE = 0,   // y (+ bias) -> out
    EPI_QKV = 1,     // y * rinv (+ bias) -> out: the q/k/v projection of a normed input
    EPI_RESID = 2,   // x += y; sum of squares per (k-block, row); pieces of g * x for the next consumer
    EPI_SILU = 3,    // silu(gate * rinv) * (up * rinv) -> pieces for the down projection
    EPI_ARGMAX = 4,  // logits y * rinv (optionally stored) -> per 32-column tile (max, index)
    EPI_MLP = 5,     // silu(gate * rinv) * (up * rinv) of the group's channels, times their columns
                     // of the down projection, added to the residual accumulator (GemvArgs::acc)
};

// The fused MLP of a bf16 layer (EPI_MLP) leaves the down projection's output
// in a fixed-point accumulator instead of x: int64 sums of round(y * 2^kAccFrac),
// exact and so independent of the order the workgroups add in. Each workgroup
// adds into copy blockIdx.x % kAccCopies (workgroup w runs on XCD w % 8, so
// the workgroups of two XCDs share a copy); a consumer sums the copies.
// Fewer copies mean fewer bytes for the consumer, more for the atomics to
// contend on. Measured on the 135M draft (cfg2, one box): 8 copies
// 2119-2123 us of draft per step, 4: 2089-2091, 2: 2111-2113, 1: 2193-2195.
// The output projection by head (k_o_heads) adds into the other accumulator,
// which the MLP reads: there each output gets one add per head (9 for the
// 135M draft) against one per MLP workgroup (96), so one copy suffices and the
// MLP's 96 workgroups read a quarter of the bytes (kAccCopiesB; with the MLP's
// accumulator at 4: draft 1861 -> 1843 us per step, 2 copies 1854; the MLP's at
// 2 copies 1865, at 8 1841).
// Layout [copy][row (4)][acc_ld]. Range: |y| < 2^26.
constexpr int kAccCopies = 4;
constexpr int kAccCopiesB = 1;
constexpr int kAccFrac = 36;

struct GemvArgs {
    const uint8_t* W = nullptr;
    const float* S = nullptr;
    int kind = 0, N = 0, KB = 0;
    const uint8_t* XA = nullptr;  // input pieces
    const float* XS = nullptr;
    int m = 0, p_total = 0;
    int nt = 2;  // n-tiles per workgroup for STORE/QKV/RESID (1 or 2; SILU takes 2*il/16)
    int il = 0;  // gate/up interleave block of the weights (EPI_SILU)
    bool mm = false;  // inputs in the MM format: the GEMM path (64 x 64 tiles)
    // GEMM split K: partial tiles [split][m][N] (kpart_cap floats available, nullptr: no split)
    float* kpart = nullptr;
    size_t kpart_cap = 0;
    int ks = 1;
    // STORE / QKV
    float* out = nullptr;
    int ldo = 0;
    const float* bias = nullptr;
    // 1/rms of the input rows from sum-of-squares partials ss_in[tile][ss_m]
    const float* ss_in = nullptr;
    int ss_tiles = 0, ss_m = 0, hidden = 0;
    float eps = 0;
    const int32_t* rows_src = nullptr;  // local row -> row of ss_in (nullptr: identity)
    // RESID / SILU
    float* x = nullptr;
    int ldx = 0;
    float* ss_out = nullptr;        // [group][ss_m] sums of squares of each group's 16*nt columns
    const float* g_next = nullptr;  // norm weight applied to the next consumer's input (nullptr: none)
    void* pa = nullptr;             // next consumer's pieces (nullptr: none)
    float* pxs = nullptr;
    int pa_kind = 0, pa_passes = 0, pa_kb = 0;  // pa_kb: the consumer's padded k-blocks
    // SILU: the activation rows also go out in f32 ([m][ldcap], nullptr: not);
    // the calibration capture of the down projection's input
    float* cap = nullptr;
    int ldcap = 0;
    // ARGMAX
    float* logits = nullptr;
    float2* best = nullptr;
    // GEMV split K (decode steps of one pass): gsplit workgroups share each
    // output group's inputs; each stores its partial tile in gpart
    // [group][split][16 rows][16 * nt] and bumps the group's counter gcnt[32 *
    // group] (zero between launches); the last to arrive sums the partials in
    // split order and runs the epilogue.
    int gsplit = 1;
    float* gpart = nullptr;
    unsigned* gcnt = nullptr;
    // RESID with am: the input is the attention output, merged in the workgroup
    // from the span partials (AttnArgs::part / mrec) instead of read as pieces
    bool am = false;
    const float* apart = nullptr;
    const int32_t* amrec = nullptr;
    int anh = 0, ankv = 0, ahd = 0, aqm = 0;
    // Fixed-point accumulators ([copy][4][acc_ld]: kAccCopies copies of the MLP's,
    // kAccCopiesB of the output projection's) of a fused layer:
    // with ax (EPI_QKV, EPI_MLP) the input rows are x + the sum of acc's copies,
    // normed here (g_in, hidden, eps) into the operand, and stored to x_alt (not
    // to x, which the launch's other workgroups are still reading); EPI_MLP adds
    // its output into acc_out. EPI_RESID reads its residual rows from x_alt when
    // set (then writes the sum to x as always). zero: zero_n words every launch
    // clears before anything else (grid-stride), for an accumulator that a
    // later kernel adds into.
    long long* acc = nullptr;
    long long* acc_out = nullptr;
    int acc_ld = 0;
    bool ax = false;
    const float* g_in = nullptr;
    float* x_alt = nullptr;
    long long* zero = nullptr;
    int zero_n = 0;
    int stamp = -1;  // timeline slot of the launch (libraries built with stamps; -1: none)
    // EPI_MLP: the down projection (bf16, the device layout) of N2 outputs, KB2 k-blocks
    const uint8_t* W2 = nullptr;
    int N2 = 0, KB2 = 0;
};

// start/stop (optional) are recorded by the dispatch itself (hipExtLaunchKernelGGL),
// so their interval is the kernel's own execution time.
void launch_gemv(hipStream_t st, int epi, const DMat& w, const GemvArgs& a, hipEvent_t start = nullptr,
                 hipEvent_t stop = nullptr);
// The output projection of a fused bf16 layer split by query head (k_o_heads):
// a.apart / a.amrec the attention's span partials and merge records, a.anh,
// a.ankv, a.ahd, a.aqm their geometry; the product is added into a.acc_out and
// a.zero is cleared. Returns -1 (nothing launched) for a head dim without an
// instance (64 and 128 have one).
int launch_o_heads(hipStream_t st, const DMat& w, const GemvArgs& a, hipEvent_t start = nullptr,
                   hipEvent_t stop = nullptr);

void launch_pieces(hipStream_t st, int consumer_kind, const float* x, int ldx, int m, int K, const float* g,
                   const int32_t* rows_src, Pieces& out);
void launch_embed(hipStream_t st, const uint32_t* tokens, int stride, const uint16_t* embed, int m, int H,
                  const float* g, float* x, float* ss, int consumer_kind, Pieces& out);

struct AttnArgs {
    const float* qkv;  // [m][ld] q, k, v of the new rows (q and k not yet rotated)
    int ld;
    float* kc;  // layer K cache [block][kv_head][bs][hd]
    float* vc;
    const float* cos_t;
    const float* sin_t;
    // [n_wi][16] per work item: row0, nrows (the row group), crow0, cpos0 (first
    // row and position of the group's chunk; rows of a chunk hold consecutive
    // positions), p0, p1 (the span, at most 128 positions), 0, 0, then the
    // span's cache block ids (up to 8).
    // A record with nrows 0 is an unused slot.
    const int32_t* wrec;
    // [rows][4] per row: first query index within its group, the group's first
    // work item, its number of spans, 0
    const int32_t* mrec;
    float* part;  // [wi][nkv][attn_qmax(hd)][hd+4]: max score, sum of exponentials, 0, 0, weighted values
    int n_wi, nh, nkv, hd, bs;
    int ns;  // sub-spans of attn_span(hd) positions per work item (1, 2 or 4; at most 128 positions)
    float scale;
    // Long chunks at hd 64 and 128: the records are parts of items of up to 2 * (32 / G)
    // rows (p0, p1 the part's positions, word 6 the offset of the chunk's block
    // table in btab, words 7 and 8 the partial slots of the two row halves);
    // n_wi counts the partial slots, two per part.
    int flash;
    const int32_t* btab;
    int maxq = 0;  // queries of the largest row group (0: unknown, the full QM)
    int stamp = -1;  // timeline slot of the launch (libraries built with stamps; -1: none)
};
// Attention over the paged cache (RoPE, K/V write of the new rows), then the
// split merge straight into the output projection's pieces (consumer_kind < 0:
// no merge, the output projection merges the spans itself). Returns -1, and
// launches nothing, for a head dim without a kernel instance (16, 32, 64, 128).
int launch_attention(hipStream_t st, const AttnArgs& a, int m, int consumer_kind, Pieces& out);
// Calibration capture: rms_norm(x) * g of m residual rows into out [m][ldo], and
// the attention output (the spans of launch_attention merged) into out [m][ldo].
void launch_cap_norm(hipStream_t st, const float* x, int m, int H, const float* g, float eps, float* out, int ldo);
int launch_cap_merge(hipStream_t st, const AttnArgs& a, int m, float* out, int ldo);

void launch_argmax_final(hipStream_t st, const float2* best, int tiles, int rows, uint32_t* argmax_out,
                         uint32_t* aux, int aux_stride, int aux_off);
void launch_accept(hipStream_t st, const uint32_t* argmax, const uint32_t* drafts, int n_seqs, int k,
                   uint32_t* out_tokens, int32_t* out_count, int32_t* out_accepted);

// Positions per attention work item and queries per work item (rows of a
// group x GQA group), by head dim.
int attn_span(int hd);
int attn_qmax(int hd);
// Queries of a work item from which attention runs on MFMA (measured: the VALU
// loops are faster for the 3 to 5 queries of decode steps, MFMA for the 20 of
// an 8B GQA verify). Plans whose row groups reach it take work items of
// several sub-spans when the launch is large (k_attn's NS): the loads of the
// next sub-span then overlap MFMA work worth hiding them behind.
constexpr int kAttnMfmaQueries = 16;
// Workgroups (kv heads x work-item slots, empty slots included) from which a
// launch of decode-sized items (one span, at most 8 queries) takes k_attn_dec,
// the kernel that keeps keys and values in registers (measured: the 135M draft
// at 32 sequences, 3 x 576 slots, draft 4886 -> 4795 us per step; the cfg2
// draft's 3 x 32 +12 us per step; the cfg2 verify's 32 x 32 unchanged).
constexpr int kAttnDecWorkgroups = 1024;
// Positions per block of the flash attention items, and per part of an item.
constexpr int kFlashBlock(int hd) { return hd >= 128 ? 32 : 64; }
constexpr int kFlashPart = 256;

// ---------------------------------------------------------------------------
// Sampling (sampling.hip). A row's distribution is stored in the reference's
// order (tok, pr) and, for top_k 1..kSampleCap, in token order (tok_id, pr_id),
// each [row][cap], with n[row] pairs; wide rows (top_k 0 or above kSampleCap)
// keep a dense by-token copy instead of the token-ordered pairs.
// ---------------------------------------------------------------------------
constexpr int kSampleCap = 1024;

struct SampleParams {  // fg_sampling; temperature <= 0 is greedy
    float temperature, top_p;
    int32_t top_k, pad;
};

struct SampleRows {
    uint32_t* tok;
    float* pr;
    uint32_t* tok_id;
    float* pr_id;
    int* n;
    int cap;    // pairs per row: kSampleCap, or the vocabulary when any row is wide
    int vocab;
    float* dense;        // wide rows: probability by token [row][cap] (null: no wide rows)
    uint32_t* scratch;   // wide rows: the sort's ping-pong keys and values [row][4 * cap]
};
// A row is wide when it samples with top_k 0 (no limit) or above kSampleCap.
__host__ __device__ inline bool sample_wide(const SampleParams& p) {
    return p.temperature > 0.0f && (p.top_k == 0 || p.top_k > kSampleCap);
}

// distributions of `rows` logits rows (row r uses prm[r / rows_per_seq])
void launch_dist(hipStream_t st, const float* logits, int rows, int vocab, int rows_per_seq, const SampleParams* prm,
                 SampleRows& out);
// a draw from each sampled row's distribution into out[r * out_stride + out_off]
// (row r uses prm[r] and rng[r]); greedy rows are left as they are
void launch_draw(hipStream_t st, int rows, const SampleParams* prm, const SampleRows& d, uint64_t* rng, uint32_t* out,
                 int out_stride, int out_off);
// the verify of a speculative step under sampling: p holds the target's
// n_seqs*(k+1) verify rows, q the draft's k rounds ([round][seq] rows)
void launch_accept_sampled(hipStream_t st, int n_seqs, int k, const SampleParams* prm, const uint32_t* vtok,
                           const uint32_t* am, const SampleRows& p, const SampleRows& q, uint64_t* rng,
                           uint32_t* out_tokens, int32_t* out_count, int32_t* out_accepted);

// Load-time quantization and the AWQ search (quant.hip). w, imp, x are f32
// device arrays; q / s the QMatrix codes and scales (src/quant.rs:64-76).
void launch_quantize(hipStream_t st, int kind, int rows, int cols, const float* w, const float* imp, uint8_t* q,
                     float* s);
void launch_scale_cols(hipStream_t st, const float* src, int64_t n, int k, const float* s, int div, float* dst);
// kind BF16: W is wf (f32, rounded to bf16 as read); INT8/INT4: the QMatrix q, s
void launch_mm_exact(hipStream_t st, int kind, const float* x, int m, int K, const float* wf, const uint8_t* q,
                     const float* s, int rows, float* y);
// out[b] = mean over t < n of (y[b * ystride + t] - yref[t])^2, f64, summed in t order
// (n a multiple of 4, ystride of 4)
void launch_sq_err(hipStream_t st, const float* y, int64_t ystride, int count, const float* yref, int64_t n,
                   double* out);

// In-kernel timeline (a library built with -DFERRO_STAMPS): thread 0 of each
// workgroup of a launch with a slot stores its s_memrealtime entry and exit
// ticks (100 MHz) into [slot][workgroup][2]. stamps_read copies the first
// `slots` slots; both return -1 in a library built without stamps.
constexpr int kStampSlots = 1024, kStampWgs = 1024;
int stamps_read(uint64_t* out, int slots);
int stamps_clear();

}  // namespace fg
