// Persistent forward of one sequence's t <= 4 new rows through a whole model
// (greedy): a draft round of the speculative step (Engine::propose,
// src/engine.rs:658-717, each round one Model::forward with Logits::Last,
// src/model.rs:269-362, then sampler::argmax, src/sampler.rs:42-51), or the
// target's verify pass over [last, d_1 .. d_k] with the greedy accept
// (src/engine.rs:563-616).
//
// As separate kernels, a layer of a batch-1 step is six dependent launches of
// 2.6 to 21 MB each, and every launch pays a kernel boundary plus the ramp of
// its first loads: a 2.6 MB read takes about 6 us as a kernel of its own on
// MI355X. Here one launch of one 512-thread workgroup per CU runs every stage,
// and the stages meet at grid barriers. What makes the difference is the order
// within a workgroup: it signals that its outputs are stored, then requests
// the weights of its next stage (or the cached keys and values of its next
// attention span), and only then waits for the barrier. The weight stream of
// the next stage is in flight while the barrier completes.
//
// Barriers: 32 counters per barrier, 1 KiB apart; workgroup g adds 1 to
// counter g % 32 (agent scope) once its stores have completed, and wave 0 of
// every waiting workgroup polls the 32 counters until each holds epoch x (its
// number of workgroups). One counter for all 256 workgroups serializes the
// atomics (3.8 us per barrier); 32 counters take 1.5 us. Counters only ever
// grow: barrier b of launch e is complete when its counters reach e times
// their workgroup counts, and the last workgroup to finish a launch advances
// the epoch. Every wait is bounded: past a.spin polls the workgroup raises
// the abort flag, which every wait also watches; the host then reports the
// step as failed and clears the counters.
//
// Stages of layer l (barrier indices 6l + 0..5 follow each):
//   QKV   x_b = embed (l = 0) or x_a + sum of down partials; its slice is
//         stored (xb); [q k v] = ((attn_norm (.) x_b) W_qkv^T) * rinv(x_b) (+ bias),
//         partial over the unit's K slice
//   ATTN  item (kv head, span of blocks): RoPE of the queries and new keys, the
//         new keys/values into their cache slots, per query the span's max
//         score, sum of exponentials and weighted values
//   MERGE one (row, query head) per wave: the spans merged (the attention output)
//   O     o = att W_o^T, partial over the unit's K slice
//   GU    x_a = x_b + sum of o partials (its slice stored, xa);
//         act = silu(g rinv(x_a)) * (u rinv(x_a)), [g u] = (mlp_norm (.) x_a) W_gu^T
//   DOWN  d = act W_down^T, partial over the unit's K slice
// then LM: x = x_a + sum of d partials, final norm, lm_head tiles, the
// workgroup's (max, first index) per selected row; the argmax over the
// workgroups (workgroup 0) and, for a verify, the accepted prefix.
//
// Exchange buffers take fresh addresses per layer and stage, are written with
// agent-scope (write-through) stores and read with plain loads after the
// barrier that follows their writes, so the 32 workgroups of an XCD share one
// L2 copy of each input; no line is read in a launch before it is written.
//
// The GEMV arithmetic is k_gemv's: pieces of the input in the MFMA A layout
// (four int8 pieces with a power-of-two block scale for quantized weights,
// four bf16 pieces for bf16 weights), v_mfma_i32_16x16x32_i8 or
// v_mfma_f32_16x16x32_bf16, the group scale applied per k-block.
#include "devutil.h"
#include "pfwd.h"

namespace fg {

namespace {

constexpr int NW = kPfWaves, NTHR = kPfThreads, HD = 64, HALF = HD / 2;
constexpr int PB = 1;      // attention blocks per wave whose keys/values are requested before the barrier (two spill)
constexpr int PSZ = 68;    // floats of an attention partial: max, sum, 0, 0, weighted values
constexpr int MQ = kPfMaxRows * kPfMaxGqa;  // queries of an attention item at most
constexpr int YS = 16 * kPfMaxNtg;          // row stride of a unit's products (yt)

template <int KIND>
struct Tr {
    static constexpr bool Q = KIND != BF16;
    static constexpr int WQ = KIND == INT4 ? 1 : KIND == INT8 ? 2 : 4;  // 16-byte words per lane per (tile, chunk)
    static constexpr int R = KIND == BF16 ? 4 : 8;                       // (tile, chunk) pairs per wave per round
    static constexpr bool NT = KIND != BF16;  // quantized weights are read once per step: non-temporal
};

template <int KIND>
struct Wreg {
    u32x4 w[Tr<KIND>::R][Tr<KIND>::WQ];
    float s[Tr<KIND>::R];
};

struct Sh {
    float* xf;     // [4][xk] staged f32 input rows
    uint8_t* pa;   // pieces [kb][64 lanes][8 int8 or 8 bf16]
    float* pxs;    // int8 block scales [kb][4 rows]
    float* red;    // [NW][kPfMaxNtg][64] products of each wave
    float* yt;     // [4][YS] products of a unit
    float* misc;   // [0..3] 1/rms of the rows, [8..15] row sums of squares by half
    int* flag;     // [0] abort seen, [1] epoch
    // attention (aliases xf / pa)
    float* qs;     // [MQ][64]
    float* kn;     // [4][64]
    float* vn;     // [4][64]
    float* wred;   // [NW][MQ][PSZ]
};

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// write-through store: visible to every XCD once complete
__device__ __forceinline__ void st_x(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned* counter(const PfArgs& a, int b, int c) {
    return a.bar + ((size_t)b * kPfCounters + c) * kPfCounterWords;
}

// This workgroup has finished barrier b's stage: its stores have completed
// (every wave waits for them), then one arrival.
__device__ __forceinline__ void arrive(const PfArgs& a, int b) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(counter(a, b, blockIdx.x % kPfCounters), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until workgroups 0 .. G - 1 have arrived at barrier b (wave 0 polls;
// the other waves wait at the workgroup barrier, their loads still in flight).
// False in every thread when the launch was aborted.
__device__ __forceinline__ bool wait_bar(const PfArgs& a, int b, unsigned epoch, const Sh& sh, int G) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const unsigned want = lane < kPfCounters ? epoch * (unsigned)((G - lane + kPfCounters - 1) / kPfCounters) : 0u;
        const unsigned* p = lane < kPfCounters ? counter(a, b, lane) : a.ctl + kPfCtlAbort;
        int spins = 0;
        bool good = true;
        while (true) {
            const unsigned v = ld_agent(p);
            if (__any(lane >= kPfCounters && v != 0u)) {
                good = false;
                break;
            }
            if (__all(lane >= kPfCounters || v >= want)) break;
            if (++spins > a.spin) {
                if (lane == 0) __hip_atomic_store(a.ctl + kPfCtlAbort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                good = false;
                break;
            }
        }
        if (lane == 0) sh.flag[0] = good ? 0 : 1;
    }
    __syncthreads();
    return sh.flag[0] == 0;
}

// ---------------------------------------------------------------------------
// GEMV work units
// ---------------------------------------------------------------------------
struct Unit {
    int t0, nt, c0, c1;  // n-tiles t0 .. t0 + nt - 1, chunks c0 .. c1 - 1
};

__device__ __forceinline__ Unit unit_of(const PfMat& m, int u, int n_tiles) {
    const int g = u / m.ks, ks = u - g * m.ks, KC = m.kb >> 2;
    Unit U;
    U.t0 = g * m.ntg;
    U.nt = min(m.ntg, n_tiles - U.t0);
    U.c0 = ks * KC / m.ks;
    U.c1 = (ks + 1) * KC / m.ks;
    return U;
}

// This wave's pairs of round `round`: pair p = wave + NW (round R + i) of the
// unit is (tile t0 + p / nch, chunk c0 + p % nch). Loads past the unit's pairs
// re-read its last pair (valid addresses; never used).
template <int KIND, bool NT = Tr<KIND>::NT>
__device__ __forceinline__ void load_w(const PfMat& m, const Unit& U, int round, Wreg<KIND>& r) {
    constexpr int R = Tr<KIND>::R;
    const int wave = wave_id(), lane = lane_id();
    const int nch = U.c1 - U.c0, np = U.nt * nch, KC = m.kb >> 2;
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int p = min(wave + NW * (round * R + i), np - 1);
        const int tile = U.t0 + p / nch, c = U.c0 + p % nch;
        if (KIND == INT4) {
            r.w[i][0] = ld_nt<NT>((const u32x4*)m.w + ((size_t)tile * KC + c) * 64 + lane);
        } else if (KIND == INT8) {
#pragma unroll
            for (int j = 0; j < 2; j++)
                r.w[i][j] = ld_nt<NT>((const u32x4*)m.w + ((size_t)tile * (m.kb >> 1) + 2 * c + j) * 64 + lane);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                r.w[i][j] = ld_nt<NT>((const u32x4*)m.w + ((size_t)tile * m.kb + 4 * c + j) * 64 + lane);
        }
        if (Tr<KIND>::Q) r.s[i] = ld_nt<NT>(m.s + ((size_t)tile * KC + c) * 64 + (lane & 15) * 4 + (lane >> 4));
    }
}

template <int KIND>
using Acc = typename std::conditional<Tr<KIND>::Q, float, f32x4>::type;

// The MFMAs of this wave's pairs of round `round`; the pieces in LDS start at
// k-block kbb.
template <int KIND>
__device__ __forceinline__ void mma_w(const Unit& U, int round, const Wreg<KIND>& r, const Sh& sh, int kbb,
                                      Acc<KIND> (&acc)[kPfMaxNtg]) {
    constexpr int R = Tr<KIND>::R;
    const int wave = wave_id(), lane = lane_id();
    const int nch = U.c1 - U.c0, np = U.nt * nch;
    const i32x4 izero = {0, 0, 0, 0};
    const float inv128 = 0.0078125f;
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int p = wave + NW * (round * R + i);
        if (p >= np) break;
        const int ti = p / nch, kl = 4 * (U.c0 + p % nch) - kbb;
        if constexpr (Tr<KIND>::Q) {
            float svj[4];
            gather_rows(r.s[i], svj);
            long bq[4];
            if constexpr (KIND == INT4) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t w = r.w[i][0][j];
                    const uint32_t lo = (w << 4) & 0xF0F0F0F0u, hi = w & 0xF0F0F0F0u;
                    bq[j] = (long)(((uint64_t)hi << 32) | lo);
                }
            } else {
                bq[0] = (long)(((uint64_t)r.w[i][0][1] << 32) | r.w[i][0][0]);
                bq[1] = (long)(((uint64_t)r.w[i][0][3] << 32) | r.w[i][0][2]);
                bq[2] = (long)(((uint64_t)r.w[i][1][1] << 32) | r.w[i][1][0]);
                bq[3] = (long)(((uint64_t)r.w[i][1][3] << 32) | r.w[i][1][2]);
            }
            float v = 0.0f;
#pragma unroll
            for (int tt = 0; tt < kPfMaxNtg; tt++)
                if (tt == ti) v = acc[tt];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const long aq = ((const long*)sh.pa)[(kl + j) * 64 + lane];
                const float sx = sh.pxs[(kl + j) * 4 + (lane >> 4)];
                const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq, bq[j], izero, 0, 0, 0);
                float comb = fmaf((float)d[3], inv128, (float)d[2]);
                comb = fmaf(comb, inv128, (float)d[1]);
                comb = fmaf(comb, inv128, (float)d[0]);
                v = fmaf(comb, svj[j] * sx, v);
            }
#pragma unroll
            for (int tt = 0; tt < kPfMaxNtg; tt++)
                if (tt == ti) acc[tt] = v;
        } else {
            f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int tt = 0; tt < kPfMaxNtg; tt++)
                if (tt == ti) v = acc[tt];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bf16x8 ab = ((const bf16x8*)sh.pa)[(kl + j) * 64 + lane];
                bf16x8 wb;
                __builtin_memcpy(&wb, &r.w[i][j], sizeof(wb));
                v = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, wb, v, 0, 0, 0);
            }
#pragma unroll
            for (int tt = 0; tt < kPfMaxNtg; tt++)
                if (tt == ti) acc[tt] = v;
        }
    }
}

// Rounds of this wave over the unit (ceil(its pairs / R)).
template <int KIND>
__device__ __forceinline__ int rounds_of(const Unit& U) {
    const int np = U.nt * (U.c1 - U.c0), wave = wave_id();
    const int mine = np > wave ? (np - wave + NW - 1) / NW : 0;
    return (mine + Tr<KIND>::R - 1) / Tr<KIND>::R;
}

// The unit's products: `r` holds round 0 (requested earlier); the other rounds
// are requested here. Result: yt[row][16 tt + n], the sums over the waves in
// wave order (D layout: lane l holds input row l / 16, column l % 16).
template <int KIND, bool NT = Tr<KIND>::NT>
__device__ __forceinline__ void gemv_unit(const PfMat& m, const Unit& U, Wreg<KIND>& r, const Sh& sh, int kbb) {
    Acc<KIND> acc[kPfMaxNtg];
#pragma unroll
    for (int tt = 0; tt < kPfMaxNtg; tt++) {
        if constexpr (Tr<KIND>::Q)
            acc[tt] = 0.0f;
        else
            acc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const int nr = rounds_of<KIND>(U);
    for (int rd = 0; rd < nr; rd++) {
        if (rd > 0) load_w<KIND, NT>(m, U, rd, r);
        mma_w<KIND>(U, rd, r, sh, kbb, acc);
    }
    const int wave = wave_id(), lane = lane_id();
#pragma unroll
    for (int tt = 0; tt < kPfMaxNtg; tt++) {
        if (tt < U.nt) {
            float v;
            if constexpr (Tr<KIND>::Q)
                v = acc[tt];
            else
                v = ((acc[tt][0] + acc[tt][1]) + acc[tt][2]) + acc[tt][3];
            sh.red[(wave * kPfMaxNtg + tt) * 64 + lane] = v;
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < U.nt * 64; idx += NTHR) {
        const int tt = idx >> 6, l = idx & 63;
        float v = 0.0f;
        for (int w = 0; w < NW; w++) v += sh.red[(w * kPfMaxNtg + tt) * 64 + l];
        sh.yt[(l >> 4) * YS + tt * 16 + (l & 15)] = v;
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Inputs
// ---------------------------------------------------------------------------
// xf[r][k - kx0] = the sum of the sources (rows of ld floats; null ones are
// skipped, each source added in order) at rows r < t, columns kx0 .. kx1 - 1.
// Every load of a thread is requested before any is used: a pass covers
// MV float4 per thread (rows past t are never read by the consumers of xf).
constexpr int MV = 4;
constexpr int MS = 3;  // sources at most: a residual and two K-slice partials (the host splits o and down in two at most)
__device__ __forceinline__ void stage_rows(const Sh& sh, int xk, int t, int kx0, int kx1, int ld,
                                           const float* const (&src)[MS]) {
    const int n4 = (kx1 - kx0) >> 2, tot = t * n4;
    for (int b = 0; b < tot; b += MV * NTHR) {
        float4 acc[MV];
#pragma unroll
        for (int u = 0; u < MV; u++) acc[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int si = 0; si < MS; si++) {
            if (!src[si]) continue;
            float4 v[MV];
#pragma unroll
            for (int u = 0; u < MV; u++) {
                const int idx = min(b + (int)threadIdx.x + u * NTHR, tot - 1), r = idx / n4;
                v[u] = *(const float4*)(src[si] + (size_t)r * ld + kx0 + 4 * (idx - r * n4));
            }
#pragma unroll
            for (int u = 0; u < MV; u++) {
                if (si == 0) {
                    acc[u] = v[u];
                } else {
                    acc[u].x += v[u].x, acc[u].y += v[u].y, acc[u].z += v[u].z, acc[u].w += v[u].w;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < MV; u++) {
            const int idx = b + (int)threadIdx.x + u * NTHR;
            if (idx < tot) {
                const int r = idx / n4;
                *(float4*)&sh.xf[r * xk + 4 * (idx - r * n4)] = acc[u];
            }
        }
    }
}

// The staged sum x = src + the ks partials of a split GEMV (ks 0: src alone;
// rows of ld floats, partial i at part + i * 4 * ld), columns kx0 .. kx1 - 1.
__device__ __forceinline__ void stage_partials(const Sh& sh, int xk, int t, int kx0, int kx1, int ld,
                                               const float* src0, const float* part, int ks) {
    const size_t st = (size_t)4 * ld;
    const float* src[MS] = {src0, ks > 0 ? part : nullptr, ks > 1 ? part + st : nullptr};
    stage_rows(sh, xk, t, kx0, kx1, ld, src);
}

// xf[r][k] = embed[tok[r]][k] for r < t (zero rows past t).
__device__ __forceinline__ void stage_embed(const PfArgs& a, const Sh& sh, int t) {
    const int H = a.H, n4 = H >> 2, tot = t * n4;
    for (int b0 = 0; b0 < tot; b0 += MV * NTHR) {
        uint2 e[MV];
#pragma unroll
        for (int u = 0; u < MV; u++) {
            const int idx = min(b0 + (int)threadIdx.x + u * NTHR, tot - 1), r = idx / n4;
            e[u] = *(const uint2*)(a.embed + (size_t)a.tok[(size_t)r * a.tok_stride] * H + 4 * (idx - r * n4));
        }
#pragma unroll
        for (int u = 0; u < MV; u++) {
            const int idx = b0 + (int)threadIdx.x + u * NTHR;
            if (idx < tot) {
                const int r = idx / n4;
                *(float4*)&sh.xf[r * a.xk + 4 * (idx - r * n4)] =
                    make_float4(bf16_bits_to_f32(e[u].x & 0xFFFFu), bf16_bits_to_f32(e[u].x >> 16),
                                bf16_bits_to_f32(e[u].y & 0xFFFFu), bf16_bits_to_f32(e[u].y >> 16));
            }
        }
    }
}

// Stores columns [w cw, (w + 1) cw) of the staged rows (cw = ceil(K / n)) to dst [4][K].
__device__ __forceinline__ void store_slice(const Sh& sh, int xk, int t, int K, int w, int n, float* dst) {
    const int cw = (K + n - 1) / n, c0 = w * cw;
    for (int idx = threadIdx.x; idx < t * cw; idx += NTHR) {
        const int r = idx / cw, c = c0 + idx - r * cw;
        if (c < K) st_x(dst + (size_t)r * K + c, sh.xf[r * xk + c]);
    }
}

// A norm weight's values for this thread: g[tid + NTHR i] (K <= MG NTHR),
// requested before the barrier (they do not depend on it).
constexpr int MG = 8;
struct Gpre {
    float g[MG];
};
__device__ __forceinline__ void load_g(const float* __restrict__ g, int K, Gpre& gp) {
#pragma unroll
    for (int i = 0; i < MG; i++) gp.g[i] = g[min((int)threadIdx.x + NTHR * i, K - 1)];
}

// 1/rms of the staged rows (full rows of K) into misc[0..3], then the rows
// multiplied by g in place. Thread j takes columns j + NTHR i of every row;
// each row's sum runs over the thread's columns in order, then a fixed tree
// over the wave and the waves in order.
__device__ __forceinline__ void rms_scale(const Sh& sh, int xk, int t, int K, const Gpre& gp, float eps) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < MG; i++) {
        const int k = threadIdx.x + NTHR * i;
        if (k < K) {
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (r < t) {
                    const float v = sh.xf[r * xk + k];
                    s[r] = fmaf(v, v, s[r]);
                    sh.xf[r * xk + k] = gp.g[i] * v;
                }
        }
    }
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float v = group_reduce<64, false>(s[r]);
        if ((threadIdx.x & 63) == 0) sh.red[wave * 4 + r] = v;
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        float v = 0.0f;
        for (int w = 0; w < NW; w++) v += sh.red[w * 4 + threadIdx.x];
        sh.misc[threadIdx.x] = (int)threadIdx.x < t ? 1.0f / sqrtf(v / (float)K + eps) : 0.0f;
    }
    __syncthreads();
}

// The pieces of one lane's eight inputs v (k_gemv's A operand; PK BF16: four
// bf16 pieces, 16 bytes; INT8: four int8 pieces at the block exponent e,
// 8 bytes). Called by a whole wave: the int8 exponent is reduced over the
// lanes l, l^16, l^32, l^48 that hold the row's 32 inputs.
template <int PK>
__device__ __forceinline__ void kb_pieces(const float (&v)[8], int piece, u32x4& ob, uint64_t& oi, int& e) {
    if (PK == BF16) {
        u16x8 o;
#pragma unroll
        for (int s = 0; s < 8; s++) o[s] = (uint16_t)bf16_piece(v[s], piece);
        __builtin_memcpy(&ob, &o, sizeof(ob));
        e = 0;
    } else {
        float mx = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; s++) mx = fmaxf(mx, fabsf(v[s]));
        e = int8_block_exp(mx);
        i8x8 o;
#pragma unroll
        for (int s = 0; s < 8; s++) o[s] = (int8_t)int8_piece(v[s], e, piece);
        __builtin_memcpy(&oi, &o, sizeof(oi));
    }
}

// Pieces of the staged rows for k-blocks kb0 .. kb1 - 1, stored from local
// k-block 0; xf's column 0 is input kx0; inputs past K and rows past t are
// zero. One wave per k-block, two k-blocks in flight per wave (independent
// chains the scheduler interleaves).
template <int PK>  // BF16 or INT8 pieces
__device__ __forceinline__ void build_pieces(const Sh& sh, int xk, int kx0, int K, int kb0, int kb1, int t) {
    const int wave = wave_id(), lane = lane_id();
    const int c = lane & 15, row = c >> 2, piece = c & 3, q = lane >> 4;
    for (int kbA = kb0 + wave; kbA < kb1; kbA += 2 * NW) {
        const int kbB = kbA + NW;
        const bool hasB = kbB < kb1;  // uniform
        float va[8], vb[8];
        const int ka = kbA * 32 + q * 8, kbq = kbB * 32 + q * 8;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            va[s] = (row < t && ka + s < K) ? sh.xf[row * xk + (ka + s - kx0)] : 0.0f;
            vb[s] = (hasB && row < t && kbq + s < K) ? sh.xf[row * xk + (kbq + s - kx0)] : 0.0f;
        }
        u32x4 oba, obb;
        uint64_t oia, oib;
        int ea, eb;
        kb_pieces<PK>(va, piece, oba, oia, ea);
        kb_pieces<PK>(vb, piece, obb, oib, eb);
        if (PK == BF16) {
            ((u32x4*)sh.pa)[(kbA - kb0) * 64 + lane] = oba;
            if (hasB) ((u32x4*)sh.pa)[(kbB - kb0) * 64 + lane] = obb;
        } else {
            ((uint64_t*)sh.pa)[(kbA - kb0) * 64 + lane] = oia;
            if (hasB) ((uint64_t*)sh.pa)[(kbB - kb0) * 64 + lane] = oib;
            if (lane < 16 && (lane & 3) == 0) {
                sh.pxs[(kbA - kb0) * 4 + row] = ldexpf(1.0f, ea);
                if (hasB) sh.pxs[(kbB - kb0) * 4 + row] = ldexpf(1.0f, eb);
            }
        }
    }
}

// Slot bytes of one k-block of pieces: 64 lanes x 16 (bf16) or 8 (int8) bytes.
template <int PK>
constexpr int kb_bytes() { return PK == BF16 ? 1024 : 512; }

// A producer's pieces of k-block kb (the consumer's input, written once for
// every consumer): src[row * lds + 8 (q - q0) + s] holds input 8 q + s of the
// k-block for rows < t and input groups q0 <= q < q1 (others are zero); the
// lanes whose row lies in [r0, r1) and whose group in [q0, q1) store their
// slot (write-through) into dst [kb][64 lanes][slot], the int8 block scales
// into dxs [kb][4 rows]. Called by a whole wave.
template <int PK>
__device__ __forceinline__ void put_kb_pieces(const float* src, int lds, int t, int kb, int r0, int r1, int q0, int q1,
                                              uint8_t* dst, float* dxs) {
    const int lane = lane_id(), c = lane & 15, row = c >> 2, piece = c & 3, q = lane >> 4;
    const bool in = row < t && q >= q0 && q < q1;
    float v[8];
#pragma unroll
    for (int s = 0; s < 8; s++) v[s] = in ? src[row * lds + 8 * (q - q0) + s] : 0.0f;
    u32x4 ob;
    uint64_t oi;
    int e;
    kb_pieces<PK>(v, piece, ob, oi, e);
    if (row >= r0 && row < r1 && q >= q0 && q < q1) {
        uint64_t* d = (uint64_t*)(dst + ((size_t)kb * 64 + lane) * (PK == BF16 ? 16 : 8));
        if (PK == BF16) {
            __hip_atomic_store(d, ((uint64_t)ob[1] << 32) | ob[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(d + 1, ((uint64_t)ob[3] << 32) | ob[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            __hip_atomic_store(d, oi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (piece == 0 && q == q0) st_x(dxs + (size_t)kb * 4 + row, ldexpf(1.0f, e));
        }
    }
}

// The pieces of k-blocks kb0 .. kb0 + nkb - 1 (and their int8 block scales)
// from a producers' buffer into LDS; every load of a thread requested first.
// Zero pieces (and scales) in LDS for the k-blocks kb0 .. kb1 - 1 at or past
// kb_end (the input's padding: no producer writes them).
template <int PK>
__device__ __forceinline__ void zero_pad_pieces(const Sh& sh, int kb0, int kb1, int kb_end);

template <int PK>
__device__ __forceinline__ void load_pieces(const Sh& sh, const uint8_t* src, const float* sxs, int kb0, int nkb) {
    // global -> LDS directly (global_load_lds_dwordx4: lane l's 16 bytes land at
    // the wave's LDS base + 16 l), one 1 KiB piece of the copy per wave
    // instruction, no registers held
    const int wave = wave_id(), lane = lane_id();
    const int nkib = nkb * kb_bytes<PK>() / 1024;
    const uint8_t* s0 = src + (size_t)kb0 * kb_bytes<PK>();
    for (int i = wave; i < nkib; i += NW)
        __builtin_amdgcn_global_load_lds((const void*)(s0 + (size_t)i * 1024 + lane * 16),
                                         (__attribute__((address_space(3))) void*)(sh.pa + (size_t)i * 1024), 16, 0, 0);
    if (PK != BF16)
        for (int idx = threadIdx.x; idx < nkb * 4; idx += NTHR) sh.pxs[idx] = sxs[(size_t)kb0 * 4 + idx];
    __builtin_amdgcn_s_waitcnt(0);
}

template <int PK>
__device__ __forceinline__ void zero_pad_pieces(const Sh& sh, int kb0, int kb1, int kb_end) {
    // after the copy of load_pieces: order the zeros behind it
    __syncthreads();
    const int z0 = max(kb0, kb_end);
    const int n16 = (kb1 - z0) * kb_bytes<PK>() / 16;
    for (int idx = threadIdx.x; idx < n16; idx += NTHR)
        ((u32x4*)(sh.pa + (size_t)(z0 - kb0) * kb_bytes<PK>()))[idx] = u32x4{0u, 0u, 0u, 0u};
    if (PK != BF16)
        for (int idx = threadIdx.x; idx < (kb1 - z0) * 4; idx += NTHR) sh.pxs[(z0 - kb0) * 4 + idx] = 0.0f;
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

}  // namespace

template <int KIND>
__global__ __launch_bounds__(NTHR) void k_pfwd(const PfArgs a) {
    constexpr int PK = KIND == BF16 ? BF16 : INT8;  // pieces format of the layer matrices
    extern __shared__ __align__(16) float lds[];
    Sh sh;
    {
        // pkb covers the lm_head's bf16 pieces too (the host sizes it)
        const size_t pa_bytes = (size_t)a.pkb * (PK == BF16 ? 1024 : 512);
        sh.xf = lds;
        sh.pa = (uint8_t*)(lds + 4 * a.xk);
        sh.pxs = (float*)(sh.pa + pa_bytes);
        float* after = sh.pxs + 4 * a.pkb;
        // the attention region aliases xf, pa and pxs; it may be the larger
        sh.qs = lds;
        sh.kn = sh.qs + MQ * HD;
        sh.vn = sh.kn + 4 * HD;
        sh.wred = sh.vn + 4 * HD;
        float* att_end = sh.wred + NW * MQ * PSZ;
        if (att_end > after) after = att_end;
        sh.red = after;
        sh.yt = sh.red + NW * kPfMaxNtg * 64;
        sh.misc = sh.yt + 4 * YS;
        sh.flag = (int*)(sh.misc + 16);  // [0] abort seen, [1] epoch, [8..15] argmax tokens
    }
    const int tid = threadIdx.x, lane = tid & 63, G = gridDim.x, wg = blockIdx.x;
    const int GL = a.gl;  // workgroups 0 .. GL - 1 run the layers; all of them the lm_head
    const int t = a.t, H = a.H, I = a.I, nkv = a.nkv, GQ = a.nh / a.nkv, qd = a.qd, kvd = a.kvd;
    const int qkvd = qd + 2 * kvd;
    if (tid == 0) {
        sh.flag[1] = (int)ld_agent(a.ctl + kPfCtlEpoch);
        sh.flag[0] = ld_agent(a.ctl + kPfCtlAbort) != 0u;
    }
    __syncthreads();
    const unsigned epoch = (unsigned)sh.flag[1];
    if (sh.flag[0]) return;  // an earlier launch aborted; the host resets the words before the next step
    const int pos0 = *a.pos0, ctx = pos0 + t;
    const int nblk = (ctx + 15) >> 4;
    // attention spans per kv head: at most one block per wave when that many
    // items fit the grid, else G / nkv spans of several blocks
    int S = min(max(1, GL / nkv), (nblk + NW - 1) / NW);
    const int BPS = (nblk + S - 1) / S;
    S = (nblk + BPS - 1) / BPS;
    bool ok = true;
    const PfXch& xo = a.xo;

    for (int l = 0; l < a.L && ok && wg < GL; l++) {
        const PfLayer& Ly = a.layers[l];
        float* const X = a.x + (size_t)l * xo.layer;
        const float* const Xp = l > 0 ? X - xo.layer : nullptr;
        float* const kc = a.kc + (size_t)l * a.layer_floats;
        float* const vc = a.vc + (size_t)l * a.layer_floats;
        const int b0 = 6 * l;
        // ---- QKV
        {
            const PfMat& M = Ly.qkv;
            const int ntl = qkvd / 16;
            if (wg < M.units) {
                const Unit U = unit_of(M, wg, ntl);
                Wreg<KIND> wr;
                load_w<KIND>(M, U, 0, wr);
                Gpre gp;
                load_g(Ly.attn_norm, H, gp);
                if (l > 0 && !(ok = wait_bar(a, b0 - 1, epoch, sh, GL))) break;
                if (l == 0)
                    stage_embed(a, sh, t);
                else
                    stage_partials(sh, a.xk, t, 0, H, H, Xp + xo.xa, Xp + xo.d, a.layers[l - 1].down.ks);
                __syncthreads();
                store_slice(sh, a.xk, t, H, wg, M.units, X + xo.xb);
                __syncthreads();
                rms_scale(sh, a.xk, t, H, gp, a.eps);
                build_pieces<PK>(sh, a.xk, 0, H, 4 * U.c0, 4 * U.c1, t);
                __syncthreads();
                gemv_unit<KIND>(M, U, wr, sh, 4 * U.c0);
                const int ks = wg % M.ks, cols = U.nt * 16;
                for (int idx = tid; idx < t * cols; idx += NTHR) {
                    const int r = idx / cols, cc = idx - r * cols, col = U.t0 * 16 + cc;
                    float v = sh.yt[r * YS + cc] * sh.misc[r];
                    if (Ly.bqkv && ks == 0) v += Ly.bqkv[col];
                    st_x(X + xo.qkv + ((size_t)ks * 4 + r) * qkvd + col, v);
                }
            }
            arrive(a, b0);
        }
        // ---- ATTN: item wg = (kv head h, span sp)
        {
            const int items = nkv * S;
            if (wg < items) {
                const int h = wg / S, sp = wg - h * S;
                const int bA = sp * BPS, nb = min(nblk, bA + BPS) - bA;
                const int wave = wave_id();
                float4 kr[PB][4], vr[PB][4];
#pragma unroll
                for (int pb = 0; pb < PB; pb++) {
                    const int lb = min(wave + NW * pb, nb - 1);
                    const size_t base = ((size_t)(uint32_t)a.blocks[bA + lb] * nkv + h) * 16 * HD;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const size_t at = base + (size_t)(4 * j + (lane >> 4)) * HD + 4 * (lane & 15);
                        kr[pb][j] = ld_nt_f4(kc + at);
                        vr[pb][j] = ld_nt_f4(vc + at);
                    }
                }
                // the rotation of this thread's query / new-key pairs (at most (MQ + 4) HALF
                // of them, two per thread), also requested before the barrier
                const int Q = t * GQ;
                float rc[2], rsn[2];
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int idx = min(tid + u * NTHR, (Q + t) * HALF - 1);
                    const bool isq = idx < Q * HALF;
                    const int i = isq ? idx / HALF : (idx - Q * HALF) / HALF, d = idx % HALF;
                    const int pos = pos0 + (isq ? i / GQ : i);
                    rc[u] = a.cos_t[(size_t)pos * HALF + d];
                    rsn[u] = a.sin_t[(size_t)pos * HALF + d];
                }
                if (!(ok = wait_bar(a, b0, epoch, sh, GL))) break;
                // q / k / v of this kv head for the t rows (sums of the K-slice partials;
                // every load of a thread requested first)
                const PfMat& Mq = Ly.qkv;
                const int per = (GQ + 2) * HD;
                {
                    constexpr int MU = (kPfMaxRows * (kPfMaxGqa + 2) * HD + NTHR - 1) / NTHR;
                    float v[MU][4];
#pragma unroll
                    for (int u = 0; u < MU; u++) {
                        const int idx = min(tid + u * NTHR, t * per - 1);
                        const int r = idx / per, rem = idx - r * per, j = rem / HD, d = rem - j * HD;
                        const int col = j < GQ ? (h * GQ + j) * HD + d : j == GQ ? qd + h * HD + d : qd + kvd + h * HD + d;
#pragma unroll
                        for (int ks = 0; ks < 4; ks++)
                            v[u][ks] = X[xo.qkv + ((size_t)min(ks, Mq.ks - 1) * 4 + r) * qkvd + col];
                    }
#pragma unroll
                    for (int u = 0; u < MU; u++) {
                        const int idx = tid + u * NTHR;
                        if (idx < t * per) {
                            const int r = idx / per, rem = idx - r * per, j = rem / HD, d = rem - j * HD;
                            float x = v[u][0];
#pragma unroll
                            for (int ks = 1; ks < 4; ks++)
                                if (ks < Mq.ks) x += v[u][ks];
                            if (j < GQ)
                                sh.qs[(r * GQ + j) * HD + d] = x;
                            else if (j == GQ)
                                sh.kn[r * HD + d] = x;
                            else
                                sh.vn[r * HD + d] = x;
                        }
                    }
                }
                __syncthreads();
                // RoPE (rotate-half, src/model.rs:451-459): the queries at their row's
                // position, the new keys at theirs
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int idx = tid + u * NTHR;
                    if (idx < (Q + t) * HALF) {
                        const bool isq = idx < Q * HALF;
                        const int i = isq ? idx / HALF : (idx - Q * HALF) / HALF, d = idx % HALF;
                        float* x = isq ? sh.qs + i * HD : sh.kn + i * HD;
                        const float c = rc[u], sn = rsn[u];
                        const float x1 = x[d], x2 = x[d + HALF];
                        x[d] = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(-x2, sn));
                        x[d + HALF] = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, sn));
                    }
                }
                __syncthreads();
                // the new rows' keys and values into their cache slots (KvCache::write,
                // src/kv.rs:48-56), by the item whose span holds their block
                for (int idx = tid; idx < t * HD; idx += NTHR) {
                    const int r = idx / HD, d = idx - r * HD, p = pos0 + r, blk = p >> 4;
                    if (blk >= bA && blk < bA + nb) {
                        const size_t at = (((size_t)(uint32_t)a.blocks[blk] * nkv + h) * 16 + (p & 15)) * HD + d;
                        kc[at] = sh.kn[r * HD + d];
                        vc[at] = sh.vn[r * HD + d];
                    }
                }
                // this wave's blocks, four queries at a time: scores (lane l holds dims
                // 4 (l % 16) .. + 3 of position 4 j + l / 16 of the block), a running
                // max, sum of exponentials and weighted values per query
                const int dq = 4 * (lane & 15), pg = lane >> 4;
                for (int q0 = 0; q0 < Q; q0 += 4) {
                    const int nq = min(4, Q - q0);
                    float4 qv[4];
                    float m[4], ls[4];
                    float4 o[4];
#pragma unroll
                    for (int qi = 0; qi < 4; qi++) {
                        qv[qi] = qi < nq ? *(const float4*)&sh.qs[(q0 + qi) * HD + dq] : make_float4(0, 0, 0, 0);
                        m[qi] = -INFINITY;
                        ls[qi] = 0.0f;
                        o[qi] = make_float4(0, 0, 0, 0);
                    }
                    int pb = 0;
                    for (int lb = wave; lb < nb; lb += NW, pb++) {
                        float4 K[4], V[4];
                        static_assert(PB == 1, "one prefetched block per wave");
                        if (pb < PB) {
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                K[j] = kr[0][j];
                                V[j] = vr[0][j];
                            }
                        } else {
                            const size_t base = ((size_t)(uint32_t)a.blocks[bA + lb] * nkv + h) * 16 * HD;
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                const size_t at = base + (size_t)(4 * j + pg) * HD + dq;
                                K[j] = ld_nt_f4(kc + at);
                                V[j] = ld_nt_f4(vc + at);
                            }
                        }
                        const int pbase = (bA + lb) * 16;
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int p = pbase + 4 * j + pg;
                            if (p >= pos0 && p < ctx) {  // a new row: its rotated key and value
                                K[j] = *(const float4*)&sh.kn[(p - pos0) * HD + dq];
                                V[j] = *(const float4*)&sh.vn[(p - pos0) * HD + dq];
                            }
                        }
#pragma unroll
                        for (int qi = 0; qi < 4; qi++) {
                            if (qi >= nq) break;
                            const int lim = pos0 + (q0 + qi) / GQ;
                            float s[4];
                            float bm = -INFINITY;
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                float d = qv[qi].x * K[j].x;
                                d = fmaf(qv[qi].y, K[j].y, d);
                                d = fmaf(qv[qi].z, K[j].z, d);
                                d = fmaf(qv[qi].w, K[j].w, d);
                                d = group_reduce<16, false>(d);
                                const int p = pbase + 4 * j + pg;
                                s[j] = p <= lim ? d * a.scale : -INFINITY;
                                bm = fmaxf(bm, s[j]);
                            }
                            bm = reduce_rows<true, true>(bm);
                            const float nm = fmaxf(m[qi], bm);
                            if (nm == -INFINITY) continue;
                            const float f = m[qi] == -INFINITY ? 0.0f : dev_exp(m[qi] - nm);
                            ls[qi] *= f;
                            o[qi].x *= f, o[qi].y *= f, o[qi].z *= f, o[qi].w *= f;
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                const float e = s[j] == -INFINITY ? 0.0f : dev_exp(s[j] - nm);
                                ls[qi] += e;
                                o[qi].x = fmaf(e, V[j].x, o[qi].x);
                                o[qi].y = fmaf(e, V[j].y, o[qi].y);
                                o[qi].z = fmaf(e, V[j].z, o[qi].z);
                                o[qi].w = fmaf(e, V[j].w, o[qi].w);
                            }
                            m[qi] = nm;
                        }
                    }
                    // sums over the four position groups; lanes 0..15 publish the wave's
                    // partial of each query
#pragma unroll
                    for (int qi = 0; qi < 4; qi++) {
                        if (qi >= nq) break;
                        const float L = reduce_rows<false, true>(ls[qi]);
                        const float ox = reduce_rows<false, true>(o[qi].x), oy = reduce_rows<false, true>(o[qi].y);
                        const float oz = reduce_rows<false, true>(o[qi].z), ow = reduce_rows<false, true>(o[qi].w);
                        float* wr = sh.wred + (wave * MQ + q0 + qi) * PSZ;
                        if (lane < 16) *(float4*)&wr[4 + dq] = make_float4(ox, oy, oz, ow);
                        if (lane == 0) {
                            wr[0] = m[qi];
                            wr[1] = L;
                        }
                    }
                }
                __syncthreads();
                // the waves' partials merged in wave order: the item's partial per query
                float* part = X + xo.part;
                for (int idx = tid; idx < Q * HD; idx += NTHR) {
                    const int q = idx >> 6, d = idx & 63;
                    float M = -INFINITY, L = 0.0f, O = 0.0f;
                    for (int w = 0; w < NW; w++) {
                        const float* wr = sh.wred + (w * MQ + q) * PSZ;
                        const float mw = wr[0];
                        if (mw == -INFINITY) continue;
                        const float nM = fmaxf(M, mw);
                        const float fo = M == -INFINITY ? 0.0f : dev_exp(M - nM), fn = dev_exp(mw - nM);
                        L = fmaf(wr[1], fn, L * fo);
                        O = fmaf(wr[4 + d], fn, O * fo);
                        M = nM;
                    }
                    const int r = q / GQ, j = q - r * GQ;
                    float* dst = part + (((size_t)wg * 4 + r) * GQ + j) * PSZ;
                    if (d == 0) {
                        st_x(dst, M);
                        st_x(dst + 1, L);
                    }
                    st_x(dst + 4 + d, O);
                }
            }
            arrive(a, b0 + 1);
        }
        // ---- MERGE: (row r, query head qh) per wave
        {
            const int n = t * a.nh;
            if (wg * NW < n) {
                if (!(ok = wait_bar(a, b0 + 1, epoch, sh, GL))) break;
                const int i = wg * NW + wave_id();
                if (i < n) {
                    const int r = i / a.nh, qh = i - r * a.nh, h = qh / GQ, j = qh - h * GQ;
                    const float* part = X + xo.part;
                    float M = -INFINITY, L = 0.0f, O = 0.0f;
                    constexpr int MB = 8;
                    for (int s0 = 0; s0 < S; s0 += MB) {
                        float mv[MB], lv[MB], ov[MB];
#pragma unroll
                        for (int u = 0; u < MB; u++) {
                            const int sp = min(s0 + u, S - 1);
                            const float* src = part + ((((size_t)h * S + sp) * 4 + r) * GQ + j) * PSZ;
                            mv[u] = src[0];
                            lv[u] = src[1];
                            ov[u] = src[4 + lane];
                        }
#pragma unroll
                        for (int u = 0; u < MB; u++) {
                            if (s0 + u >= S || mv[u] == -INFINITY) continue;
                            const float nM = fmaxf(M, mv[u]);
                            const float fo = M == -INFINITY ? 0.0f : dev_exp(M - nM), fn = dev_exp(mv[u] - nM);
                            L = fmaf(lv[u], fn, L * fo);
                            O = fmaf(ov[u], fn, O * fo);
                            M = nM;
                        }
                    }
                    // the o projection's pieces of this row's two k-blocks of the head
                    float* wb = sh.red + wave_id() * 64;
                    wb[lane] = O / L;
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                    for (int hh = 0; hh < 2; hh++)
                        put_kb_pieces<PK>(wb + 32 * hh, 0, t, 2 * qh + hh, r, r + 1, 0, 4, (uint8_t*)(X + xo.opa),
                                          X + xo.oxs);
                }
            }
            arrive(a, b0 + 2);
        }
        // ---- O: partial products of the attention output
        {
            const PfMat& M = Ly.o;
            if (wg < M.units) {
                const Unit U = unit_of(M, wg, H / 16);
                Wreg<KIND> wr;
                load_w<KIND>(M, U, 0, wr);
                if (!(ok = wait_bar(a, b0 + 2, epoch, sh, GL))) break;
                load_pieces<PK>(sh, (const uint8_t*)(X + xo.opa), X + xo.oxs, 4 * U.c0, 4 * (U.c1 - U.c0));
                zero_pad_pieces<PK>(sh, 4 * U.c0, 4 * U.c1, qd / 32);
                __syncthreads();
                gemv_unit<KIND>(M, U, wr, sh, 4 * U.c0);
                const int ks = wg % M.ks, cols = U.nt * 16;
                for (int idx = tid; idx < t * cols; idx += NTHR) {
                    const int r = idx / cols, cc = idx - r * cols;
                    st_x(X + xo.o + ((size_t)ks * 4 + r) * H + U.t0 * 16 + cc, sh.yt[r * YS + cc]);
                }
            }
            arrive(a, b0 + 3);
        }
        // ---- GU: x_a, its norm, gate/up and SiLU
        {
            const PfMat& M = Ly.gu;
            if (wg < M.units) {
                const Unit U = unit_of(M, wg, 2 * I / 16);
                Wreg<KIND> wr;
                load_w<KIND>(M, U, 0, wr);
                Gpre gp;
                load_g(Ly.mlp_norm, H, gp);
                if (!(ok = wait_bar(a, b0 + 3, epoch, sh, GL))) break;
                stage_partials(sh, a.xk, t, 0, H, H, X + xo.xb, X + xo.o, Ly.o.ks);
                __syncthreads();
                store_slice(sh, a.xk, t, H, wg, M.units, X + xo.xa);
                __syncthreads();
                rms_scale(sh, a.xk, t, H, gp, a.eps);
                build_pieces<PK>(sh, a.xk, 0, H, 4 * U.c0, 4 * U.c1, t);
                __syncthreads();
                gemv_unit<KIND>(M, U, wr, sh, 4 * U.c0);
                // [gate il channels | up il channels] of the unit's 2 il rows: the
                // activation of il channels, then the down projection's pieces of them
                // (a whole k-block for il 32, half of one for il 16)
                const int il = a.il, ng = U.nt * 16 / (2 * il);  // interleave groups of the unit
                for (int idx = tid; idx < ng * 4 * il; idx += NTHR) {
                    const int j = idx / (4 * il), r = (idx / il) & 3, c = idx % il;
                    const float gt = sh.yt[r * YS + j * 2 * il + c] * sh.misc[r];
                    const float up = sh.yt[r * YS + j * 2 * il + il + c] * sh.misc[r];
                    sh.xf[idx] = r < t ? gt / (1.0f + dev_exp(-gt)) * up : 0.0f;
                }
                __syncthreads();
                const int wave = wave_id();
                if (wave < ng) {
                    const int ch0 = (U.t0 * 16 + wave * 2 * il) / 2;
                    const int q0 = il == 32 ? 0 : 2 * ((ch0 >> 4) & 1);
                    put_kb_pieces<PK>(sh.xf + wave * 4 * il, il, t, ch0 >> 5, 0, 4, q0, q0 + il / 8,
                                      (uint8_t*)(X + xo.dpa), X + xo.dxs);
                }
            }
            arrive(a, b0 + 4);
        }
        // ---- DOWN: partial products of the activation
        {
            const PfMat& M = Ly.down;
            if (wg < M.units) {
                const Unit U = unit_of(M, wg, H / 16);
                Wreg<KIND> wr;
                load_w<KIND>(M, U, 0, wr);
                if (!(ok = wait_bar(a, b0 + 4, epoch, sh, GL))) break;
                load_pieces<PK>(sh, (const uint8_t*)(X + xo.dpa), X + xo.dxs, 4 * U.c0, 4 * (U.c1 - U.c0));
                zero_pad_pieces<PK>(sh, 4 * U.c0, 4 * U.c1, I / 32);
                __syncthreads();
                gemv_unit<KIND>(M, U, wr, sh, 4 * U.c0);
                const int ks = wg % M.ks, cols = U.nt * 16;
                for (int idx = tid; idx < t * cols; idx += NTHR) {
                    const int r = idx / cols, cc = idx - r * cols;
                    st_x(X + xo.d + ((size_t)ks * 4 + r) * H + U.t0 * 16 + cc, sh.yt[r * YS + cc]);
                }
            }
            arrive(a, b0 + 5);
        }
    }
    if (!ok) return;
    // ---- LM: final norm of the last layer's output, lm_head tiles [tA, tB) of
    // this workgroup in units of four, (max, first index) per selected row
    const int bl = 6 * a.L;
    {
        const int ntl = a.V / 16, tpw = (ntl + G - 1) / G, tA = min(ntl, wg * tpw), tB = min(ntl, tA + tpw);
        const int r0 = t - a.logits_rows;
        PfMat LMm;
        LMm.w = a.lm;
        LMm.s = nullptr;
        LMm.kb = a.lm_kb;
        LMm.ntg = 4;
        LMm.ks = 1;
        LMm.units = 0;
        Unit U;
        U.t0 = tA;
        U.nt = min(4, tB - tA);
        U.c0 = 0;
        U.c1 = a.lm_kb >> 2;
        const bool has = tB > tA;
        Wreg<BF16> wr;
        if (has) load_w<BF16, true>(LMm, U, 0, wr);
        Gpre gp;
        load_g(a.norm, H, gp);
        if (!(ok = wait_bar(a, bl - 1, epoch, sh, GL))) return;
        float bv = -INFINITY;  // wave r (< 4) keeps row r's best
        int bi = 0x7FFFFFFF;
        if (has) {
            const float* Xl = a.x + (size_t)(a.L - 1) * xo.layer;
            stage_partials(sh, a.xk, t, 0, H, H, Xl + xo.xa, Xl + xo.d, a.layers[a.L - 1].down.ks);
            __syncthreads();
            rms_scale(sh, a.xk, t, H, gp, a.eps);
            build_pieces<BF16>(sh, a.xk, 0, H, 0, a.lm_kb, t);
            __syncthreads();
            for (int u0 = tA; u0 < tB; u0 += 4) {
                U.t0 = u0;
                U.nt = min(4, tB - u0);
                if (u0 > tA) load_w<BF16, true>(LMm, U, 0, wr);
                gemv_unit<BF16, true>(LMm, U, wr, sh, 0);
                const int wave = wave_id();
                if (wave >= r0 && wave < t) {
                    const int r = wave;
                    const float y = sh.yt[r * YS + lane] * sh.misc[r];
                    float v = lane < U.nt * 16 ? (y != y ? -INFINITY : y) : -INFINITY;
                    int idx = lane < U.nt * 16 ? u0 * 16 + lane : 0x7FFFFFFF;
                    for (int off = 32; off >= 1; off >>= 1) {
                        const float ov = __shfl_xor(v, off);
                        const int oi = __shfl_xor(idx, off);
                        if (better(ov, oi, v, idx)) {
                            v = ov;
                            idx = oi;
                        }
                    }
                    if (better(v, idx, bv, bi)) {
                        bv = v;
                        bi = idx;
                    }
                }
                __syncthreads();
            }
        }
        const int wave = wave_id();
        if (wave < 4 && lane == 0) {
            float* dst = a.x + xo.lmb + ((size_t)wg * 4 + wave) * 2;
            st_x(dst, bv);
            st_x(dst + 1, __int_as_float(bi));
        }
    }
    arrive(a, bl);
    // ---- the argmax over the workgroups (workgroup 0): row r in wave r; then the accept
    if (wg == 0) {
        if (!(ok = wait_bar(a, bl, epoch, sh, G))) return;
        const int r0 = t - a.logits_rows, wave = wave_id();
        if (wave >= r0 && wave < t) {
            const int r = wave;
            float v = -INFINITY;
            int idx = 0x7FFFFFFF;
            for (int g0 = 0; g0 < G; g0 += 64) {
                if (g0 + lane < G) {
                    const float* src = a.x + xo.lmb + ((size_t)(g0 + lane) * 4 + r) * 2;
                    const float ov = src[0];
                    const int oi = __float_as_int(src[1]);
                    if (better(ov, oi, v, idx)) {
                        v = ov;
                        idx = oi;
                    }
                }
            }
            for (int off = 32; off >= 1; off >>= 1) {
                const float ov = __shfl_xor(v, off);
                const int oi = __shfl_xor(idx, off);
                if (better(ov, oi, v, idx)) {
                    v = ov;
                    idx = oi;
                }
            }
            if (lane == 0) {
                const uint32_t tok = idx == 0x7FFFFFFF ? 0u : (uint32_t)idx;  // all NaN: index 0, as sampler::argmax
                a.am[r - r0] = tok;
                if (a.aux) a.aux[(size_t)(r - r0) * a.aux_stride + a.aux_off] = tok;
                sh.flag[8 + r - r0] = (int)tok;
            }
        }
        __syncthreads();
        if (a.k > 0 && tid == 0) {
            // greedy accept-prefix (k_accept for one sequence): the proposals d_1 .. d_k
            // against the argmax of rows 0 .. k
            const uint32_t* d = a.vtok + 1;
            const int* am = sh.flag + 8;
            int n = 0, ac = 0;
            for (int j = 0; j < a.k; j++) {
                if ((uint32_t)am[j] == d[j]) {
                    a.out[n++] = d[j];
                    ac++;
                } else {
                    a.out[n++] = (uint32_t)am[j];
                    break;
                }
            }
            if (ac == a.k) a.out[n++] = (uint32_t)am[a.k];
            a.cnt[0] = n;
            a.acc[0] = ac;
        }
    }
    // ---- the last workgroup to finish advances the epoch for the next launch
    __syncthreads();
    if (tid == 0) {
        const unsigned done = __hip_atomic_fetch_add(a.ctl + kPfCtlDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == (unsigned)G - 1) {
            __hip_atomic_store(a.ctl + kPfCtlDone, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.ctl + kPfCtlEpoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

PfXch pfwd_xch(int kind, int L, int H, int I, int qd, int qkvd, int nkv, int gq, int ks_qkv, int ks_o, int ks_d,
               int items, int groups) {
    const size_t kbf = kind == BF16 ? 256 : 128;  // floats of pieces per k-block
    auto up = [](size_t n) { return (n + 63) / 64 * 64; };  // 256-byte boundaries
    PfXch x{};
    size_t o = 0;
    x.xb = o;
    o += up((size_t)4 * H);
    x.qkv = o;
    o += up((size_t)ks_qkv * 4 * qkvd);
    x.part = o;
    o += up((size_t)items * 4 * gq * PSZ);
    x.opa = o;
    o += up((size_t)(qd / 32 + 4) * kbf);
    x.oxs = o;
    o += up((size_t)(qd / 32 + 4) * 4);
    x.o = o;
    o += up((size_t)ks_o * 4 * H);
    x.xa = o;
    o += up((size_t)4 * H);
    x.dpa = o;
    o += up((size_t)(I / 32 + 4) * kbf);
    x.dxs = o;
    o += up((size_t)(I / 32 + 4) * 4);
    x.d = o;
    o += up((size_t)ks_d * 4 * H);
    x.layer = o;
    x.lmb = (size_t)L * o;
    x.total = x.lmb + up((size_t)groups * 4 * 2);
    (void)nkv;
    return x;
}

size_t pfwd_lds_bytes(int kind, int xk, int pkb) {
    // as k_pfwd carves it
    const size_t pa = (size_t)pkb * (kind == BF16 ? 1024 : 512);
    size_t main = (size_t)4 * xk * 4 + pa + (size_t)4 * pkb * 4;
    const size_t att = ((size_t)MQ * HD + 8 * HD + (size_t)NW * MQ * PSZ) * 4;
    if (att > main) main = att;
    return main + ((size_t)NW * kPfMaxNtg * 64 + 4 * YS + 16) * 4 + 16 * sizeof(int);
}

hipError_t pfwd_init() {
    hipError_t e = hipSuccess;
    for (const void* f : {(const void*)k_pfwd<BF16>, (const void*)k_pfwd<INT8>, (const void*)k_pfwd<INT4>}) {
        const hipError_t r = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kPfLdsMax);
        if (r != hipSuccess) e = r;
    }
    if (e != hipSuccess) (void)hipGetLastError();
    return e;
}

int pfwd_groups(int kind, int xk, int pkb) {
    int dev = 0, cus = 0, per = 0;
    const void* f = kind == BF16 ? (const void*)k_pfwd<BF16> : kind == INT8 ? (const void*)k_pfwd<INT8>
                                                                           : (const void*)k_pfwd<INT4>;
    const size_t lds = pfwd_lds_bytes(kind, xk, pkb);
    if (lds > (size_t)kPfLdsMax || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, f, NTHR, lds) != hipSuccess)
        return 0;
    return cus * per >= kPfGroups ? kPfGroups : 0;
}

void launch_pfwd(hipStream_t st, int kind, int groups, const PfArgs& a) {
    const size_t lds = pfwd_lds_bytes(kind, a.xk, a.pkb);
    if (kind == BF16)
        hipLaunchKernelGGL(k_pfwd<BF16>, dim3(groups), dim3(NTHR), lds, st, a);
    else if (kind == INT8)
        hipLaunchKernelGGL(k_pfwd<INT8>, dim3(groups), dim3(NTHR), lds, st, a);
    else
        hipLaunchKernelGGL(k_pfwd<INT4>, dim3(groups), dim3(NTHR), lds, st, a);
}

}  // namespace fg
