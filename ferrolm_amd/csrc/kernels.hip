// HIP kernels for gfx950 (MI355X): the verify-path hot ops.
//
// One transformer layer is six launches: the q/k/v GEMV, attention, the
// split merge (into the output projection's operand), and the o, gate/up
// and down GEMVs. Each GEMV workgroup owns a 32- or 64-row output tile over
// the whole input, so its epilogue sees finished outputs and does the
// elementwise work of the reference in place (residual add, the RMSNorm
// sum of squares, SiLU * up) and writes the next GEMV's operand directly.
//
// Reference counterparts (Rust, /root/reference):
//   k_embed         embedding gather + first rms_norm input  src/model.rs:295-299; src/kernels.rs:597-607
//   k_gemv          kernels::matmul / quant::panels_of        src/kernels.rs:249-376; src/quant.rs:175-454
//     EPI_QKV       rms_norm scaling + qkv bias               src/kernels.rs:597-607,268-274
//     EPI_RESID     kernels::add + rms_norm's mean square     src/kernels.rs:665-669,597-607
//     EPI_SILU      kernels::silu_mul                         src/kernels.rs:650-663
//     EPI_ARGMAX    final rms_norm + lm_head + argmax         src/model.rs:338-361; src/sampler.rs:41-51
//   k_attn          rope + KvCache::write + attend            src/model.rs:314-322,395-459; src/kv.rs:48-56;
//                                                             src/kernels.rs:703-756
//   k_attn_dec      the same, decode-sized items              src/model.rs:395-459; src/kernels.rs:703-756
//   k_merge_pieces  the softmax normalisation of attend       src/kernels.rs:722-732
//   k_accept        Engine::execute greedy accept             src/engine.rs:563-616
#include "devutil.h"

#include <hip/hip_ext.h>
#include <math.h>

#include <algorithm>
#include <type_traits>

namespace fg {

// The int8 pieces layout: a lane's slots (8 bytes: pieces of 8 inputs) of the
// four k-blocks of a chunk sit together (32 bytes), so a consumer reads them in
// two 16-byte loads; the block scales 2^e likewise, [chunk][row][4 k-blocks].
// Indices in 8-byte slots and in floats.
__device__ __forceinline__ size_t i8_slot(int kb, int pass, int passes, int lane) {
    return ((((size_t)(kb >> 2) * passes + pass) * 64 + lane) << 2) + (kb & 3);
}
__device__ __forceinline__ size_t i8_scale(int kb, int passes, int row) {
    return (((size_t)(kb >> 2) * passes * 4 + row) << 2) + (kb & 3);
}

template <int CK>
__device__ __forceinline__ void write_pieces(const float (&v)[8], int kb, int pass, int passes, int row, int piece,
                                             int lane, void* out, float* xs) {
    if (CK == MM) {
        // pieces 0 and 1 of the row's 8 inputs, at its A-operand slot
        if (piece < 2) {
            const size_t at = ((((size_t)kb * ((passes + 3) >> 2) + (row >> 4)) * 2 + piece) * 64) +
                              (lane >> 4) * 16 + (row & 15);
            u16x8 o;
#pragma unroll
            for (int s = 0; s < 8; s++) o[s] = (uint16_t)bf16_piece(v[s], piece);
            ((u16x8*)out)[at] = o;
        }
        return;
    }
    const size_t slot = ((size_t)kb * passes + pass) * 64 + lane;
    if (CK == BF16) {
        u16x8 o;
#pragma unroll
        for (int s = 0; s < 8; s++) o[s] = (uint16_t)bf16_piece(v[s], piece);
        ((u16x8*)out)[slot] = o;
    } else {
        float mx = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; s++) mx = fmaxf(mx, fabsf(v[s]));
        const int e = int8_block_exp(mx);
        i8x8 o;
#pragma unroll
        for (int s = 0; s < 8; s++) o[s] = (int8_t)int8_piece(v[s], e, piece);
        ((i8x8*)out)[i8_slot(kb, pass, passes, lane)] = o;
        if (lane < 16 && (lane & 3) == 0) xs[i8_scale(kb, passes, row)] = ldexpf(1.0f, e);
    }
}

// Inputs 2*pair and 2*pair+1 of a lane's eight (x0, x1), written as their
// part of the lane's slot (4 bytes of bf16 pieces, 2 bytes of int8); mx is the
// lane's max |input| over all eight, so the int8 block scale still covers the
// row's 32 inputs. Four calls (pair 0..3, possibly from four waves) write
// exactly what one write_pieces call writes.
template <int CK>
__device__ __forceinline__ void write_pieces_pair(float x0, float x1, float mx, int pair, int kb, int pass,
                                                  int passes, int row, int piece, int lane, void* out, float* xs) {
    if (CK == MM) {
        if (piece < 2) {
            const size_t at = ((((size_t)kb * ((passes + 3) >> 2) + (row >> 4)) * 2 + piece) * 64) +
                              (lane >> 4) * 16 + (row & 15);
            ((uint32_t*)out)[at * 4 + pair] = bf16_piece(x0, piece) | (bf16_piece(x1, piece) << 16);
        }
        return;
    }
    const size_t slot = ((size_t)kb * passes + pass) * 64 + lane;
    if (CK == BF16) {
        ((uint32_t*)out)[slot * 4 + pair] = bf16_piece(x0, piece) | (bf16_piece(x1, piece) << 16);
    } else {
        const int e = int8_block_exp(mx);
        ((uint16_t*)out)[i8_slot(kb, pass, passes, lane) * 4 + pair] =
            (uint16_t)((uint8_t)int8_piece(x0, e, piece) | ((uint32_t)(uint8_t)int8_piece(x1, e, piece) << 8));
        if (pair == 0 && lane < 16 && (lane & 3) == 0) xs[i8_scale(kb, passes, row)] = ldexpf(1.0f, e);
    }
}

__device__ __forceinline__ void write_pieces_kind(int kind, const float (&v)[8], int kb, int pass, int passes,
                                                  int row, int piece, int lane, void* out, float* xs) {
    if (kind == BF16)
        write_pieces<BF16>(v, kb, pass, passes, row, piece, lane, out, xs);
    else if (kind == MM)
        write_pieces<MM>(v, kb, pass, passes, row, piece, lane, out, xs);
    else
        write_pieces<INT8>(v, kb, pass, passes, row, piece, lane, out, xs);
}

__device__ __forceinline__ void write_pieces_pair_kind(int kind, float x0, float x1, float mx, int pair, int kb,
                                                       int pass, int passes, int row, int piece, int lane, void* out,
                                                       float* xs) {
    if (kind == BF16)
        write_pieces_pair<BF16>(x0, x1, mx, pair, kb, pass, passes, row, piece, lane, out, xs);
    else if (kind == MM)
        write_pieces_pair<MM>(x0, x1, mx, pair, kb, pass, passes, row, piece, lane, out, xs);
    else
        write_pieces_pair<INT8>(x0, x1, mx, pair, kb, pass, passes, row, piece, lane, out, xs);
}

// Merge of the spans of one (row, query head, 8 dims) at input k0 of the
// attention output: the lane takes spans phase, phase + 4, ... (phase 0..3),
// and the four lanes of an aligned quad (phases 0..3 of the same row and
// inputs, all active) combine their sums in a fixed order, so all four end
// with the same bits. mr is the row's merge record (first query index, first
// work item, spans). Spans are loaded SB per round trip (load(s0), from
// clamped, always valid addresses, every load issued before any is used) and
// folded batch by batch (fold(s0)): the running sums are rescaled once per
// batch, to the batch's maximum; spans past ns are masked out.
template <int SB>
struct SpanMerge {
    const float* base;
    size_t stride;
    int ns, d0;
    float M, L, O[8];
    float2 st[SB];
    float ov[SB][8];

    __device__ __forceinline__ void init(const float* __restrict__ part, int4 mr, int nh, int nkv, int hd, int qm,
                                         int k0) {
        const int hq = k0 / hd, G = nh / nkv, h = hq / G, j = hq % G;
        d0 = k0 % hd;
        ns = mr.z;
        stride = (size_t)nkv * qm * (hd + 4);
        base = part + ((size_t)mr.y * nkv * qm + (size_t)h * qm + mr.x + j) * (hd + 4);
        M = -INFINITY;
        L = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) O[e] = 0.0f;
    }
    __device__ __forceinline__ void load(int s0) {
#pragma unroll
        for (int b = 0; b < SB; b++) {
            const float* p = base + min(s0 + 4 * b, ns - 1) * stride;
            st[b] = *(const float2*)p;
            const float4 o0 = *(const float4*)(p + 4 + d0), o1 = *(const float4*)(p + 8 + d0);
            ov[b][0] = o0.x, ov[b][1] = o0.y, ov[b][2] = o0.z, ov[b][3] = o0.w;
            ov[b][4] = o1.x, ov[b][5] = o1.y, ov[b][6] = o1.z, ov[b][7] = o1.w;
        }
    }
    __device__ __forceinline__ void fold(int s0) {
        float nM = M;
#pragma unroll
        for (int b = 0; b < SB; b++) nM = s0 + 4 * b < ns ? fmaxf(nM, st[b].x) : nM;
        const float fo = M == -INFINITY ? 0.0f : dev_exp(M - nM);
        L *= fo;
#pragma unroll
        for (int e = 0; e < 8; e++) O[e] *= fo;
#pragma unroll
        for (int b = 0; b < SB; b++) {
            const float w = s0 + 4 * b < ns && st[b].x != -INFINITY ? dev_exp(st[b].x - nM) : 0.0f;
            L = fmaf(st[b].y, w, L);
#pragma unroll
            for (int e = 0; e < 8; e++) O[e] = fmaf(ov[b][e], w, O[e]);
        }
        M = nM;
    }
    // the four lanes of the quad, in a fixed order
    __device__ __forceinline__ void finish(float (&v)[8]) {
        float MA = fmaxf(M, lane_xor1(M));
        MA = fmaxf(MA, lane_xor2(MA));
        const float f = M == -INFINITY ? 0.0f : dev_exp(M - MA);
        L *= f;
        L += lane_xor1(L);
        L += lane_xor2(L);
        const float il = 1.0f / L;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            O[e] *= f;
            O[e] += lane_xor1(O[e]);
            O[e] += lane_xor2(O[e]);
            v[e] = O[e] * il;
        }
    }
};

template <int SB>
__device__ __forceinline__ void merge_spans(const float* __restrict__ part, int4 mr, int nh, int nkv, int hd, int qm,
                                            int k0, int phase, float (&v)[8]) {
    SpanMerge<SB> sm;
    sm.init(part, mr, nh, nkv, hd, qm, k0);
    for (int s0 = phase; s0 < sm.ns; s0 += 4 * SB) {
        sm.load(s0);
        sm.fold(s0);
    }
    sm.finish(v);
}

// Pieces of g * x[rows_src[row]] (g, rows_src optional). One wave per
// (k-block, pass).
template <int CK>
__global__ __launch_bounds__(64) void k_pieces(const float* __restrict__ x, int ldx, int m, int K,
                                               const float* __restrict__ g, const int32_t* __restrict__ rows_src,
                                               void* __restrict__ out, float* __restrict__ xs, int passes) {
    const int kb = blockIdx.x, pass = blockIdx.y, lane = threadIdx.x;
    const int c = lane & 15, row = pass * 4 + (c >> 2), piece = c & 3;
    const int k0 = kb * 32 + (lane >> 4) * 8;
    float v[8];
    const bool rv = row < m;
    const int src = rv ? (rows_src ? rows_src[row] : row) : 0;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int k = k0 + s;
        float t = 0.0f;
        if (rv && k < K) {
            t = x[(size_t)src * ldx + k];
            if (g) t = g[k] * t;
        }
        v[s] = t;
    }
    write_pieces<CK>(v, kb, pass, passes, row, piece, lane, out, xs);
}

void launch_pieces(hipStream_t st, int consumer_kind, const float* x, int ldx, int m, int K, const float* g,
                   const int32_t* rows_src, Pieces& out) {
    if (m <= 0) return;
    dim3 grid(out.kb, out.passes);
    if (consumer_kind == BF16)
        hipLaunchKernelGGL(k_pieces<BF16>, grid, dim3(64), 0, st, x, ldx, m, K, g, rows_src, out.a, out.xs,
                           out.passes);
    else if (consumer_kind == MM)
        hipLaunchKernelGGL(k_pieces<MM>, grid, dim3(64), 0, st, x, ldx, m, K, g, rows_src, out.a, out.xs,
                           out.passes);
    else
        hipLaunchKernelGGL(k_pieces<INT8>, grid, dim3(64), 0, st, x, ldx, m, K, g, rows_src, out.a, out.xs,
                           out.passes);
}

// ---------------------------------------------------------------------------
// Embedding gather (x = embed[token] as f32), the sum of squares of each
// (k-block, row) for the first RMSNorm, and the first projection's pieces
// of g * x. One wave per (k-block, pass).
// ---------------------------------------------------------------------------
template <int CK>
__global__ __launch_bounds__(64) void k_embed(const uint32_t* __restrict__ tok, int stride,
                                              const uint16_t* __restrict__ E, int m, int H,
                                              const float* __restrict__ g, float* __restrict__ x,
                                              float* __restrict__ ss, void* __restrict__ out,
                                              float* __restrict__ xs, int passes) {
    const int kb = blockIdx.x, pass = blockIdx.y, lane = threadIdx.x;
    const int c = lane & 15, row = pass * 4 + (c >> 2), piece = c & 3, q = lane >> 4;
    const int k0 = kb * 32 + q * 8;
    float v[8];
    const bool rv = row < m;
    const uint16_t* e = rv ? E + (size_t)tok[(size_t)row * stride] * H : E;
#pragma unroll
    for (int s = 0; s < 8; s++) v[s] = (rv && k0 + s < H) ? bf16_bits_to_f32(e[k0 + s]) : 0.0f;
    float sq = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; s++) sq = fmaf(v[s], v[s], sq);
    sq = reduce_rows<false, true>(sq);
    if (rv && piece == 0) {
#pragma unroll
        for (int s = 0; s < 8; s++)
            if (k0 + s < H) x[(size_t)row * H + k0 + s] = v[s];
        if (q == 0 && kb * 32 < H) ss[(size_t)kb * m + row] = sq;
    }
    float gv[8];
#pragma unroll
    for (int s = 0; s < 8; s++) gv[s] = (k0 + s < H && g) ? g[k0 + s] * v[s] : v[s];
    write_pieces<CK>(gv, kb, pass, passes, row, piece, lane, out, xs);
}

void launch_embed(hipStream_t st, const uint32_t* tokens, int stride, const uint16_t* embed, int m, int H,
                  const float* g, float* x, float* ss, int consumer_kind, Pieces& out) {
    if (m <= 0) return;
    dim3 grid(out.kb, out.passes);
    if (consumer_kind == BF16)
        hipLaunchKernelGGL(k_embed<BF16>, grid, dim3(64), 0, st, tokens, stride, embed, m, H, g, x, ss, out.a,
                           out.xs, out.passes);
    else if (consumer_kind == MM)
        hipLaunchKernelGGL(k_embed<MM>, grid, dim3(64), 0, st, tokens, stride, embed, m, H, g, x, ss, out.a,
                           out.xs, out.passes);
    else
        hipLaunchKernelGGL(k_embed<INT8>, grid, dim3(64), 0, st, tokens, stride, embed, m, H, g, x, ss, out.a,
                           out.xs, out.passes);
}

// ---------------------------------------------------------------------------
// GEMV / skinny GEMM over up to 16 activation rows per workgroup (grid.z
// walks groups of 4 passes). A workgroup owns NT n-tiles (16*NT output
// rows) and the whole input: its waves split the 4-k-block chunks, keep the
// activation operand of U chunks in registers, stream the weights through
// the MFMA B-operand and reduce across waves in LDS.
//   int4/int8: v_mfma_i32_16x16x32_i8, one MFMA per (tile, k-block, pass),
//     then the group's scale: acc += (D0 + D1/128 + D2/128^2 + D3/128^3) *
//     s_w[n][kb] * s_x[row][kb].
//   bf16: v_mfma_f32_16x16x32_bf16 accumulating over k; the four pieces
//     are summed at the end.
// D layout of a 16x16 MFMA: lane l holds rows 4*(l/16)+r (r = 0..3, the
// four pieces of activation row l/16 of the pass) of column l%16 (output n).
// ---------------------------------------------------------------------------

// AM: the input is the attention output, merged by the workgroup itself from
// the span partials (instead of a separate merge kernel writing pieces):
// bf16 weights, one pass, at most 1024 inputs.
// AX: the input is the residual x plus a fixed-point accumulator (the previous
// fused stage's output), normed by the workgroup itself (sum of squares over
// the whole row, 1/rms in the epilogue, g_in as the norm weight): bf16 q/k/v
// or fused MLP, one pass, at most 1024 inputs; x + acc is stored to x_alt.
template <int KIND, int NT, int EPI, int PG, int WMAX = 8, bool AM = false, bool AX = false>
__global__ __launch_bounds__(64 * WMAX) void k_gemv(const GemvArgs a) {
    constexpr bool Q = KIND != BF16;
    // weights read once per step: quantized ones and the lm_heads (non-temporal loads)
    constexpr bool WNT = Q || EPI == EPI_ARGMAX;
    // chunks loaded ahead per wave: about 16 B x 4 per lane and tile of weights in
    // flight; with 16 waves (4 per SIMD, 128 VGPRs) half as many, the other waves
    // of the SIMD covering each one's wait
    constexpr int U = PG == 1 ? (KIND == INT4 ? 4 : NT >= 6 ? 1 : 2) / (WMAX == 16 ? 2 : 1) : 1;
    // 1/rms of the input rows from the producers' sum-of-squares partials (AX forms its own)
    constexpr bool NEED_R = (EPI == EPI_QKV || EPI == EPI_SILU || EPI == EPI_ARGMAX || EPI == EPI_MLP) && !AX;
    constexpr int YS = NT * 16 > 64 ? NT * 16 : 64;  // row stride of the output tile in LDS
    // finished output columns per group (EPI_RESID, EPI_SILU): 16 or 32, a half
    // or a whole k-block of the next consumer; EPI_MLP: its channels
    constexpr int OC = EPI == EPI_SILU || EPI == EPI_MLP ? NT * 8 : NT * 16;
    __shared__ float red[WMAX * NT * PG * 64];
    __shared__ __align__(16) float yt[16 * YS];
    __shared__ float rs[16];
    __shared__ float rtmp[16 * 17];
    __shared__ __align__(16) float et[16 * YS];  // epilogue inputs: x tile (EPI_RESID) or bias
    __shared__ __align__(16) float gs[32];       // g_next of this group's 32 columns (EPI_RESID)
    __shared__ __align__(16) float vt[16 * YS];  // finished values for the next consumer's pieces
    constexpr int AMKB = 32;  // AM: the operand of up to 32 k-blocks, [kb][lane] bf16 pieces as in global memory
    __shared__ __align__(16) u16x8 xm[AM ? AMKB * 64 : 1];
    // AX: the operand as bf16 pieces [piece][row][XPK]: a row pitch of 8 (mod 128)
    // bf16 puts the 16 (piece, row) rows of an MFMA read 4 banks apart, and
    // lanes writing consecutive inputs of one row hit consecutive banks
    constexpr int XPK = AMKB * 32 + 8;
    __shared__ __align__(16) uint16_t xp[AX ? 16 * XPK : 1];
    static_assert(!AX || (KIND == BF16 && PG == 1 && (EPI == EPI_QKV || EPI == EPI_MLP)), "AX: bf16 q/k/v or MLP of one pass");
    static_assert(EPI != EPI_MLP || (KIND == BF16 && PG == 1 && NT == 2), "EPI_MLP: bf16 gate/up of one pass");

    const Stamp stamp(a.stamp);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int tile0 = blockIdx.x * NT;
    const int pass0 = blockIdx.z * PG;

    // AM: the merge records of the (at most four) rows (uniform loads; the
    // records sit in a 64-word padded region) and the first span batch of the
    // thread's first merge item are requested before anything else, so that
    // the merge waits on nothing issued later (vector loads retire in order).
    // Rows past m take the last row's partials (valid addresses, discarded).
    constexpr int AMSB = 5;
    SpanMerge<AMSB> sm;
    int4 amr0, amr1, amr2, amr3;
    const int am_per_row = AM ? a.anh * a.ahd / 2 : 1;  // items per row: 8 inputs x 4 phases
    auto am_item = [&](int item, int& row, int& k0, int& phase) {
        row = item / am_per_row;
        const int rem = item % am_per_row;
        k0 = (rem >> 2) * 8;
        phase = rem & 3;
    };
    auto am_start = [&](int item) {
        int row, k0, phase;
        am_item(item, row, k0, phase);
        const int r = min(row, a.m - 1);
        const int4 mr = r == 0 ? amr0 : r == 1 ? amr1 : r == 2 ? amr2 : amr3;
        sm.init(a.apart, mr, a.anh, a.ankv, a.ahd, a.aqm, k0);
        sm.load(phase);
    };
    if constexpr (AM) {
        const int4* mrp = (const int4*)a.amrec;
        amr0 = mrp[0];
        amr1 = mrp[1];
        amr2 = mrp[2];
        amr3 = mrp[3];
        am_start(threadIdx.x);
    }
    const int np = min(PG, a.p_total - pass0);
    const int KB = a.KB, KC = KB >> 2;
    // split K (gridDim.y > 1): this workgroup's share of the chunks, split among its waves
    const int ks = gridDim.y, split = blockIdx.y;
    const int cs0 = split * KC / ks, cs1 = (split + 1) * KC / ks;
    const int c0 = cs0 + wave * (cs1 - cs0) / W, c1 = cs0 + (wave + 1) * (cs1 - cs0) / W;

    // 1/rms of the input rows from the producers' sum-of-squares partials
    // ss_in[tile][row]: slot (row r, j) sums tiles j, j + 16, ... The fast path
    // only issues the loads here, into registers, and folds them after the main
    // loop so that their latency hides under the weight stream.
    constexpr int RL = 8;
    const int rslots = np * 64;
    const bool rfast = rslots <= (int)blockDim.x && a.ss_tiles <= 16 * RL;
    float rv[RL];
#pragma unroll
    for (int i = 0; i < RL; i++) rv[i] = 0.0f;
    if (NEED_R) {
        if (rfast) {
            const int r = threadIdx.x >> 4, j = threadIdx.x & 15, row = pass0 * 4 + r;
            if ((int)threadIdx.x < rslots && row < a.m) {
                const int src = a.rows_src ? a.rows_src[row] : row;
#pragma unroll
                for (int i = 0; i < RL; i++)
                    if (j + 16 * i < a.ss_tiles) rv[i] = a.ss_in[(size_t)(j + 16 * i) * a.ss_m + src];
            }
        } else {
            for (int idx = threadIdx.x; idx < 256; idx += blockDim.x) {
                const int r = idx >> 4, j = idx & 15, row = pass0 * 4 + r;
                float v = 0.0f;
                if (r < np * 4 && row < a.m) {
                    const int src = a.rows_src ? a.rows_src[row] : row;
                    for (int t = j; t < a.ss_tiles; t += 16) v += a.ss_in[(size_t)t * a.ss_m + src];
                }
                rtmp[r * 17 + j] = v;
            }
        }
    }

    // epilogue inputs (the x tile of EPI_RESID, the bias), fetched now so their
    // latency hides under the main loop; element it of this thread is
    // idx = threadIdx.x + it * blockDim.x
    constexpr int COLS = NT * 16;
    constexpr int EPI_IT = (16 * COLS + 63) / 64;
    const int rows = np * 4;
    float pre[EPI_IT];
#pragma unroll
    for (int it = 0; it < EPI_IT; it++) {
        const int idx = threadIdx.x + it * blockDim.x;
        pre[it] = 0.0f;
        if (idx < rows * COLS) {
            const int r = idx / COLS, cc = idx % COLS, row = pass0 * 4 + r;
            if (EPI == EPI_RESID && row < a.m)
                pre[it] = (a.x_alt ? a.x_alt : a.x)[(size_t)row * a.ldx + blockIdx.x * OC + cc];
            if ((EPI == EPI_QKV || EPI == EPI_STORE) && a.bias) pre[it] = a.bias[tile0 * 16 + cc];
        }
    }
    float gv = 1.0f;
    if (EPI == EPI_RESID && a.g_next && threadIdx.x < OC) gv = a.g_next[blockIdx.x * OC + threadIdx.x];
    // EPI_MLP: the down projection's columns of this group's 16 channels (half
    // of k-block blockIdx.x / 2: 512 bytes of each n-tile), requested now so
    // they arrive with the gate/up weights; item i = (n-tile i / 32, lane 32 h +
    // i % 32), items past the last re-read it (unconditional loads)
    constexpr int DWI = EPI == EPI_MLP ? 4 : 1;
    u32x4 dw[DWI];
    if constexpr (EPI == EPI_MLP) {
        const int n_items = (a.N2 >> 4) * 32, kb2 = blockIdx.x >> 1, hh = blockIdx.x & 1;
#pragma unroll
        for (int it = 0; it < DWI; it++) {
            const int i = min((int)threadIdx.x + it * (int)blockDim.x, n_items - 1);
            dw[it] = ((const u32x4*)a.W2)[((size_t)(i >> 5) * a.KB2 + kb2) * 64 + 32 * hh + (i & 31)];
        }
    }

    float accq[NT][PG];
    f32x4 accb[NT][PG];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int p = 0; p < PG; p++) {
            accq[t][p] = 0.0f;
            accb[t][p] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
    const i32x4 izero = {0, 0, 0, 0};
    const float inv128 = 0.0078125f;

    // The main loop: batches of UU chunks whose loads are all issued before
    // the first MFMA. Every load is unconditional (full batches, then single
    // chunks; passes past np re-read the last one and are masked out), so no
    // register carries a possibly pending load across iterations and nothing
    // waits before the first weights are requested.
    // whether this lane's input row (row 4 pp + (lane % 16) / 4 of the A operand) is below m
    auto lane_alive = [&](int pp) { return pp * 4 + ((lane & 15) >> 2) < a.m; };
    auto chunks = [&](int c, auto uu) {
        constexpr int UU = decltype(uu)::value;
        long aq[UU][4][PG];
        bf16x8 ab[UU][4][PG];
        float sx[UU][4][PG];
        u32x4 wq[UU][NT][2];
        bf16x8 wb[UU][NT][4];
        float sv[UU][NT];  // group scale of (row lane % 16, k-block lane / 16) of the chunk
#pragma unroll
        for (int u = 0; u < UU; u++) {
            const int cc = c + u, kb = cc * 4;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int p = 0; p < PG; p++) {
                    const int pp = pass0 + (PG == 1 ? 0 : min(p, np - 1));
                    // lanes of input rows past m read row 4 pp's slot instead (the same
                    // addresses as its lanes, so no extra bytes move; those output rows
                    // are dropped): at one row, a quarter of the operand's bytes
                    const int al = lane_alive(pp) ? lane : (lane & ~12);
                    if (Q) {
                        aq[u][j][p] = ((const long*)a.XA)[i8_slot(kb + j, pp, a.p_total, al)];
                        sx[u][j][p] = a.XS[i8_scale(kb + j, a.p_total, pp * 4 + (lane >> 4))];
                    } else {
                        const size_t idx = ((size_t)(kb + j) * a.p_total + pp) * 64 + al;
                        ab[u][j][p] = ((const bf16x8*)a.XA)[idx];
                    }
                }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const size_t tile = tile0 + t;
                if (KIND == INT4) {
                    wq[u][t][0] = ld_nt<WNT>((const u32x4*)a.W + (tile * KC + cc) * 64 + lane);
                } else if (KIND == INT8) {
                    wq[u][t][0] = ld_nt<WNT>((const u32x4*)a.W + (tile * (KB >> 1) + 2 * cc) * 64 + lane);
                    wq[u][t][1] = ld_nt<WNT>((const u32x4*)a.W + (tile * (KB >> 1) + 2 * cc + 1) * 64 + lane);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        wb[u][t][j] = ld_nt<WNT>((const bf16x8*)a.W + (tile * KB + kb + j) * 64 + lane);
                }
                if (Q) sv[u][t] = ld_nt<WNT>(a.S + (tile * KC + cc) * 64 + (lane & 15) * 4 + (lane >> 4));
            }
        }
        // keep the scheduler from sinking loads of the batch below its first MFMA
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < UU; u++) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (Q) {
                    // each lane's row scales for the chunk's four k-blocks, gathered from
                    // the four 16-lane rows (one scale per lane loaded: 256 B a wave)
                    float svj[4];
                    gather_rows(sv[u][t], svj);
                    long bq[4];
                    if (KIND == INT4) {
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const uint32_t w = wq[u][t][0][j];
                            const uint32_t lo = (w << 4) & 0xF0F0F0F0u, hi = w & 0xF0F0F0F0u;
                            bq[j] = (long)(((uint64_t)hi << 32) | lo);
                        }
                    } else {
                        bq[0] = (long)(((uint64_t)wq[u][t][0][1] << 32) | wq[u][t][0][0]);
                        bq[1] = (long)(((uint64_t)wq[u][t][0][3] << 32) | wq[u][t][0][2]);
                        bq[2] = (long)(((uint64_t)wq[u][t][1][1] << 32) | wq[u][t][1][0]);
                        bq[3] = (long)(((uint64_t)wq[u][t][1][3] << 32) | wq[u][t][1][2]);
                    }
#pragma unroll
                    for (int j = 0; j < 4; j++)
#pragma unroll
                        for (int p = 0; p < PG; p++)
                            if (p < np) {
                                const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq[u][j][p], bq[j], izero, 0, 0, 0);
                                float comb = fmaf((float)d[3], inv128, (float)d[2]);
                                comb = fmaf(comb, inv128, (float)d[1]);
                                comb = fmaf(comb, inv128, (float)d[0]);
                                accq[t][p] = fmaf(comb, svj[j] * sx[u][j][p], accq[t][p]);
                            }
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
#pragma unroll
                        for (int p = 0; p < PG; p++)
                            if (p < np)
                                accb[t][p] =
                                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab[u][j][p], wb[u][t][j], accb[t][p], 0, 0, 0);
                }
            }
        }
    };
    if constexpr (AM) {
        // The weights of the wave's chunks are requested first; meanwhile every
        // thread merges (row, 8 inputs, span phase) items and writes piece
        // `phase` of the 8 merged values into xm at its operand slot (the four
        // phases of an item are its four pieces), and each wave then reads its
        // operand from xm. This is k_merge_pieces' arithmetic: the same bits
        // wherever both take a row's spans in one batch (up to 20 spans).
        static_assert(KIND == BF16 && PG == 1, "bf16 weights, one pass");
        constexpr int AMC = 1;  // chunks per wave: AMKB k-blocks are at most 8 chunks, one per wave
        const int wv = __builtin_amdgcn_readfirstlane(wave);
        const int a0 = wv * KC / W, a1 = (wv + 1) * KC / W;
        bf16x8 wm[AMC][NT][4];
#pragma unroll
        for (int u = 0; u < AMC; u++) {
            const int cc = min(a0 + u, KC - 1);
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    wm[u][t][j] = ((const bf16x8*)a.W)[((size_t)(tile0 + t) * KB + cc * 4 + j) * 64 + lane];
        }
        const int K = a.anh * a.ahd;
        // zero slots: rows past m, inputs past K
        for (int i = threadIdx.x; i < KB * 64; i += blockDim.x) {
            const int l = i & 63, row = (l & 15) >> 2, kin = (i >> 6) * 32 + (l >> 4) * 8;
            if (row >= a.m || kin >= K) xm[i] = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
        }
        // whole quads take part in every step (am_per_row and blockDim are multiples of 4)
        for (int i0 = 0; i0 < a.m * am_per_row; i0 += blockDim.x) {
            if (i0 > 0) am_start(i0 + threadIdx.x);
            int row, k0, phase;
            am_item(i0 + threadIdx.x, row, k0, phase);
            sm.fold(phase);
            for (int s0 = phase + 4 * AMSB; s0 < sm.ns; s0 += 4 * AMSB) {
                sm.load(s0);
                sm.fold(s0);
            }
            float v[8];
            sm.finish(v);
            if (row < a.m) {
                u16x8 o;
#pragma unroll
                for (int e = 0; e < 8; e++) o[e] = (uint16_t)bf16_piece(v[e], phase);
                xm[(k0 >> 5) * 64 + ((k0 & 31) >> 3) * 16 + row * 4 + phase] = o;
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < AMC; u++) {
            if (a0 + u < a1) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const u16x8 o = xm[((a0 + u) * 4 + j) * 64 + lane];
                    bf16x8 ab;
                    __builtin_memcpy(&ab, &o, sizeof(ab));
#pragma unroll
                    for (int t = 0; t < NT; t++)
                        accb[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, wm[u][t][j], accb[t][0], 0, 0, 0);
                }
            }
        }
    } else if constexpr (AX) {
        // The wave's weights first; then per item (row slot, two inputs): x + acc
        // (every copy requested before any is added; the copies sum exactly),
        // stored to x_alt by one workgroup per item, the four bf16 pieces of
        // g * (x + acc) straight into their operand slots (rows past m and
        // inputs past the row: zero), and the row's sum of squares; the rows'
        // 1/rms (the waves' sums in wave order) is needed only by the epilogue.
        // Two inputs per item spread the loads and conversions over every wave.
        const int wv = __builtin_amdgcn_readfirstlane(wave);
        const int a0 = wv * KC / W, a1 = (wv + 1) * KC / W;
        bf16x8 wm[NT][4];
        {
            const int cc = min(a0, KC - 1);
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    wm[t][j] = ((const bf16x8*)a.W)[((size_t)(tile0 + t) * KB + cc * 4 + j) * 64 + lane];
        }
        const int H = a.hidden, KP = KB * 16;  // input pairs of the padded row
        uint32_t* xw = (uint32_t*)xp;
        float sq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if (r >= a.m) break;  // uniform
            for (int kp = threadIdx.x; kp < KP; kp += blockDim.x) {
                const int k = 2 * kp;
                float v0 = 0.0f, v1 = 0.0f;
                if (k < H) {  // (H is even)
                    const float2 xv = *(const float2*)(a.x + (size_t)r * a.ldx + k);
                    constexpr int NCP = EPI == EPI_MLP ? kAccCopiesB : kAccCopies;  // the MLP reads k_o_heads' sums
                    i64x2 cv[NCP];
#pragma unroll
                    for (int c = 0; c < NCP; c++)
                        cv[c] = *(const i64x2*)(a.acc + ((size_t)c * 4 + r) * a.acc_ld + k);
                    const float2 gv = *(const float2*)(a.g_in + k);
                    long long s0 = 0, s1 = 0;
#pragma unroll
                    for (int c = 0; c < NCP; c++) {
                        s0 += cv[c][0];
                        s1 += cv[c][1];
                    }
                    const float unit = 1.0f / (float)(1ll << kAccFrac);
                    const float x0 = xv.x + (float)s0 * unit, x1 = xv.y + (float)s1 * unit;
                    if (blockIdx.x == 0) *(float2*)(a.x_alt + (size_t)r * a.ldx + k) = make_float2(x0, x1);
                    sq[r] += fmaf(x1, x1, x0 * x0);
                    v0 = gv.x * x0;
                    v1 = gv.y * x1;
                }
                // the four pieces (bf16_piece's successive roundings) of inputs k, k + 1
#pragma unroll
                for (int pc = 0; pc < 4; pc++) {
                    const uint32_t h0 = f32_to_bf16_bits(v0), h1 = f32_to_bf16_bits(v1);
                    xw[((pc * 4 + r) * XPK + k) >> 1] = h0 | (h1 << 16);
                    v0 = v0 - bf16_bits_to_f32(h0);
                    v1 = v1 - bf16_bits_to_f32(h1);
                }
            }
        }
        // rows past m: zero pieces (four 16-byte words per thread-step, consecutive)
        for (int i = threadIdx.x; i < 4 * (4 - a.m) * (KB * 4); i += blockDim.x) {
            const int pr = i / (KB * 4), kg = i - pr * (KB * 4), pc = pr & 3, r = a.m + (pr >> 2);
            *(u16x8*)&xp[(pc * 4 + r) * XPK + kg * 8] = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
        }
        // (the partials go to rtmp, which nothing else uses here: red is
        // rewritten by the waves' products while these are being summed)
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const float v = group_reduce<64, false>(sq[rr]);
            if (lane == 0) rtmp[wave * 4 + rr] = v;
        }
        __syncthreads();
        if (threadIdx.x < 4) {
            float v = 0.0f;
            for (int w = 0; w < W; w++) v += rtmp[w * 4 + threadIdx.x];
            rs[threadIdx.x] = 1.0f / sqrtf(v / (float)H + a.eps);
        }
        if (a0 < a1) {
            // lane l: piece l % 4 of row (l % 16) / 4, inputs 8 (l / 16) .. + 7 of the k-block
            const uint16_t* xl = xp + ((lane & 3) * 4 + ((lane & 15) >> 2)) * XPK + 8 * (lane >> 4);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const u16x8 o = *(const u16x8*)(xl + (a0 * 4 + j) * 32);
                bf16x8 ab;
                __builtin_memcpy(&ab, &o, sizeof(ab));
#pragma unroll
                for (int t = 0; t < NT; t++)
                    accb[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, wm[t][j], accb[t][0], 0, 0, 0);
            }
        }
    } else {
        int c = c0;
        for (; c + U <= c1; c += U) chunks(c, std::integral_constant<int, U>{});
        if constexpr (U > 2)
            for (; c + 2 <= c1; c += 2) chunks(c, std::integral_constant<int, 2>{});
        if constexpr (U > 1)
            for (; c < c1; c++) chunks(c, std::integral_constant<int, 1>{});
    }

    // Park the prologue's values in LDS. Their loads completed with the main
    // loop's; reading them back from LDS later keeps the epilogue from waiting
    // on its own global stores (stores and loads share one counter). The empty
    // asm statements pin the first use of each value here, so the compiler
    // neither folds it into the load's branch nor hoists the LDS write above
    // the weight loads (either would wait on the load before the stream starts).
#pragma unroll
    for (int i = 0; i < RL; i++) asm volatile("" : "+v"(rv[i]));
#pragma unroll
    for (int it = 0; it < EPI_IT; it++) asm volatile("" : "+v"(pre[it]));
    asm volatile("" : "+v"(gv));
#pragma unroll
    for (int it = 0; it < DWI; it++) asm volatile("" : "+v"(dw[it]));
    if (NEED_R && rfast && (int)threadIdx.x < rslots) {
        // the 16 partials of a row sit in 16 consecutive lanes (whole waves take part)
        float v = 0.0f;
#pragma unroll
        for (int i = 0; i < RL; i++) v += rv[i];
        v = group_reduce<16, false>(v);
        if ((threadIdx.x & 15) == 0) rs[threadIdx.x >> 4] = 1.0f / sqrtf(v / (float)a.hidden + a.eps);
    }
    if (EPI == EPI_RESID || ((EPI == EPI_QKV || EPI == EPI_STORE) && a.bias)) {
#pragma unroll
        for (int it = 0; it < EPI_IT; it++) {
            const int idx = threadIdx.x + it * blockDim.x;
            if (idx < rows * COLS) et[(idx / COLS) * YS + idx % COLS] = pre[it];
        }
    }
    if (EPI == EPI_RESID && threadIdx.x < OC) gs[threadIdx.x] = gv;

    // an accumulator a later kernel adds into starts at zero (stored only now:
    // loads and stores retire in order, so earlier stores would hold up every
    // wait on the loads above)
    if (a.zero) {
        const int nthr = (int)(blockDim.x * gridDim.x * gridDim.y * gridDim.z);
        const int g = (int)threadIdx.x + (int)blockDim.x * (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
        for (int i = g; i < a.zero_n; i += nthr) a.zero[i] = 0;
    }
    // reduce across waves
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int p = 0; p < PG; p++)
            if (p < np)
                red[((wave * NT + t) * PG + p) * 64 + lane] =
                    Q ? accq[t][p] : ((accb[t][p][0] + accb[t][p][1]) + accb[t][p][2]) + accb[t][p][3];
    __syncthreads();
    if (NEED_R && !rfast && threadIdx.x < 16) {
        float s = 0.0f;
        for (int j = 0; j < 16; j++) s += rtmp[threadIdx.x * 17 + j];
        rs[threadIdx.x] = 1.0f / sqrtf(s / (float)a.hidden + a.eps);
    }
    for (int idx = threadIdx.x; idx < NT * np * 64; idx += blockDim.x) {
        const int t = idx / (np * 64), rem = idx % (np * 64), p = rem >> 6, l = rem & 63;
        float v = 0.0f;
        for (int w = 0; w < W; w++) v += red[((w * NT + t) * PG + p) * 64 + l];
        yt[(p * 4 + (l >> 4)) * YS + t * 16 + (l & 15)] = v;
    }
    __syncthreads();
    if (EPI != EPI_ARGMAX && ks > 1) {
        // The workgroups of the group meet: each stores its partial tile with
        // agent-coherent (L2-bypassing) stores and, once they have completed,
        // bumps the group's counter; the last to arrive reads every partial the
        // same way and sums them in split order (the same bits whichever
        // arrives last), then runs the epilogue. The counter is reset for the
        // next launch by that last workgroup.
        __shared__ int last;
        float* gp = a.gpart + (size_t)blockIdx.x * ks * (16 * COLS);
        for (int idx = threadIdx.x; idx < rows * COLS; idx += blockDim.x)
            __hip_atomic_store(gp + (size_t)split * 16 * COLS + idx, yt[(idx / COLS) * YS + idx % COLS],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned* cnt = a.gcnt + (size_t)blockIdx.x * 32;
            const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = old == (unsigned)ks - 1;
            if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last) {
            stamp.end();
            return;
        }
        constexpr int KSMAX = 8;
        for (int idx = threadIdx.x; idx < rows * COLS; idx += blockDim.x) {
            float pv[KSMAX];
#pragma unroll
            for (int s = 0; s < KSMAX; s++)
                pv[s] = s >= ks ? 0.0f
                                : __hip_atomic_load(gp + (size_t)s * 16 * COLS + idx, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
            float v = pv[0];
#pragma unroll
            for (int s = 1; s < KSMAX; s++)
                if (s < ks) v += pv[s];
            yt[(idx / COLS) * YS + idx % COLS] = v;
        }
        __syncthreads();
    }

    if constexpr (EPI == EPI_MLP) {
        // The activations of the group's 16 channels (the EPI_SILU arithmetic),
        // then each output n of the down projection from these channels: an item
        // holds 8 channels of one output (one fma chain), the other 8 sit in lane
        // ^ 16 (row swap; both lanes end with the same sum), and the sum goes into
        // this XCD's accumulator copy as round(y * 2^kAccFrac).
        for (int idx = threadIdx.x; idx < rows * OC; idx += blockDim.x) {
            const int r = idx / OC, cc = idx % OC, row = pass0 * 4 + r;
            const float gt = yt[r * YS + cc] * rs[r], up = yt[r * YS + OC + cc] * rs[r];
            vt[r * YS + cc] = row < a.m ? gt / (1.0f + dev_exp(-gt)) * up : 0.0f;
        }
        __syncthreads();
        const int n_items = (a.N2 >> 4) * 32, qq = (lane >> 4) & 1;
        long long* accp = a.acc_out + (size_t)(blockIdx.x % kAccCopies) * 4 * a.acc_ld;
#pragma unroll
        for (int it = 0; it < DWI; it++) {
            const int i = (int)threadIdx.x + it * (int)blockDim.x;
            const int n = (min(i, n_items - 1) >> 5) * 16 + (lane & 15);
            float w8[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                w8[2 * e] = bf16_bits_to_f32(dw[it][e] & 0xFFFFu);
                w8[2 * e + 1] = bf16_bits_to_f32(dw[it][e] >> 16);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (pass0 * 4 + r >= a.m) break;  // uniform: the live rows only
                const float* vr = &vt[r * YS + 8 * qq];
                float y = w8[0] * vr[0];
#pragma unroll
                for (int e = 1; e < 8; e++) y = fmaf(w8[e], vr[e], y);
                y = reduce_rows<false, false>(y);
                if (qq == 0 && i < n_items) {
                    const double d = fmin(fmax((double)y * (double)(1ll << kAccFrac), -4.0e18), 4.0e18);
                    __hip_atomic_fetch_add(accp + (size_t)r * a.acc_ld + n, (long long)rint(d), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        stamp.end();
        return;
    }
    if (EPI == EPI_STORE || EPI == EPI_QKV) {
#pragma unroll
        for (int it = 0; it < EPI_IT; it++) {
            const int idx = threadIdx.x + it * blockDim.x;
            if (idx < rows * COLS) {
                const int r = idx / COLS, cc = idx % COLS, row = pass0 * 4 + r, col = tile0 * 16 + cc;
                if (row < a.m) {
                    float v = yt[r * YS + cc];
                    if (EPI == EPI_QKV) v *= rs[r];
                    if (a.bias) v += et[r * YS + cc];
                    a.out[(size_t)row * a.ldo + col] = v;
                }
            }
        }
        stamp.end();
        return;
    }
    if (EPI == EPI_ARGMAX) {
        for (int idx = threadIdx.x; idx < rows * COLS; idx += blockDim.x) {
            const int r = idx / COLS, cc = idx % COLS, row = pass0 * 4 + r, col = tile0 * 16 + cc;
            const float v = yt[r * YS + cc] * rs[r];
            if (row < a.m && a.logits) a.logits[(size_t)row * a.N + col] = v;
            yt[r * YS + cc] = v != v ? -INFINITY : v;
        }
        __syncthreads();
        // (max, first index) of each row in each 32-column tile of the group
        constexpr int SUB = COLS / 32;
        if ((int)threadIdx.x < rows * SUB) {
            const int r = threadIdx.x / SUB, j = threadIdx.x % SUB, row = pass0 * 4 + r;
            if (row < a.m) {
                const float* yr = &yt[r * YS + j * 32];
                float bv = yr[0];
                int bi = 0;
                for (int cc = 1; cc < 32; cc++)
                    if (yr[cc] > bv) {
                        bv = yr[cc];
                        bi = cc;
                    }
                a.best[((size_t)blockIdx.x * SUB + j) * a.m + row] =
                    make_float2(bv, __int_as_float(tile0 * 16 + j * 32 + bi));
            }
        }
        stamp.end();
        return;
    }
    // EPI_RESID / EPI_SILU finish the group's OC output columns: one k-block of
    // the next consumer (OC 32), or half of one (OC 16, bf16 pieces only: they
    // carry no per-block scale). (A) every thread finishes some of the rows x OC
    // values into LDS; (B) one wave forms each row's sum of squares (EPI_RESID);
    // (C) up to four waves per pass write the pieces, two of a lane's eight
    // inputs each, so the conversions run on several SIMDs at once.
    static_assert(EPI != EPI_RESID && EPI != EPI_SILU || OC == 16 || OC == 32, "16 or 32 finished columns");
    for (int idx = threadIdx.x; idx < rows * OC; idx += blockDim.x) {
        const int r = idx / OC, cc = idx % OC, row = pass0 * 4 + r;
        const bool live = row < a.m;
        if (EPI == EPI_RESID) {
            const float xn = live ? et[r * YS + cc] + yt[r * YS + cc] : 0.0f;
            if (live) a.x[(size_t)row * a.ldx + blockIdx.x * OC + cc] = xn;
            yt[r * YS + cc] = xn;
            vt[r * YS + cc] = a.g_next ? gs[cc] * xn : xn;
        } else {
            const float gt = yt[r * YS + cc] * rs[r], up = yt[r * YS + OC + cc] * rs[r];
            const float v = live ? gt / (1.0f + dev_exp(-gt)) * up : 0.0f;
            vt[r * YS + cc] = v;
            if (a.cap && live) a.cap[(size_t)row * a.ldcap + blockIdx.x * OC + cc] = v;
        }
    }
    __syncthreads();
    if (EPI == EPI_RESID && wave == W - 1)
        for (int p = 0; p < np; p++) {
            // row 4p + lane/16: lane j of 16 takes columns j*OC/16 .. +OC/16-1
            const int r = p * 4 + (lane >> 4), j = lane & 15, row = pass0 * 4 + r;
            float ssq;
            if (OC == 32) {
                const float x0 = yt[r * YS + 2 * j], x1 = yt[r * YS + 2 * j + 1];
                ssq = fmaf(x1, x1, x0 * x0);
            } else {
                const float x0 = yt[r * YS + j];
                ssq = x0 * x0;
            }
            ssq = group_reduce<16, false>(ssq);
            if (j == 0 && row < a.m) a.ss_out[(size_t)blockIdx.x * a.ss_m + row] = ssq;
        }
    // the consumer's k-block and, for OC 16, which half of it (lanes 32h .. 32h+31)
    const int pkb = blockIdx.x * OC / 32, half = OC == 16 ? (int)(blockIdx.x & 1) : 0;
    if (a.pa)
        for (int t = wave; t < np * 4; t += W) {
            const int p = t >> 2, pair = t & 3;
            const int c = lane & 15, r = p * 4 + (c >> 2), q = lane >> 4;
            if (OC == 16 && (q >> 1) != half) continue;
            const float* vr = &vt[r * YS + (OC == 16 ? q & 1 : q) * 8];
            const float4 v0 = *(const float4*)vr, v1 = *(const float4*)(vr + 4);
            const float2 xp = *(const float2*)(vr + 2 * pair);
            if (OC == 16) {  // bf16 or MM pieces: no block scale
                if (a.pa_kind == MM)
                    write_pieces_pair<MM>(xp.x, xp.y, 0.0f, pair, pkb, pass0 + p, a.pa_passes, pass0 * 4 + r,
                                          c & 3, lane, a.pa, a.pxs);
                else
                    write_pieces_pair<BF16>(xp.x, xp.y, 0.0f, pair, pkb, pass0 + p, a.pa_passes, pass0 * 4 + r,
                                            c & 3, lane, a.pa, a.pxs);
            } else {
                const float mx = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                                       fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
                write_pieces_pair_kind(a.pa_kind, xp.x, xp.y, mx, pair, pkb, pass0 + p, a.pa_passes, pass0 * 4 + r,
                                       c & 3, lane, a.pa, a.pxs);
            }
        }
    // the consumer's zero padding past the last k-block, one wave per (k-block, pass)
    if (a.pa && blockIdx.x == gridDim.x - 1) {
        const float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        const int c = lane & 15, covered = (int)gridDim.x * OC / 32;
        for (int idx = wave; idx < (a.pa_kb - covered) * np; idx += W) {
            const int kb2 = covered + idx / np, p = idx % np;
            write_pieces_kind(a.pa_kind, z, kb2, pass0 + p, a.pa_passes, pass0 * 4 + p * 4 + (c >> 2), c & 3, lane,
                              a.pa, a.pxs);
        }
    }
    stamp.end();
}

template <class K>
static void launch_timed(K kernel, dim3 grid, dim3 block, hipStream_t st, const GemvArgs& a, hipEvent_t e0,
                         hipEvent_t e1) {
    if (e0 || e1)
        hipExtLaunchKernelGGL(kernel, grid, block, 0, st, e0, e1, 0, a);
    else
        hipLaunchKernelGGL(kernel, grid, block, 0, st, a);
}

// ---------------------------------------------------------------------------
// GEMM for more than 16 activation rows (batched verify, prefill chunks):
// bf16 MFMA (v_mfma_f32_16x16x32_bf16) on activations in the MM format (x =
// hi + lo, two bf16 pieces: 16 significant bits) and on weights converted to
// bf16 exactly (int8 codes, int4 codes x 16, bf16 as stored); the group
// scale is applied once per k-block after the hi and lo products, as the
// reference applies it to each group's dot product (src/quant.rs:331-374).
// A workgroup owns a 64-row x 64-column output tile; its eight waves are two
// halves of K x four 32 x 32 sub-tiles (2 row tiles x 2 n-tiles each), whose
// operands each wave loads straight into registers (the other waves' copies
// hit in L1); a chunk's loads are all issued before its first MFMA. The two
// K halves meet in LDS, then the same epilogues as the GEMV run on the tile.
// ---------------------------------------------------------------------------

// bytes b, b+1 of w (two's-complement int8) as two bf16, exactly
__device__ __forceinline__ uint32_t bf16x2_i8(uint32_t w, int b) {
    const float f0 = (float)(int8_t)(w >> (8 * b)), f1 = (float)(int8_t)(w >> (8 * b + 8));
    return (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
}

// The GEMM epilogues on the finished 64 x 64 tile yt (rows [row0, row0 + rows),
// columns from col0): 1/rms from the producers' sums of squares, then the
// GEMV's epilogues (internal.h) with the next operand in the MM format.
template <int EPI, int NTHR, int MR>
__device__ void gemm_epilogue(const GemvArgs& a, float* yt, float* part, float* rs, int row0, int rows, int col0) {
    constexpr bool NEED_R = EPI == EPI_QKV || EPI == EPI_SILU || EPI == EPI_ARGMAX;
    constexpr int YS = 68;
    static_assert(MR * 4 <= NTHR, "four lanes per row");
    const int tid = threadIdx.x;
    // the tile's place among the output's 64-column tiles (col0 is a multiple of 64)
    const int tile = col0 / 64, ntiles = (a.N + 63) / 64;
    __syncthreads();
    // 1/rms of each row from the producers' sums of squares: four lanes per row
    if (NEED_R && tid < MR * 4) {
        const int rr = tid >> 2, q4 = tid & 3, row = row0 + rr;
        float v = 0.0f;
        if (rr < rows) {
            const int src = a.rows_src ? a.rows_src[row] : row;
            for (int t = q4; t < a.ss_tiles; t += 4) v += a.ss_in[(size_t)t * a.ss_m + src];
        }
        v = group_reduce<4, false>(v);
        if (q4 == 0) rs[rr] = 1.0f / sqrtf(v / (float)a.hidden + a.eps);
    }
    __syncthreads();

    if (EPI == EPI_STORE || EPI == EPI_QKV) {
        for (int idx = tid; idx < MR * 64; idx += NTHR) {
            const int rr = idx >> 6, cc = idx & 63, row = row0 + rr, col = col0 + cc;
            if (rr < rows && col < a.N) {
                float v = yt[rr * YS + cc];
                if (EPI == EPI_QKV) v *= rs[rr];
                if (a.bias) v += a.bias[col];
                a.out[(size_t)row * a.ldo + col] = v;
            }
        }
        return;
    }
    if (EPI == EPI_ARGMAX) {
        for (int idx = tid; idx < MR * 64; idx += NTHR) {
            const int rr = idx >> 6, cc = idx & 63, row = row0 + rr, col = col0 + cc;
            const float v = yt[rr * YS + cc] * rs[rr];
            if (rr < rows && col < a.N && a.logits) a.logits[(size_t)row * a.N + col] = v;
            yt[rr * YS + cc] = v != v ? -INFINITY : v;
        }
        __syncthreads();
        // (max, first index) of each row in each 32-column tile
        if (tid < MR * 2) {
            const int rr = tid >> 1, j = tid & 1, row = row0 + rr;
            if (rr < rows && col0 + j * 32 < a.N) {
                const float* yr = &yt[rr * YS + j * 32];
                float bv = yr[0];
                int bi = 0;
                for (int cc = 1; cc < 32; cc++)
                    if (yr[cc] > bv) {
                        bv = yr[cc];
                        bi = cc;
                    }
                a.best[((size_t)tile * 2 + j) * a.m + row] = make_float2(bv, __int_as_float(col0 + j * 32 + bi));
            }
        }
        return;
    }
    // EPI_RESID / EPI_SILU: the finished values of the group's output columns
    // (64 for RESID, the 32 channels of SILU) go to LDS, then out as the next
    // GEMM's MM pieces (two bf16 pieces per value) in 16-byte slots.
    constexpr int OC = EPI == EPI_RESID ? 64 : 32;
    float* vt = part;  // free again after the tree
    for (int idx = tid; idx < MR * OC; idx += NTHR) {
        const int rr = idx / OC, cc = idx % OC, row = row0 + rr;
        const bool live = rr < rows && (EPI == EPI_SILU || col0 + cc < a.N);
        if (EPI == EPI_RESID) {
            const size_t at = (size_t)row * a.ldx + col0 + cc;
            const float xn = live ? a.x[at] + yt[rr * YS + cc] : 0.0f;
            if (live) a.x[at] = xn;
            yt[rr * YS + cc] = xn;
            vt[rr * YS + cc] = live && a.g_next ? a.g_next[col0 + cc] * xn : xn;
        } else {
            // channel cc: block b of the [gate il, up il] interleave, position j in it
            const int b = cc / a.il, j = cc % a.il;
            const float gt = yt[rr * YS + b * 2 * a.il + j] * rs[rr], up = yt[rr * YS + b * 2 * a.il + a.il + j] * rs[rr];
            const float v = live ? gt / (1.0f + dev_exp(-gt)) * up : 0.0f;
            vt[rr * YS + cc] = v;
            if (a.cap && live) a.cap[(size_t)row * a.ldcap + tile * 32 + cc] = v;
        }
    }
    __syncthreads();
    if (EPI == EPI_RESID && tid < MR * 4) {
        // each row's sum of squares over the group's columns: four lanes per row
        const int rr = tid >> 2, q4 = tid & 3, row = row0 + rr;
        float ssq = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const float x = yt[rr * YS + q4 * 16 + e];
            ssq = fmaf(x, x, ssq);
        }
        ssq = group_reduce<4, false>(ssq);
        if (q4 == 0 && rr < rows) a.ss_out[(size_t)tile * a.ss_m + row] = ssq;
    }
    if (a.pa) {
        // slot (k-block, row tile, piece h, lane q8 * 16 + row % 16) holds 8 values
        const int prt = (a.pa_passes + 3) >> 2, kb0 = col0 / 32;
        constexpr int Q8 = OC / 8;
        for (int idx = tid; idx < MR * Q8 * 2; idx += NTHR) {
            const int h = idx & 1, q8 = (idx >> 1) % Q8, rr = (idx >> 1) / Q8, row = row0 + rr;
            if (rr >= rows) continue;
            const int kb = (EPI == EPI_RESID ? kb0 : tile) + q8 / 4;
            const float* vr = &vt[rr * YS + q8 * 8];
            u16x8 o;
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = (uint16_t)bf16_piece(vr[e], h);
            ((u16x8*)a.pa)[(((size_t)kb * prt + (row >> 4)) * 2 + h) * 64 + (q8 & 3) * 16 + (row & 15)] = o;
        }
        // the consumer's zero padding past the last k-block
        if (tile == ntiles - 1) {
            const int covered = EPI == EPI_RESID ? (a.N + 31) / 32 : ntiles;
            const u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int idx = tid; idx < (a.pa_kb - covered) * MR * 8; idx += NTHR) {
                const int kb = covered + idx / (MR * 8), rem = idx % (MR * 8), h = rem & 1, q8 = (rem >> 1) & 3,
                          rr = rem >> 3, row = row0 + rr;
                if (rr < rows)
                    ((u16x8*)a.pa)[(((size_t)kb * prt + (row >> 4)) * 2 + h) * 64 + q8 * 16 + (row & 15)] = z;
            }
        }
    }
}

// CS 2 (steps of 256 rows or more): the eight waves form two sets of four, one
// per 64-column half of a 128-column tile, each set splitting K in quarters, so
// that a workgroup reads its activation rows once for twice the columns.
template <int KIND, int EPI, int RTW, int CS = 1>
__global__ __launch_bounds__(512) void k_gemm(const GemvArgs a) {
    constexpr int NW = 8, NTHR = 64 * NW, NKW = NW / CS;
    static_assert(CS == 1 || CS == 2, "one or two column sets");
    constexpr bool Q = KIND != BF16;
    constexpr bool WNT = Q || EPI == EPI_ARGMAX;  // weights read once per step: non-temporal
    constexpr bool NEED_R = EPI == EPI_QKV || EPI == EPI_SILU || EPI == EPI_ARGMAX;
    constexpr int YS = 68;  // LDS row stride of the 16 RTW x 64 tile
    // the cross-wave tree: four partial tiles (the lanes' layout), then the tile
    __shared__ __align__(16) float part[4 * RTW * 4 * 256];
    __shared__ __align__(16) float yt[16 * RTW * YS];
    __shared__ float rs[16 * RTW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar registers, no divergence
    const int RT = (a.p_total + 3) >> 2;                         // row tiles of the activation buffer
    const int cs = CS == 1 ? 0 : wave / NKW, kw = wave % NKW;  // column set, K share
    const int rtb = blockIdx.y * RTW, tb = blockIdx.x * 4 * CS + cs * 4;
    const int row0 = rtb * 16, col0 = blockIdx.x * 64 * CS;
    const int rows = min(16 * RTW, a.m - row0);  // rows of this tile that exist (others are discarded)
    const int ntl = a.N >> 4, KB = a.KB, KC = KB >> 2;
    // row tiles / n-tiles past the end re-read the last one (their results are discarded)
    int rt_[RTW], t_[4];
#pragma unroll
    for (int i = 0; i < RTW; i++) rt_[i] = min(rtb + i, RT - 1);
#pragma unroll
    for (int t = 0; t < 4; t++) t_[t] = min(tb + t, ntl - 1);
    // k-block pairs: this workgroup's share of K (blockIdx.z of gridDim.z), an
    // eighth of it per wave
    const int NP = KB >> 1, ks = gridDim.z;
    const int g0 = blockIdx.z * NP / ks, g1 = (blockIdx.z + 1) * NP / ks;
    const int p0 = g0 + kw * (g1 - g0) / NKW, p1 = g0 + (kw + 1) * (g1 - g0) / NKW;

    f32x4 acc[RTW][4];
#pragma unroll
    for (int i = 0; i < RTW; i++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[i][t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 fzero = {0.0f, 0.0f, 0.0f, 0.0f};

    for (int pr = p0; pr < p1; pr++) {
        const int kb0 = 2 * pr, c = kb0 >> 2, half = (kb0 >> 1) & 1;
        // every operand of the pair in flight before the first MFMA
        bf16x8 A[2][RTW][2];  // [k-block][row tile][hi/lo]
        uint2 w4[4];          // int4: the pair's two 4-byte words
        u32x4 w8[4];          // int8: the pair's 16 bytes
        bf16x8 wb[4][2];
        float2 sv[4];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < RTW; i++)
#pragma unroll
                for (int h = 0; h < 2; h++)
                    A[j][i][h] = ((const bf16x8*)a.XA)[((((size_t)(kb0 + j) * RT + rt_[i]) * 2 + h) * 64) + lane];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const size_t tile = t_[t];
            if (KIND == INT4) {
                const u32x2 v = ld_nt<WNT>((const u32x2*)a.W + ((tile * KC + c) * 64 + lane) * 2 + half);
                w4[t] = make_uint2(v[0], v[1]);
            } else if (KIND == INT8) {
                w8[t] = ld_nt<WNT>((const u32x4*)a.W + (tile * (KB >> 1) + pr) * 64 + lane);
            } else {
#pragma unroll
                for (int j = 0; j < 2; j++) wb[t][j] = ld_nt<WNT>((const bf16x8*)a.W + (tile * KB + kb0 + j) * 64 + lane);
            }
            if (Q) {
                const f32x2 v = ld_nt<WNT>((const f32x2*)a.S + ((tile * KC + c) * 16 + (lane & 15)) * 2 + half);
                sv[t] = make_float2(v[0], v[1]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                bf16x8 B;
                if (KIND == INT4) {
                    const uint32_t w = j ? w4[t].y : w4[t].x;
                    const uint32_t lo = (w << 4) & 0xF0F0F0F0u, hi = w & 0xF0F0F0F0u;
                    const u32x4 bw = {bf16x2_i8(lo, 0), bf16x2_i8(lo, 2), bf16x2_i8(hi, 0), bf16x2_i8(hi, 2)};
                    B = __builtin_bit_cast(bf16x8, bw);
                } else if (KIND == INT8) {
                    const uint32_t w0 = w8[t][2 * j], w1 = w8[t][2 * j + 1];
                    const u32x4 bw = {bf16x2_i8(w0, 0), bf16x2_i8(w0, 2), bf16x2_i8(w1, 0), bf16x2_i8(w1, 2)};
                    B = __builtin_bit_cast(bf16x8, bw);
                } else {
                    B = wb[t][j];
                }
                const float sj = Q ? (j == 0 ? sv[t].x : sv[t].y) : 1.0f;
#pragma unroll
                for (int i = 0; i < RTW; i++) {
                    if (Q) {
                        f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[j][i][0], B, fzero, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[j][i][1], B, d, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[i][t][r] = fmaf(d[r], sj, acc[i][t][r]);
                    } else {
                        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[j][i][0], B, acc[i][t], 0, 0, 0);
                        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[j][i][1], B, acc[i][t], 0, 0, 0);
                    }
                }
            }
    }
    // Eight partial tiles to one, in a fixed order: waves 4-7 hand theirs to 0-3,
    // then 2-3 to 0-1, then 1 to 0 (each hand-off in the lanes' own layout).
    auto put = [&](int slot) {
#pragma unroll
        for (int i = 0; i < RTW; i++)
#pragma unroll
            for (int t = 0; t < 4; t++)
                *(f32x4*)&part[((slot * RTW * 4 + i * 4 + t) * 64 + lane) * 4] = acc[i][t];
    };
    auto take = [&](int slot) {
#pragma unroll
        for (int i = 0; i < RTW; i++)
#pragma unroll
            for (int t = 0; t < 4; t++) acc[i][t] += *(const f32x4*)&part[((slot * RTW * 4 + i * 4 + t) * 64 + lane) * 4];
    };
    if constexpr (CS == 1) {
        if (wave >= 4) put(wave - 4);
        __syncthreads();
        if (wave < 4) take(wave);
        __syncthreads();
    }
    // (CS 2: each set's four partial tiles, in the same order, in slots 2 cs and 2 cs + 1)
    if (kw == 2 || kw == 3) put(cs * 2 + kw - 2);
    __syncthreads();
    if (kw < 2) take(cs * 2 + kw);
    __syncthreads();
    if (kw == 1) put(cs * 2);
    __syncthreads();
    if (kw == 0) take(cs * 2);
    if (CS == 1 && RTW <= 2 && ks > 1 && a.gcnt) {
        // Split K finished in place (tiles of at most 32 rows: the 1B draft's
        // 16-row rounds of cfg4, 6595-6601 -> 6410-6418 us per step in a same-box
        // A/B; the target's 48- and 80-row tiles were slower this way, cfg4
        // verify 8796 -> 9091 us, and keep k_gemm_finish): each workgroup of the
        // tile stores its partial
        // with agent-coherent (L2-bypassing) stores and, once they have completed,
        // bumps the tile's counter; the last to arrive reads every partial the
        // same way, sums them in split order (k_gemm_finish's order: the same bits
        // whichever arrives last) and runs the epilogue. It resets the counter
        // for the next launch.
        __shared__ int last;
        if (wave == 0)
#pragma unroll
            for (int i = 0; i < RTW; i++)
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int rr = i * 16 + 4 * (lane >> 4) + r, cc = t * 16 + (lane & 15);
                        if (rr < rows && col0 + cc < a.N)
                            __hip_atomic_store(a.kpart + ((size_t)blockIdx.z * a.m + row0 + rr) * a.N + col0 + cc,
                                               acc[i][t][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            unsigned* cnt = a.gcnt + ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 32;
            const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = old == (unsigned)ks - 1;
            if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last) return;
        constexpr int KSMAX = 8;
        for (int idx = tid; idx < 16 * RTW * 64; idx += NTHR) {
            const int rr = idx >> 6, cc = idx & 63;
            const bool live = rr < rows && col0 + cc < a.N;
            const size_t at = ((size_t)min(row0 + rr, a.m - 1)) * a.N + min(col0 + cc, a.N - 1);
            float pv[KSMAX];
#pragma unroll
            for (int z = 0; z < KSMAX; z++)
                pv[z] = z < ks ? __hip_atomic_load(a.kpart + (size_t)z * a.m * a.N + at, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                               : 0.0f;
            float v = pv[0];
#pragma unroll
            for (int z = 1; z < KSMAX; z++)
                if (z < ks) v += pv[z];
            yt[rr * YS + cc] = live ? v : 0.0f;
        }
        if (col0 < a.N) gemm_epilogue<EPI, NTHR, 16 * RTW>(a, yt, part, rs, row0, rows, col0);
        return;
    }
    for (int c = 0; c < CS; c++) {
    if (c > 0) __syncthreads();  // the previous column set's epilogue is done with yt
    const int colc = col0 + c * 64;
    if (wave == c * NKW) {
        if (ks > 1) {
            // split K: this workgroup's partial tile goes to kpart[z][row][col]; k_gemm_finish sums
            // the splits in order and runs the epilogue
#pragma unroll
            for (int i = 0; i < RTW; i++)
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int rr = i * 16 + 4 * (lane >> 4) + r, cc = t * 16 + (lane & 15);
                        if (rr < rows && colc + cc < a.N)
                            a.kpart[((size_t)blockIdx.z * a.m + row0 + rr) * a.N + colc + cc] = acc[i][t][r];
                    }
        } else {
        // D of a 16 x 16 tile has row 4 (l / 16) + r, column l % 16 in lane l
#pragma unroll
        for (int i = 0; i < RTW; i++)
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) yt[(i * 16 + 4 * (lane >> 4) + r) * YS + t * 16 + (lane & 15)] = acc[i][t][r];
        }
    }
    if (ks == 1 && colc < a.N) gemm_epilogue<EPI, NTHR, 16 * RTW>(a, yt, part, rs, row0, rows, colc);
    }
}

// The split-K sum (splits in order, so the result does not depend on which
// workgroup finished first) and the epilogue of one 16 RTW x 64 tile (launched
// on 16-row slabs, RTW 1, for more workgroups).
template <int EPI, int RTW>
__global__ __launch_bounds__(256) void k_gemm_finish(const GemvArgs a) {
    constexpr int YS = 68;
    __shared__ __align__(16) float vt[64 * YS];
    __shared__ __align__(16) float yt[64 * YS];
    __shared__ float rs[64];
    const int row0 = blockIdx.y * RTW * 16, col0 = blockIdx.x * 64;
    const int rows = min(16 * RTW, a.m - row0);
    // RTW 4-column slots per thread (16 RTW rows x 16 slots), every split's load
    // issued before the sums (clamped addresses; splits past ks and slots past
    // the tile are masked)
    constexpr int KSMAX = 8;
    float4 v[RTW][KSMAX];
#pragma unroll
    for (int it = 0; it < RTW; it++) {
        const int slot = threadIdx.x + it * 256, rr = min(slot >> 4, rows - 1), c = min(col0 + (slot & 15) * 4, a.N - 4);
#pragma unroll
        for (int z = 0; z < KSMAX; z++)
            v[it][z] = *(const float4*)&a.kpart[((size_t)min(z, a.ks - 1) * a.m + row0 + rr) * a.N + c];
    }
#pragma unroll
    for (int it = 0; it < RTW; it++) {
        const int slot = threadIdx.x + it * 256, rr = slot >> 4, cc = (slot & 15) * 4;
        const bool live = rr < rows && col0 + cc < a.N;
        float4 t = v[it][0];
#pragma unroll
        for (int z = 1; z < KSMAX; z++)
            if (z < a.ks) {
                t.x += v[it][z].x;
                t.y += v[it][z].y;
                t.z += v[it][z].z;
                t.w += v[it][z].w;
            }
        *(float4*)&yt[rr * YS + cc] = live ? t : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    gemm_epilogue<EPI, 256, 16 * RTW>(a, yt, vt, rs, row0, rows, col0);
}

template <int KIND, int RTW, int CS>
static void gemm_rtw(hipStream_t st, int epi, const DMat& w, const GemvArgs& a0, int groups, hipEvent_t e0,
                     hipEvent_t e1) {
    // Split K across workgroups when the tiles alone leave most CUs idle: up
    // to 256 workgroups, at least one k-block pair per wave and split, and the
    // partial tiles within the workspace's kpart buffer.
    GemvArgs a = a0;
    const int cg = (w.n_tiles + 4 * CS - 1) / (4 * CS), cg64 = (w.n_tiles + 3) / 4, np = w.kb / 2;
    int ks = 1;
    if (a.kpart)
        while (ks < 8 && cg * groups * ks * 2 <= 256 && np / (ks * 2) >= 8 &&
               (size_t)ks * 2 * a.m * a.N <= a.kpart_cap)
            ks *= 2;
    a.ks = ks;
    const dim3 grid(cg, groups, ks);
    // timed from the start of the main kernel to the end of the split's finish
    auto run = [&](auto kern, auto fin) {
        // one column set of at most two row tiles, with meeting counters: the
        // split is finished in the kernel
        if (ks == 1 || (CS == 1 && RTW <= 2 && a.gcnt)) {
            launch_timed(kern, grid, dim3(512), st, a, e0, e1);
        } else {
            launch_timed(kern, grid, dim3(512), st, a, e0, nullptr);
            launch_timed(fin, dim3(cg64, (a.m + 15) / 16), dim3(256), st, a, nullptr, e1);
        }
    };
    switch (epi) {
        case EPI_STORE: run(k_gemm<KIND, EPI_STORE, RTW, CS>, k_gemm_finish<EPI_STORE, 1>); break;
        case EPI_QKV: run(k_gemm<KIND, EPI_QKV, RTW, CS>, k_gemm_finish<EPI_QKV, 1>); break;
        case EPI_RESID: run(k_gemm<KIND, EPI_RESID, RTW, CS>, k_gemm_finish<EPI_RESID, 1>); break;
        case EPI_SILU: run(k_gemm<KIND, EPI_SILU, RTW, CS>, k_gemm_finish<EPI_SILU, 1>); break;
        case EPI_ARGMAX: run(k_gemm<KIND, EPI_ARGMAX, RTW, CS>, k_gemm_finish<EPI_ARGMAX, 1>); break;
    }
}

template <int KIND>
static void gemm_kind(hipStream_t st, int epi, const DMat& w, const GemvArgs& a, hipEvent_t e0, hipEvent_t e1) {
    const int rt = (a.p_total + 3) / 4, groups = (rt + 4) / 5, rtw = (rt + groups - 1) / groups;
    // 128-column tiles (CS 2) for steps of 256 rows or more when they still make
    // 512 workgroups (measured on the 1.7B int4 prefill of 1024 tokens: 14.45
    // against 15.3 ms; with fewer workgroups, the 135M draft's prefill and the
    // 160-row verify steps ran slower: 4.54 against 4.0 ms, 7.42 against 6.80 ms)
    // Steps of 256 rows or more into fewer than 4096 outputs: row groups of two
    // tiles, for more workgroups (measured on the cfg2 prompt's forwards: the
    // 135M draft 3.97 -> 3.31 ms, the 1.7B target's o and down 14.13 -> 14.03 ms
    // per forward)
    // 80 to 160 rows into 16384 or more outputs (gate/up and the lm_heads of the
    // batched verifies): 128-column tiles too. Same-box A/B: cfg4 verify
    // 8644-8650 -> 8383-8386 us, cfg3 at 32 sequences 5682 -> 5485 us. At 40
    // rows (three-tile groups) they were slower: cfg3 at 8 sequences 2562 ->
    // 2690 us.
    if (rt >= 5 && rt < 16 && rtw == 5 && w.n_tiles >= 1024) {
        gemm_rtw<KIND, 5, 2>(st, epi, w, a, groups, e0, e1);
        return;
    }
    if (rt >= 16 && w.n_tiles < 256)
        gemm_rtw<KIND, 2, 1>(st, epi, w, a, (rt + 1) / 2, e0, e1);
    else
    if (rt >= 16 && (w.n_tiles + 7) / 8 * groups >= 512)
        gemm_rtw<KIND, 5, 2>(st, epi, w, a, groups, e0, e1);
    else if (rtw <= 2)
        gemm_rtw<KIND, 2, 1>(st, epi, w, a, (rt + 1) / 2, e0, e1);
    else if (rtw == 3)
        gemm_rtw<KIND, 3, 1>(st, epi, w, a, (rt + 2) / 3, e0, e1);
    else if (rtw == 4)
        gemm_rtw<KIND, 4, 1>(st, epi, w, a, (rt + 3) / 4, e0, e1);
    else
        gemm_rtw<KIND, 5, 1>(st, epi, w, a, groups, e0, e1);
}

template <int KIND, int NT, int EPI>
static void gemv_pg(hipStream_t st, const DMat& w, const GemvArgs& a, hipEvent_t e0, hipEvent_t e1) {
    const int groups = w.n_tiles / NT;
    const int KC = w.kb / 4;
    const int maxw = 8;  // waves per group: launch bounds of k_gemv
    if (a.p_total == 1) {
        if (a.gsplit > 1) {
            // split K: up to 8 waves over each workgroup's share of the chunks
            const int W = std::max(1, std::min(maxw, KC / a.gsplit));
            launch_timed(k_gemv<KIND, NT, EPI, 1>, dim3(groups, a.gsplit, 1), dim3(64 * W), st, a, e0, e1);
            return;
        }
        if constexpr (KIND == INT4 && NT == 2) {
            if (KC >= 16) {
                // 16 waves (4 per SIMD) cover each other's waits on the big int4 matrices
                launch_timed(k_gemv<KIND, NT, EPI, 1, 16>, dim3(groups, 1, 1), dim3(64 * 16), st, a, e0, e1);
                return;
            }
        }
        const int W = std::max(1, std::min(maxw, KC));
        launch_timed(k_gemv<KIND, NT, EPI, 1>, dim3(groups, 1, 1), dim3(64 * W), st, a, e0, e1);
    } else if constexpr (NT <= 4) {
        // Up to 8 passes (32 rows): one pass per workgroup along z, each reading
        // the weights again from L2, for 8x the workgroups of a decode launch
        // (cfg3's 135M draft rounds at 32 sequences: draft 5374-5377 -> 5015-5025
        // us per step, at 8 sequences 3828 -> 3457 us). More passes take groups
        // of four, which share one weight read; for gate/up, whose weights are
        // the largest, already past 4 passes (at 32 sequences draft 5078-5080 ->
        // 4929-4954 us; at 8 sequences, 2 passes, one per workgroup stays faster:
        // 3457 against 3559 us).
        if (a.p_total <= (EPI == EPI_SILU ? 4 : 8)) {
            const int W = std::max(1, std::min(maxw, KC));
            launch_timed(k_gemv<KIND, NT, EPI, 1>, dim3(groups, 1, a.p_total), dim3(64 * W), st, a, e0, e1);
            return;
        }
        const int pg = (a.p_total + 3) / 4;
        int W = (4096 + groups * pg - 1) / (groups * pg);
        W = std::max(1, std::min(std::min(W, maxw), KC));
        launch_timed(k_gemv<KIND, NT, EPI, 4>, dim3(groups, 1, pg), dim3(64 * W), st, a, e0, e1);
    }
}

template <int KIND>
static void gemv_kind(hipStream_t st, int epi, const DMat& w, const GemvArgs& a, hipEvent_t e0, hipEvent_t e1) {
    switch (epi) {
        case EPI_STORE: gemv_pg<KIND, 2, EPI_STORE>(st, w, a, e0, e1); break;
        case EPI_QKV:
            if constexpr (KIND == BF16) {
                if (a.ax) {
                    // input formed in the workgroup: one chunk per wave
                    const int W = std::max(1, std::min(8, w.kb / 4));
                    if (a.nt == 1)
                        launch_timed(k_gemv<BF16, 1, EPI_QKV, 1, 8, false, true>, dim3(w.n_tiles, 1, 1), dim3(64 * W),
                                     st, a, e0, e1);
                    else
                        launch_timed(k_gemv<BF16, 2, EPI_QKV, 1, 8, false, true>, dim3(w.n_tiles / 2, 1, 1),
                                     dim3(64 * W), st, a, e0, e1);
                    break;
                }
            }
            if (a.nt == 1)
                gemv_pg<KIND, 1, EPI_QKV>(st, w, a, e0, e1);
            else
                gemv_pg<KIND, 2, EPI_QKV>(st, w, a, e0, e1);
            break;
        case EPI_RESID:
            if constexpr (KIND == BF16) {
                if (a.am) {
                    // the launch shape of the two-kernel path (waves = chunks, up to 8)
                    const int W = std::max(1, std::min(8, w.kb / 4));
                    if (a.nt == 1)
                        launch_timed(k_gemv<BF16, 1, EPI_RESID, 1, 8, true>, dim3(w.n_tiles, 1, 1), dim3(64 * W), st,
                                     a, e0, e1);
                    else
                        launch_timed(k_gemv<BF16, 2, EPI_RESID, 1, 8, true>, dim3(w.n_tiles / 2, 1, 1), dim3(64 * W),
                                     st, a, e0, e1);
                    break;
                }
            }
            if (a.nt == 1)
                gemv_pg<KIND, 1, EPI_RESID>(st, w, a, e0, e1);
            else
                gemv_pg<KIND, 2, EPI_RESID>(st, w, a, e0, e1);
            break;
        case EPI_SILU:
            if (w.il == 16)
                gemv_pg<KIND, 2, EPI_SILU>(st, w, a, e0, e1);
            else
                gemv_pg<KIND, 4, EPI_SILU>(st, w, a, e0, e1);
            break;
        case EPI_MLP:
            if constexpr (KIND == BF16) {
                const int W = std::max(1, std::min(8, w.kb / 4));
                if (a.ax)
                    launch_timed(k_gemv<BF16, 2, EPI_MLP, 1, 8, false, true>, dim3(w.n_tiles / 2, 1, 1), dim3(64 * W),
                                 st, a, e0, e1);
                else
                    launch_timed(k_gemv<BF16, 2, EPI_MLP, 1>, dim3(w.n_tiles / 2, 1, 1), dim3(64 * W), st, a, e0, e1);
            }
            break;
        case EPI_ARGMAX:
            // bf16 lm_head when decoding: 96 or 128 columns per group (fewer, fuller
            // workgroups); 96 when the groups then fill the 256 CUs evenly (a
            // multiple of 256 groups)
            if constexpr (KIND == BF16) {
                if (a.p_total == 1 && w.n_tiles % 6 == 0 && (w.n_tiles / 6) % 256 == 0) {
                    gemv_pg<KIND, 6, EPI_ARGMAX>(st, w, a, e0, e1);
                    break;
                }
                if (a.p_total == 1 && w.n_tiles % 8 == 0) {
                    gemv_pg<KIND, 8, EPI_ARGMAX>(st, w, a, e0, e1);
                    break;
                }
            }
            gemv_pg<KIND, 2, EPI_ARGMAX>(st, w, a, e0, e1);
            break;
    }
}

void launch_gemv(hipStream_t st, int epi, const DMat& w, const GemvArgs& a, hipEvent_t start, hipEvent_t stop) {
    if (a.m <= 0) return;
    if (a.mm) {
        if (w.kind == INT4)
            gemm_kind<INT4>(st, epi, w, a, start, stop);
        else if (w.kind == INT8)
            gemm_kind<INT8>(st, epi, w, a, start, stop);
        else
            gemm_kind<BF16>(st, epi, w, a, start, stop);
        return;
    }
    if (w.kind == INT4)
        gemv_kind<INT4>(st, epi, w, a, start, stop);
    else if (w.kind == INT8)
        gemv_kind<INT8>(st, epi, w, a, start, stop);
    else
        gemv_kind<BF16>(st, epi, w, a, start, stop);
}

// The V tile in LDS (f32, rows = positions): at HD >= 64 rows are unpadded and
// the four 16-float quarters of row r are permuted by r % 4 (an XOR of column
// bits 4-5). The PV products read, per MFMA, 16 consecutive columns of 4
// consecutive rows (B[k][j] in lane j + 16k): with the permutation the 64 lanes
// hit 64 distinct banks; with rows padded by 4 floats they met 4 to a bank.
constexpr int vstride(int hd) { return hd >= 64 ? hd : hd + 4; }
template <int HD>
__device__ __forceinline__ int vcol(int r, int d) {
    return HD >= 64 ? d ^ ((r & 3) << 4) : d;
}

// ---------------------------------------------------------------------------
// Paged attention, split over the context (flash-decoding). A work item is
// (row group, span of P positions) x kv head: the rows of a group are
// consecutive rows of one chunk (<= 16), their queries (rows x GQA group)
// share the span's keys/values, loaded into LDS in one pass, and each row is
// causally limited to positions <= its own. q and the chunk's new keys are
// rotated here (rotate-half RoPE, src/model.rs:451-459); the new keys/values
// come from the q/k/v rows and are written to the cache slot of their row by
// the one item that covers it (KvCache::write, src/kv.rs:48-56). Each item
// writes per query the span's max score, sum of exponentials and weighted
// values; k_merge_pieces combines the spans.
// ---------------------------------------------------------------------------
// A work item covers NS consecutive sub-spans of P positions (at most 128
// positions: the eight cache blocks of its record). With NS > 1 the next
// sub-span's keys and values are loaded into registers while the current one
// is scored from LDS, and the softmax runs online across sub-spans: a
// running max and sum per query, the weighted values rescaled by
// exp(old max - new max) (flash-decoding within the work item).
//
// QM is the partials' query stride (the merge's layout); QL <= QM the queries an
// item holds (its LDS and registers), chosen per launch from the plan's largest
// row group so that small items leave room for more workgroups per CU. MINW:
// waves per SIMD the launch bounds ask for (3 lets three items share a CU).
template <int HD, int P, int QM, int NS, int QL = QM, int MINW = 2>
__global__ __launch_bounds__(256, MINW) void k_attn(AttnArgs a) {
    constexpr int HALF = HD / 2;
    // Items of several sub-spans at head_dim 128 with 16 or more queries (GQA
    // verify batches) score and weigh on bf16 MFMA with split operands: every f32
    // value x of q, k, the probabilities and v is held as hi = bf16(x) and lo =
    // bf16(x - hi), and a product as lo*hi + hi*lo + hi*hi
    // (v_mfma_f32_16x16x32_bf16, three per 32 inputs, f32 accumulation): 2^-16 of
    // each term against the f32 MFMA's 2^-24, at five times its rate. (cfg4's 8B
    // target: 92.6 -> 82.2 us per layer. At head_dim 64 with 8 queries the
    // splitting and the column reads of v cost more than the MFMA saves: 112.3
    // -> 126.7 us per layer for cfg3's target at 32 sequences.)
    constexpr bool BF = NS > 1 && HD >= 128 && HD % 32 == 0 && P % 32 == 0 && QL >= 16;
    // f32 rows padded by 4 floats (16-byte aligned): lanes reading one column of
    // consecutive rows (the MFMA operands) hit distinct banks
    __shared__ __align__(16) float ks[BF ? 1 : P][HD + 4];
    __shared__ __align__(16) float vs[BF ? 1 : P][vstride(HD)];
    __shared__ __align__(16) float qs[BF ? 1 : QL][HD + 4];
    // (BF) the pieces: q and k rows read 8 inputs per lane (16 bytes; rows 16
    // bytes apart in the bank map), v columns 2 bytes per lane (rows 8 bytes apart)
    __shared__ __align__(16) uint16_t qh[BF ? QL : 1][HD + 8], ql[BF ? QL : 1][HD + 8];
    __shared__ __align__(16) uint16_t kh[BF ? P : 1][HD + 8], kl[BF ? P : 1][HD + 8];
    __shared__ __align__(16) uint16_t vh[BF ? P : 1][HD + 4], vl[BF ? P : 1][HD + 4];
    // scores; (BF) after the softmax each slot holds its probability's pieces,
    // hi in the low half (written by the thread that read the score)
    __shared__ __align__(16) float pr[QL][P + 4];
    __shared__ int lim[QL];
    __shared__ float mrun[NS > 1 ? QL : 1], lrun[NS > 1 ? QL : 1], fac[NS > 1 ? QL : 1];

    static_assert(P <= 64 && P % 16 == 0 && 64 % P == 0, "a sub-span covers at most four cache blocks");
    static_assert(NS * P <= 128, "a work item covers at most the eight cache blocks of its record");
    static_assert(QL <= QM && QL % 8 == 0, "an item's queries fit the partials' stride");
    // grid (kv head, work item): every real item is dispatched before the
    // launch's unused capacity slots, which exit at once
    const Stamp stamp(a.stamp);
    const int h = blockIdx.x, wi = blockIdx.y;
    // the work item's record: one 64-byte read, everything else is arithmetic
    const int4* rec = (const int4*)(a.wrec + (size_t)wi * 16);
    const int4 r0 = rec[0], r1 = rec[1], rb = rec[2], rb2 = rec[3];
    const int row0 = r0.x, nrows = r0.y, crow0 = r0.z, cpos0 = r0.w;
    const int p0 = r1.x, p1 = r1.y;
    if (nrows == 0) return;  // an unused slot of the launch's capacity
    const int G = a.nh / a.nkv;
    const int Q = nrows * G;
    const int qd = a.nh * HD, kvd = a.nkv * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    auto blk = [&](int j) -> size_t {
        const int4 b = j < 4 ? rb : rb2;
        const int jj = j & 3;
        return (uint32_t)(jj == 0 ? b.x : jj == 1 ? b.y : jj == 2 ? b.z : b.w);
    };
    // rows of a chunk hold consecutive positions: row r sees positions <= its own
    const int pos_of_row0 = cpos0 + row0 - crow0;
    for (int q = tid; q < Q; q += 256) {
        lim[q] = pos_of_row0 + q / G;
        if (NS > 1) {
            mrun[q] = -INFINITY;
            lrun[q] = 0.0f;
        }
    }
    // A sub-span's loads are all issued before anything waits on one: the keys
    // and values (from the cache, or from the q/k/v rows for this chunk's new
    // positions) with the cos/sin of their positions, into registers. The
    // loads take no branches (a value loaded under a condition gets copied at
    // the join, which waits on it): positions past the sub-span read its last
    // position, and the LDS stores below select.
    constexpr int KI = P * (HALF / 4), KIT = (KI + 255) / 256;
    constexpr int VI = P * (HD / 4), VIT = (VI + 255) / 256;
    float4 ku[KIT], kw[KIT], kcs[KIT], ksn[KIT], vv[VIT];
    auto src_of = [&](int p, int col) -> const float* {  // position p's key (col 0) or value (col kvd)
        const bool cached = p < cpos0;
        const size_t crow = cached ? 0 : (size_t)(crow0 + p - cpos0);
        return cached ? (col ? a.vc : a.kc) + ((blk((p - p0) >> 4) * a.nkv + h) * 16 + (p & 15)) * HD
                      : a.qkv + crow * a.ld + qd + col + h * HD;
    };
    auto load_sub = [&](int sp0, int sp1) {
#pragma unroll
        for (int it = 0; it < KIT; it++) {
            const int i = min(tid + it * 256, KI - 1);
            const int d = (i % (HALF / 4)) * 4, p = min(sp0 + i / (HALF / 4), sp1 - 1);
            const float* kp = src_of(p, 0);
            ku[it] = ld_nt_f4(kp + d);
            kw[it] = ld_nt_f4(kp + d + HALF);
            // only new keys are rotated: cached positions all read the chunk's first
            // position (one cache line instead of a table row each)
            const int pr = max(p, cpos0);
            kcs[it] = *(const float4*)(a.cos_t + (size_t)pr * HALF + d);
            ksn[it] = *(const float4*)(a.sin_t + (size_t)pr * HALF + d);
        }
#pragma unroll
        for (int it = 0; it < VIT; it++) {
            const int i = min(tid + it * 256, VI - 1);
            const int d = (i % (HD / 4)) * 4, p = min(sp0 + i / (HD / 4), sp1 - 1);
            vv[it] = ld_nt_f4(src_of(p, kvd) + d);
        }
    };
    // q's loads go first: loads retire in order, so staging q then waits on q
    // alone while the keys and values are still in flight (and, on the VALU path
    // of one sub-span, the scores wait on the keys alone). 4 (d, d + HALF) pairs
    // per item; past the item's queries the last is loaded again (unconditional
    // loads) and not stored.
    constexpr int QI = QL * (HALF / 4), QIT = (QI + 255) / 256;
    const int qn = Q * (HALF / 4);
    float4 qx1[QIT], qx2[QIT], qcs[QIT], qsn[QIT];
#pragma unroll
    for (int it = 0; it < QIT; it++) {
        const int i = min(tid + it * 256, qn - 1);
        const int q = i / (HALF / 4), d = (i % (HALF / 4)) * 4, r = q / G, j = q % G, row = row0 + r;
        const int pos = pos_of_row0 + r;
        const float* src = a.qkv + (size_t)row * a.ld + (size_t)(h * G + j) * HD;
        qx1[it] = *(const float4*)(src + d);
        qx2[it] = *(const float4*)(src + d + HALF);
        qcs[it] = *(const float4*)(a.cos_t + (size_t)pos * HALF + d);
        qsn[it] = *(const float4*)(a.sin_t + (size_t)pos * HALF + d);
    }
    load_sub(p0, min(p0 + P, p1));
    // q, rotated
#pragma unroll
    for (int it = 0; it < QIT; it++) {
        const int i = tid + it * 256;
        if (i < qn) {
            const int q = i / (HALF / 4), d = (i % (HALF / 4)) * 4;
            const float a1[4] = {qx1[it].x, qx1[it].y, qx1[it].z, qx1[it].w};
            const float a2[4] = {qx2[it].x, qx2[it].y, qx2[it].z, qx2[it].w};
            const float cc[4] = {qcs[it].x, qcs[it].y, qcs[it].z, qcs[it].w};
            const float ss[4] = {qsn[it].x, qsn[it].y, qsn[it].z, qsn[it].w};
            float r1[4], r2[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                r1[e] = __fadd_rn(__fmul_rn(a1[e], cc[e]), __fmul_rn(-a2[e], ss[e]));
                r2[e] = __fadd_rn(__fmul_rn(a2[e], cc[e]), __fmul_rn(a1[e], ss[e]));
            }
            if constexpr (BF) {
                split4(r1, &qh[q][d], &ql[q][d]);
                split4(r2, &qh[q][d + HALF], &ql[q][d + HALF]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    qs[q][d + e] = r1[e];
                    qs[q][d + HALF + e] = r2[e];
                }
            }
        }
    }
    // From kAttnMfmaQueries queries on, the scores and the weighted values run on f32 MFMA
    // (v_mfma_f32_16x16x4f32; A[i][k] in lane i + 16k, B[k][j] in lane j + 16k,
    // D[4(l/16) + r][l%16] in register r of lane l) over 16 x 16 tiles, with
    // operands from LDS; fewer queries take the VALU loops. Rows of qs and pr
    // past Q hold stale values: they only reach output rows that are dropped.
    // items of several sub-spans exist only in launches whose largest row group
    // has kAttnMfmaQueries queries: all of them take the MFMA path (rows past Q
    // are dropped), so the VALU path's registers are not carried across sub-spans
    const bool mf = NS > 1 || Q >= kAttnMfmaQueries;
    const int mtu = (Q + 15) >> 4;
    constexpr int NTD = HD / 16;
    constexpr int TPW = ((QL + 15) / 16 * NTD + 3) / 4;  // weighted-value tiles per wave (MFMA)
    constexpr int OI = (QL * HD + 255) / 256;            // weighted values per thread (VALU)
    // MFMA rows past QL (a 16-row tile of fewer queries) read the last row and are dropped
    auto qrow = [&](int r) { return min(r, QL - 1); };
    f32x4 oc[TPW];
    float ov[OI];
#pragma unroll
    for (int j = 0; j < TPW; j++) oc[j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < OI; j++) ov[j] = 0.0f;
    float* partq = a.part + ((size_t)wi * a.nkv + h) * QM * (HD + 4);
    for (int s = 0; s < NS; s++) {
        const int sp0 = p0 + s * P;
        if (sp0 >= p1) break;
        const int sp1 = min(sp0 + P, p1);
        if (s > 0) __syncthreads();  // the previous sub-span's readers of ks, vs and pr are done
        // (BF) this group's new rows in the sub-span: written to the cache from
        // the staging registers (the pieces in LDS are not the f32 values)
        const int nr0 = max(max(sp0, cpos0), cpos0 + row0 - crow0);
        const int nr1 = min(sp1, cpos0 + row0 + nrows - crow0);
        auto cache_at = [&](int p, int d) {
            return ((blk((p - p0) >> 4) * a.nkv + h) * 16 + (p & 15)) * HD + d;
        };
        // keys (rotated when new) and values to LDS
#pragma unroll
        for (int it = 0; it < KIT; it++) {
            const int i = tid + it * 256;
            if (i < KI) {
                const int o = i / (HALF / 4), d = (i % (HALF / 4)) * 4, p = sp0 + o;
                const float a1[4] = {ku[it].x, ku[it].y, ku[it].z, ku[it].w};
                const float a2[4] = {kw[it].x, kw[it].y, kw[it].z, kw[it].w};
                const float cc[4] = {kcs[it].x, kcs[it].y, kcs[it].z, kcs[it].w};
                const float ss[4] = {ksn[it].x, ksn[it].y, ksn[it].z, ksn[it].w};
                const bool live = p < sp1, rot = live && p >= cpos0;
                float r1[4], r2[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float x1 = rot ? __fadd_rn(__fmul_rn(a1[e], cc[e]), __fmul_rn(-a2[e], ss[e])) : a1[e];
                    const float x2 = rot ? __fadd_rn(__fmul_rn(a2[e], cc[e]), __fmul_rn(a1[e], ss[e])) : a2[e];
                    r1[e] = live ? x1 : 0.0f;
                    r2[e] = live ? x2 : 0.0f;
                }
                if constexpr (BF) {
                    split4(r1, &kh[o][d], &kl[o][d]);
                    split4(r2, &kh[o][d + HALF], &kl[o][d + HALF]);
                    if (p >= nr0 && p < nr1) {
                        *(float4*)(a.kc + cache_at(p, d)) = make_float4(r1[0], r1[1], r1[2], r1[3]);
                        *(float4*)(a.kc + cache_at(p, d + HALF)) = make_float4(r2[0], r2[1], r2[2], r2[3]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        ks[o][d + e] = r1[e];
                        ks[o][d + HALF + e] = r2[e];
                    }
                }
            }
        }
        auto store_v = [&]() {
#pragma unroll
            for (int it = 0; it < VIT; it++) {
                const int i = tid + it * 256;
                if (i < VI) {
                    const int o = i / (HD / 4), d = (i % (HD / 4)) * 4, p = sp0 + o;
                    const bool live = p < sp1;
                    const float v4[4] = {live ? vv[it].x : 0.0f, live ? vv[it].y : 0.0f, live ? vv[it].z : 0.0f,
                                         live ? vv[it].w : 0.0f};
                    if constexpr (BF) {
                        split4(v4, &vh[o][d], &vl[o][d]);
                        if (p >= nr0 && p < nr1) *(float4*)(a.vc + cache_at(p, d)) = make_float4(v4[0], v4[1], v4[2], v4[3]);
                    } else {
                        *(float4*)&vs[o][vcol<HD>(o, d)] = make_float4(v4[0], v4[1], v4[2], v4[3]);
                    }
                }
            }
        };
        // this group's new rows in the sub-span go to the cache (from ks and vs;
        // other items read new positions from the q/k/v rows, never the cache)
        auto new_rows_to_cache = [&]() {
            if constexpr (!BF) {
                for (int i = tid; i < (nr1 - nr0) * HD; i += 256) {
                    const int p = nr0 + i / HD, d = i % HD, o = p - sp0;
                    const size_t at = cache_at(p, d);
                    a.kc[at] = ks[o][d];
                    a.vc[at] = vs[o][vcol<HD>(o, d)];
                }
            }
        };
        // An item of one sub-span scores its keys while its values are still
        // arriving: the values go to LDS after the softmax (before the barrier
        // that precedes the weighted values). With more sub-spans the next one's
        // loads reuse the value registers right after the first barrier.
        constexpr bool late_v = NS == 1;
        if (!late_v) store_v();
        __syncthreads();
        // the next sub-span's loads fly while this one is scored
        if (NS > 1 && sp1 < p1) load_sub(sp1, min(sp1 + P, p1));
        if (!late_v) new_rows_to_cache();
        if (mf) {
            // scores, scaled, into pr
            constexpr int NTP = P / 16;
            for (int ti = wave; ti < mtu * NTP; ti += 4) {
                const int mt = ti / NTP, nt = ti % NTP, kk = lane >> 4;
                f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (BF) {
                    // A: q row mt*16 + lane%16, inputs d0 + 8 (lane/16) .. + 7; B: the same inputs of key nt*16 + lane%16
                    const int qr = qrow(mt * 16 + (lane & 15)), kr = nt * 16 + (lane & 15);
#pragma unroll
                    for (int d0 = 0; d0 < HD; d0 += 32) {
                        const int dd = d0 + 8 * kk;
                        const bf16x8 ah = as_bf16x8(*(const u16x8*)&qh[qr][dd]), al = as_bf16x8(*(const u16x8*)&ql[qr][dd]);
                        const bf16x8 bh = as_bf16x8(*(const u16x8*)&kh[kr][dd]), bl = as_bf16x8(*(const u16x8*)&kl[kr][dd]);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
                    }
                } else {
                    const float* qa = &qs[qrow(mt * 16 + (lane & 15))][kk];
                    const float* kb = &ks[nt * 16 + (lane & 15)][kk];
#pragma unroll
                    for (int d0 = 0; d0 < HD; d0 += 4) c = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[d0], kb[d0], c, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (mt * 16 + 4 * kk + r < QL) pr[mt * 16 + 4 * kk + r][nt * 16 + (lane & 15)] = c[r] * a.scale;
            }
            __syncthreads();
        }
        // Scores and their softmax statistics in one pass: item i = q * P + o, so
        // each wave holds whole queries (one per P lanes) and reduces them in
        // registers. Across sub-spans the exponentials are taken against the
        // running max, and the running sum is rescaled to it.
        // (unrolled to its bound: a loop here would make the compiler drain the
        // value loads still in flight before entering it)
#pragma unroll
        for (int pass = 0; pass < (QL * P + 255) / 256; pass++) {
            const int base = wave * 64 + pass * 256;
            if (base >= Q * P) break;
            const int i = base + lane, q = i / P, o = i % P, p = sp0 + o;
            float sc = -INFINITY;
            if (q < Q && p < sp1 && p <= lim[q] && mf) {
                sc = pr[q][o];
            } else if (!BF && q < Q && p < sp1 && p <= lim[q]) {
                const float4* kr = (const float4*)&ks[o][0];
                const float4* qr = (const float4*)&qs[q][0];
                float acc = 0.0f;
#pragma unroll
                for (int e4 = 0; e4 < HD / 4; e4++) {
                    const float4 kv = kr[e4], qv = qr[e4];
                    acc = fmaf(qv.x, kv.x, acc);
                    acc = fmaf(qv.y, kv.y, acc);
                    acc = fmaf(qv.z, kv.z, acc);
                    acc = fmaf(qv.w, kv.w, acc);
                }
                sc = acc * a.scale;
            }
            float mx = group_reduce<P, true>(sc), mold = -INFINITY;
            if (NS > 1) {
                mold = q < Q ? mrun[q] : -INFINITY;
                mx = fmaxf(mold, mx);
            }
            const float e = (sc == -INFINITY) ? 0.0f : dev_exp(sc - mx);
            const float sum = group_reduce<P, false>(e);
            if (q < Q) {
                if constexpr (BF) {
                    const uint32_t eh = f32_to_bf16_bits(e), el = f32_to_bf16_bits(e - bf16_bits_to_f32(eh));
                    ((uint32_t*)&pr[q][0])[o] = eh | (el << 16);
                } else {
                    pr[q][o] = e;
                }
                if (o == 0) {
                    if (NS == 1) {
                        partq[q * (HD + 4)] = mx;
                        partq[q * (HD + 4) + 1] = sum;
                    } else {
                        const float f = mold == -INFINITY ? 0.0f : dev_exp(mold - mx);
                        fac[q] = f;
                        lrun[q] = fmaf(lrun[q], f, sum);
                        mrun[q] = mx;
                    }
                }
            }
        }
        if (late_v) store_v();
        __syncthreads();
        if (late_v) new_rows_to_cache();
        if (mf) {
            // weighted values: O = fac O + P V, tile ti = wave + 4 j
#pragma unroll
            for (int j = 0; j < TPW; j++) {
                const int ti = wave + 4 * j;
                if (ti < mtu * NTD) {
                    const int mt = ti / NTD, nd = ti % NTD, kk = lane >> 4;
                    if (NS > 1) {
#pragma unroll
                        for (int r = 0; r < 4; r++) oc[j][r] *= fac[qrow(mt * 16 + 4 * kk + r)];
                    }
                    if constexpr (BF) {
                        // A: the probabilities of row mt*16 + lane%16 at positions k0 + 8 (lane/16) .. + 7
                        // (pairs (hi, lo) per slot, split here); B: value column nd*16 + lane%16 at the same positions
                        const uint32_t* prow = (const uint32_t*)&pr[qrow(mt * 16 + (lane & 15))][0];
                        const int vc = nd * 16 + (lane & 15);
#pragma unroll
                        for (int k0 = 0; k0 < P; k0 += 32) {
                            const int kp = k0 + 8 * kk;
                            const u32x4 w0 = *(const u32x4*)&prow[kp], w1 = *(const u32x4*)&prow[kp + 4];
                            u32x4 ah4, al4, bh4, bl4;
#pragma unroll
                            for (int e = 0; e < 2; e++) {
                                ah4[e] = (w0[2 * e] & 0xFFFFu) | (w0[2 * e + 1] << 16);
                                al4[e] = (w0[2 * e] >> 16) | (w0[2 * e + 1] & 0xFFFF0000u);
                                ah4[e + 2] = (w1[2 * e] & 0xFFFFu) | (w1[2 * e + 1] << 16);
                                al4[e + 2] = (w1[2 * e] >> 16) | (w1[2 * e + 1] & 0xFFFF0000u);
                            }
#pragma unroll
                            for (int e = 0; e < 4; e++) {
                                bh4[e] = (uint32_t)vh[kp + 2 * e][vc] | ((uint32_t)vh[kp + 2 * e + 1][vc] << 16);
                                bl4[e] = (uint32_t)vl[kp + 2 * e][vc] | ((uint32_t)vl[kp + 2 * e + 1][vc] << 16);
                            }
                            const bf16x8 ah = as_bf16x8(ah4), al = as_bf16x8(al4), bh = as_bf16x8(bh4), bl = as_bf16x8(bl4);
                            oc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, oc[j], 0, 0, 0);
                            oc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, oc[j], 0, 0, 0);
                            oc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, oc[j], 0, 0, 0);
                        }
                    } else {
                        const float* pa = &pr[qrow(mt * 16 + (lane & 15))][kk];
                        const float* vb = &vs[kk][vcol<HD>(kk, nd * 16 + (lane & 15))];  // rows kk + k0: k0 % 4 == 0
#pragma unroll
                        for (int k0 = 0; k0 < P; k0 += 4)
                            oc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[k0], vb[k0 * vstride(HD)], oc[j], 0, 0, 0);
                    }
                }
            }
        } else {
            // weighted values: item tid + 256 j is (query, dim)
#pragma unroll
            for (int j = 0; j < OI; j++) {
                const int i = tid + j * 256;
                if (i < Q * HD) {
                    const int q = i / HD, d = i % HD;
                    const float4* prr = (const float4*)&pr[q][0];
                    float acc = NS > 1 ? ov[j] * fac[q] : 0.0f;
#pragma unroll
                    for (int o4 = 0; o4 < P / 4; o4++) {
                        const float4 w = prr[o4];
                        acc = fmaf(w.x, vs[4 * o4][vcol<HD>(0, d)], acc);
                        acc = fmaf(w.y, vs[4 * o4 + 1][vcol<HD>(1, d)], acc);
                        acc = fmaf(w.z, vs[4 * o4 + 2][vcol<HD>(2, d)], acc);
                        acc = fmaf(w.w, vs[4 * o4 + 3][vcol<HD>(3, d)], acc);
                    }
                    ov[j] = acc;
                }
            }
        }
    }
    // the work item's partial: max score, sum of exponentials, weighted values
    if (NS > 1)
        for (int q = tid; q < Q; q += 256) {
            partq[q * (HD + 4)] = mrun[q];
            partq[q * (HD + 4) + 1] = lrun[q];
        }
    if (mf) {
#pragma unroll
        for (int j = 0; j < TPW; j++) {
            const int ti = wave + 4 * j;
            if (ti < mtu * NTD) {
                const int mt = ti / NTD, nd = ti % NTD, kk = lane >> 4;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int q = mt * 16 + 4 * kk + r;
                    if (q < Q) partq[q * (HD + 4) + 4 + nd * 16 + (lane & 15)] = oc[j][r];
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < OI; j++) {
            const int i = tid + j * 256;
            if (i < Q * HD) partq[(i / HD) * (HD + 4) + 4 + i % HD] = ov[j];
        }
    }
    stamp.end();
}

// Long-chunk attention (prefill at hd 64 and 128): one workgroup per (kv head, item),
// an item being up to 2 * (32 / G) consecutive rows of one chunk (at most 64
// queries, G query heads per kv head). The workgroup walks every position the
// item's last row sees (or a part of them) in blocks of P (64 at hd 64, 32 at
// hd 128, so that two workgroups fit a CU's LDS): keys (rotated when new) and values go
// through LDS, shared by the four waves; each wave owns 16 queries and keeps
// their online softmax (running max and sum, weighted values) in registers,
// scores and weighted values on f32 MFMA. The next block's loads are issued
// before the current one is scored. The item's two row halves write their
// partials (max score, sum of exponentials, weighted values) to the work-item
// slots their record names: the layout the span merge reads, one span per part.
template <int HD, int P>
__global__ __launch_bounds__(256, 2) void k_attn_flash(AttnArgs a) {
    constexpr int HALF = HD / 2, QM = 32, NTD = HD / 16;
    static_assert(P % 16 == 0 && 64 % P == 0, "blocks of whole 16-position MFMA tiles");
    __shared__ __align__(16) float ks[P][HD + 4];
    __shared__ __align__(16) float vs[P][vstride(HD)];
    __shared__ __align__(16) float qs[64][HD + 4];
    __shared__ __align__(16) float pw[4][16][P + 4];
    __shared__ int lim[64];

    const int h = blockIdx.x, fi = blockIdx.y;
    const int4* rec = (const int4*)(a.wrec + (size_t)fi * 16);
    const int4 r0 = rec[0], r1 = rec[1], r2 = rec[2];
    const int row0 = r0.x, nrows = r0.y, crow0 = r0.z, cpos0 = r0.w;
    // the part's positions [p0, L), the chunk's block table, the partial slots of the two row halves
    const int p0 = r1.x, L = r1.y, boff = r1.z, slot0 = r1.w, slot1 = r2.x;
    if (nrows == 0) return;  // an unused slot of the launch's capacity
    const int G = a.nh / a.nkv, Q = nrows * G, RQ = QM / G;
    const int qd = a.nh * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kk = lane >> 4, c16 = lane & 15;
    const int32_t* bt = a.btab + boff;
    const int pos_of_row0 = cpos0 + row0 - crow0;
    for (int q = tid; q < 64; q += 256) lim[q] = q < Q ? pos_of_row0 + q / G : -1;

    // position p's key (col 0) or value (col HD * nkv): the cache, or this chunk's q/k/v rows
    auto src_of = [&](int p, int col) -> const float* {
        return p < cpos0 ? (col ? a.vc : a.kc) + (((size_t)(uint32_t)bt[p >> 4] * a.nkv + h) * 16 + (p & 15)) * HD
                         : a.qkv + (size_t)(crow0 + p - cpos0) * a.ld + qd + col + h * HD;
    };
    constexpr int KIT = P * (HALF / 4) / 256, VIT = P * (HD / 4) / 256;
    static_assert(KIT * 256 == P * (HALF / 4) && VIT * 256 == P * (HD / 4), "whole iterations");
    float4 ku[KIT], kw[KIT], kcs[KIT], ksn[KIT], vv[VIT];
    auto load_blk = [&](int b0) {
#pragma unroll
        for (int it = 0; it < KIT; it++) {
            const int i = tid + it * 256, d = (i % (HALF / 4)) * 4, p = min(b0 + i / (HALF / 4), L - 1);
            const float* kp = src_of(p, 0);
            ku[it] = ld_nt_f4(kp + d);
            kw[it] = ld_nt_f4(kp + d + HALF);
            const int pr = max(p, cpos0);
            kcs[it] = *(const float4*)(a.cos_t + (size_t)pr * HALF + d);
            ksn[it] = *(const float4*)(a.sin_t + (size_t)pr * HALF + d);
        }
#pragma unroll
        for (int it = 0; it < VIT; it++) {
            const int i = tid + it * 256, d = (i % (HD / 4)) * 4, p = min(b0 + i / (HD / 4), L - 1);
            vv[it] = ld_nt_f4(src_of(p, a.nkv * HD) + d);
        }
    };
    load_blk(p0);
    // the queries, rotated; rows past Q are zero
    for (int i = tid; i < 64 * (HALF / 4); i += 256) {
        const int q = i / (HALF / 4), d = (i % (HALF / 4)) * 4;
        float r1v[4] = {0, 0, 0, 0}, r2v[4] = {0, 0, 0, 0};
        if (q < Q) {
            const int r = q / G, j = q % G, pos = pos_of_row0 + r;
            const float* src = a.qkv + (size_t)(row0 + r) * a.ld + (size_t)(h * G + j) * HD;
            const float4 x1 = *(const float4*)(src + d), x2 = *(const float4*)(src + d + HALF);
            const float4 c = *(const float4*)(a.cos_t + (size_t)pos * HALF + d);
            const float4 sn = *(const float4*)(a.sin_t + (size_t)pos * HALF + d);
            const float a1[4] = {x1.x, x1.y, x1.z, x1.w}, a2[4] = {x2.x, x2.y, x2.z, x2.w};
            const float cc[4] = {c.x, c.y, c.z, c.w}, ss[4] = {sn.x, sn.y, sn.z, sn.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                r1v[e] = __fadd_rn(__fmul_rn(a1[e], cc[e]), __fmul_rn(-a2[e], ss[e]));
                r2v[e] = __fadd_rn(__fmul_rn(a2[e], cc[e]), __fmul_rn(a1[e], ss[e]));
            }
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            qs[q][d + e] = r1v[e];
            qs[q][d + HALF + e] = r2v[e];
        }
    }

    float mrow[4], lrow[4];
    f32x4 oc[NTD];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        mrow[r] = -INFINITY;
        lrow[r] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < NTD; j++) oc[j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    const int nblk = (L - p0 + P - 1) / P;
    const int q0 = wave * 16;
    for (int b = 0; b < nblk; b++) {
        const int b0 = p0 + b * P;
        if (b > 0) __syncthreads();  // the previous block's readers of ks, vs and pw are done
#pragma unroll
        for (int it = 0; it < KIT; it++) {
            const int i = tid + it * 256, o = i / (HALF / 4), d = (i % (HALF / 4)) * 4, p = b0 + o;
            const float a1[4] = {ku[it].x, ku[it].y, ku[it].z, ku[it].w};
            const float a2[4] = {kw[it].x, kw[it].y, kw[it].z, kw[it].w};
            const float cc[4] = {kcs[it].x, kcs[it].y, kcs[it].z, kcs[it].w};
            const float ss[4] = {ksn[it].x, ksn[it].y, ksn[it].z, ksn[it].w};
            const bool live = p < L, rot = live && p >= cpos0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x1 = rot ? __fadd_rn(__fmul_rn(a1[e], cc[e]), __fmul_rn(-a2[e], ss[e])) : a1[e];
                const float x2 = rot ? __fadd_rn(__fmul_rn(a2[e], cc[e]), __fmul_rn(a1[e], ss[e])) : a2[e];
                ks[o][d + e] = live ? x1 : 0.0f;
                ks[o][d + HALF + e] = live ? x2 : 0.0f;
            }
        }
#pragma unroll
        for (int it = 0; it < VIT; it++) {
            const int i = tid + it * 256, o = i / (HD / 4), d = (i % (HD / 4)) * 4;
            const bool live = b0 + o < L;
            *(float4*)&vs[o][vcol<HD>(o, d)] = make_float4(live ? vv[it].x : 0.0f, live ? vv[it].y : 0.0f,
                                              live ? vv[it].z : 0.0f, live ? vv[it].w : 0.0f);
        }
        __syncthreads();
        if (b + 1 < nblk) load_blk(b0 + P);
        // this item's new rows in the block go to the cache
        {
            const int n0 = max(b0, pos_of_row0), n1 = min(b0 + P, pos_of_row0 + nrows);
            for (int i = tid; i < (n1 - n0) * HD; i += 256) {
                const int p = n0 + i / HD, d = i % HD, o = p - b0;
                const size_t at = (((size_t)(uint32_t)bt[p >> 4] * a.nkv + h) * 16 + (p & 15)) * HD + d;
                a.kc[at] = ks[o][d];
                a.vc[at] = vs[o][vcol<HD>(o, d)];
            }
        }
        // the wave's 16 x 64 scores (v_mfma_f32_16x16x4f32: A[i][k] in lane i + 16k,
        // B[k][j] in lane j + 16k, D[4(l/16) + r][l%16] in register r of lane l)
        f32x4 sc[P / 16];
#pragma unroll
        for (int nt = 0; nt < P / 16; nt++) {
            const float* qa = &qs[q0 + c16][kk];
            const float* kb = &ks[nt * 16 + c16][kk];
            f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int d0 = 0; d0 < HD; d0 += 4) c = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[d0], kb[d0], c, 0, 0, 0);
            sc[nt] = c;
        }
        // online softmax of each of the lane's four query rows; a row's 64 scores
        // sit in the 16 lanes of its lane group, four per lane
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int lq = lim[q0 + 4 * kk + r];
            float mx = -INFINITY;
#pragma unroll
            for (int nt = 0; nt < P / 16; nt++) {
                const float v = b0 + nt * 16 + c16 <= lq ? sc[nt][r] * a.scale : -INFINITY;
                sc[nt][r] = v;
                mx = fmaxf(mx, v);
            }
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 16));
            const float mn = fmaxf(mrow[r], mx);
            const float f = mrow[r] == -INFINITY ? 0.0f : dev_exp(mrow[r] - mn);
            float sum = 0.0f;
#pragma unroll
            for (int nt = 0; nt < P / 16; nt++) {
                const float e = sc[nt][r] == -INFINITY ? 0.0f : dev_exp(sc[nt][r] - mn);
                pw[wave][4 * kk + r][nt * 16 + c16] = e;
                sum += e;
            }
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 16);
            lrow[r] = fmaf(lrow[r], f, sum);
            mrow[r] = mn;
#pragma unroll
            for (int j = 0; j < NTD; j++) oc[j][r] *= f;
        }
        __syncthreads();  // pw rows are read across the wave's lanes
        // weighted values: O += P V over the block's 64 positions
#pragma unroll
        for (int j = 0; j < NTD; j++) {
            const float* pa = &pw[wave][c16][kk];
            const float* vb = &vs[kk][vcol<HD>(kk, j * 16 + c16)];  // rows kk + k0: k0 % 4 == 0
#pragma unroll
            for (int k0 = 0; k0 < P; k0 += 4)
                oc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[k0], vb[k0 * vstride(HD)], oc[j], 0, 0, 0);
        }
    }
    // the partials of the item's two row halves
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int q = q0 + 4 * kk + r;
        if (q < Q) {
            const int half = q / G >= RQ ? 1 : 0;
            float* pq = a.part + (((size_t)(half ? slot1 : slot0) * a.nkv + h) * QM + (q - half * RQ * G)) * (HD + 4);
            if (c16 == 0) {
                pq[0] = mrow[r];
                pq[1] = lrow[r];
            }
#pragma unroll
            for (int j = 0; j < NTD; j++) pq[4 + j * 16 + c16] = oc[j][r];
        }
    }
}

// Merge of the spans of each (row, head) into the attention output, written
// as the output projection's pieces. One wave per (k-block, pass), KBW waves
// (consecutive k-blocks) per workgroup; the four lanes of a (row, 8 dims) pair
// (one per piece) share the spans.
template <int HD, int QM, int CK, int KBW = 1>
__global__ __launch_bounds__(64 * KBW) void k_merge_pieces(AttnArgs a, int m, void* __restrict__ out,
                                                           float* __restrict__ xs, int passes) {
    const Stamp stamp(a.stamp);
    const int kb = blockIdx.x * KBW + (int)(threadIdx.x >> 6), pass = blockIdx.y, lane = threadIdx.x & 63;
    const int c = lane & 15, row = pass * 4 + (c >> 2), piece = c & 3;
    const int k0 = kb * 32 + (lane >> 4) * 8;
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (row < m && k0 < a.nh * HD)
        merge_spans<8>(a.part, *(const int4*)(a.mrec + (size_t)row * 4), a.nh, a.nkv, HD, QM, k0, piece, v);
    write_pieces<CK>(v, kb, pass, passes, row, piece, lane, out, xs);
    stamp.end();
}

// Decode attention for items of one span and at most QL <= 8 queries (the
// rows of a decode or verify step x the GQA group), with the keys and values
// used from the registers they are loaded into. KL = HD/8 lanes hold a key
// (4 + 4 inputs of its rotation pairs each): they dot it with every query
// (rotated queries read from LDS) and sum across their group. HD/4 lanes hold a
// value row (4 dims each): each weighs its rows by the probabilities and the
// partial sums meet across the wave's rows (lane swaps) and the four waves (LDS,
// summed in wave order). Only the queries, the scores and the per-wave sums go
// through LDS (6 or 12 KB at hd 64 for 4 or 8 queries), so registers, not LDS,
// bound the launch.
// Same records, partials and cache writes as k_attn.
template <int HD, int P, int QM, int QL, int MINW>
__global__ __launch_bounds__(256, MINW) void k_attn_dec(AttnArgs a) {
    constexpr int HALF = HD / 2;
    constexpr int KL = HALF / 4, KIT = P * KL / 256;  // lanes per key, key passes
    constexpr int VL = HD / 4, VIT = P * VL / 256;    // lanes per value row, value passes
    static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
    static_assert(KIT >= 1 && P * KL % 256 == 0 && VIT >= 1 && P * VL % 256 == 0, "whole passes of 256 lanes");
    static_assert(QL <= 8 && QL <= QM, "decode-sized items");
    __shared__ __align__(16) float qs[QL][HD];
    __shared__ __align__(16) float pr[QL][P + 4];
    __shared__ __align__(16) float ow[4][QL][HD];
    __shared__ int lim[QL];
    const Stamp stamp(a.stamp);
    const int h = blockIdx.x, wi = blockIdx.y;
    const int4* rec = (const int4*)(a.wrec + (size_t)wi * 16);
    const int4 r0 = rec[0], r1 = rec[1], rb = rec[2], rb2 = rec[3];
    const int row0 = r0.x, nrows = r0.y, crow0 = r0.z, cpos0 = r0.w;
    const int p0 = r1.x, p1 = r1.y;
    if (nrows == 0) return;  // an unused slot of the launch's capacity
    const int G = a.nh / a.nkv, Q = nrows * G;
    const int qd = a.nh * HD, kvd = a.nkv * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    auto blk = [&](int j) -> size_t {
        const int4 b = j < 4 ? rb : rb2;
        const int jj = j & 3;
        return (uint32_t)(jj == 0 ? b.x : jj == 1 ? b.y : jj == 2 ? b.z : b.w);
    };
    auto cache_at = [&](int p, int d) -> size_t { return ((blk((p - p0) >> 4) * a.nkv + h) * 16 + (p & 15)) * HD + d; };
    auto src_of = [&](int p, int col) -> const float* {  // position p's key (col 0) or value (col kvd)
        return p < cpos0 ? (col ? a.vc : a.kc) + cache_at(p, 0)
                         : a.qkv + (size_t)(crow0 + p - cpos0) * a.ld + qd + col + h * HD;
    };
    const int pos_of_row0 = cpos0 + row0 - crow0;
    // this group's new rows in the span (written to the cache by this item)
    const int nr0 = max(max(p0, cpos0), pos_of_row0), nr1 = min(p1, pos_of_row0 + nrows);
    for (int q = tid; q < Q; q += 256) lim[q] = pos_of_row0 + q / G;
    // loads, none of them under a branch: q, the keys (with the cos/sin of new
    // positions), the values; positions past the span read its last position
    constexpr int QI = QL * (HALF / 4), QIT = (QI + 255) / 256;
    const int qn = Q * (HALF / 4);
    float4 qx1[QIT], qx2[QIT], qcs[QIT], qsn[QIT];
#pragma unroll
    for (int it = 0; it < QIT; it++) {
        const int i = min(tid + it * 256, qn - 1);
        const int q = i / (HALF / 4), d = (i % (HALF / 4)) * 4, r = q / G, j = q % G;
        const float* src = a.qkv + (size_t)(row0 + r) * a.ld + (size_t)(h * G + j) * HD;
        qx1[it] = *(const float4*)(src + d);
        qx2[it] = *(const float4*)(src + d + HALF);
        qcs[it] = *(const float4*)(a.cos_t + (size_t)(pos_of_row0 + r) * HALF + d);
        qsn[it] = *(const float4*)(a.sin_t + (size_t)(pos_of_row0 + r) * HALF + d);
    }
    const int kd = (tid % KL) * 4, vd = (tid % VL) * 4;
    float4 ku[KIT], kw[KIT], kcs[KIT], ksn[KIT], vv[VIT];
#pragma unroll
    for (int it = 0; it < KIT; it++) {
        const int p = min(p0 + tid / KL + it * (256 / KL), p1 - 1);
        const float* kp = src_of(p, 0);
        ku[it] = ld_nt_f4(kp + kd);
        kw[it] = ld_nt_f4(kp + kd + HALF);
        const int pc = max(p, cpos0);  // cached keys are not rotated: one table row for all
        kcs[it] = *(const float4*)(a.cos_t + (size_t)pc * HALF + kd);
        ksn[it] = *(const float4*)(a.sin_t + (size_t)pc * HALF + kd);
    }
#pragma unroll
    for (int it = 0; it < VIT; it++) {
        const int p = min(p0 + tid / VL + it * (256 / VL), p1 - 1);
        vv[it] = ld_nt_f4(src_of(p, kvd) + vd);
    }
    // q, rotated
#pragma unroll
    for (int it = 0; it < QIT; it++) {
        const int i = tid + it * 256;
        if (i < qn) {
            const int q = i / (HALF / 4), d = (i % (HALF / 4)) * 4;
            const float a1[4] = {qx1[it].x, qx1[it].y, qx1[it].z, qx1[it].w};
            const float a2[4] = {qx2[it].x, qx2[it].y, qx2[it].z, qx2[it].w};
            const float cc[4] = {qcs[it].x, qcs[it].y, qcs[it].z, qcs[it].w};
            const float ss[4] = {qsn[it].x, qsn[it].y, qsn[it].z, qsn[it].w};
            float4 o1, o2;
            o1.x = __fadd_rn(__fmul_rn(a1[0], cc[0]), __fmul_rn(-a2[0], ss[0]));
            o1.y = __fadd_rn(__fmul_rn(a1[1], cc[1]), __fmul_rn(-a2[1], ss[1]));
            o1.z = __fadd_rn(__fmul_rn(a1[2], cc[2]), __fmul_rn(-a2[2], ss[2]));
            o1.w = __fadd_rn(__fmul_rn(a1[3], cc[3]), __fmul_rn(-a2[3], ss[3]));
            o2.x = __fadd_rn(__fmul_rn(a2[0], cc[0]), __fmul_rn(a1[0], ss[0]));
            o2.y = __fadd_rn(__fmul_rn(a2[1], cc[1]), __fmul_rn(a1[1], ss[1]));
            o2.z = __fadd_rn(__fmul_rn(a2[2], cc[2]), __fmul_rn(a1[2], ss[2]));
            o2.w = __fadd_rn(__fmul_rn(a2[3], cc[3]), __fmul_rn(a1[3], ss[3]));
            *(float4*)&qs[q][d] = o1;
            *(float4*)&qs[q][d + HALF] = o2;
        }
    }
    __syncthreads();
    // scores: each key group dots its key with every query, sums across its KL
    // lanes, and the group's first lane stores the scaled score (or -inf past
    // the span or the query's own position)
#pragma unroll
    for (int it = 0; it < KIT; it++) {
        const int o = tid / KL + it * (256 / KL), p = p0 + o;
        const bool live = p < p1, rot = live && p >= cpos0;
        const float a1[4] = {ku[it].x, ku[it].y, ku[it].z, ku[it].w};
        const float a2[4] = {kw[it].x, kw[it].y, kw[it].z, kw[it].w};
        const float cc[4] = {kcs[it].x, kcs[it].y, kcs[it].z, kcs[it].w};
        const float ss[4] = {ksn[it].x, ksn[it].y, ksn[it].z, ksn[it].w};
        float k1[4], k2[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            k1[e] = rot ? __fadd_rn(__fmul_rn(a1[e], cc[e]), __fmul_rn(-a2[e], ss[e])) : a1[e];
            k2[e] = rot ? __fadd_rn(__fmul_rn(a2[e], cc[e]), __fmul_rn(a1[e], ss[e])) : a2[e];
        }
        if (p >= nr0 && p < nr1) {
            *(float4*)(a.kc + cache_at(p, kd)) = make_float4(k1[0], k1[1], k1[2], k1[3]);
            *(float4*)(a.kc + cache_at(p, kd + HALF)) = make_float4(k2[0], k2[1], k2[2], k2[3]);
        }
#pragma unroll
        for (int q = 0; q < QL; q++) {
            const float4 x1 = *(const float4*)&qs[q][kd], x2 = *(const float4*)&qs[q][kd + HALF];
            float s = 0.0f;
            s = fmaf(x1.x, k1[0], s);
            s = fmaf(x1.y, k1[1], s);
            s = fmaf(x1.z, k1[2], s);
            s = fmaf(x1.w, k1[3], s);
            s = fmaf(x2.x, k2[0], s);
            s = fmaf(x2.y, k2[1], s);
            s = fmaf(x2.z, k2[2], s);
            s = fmaf(x2.w, k2[3], s);
            s = group_reduce<KL, false>(s);
            if (tid % KL == 0 && q < Q) pr[q][o] = (live && p <= lim[q]) ? s * a.scale : -INFINITY;
        }
    }
    __syncthreads();
    // softmax statistics per query (one query per P lanes), exponentials in place
    float* partq = a.part + ((size_t)wi * a.nkv + h) * QM * (HD + 4);
#pragma unroll
    for (int pass = 0; pass < (QL * P + 255) / 256; pass++) {
        const int base = wave * 64 + pass * 256;
        if (base >= Q * P) break;
        const int i = base + lane, q = i / P, o = i % P;
        const float sc = q < Q ? pr[q][o] : -INFINITY;
        const float mx = group_reduce<P, true>(sc);
        const float e = (sc == -INFINITY) ? 0.0f : dev_exp(sc - mx);
        const float sum = group_reduce<P, false>(e);
        if (q < Q) {
            pr[q][o] = e;
            if (o == 0) {
                partq[q * (HD + 4)] = mx;
                partq[q * (HD + 4) + 1] = sum;
            }
        }
    }
    __syncthreads();
    // weighted values: this lane's value rows, then the wave's other rows of the
    // same dims, then the four waves
    float acc[QL][4];
#pragma unroll
    for (int q = 0; q < QL; q++) acc[q][0] = acc[q][1] = acc[q][2] = acc[q][3] = 0.0f;
#pragma unroll
    for (int it = 0; it < VIT; it++) {
        const int o = tid / VL + it * (256 / VL), p = p0 + o;
        if (p >= nr0 && p < nr1) *(float4*)(a.vc + cache_at(p, vd)) = vv[it];
#pragma unroll
        for (int q = 0; q < QL; q++) {
            const float w = pr[q][o];  // 0 past the span and the query's position
            acc[q][0] = fmaf(w, vv[it].x, acc[q][0]);
            acc[q][1] = fmaf(w, vv[it].y, acc[q][1]);
            acc[q][2] = fmaf(w, vv[it].z, acc[q][2]);
            acc[q][3] = fmaf(w, vv[it].w, acc[q][3]);
        }
    }
#pragma unroll
    for (int q = 0; q < QL; q++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float v = acc[q][e];
            if constexpr (VL == 16) {
                v = reduce_rows<false, true>(v);  // lanes l, l^16, l^32, l^48
            } else {
                const auto hh = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
                v = __uint_as_float(hh[0]) + __uint_as_float(hh[1]);  // lanes l, l^32
            }
            acc[q][e] = v;
        }
        if (lane < VL) *(float4*)&ow[wave][q][vd] = make_float4(acc[q][0], acc[q][1], acc[q][2], acc[q][3]);
    }
    __syncthreads();
    for (int i = tid; i < Q * HD; i += 256) {
        const int q = i / HD, d = i % HD;
        partq[q * (HD + 4) + 4 + d] = ((ow[0][q][d] + ow[1][q][d]) + ow[2][q][d]) + ow[3][q][d];
    }
    stamp.end();
}

template <int HD, int P, int QM, int QL, int MINW>
static void attn_ns(hipStream_t st, const AttnArgs& a) {
    if (a.ns >= 4 && 4 * P <= 128)
        hipLaunchKernelGGL((k_attn<HD, P, QM, (4 * P <= 128 ? 4 : 1), QL, MINW>), dim3(a.nkv, a.n_wi), dim3(256), 0,
                           st, a);
    else if (a.ns >= 2 && 2 * P <= 128)
        hipLaunchKernelGGL((k_attn<HD, P, QM, (2 * P <= 128 ? 2 : 1), QL, MINW>), dim3(a.nkv, a.n_wi), dim3(256), 0,
                           st, a);
    else
        hipLaunchKernelGGL((k_attn<HD, P, QM, 1, QL, MINW>), dim3(a.nkv, a.n_wi), dim3(256), 0, st, a);
}

template <int HD, int P, int QM>
static void attention_hd(hipStream_t st, const AttnArgs& a, int m, int ck, Pieces& out) {
    if constexpr ((HD == 64 || HD == 128) && QM == 32) {
        if (a.flash) {
            hipLaunchKernelGGL((k_attn_flash<HD, kFlashBlock(HD)>), dim3(a.nkv, a.n_wi / 2), dim3(256), 0, st, a);
            goto merge;
        }
    }
    // items of at most 8 or 24 queries hold fewer (three workgroups per CU);
    // large launches of decode-sized items of one span at hd 64 and 128 keep
    // their keys and values in registers (small ones: the general kernel's
    // shorter chain of barriers finishes a lone item sooner)
    if constexpr ((HD == 64 || HD == 128) && QM >= 8) {
        if (a.ns == 1 && a.maxq > 0 && a.maxq <= 8 && (int64_t)a.nkv * a.n_wi >= kAttnDecWorkgroups) {
            if (a.maxq <= 4)
                hipLaunchKernelGGL((k_attn_dec<HD, P, QM, 4, 4>), dim3(a.nkv, a.n_wi), dim3(256), 0, st, a);
            else
                hipLaunchKernelGGL((k_attn_dec<HD, P, QM, 8, 4>), dim3(a.nkv, a.n_wi), dim3(256), 0, st, a);
            goto merge;
        }
    }
    if (QM > 8 && a.maxq > 0 && a.maxq <= 8)
        attn_ns<HD, P, QM, 8, 3>(st, a);
    else if (QM > 24 && a.maxq > 0 && a.maxq <= 24)
        attn_ns<HD, P, QM, 24, 3>(st, a);
    else
        attn_ns<HD, P, QM, QM, 2>(st, a);
merge:
    if (ck < 0) return;  // the consumer merges the spans itself
    AttnArgs am = a;
    am.stamp = a.stamp >= 0 ? a.stamp + 1 : -1;  // the merge's timeline slot follows the attention's
    if (ck == BF16)
        hipLaunchKernelGGL((k_merge_pieces<HD, QM, BF16>), dim3(out.kb, out.passes), dim3(64), 0, st, am, m, out.a,
                           out.xs, out.passes);
    // GEMM consumers of 1024 or more (k-block, pass) waves: four consecutive k-blocks
    // per workgroup (cfg4 at 16 sequences, 2,560 waves: verify 8185-8197 -> 8096-8099
    // us per step; eight per workgroup 8094 against 8043-8046 us on another box)
    else if (ck == MM && out.kb % 4 == 0 && out.kb * out.passes >= 1024)
        hipLaunchKernelGGL((k_merge_pieces<HD, QM, MM, 4>), dim3(out.kb / 4, out.passes), dim3(256), 0, st, am, m,
                           out.a, out.xs, out.passes);
    else if (ck == MM)
        hipLaunchKernelGGL((k_merge_pieces<HD, QM, MM>), dim3(out.kb, out.passes), dim3(64), 0, st, am, m, out.a,
                           out.xs, out.passes);
    else
        hipLaunchKernelGGL((k_merge_pieces<HD, QM, INT8>), dim3(out.kb, out.passes), dim3(64), 0, st, am, m, out.a,
                           out.xs, out.passes);
}

int attn_span(int hd) { return hd >= 128 ? 32 : 64; }
int attn_qmax(int hd) { return hd >= 64 ? 32 : 64; }

// ---------------------------------------------------------------------------
// Calibration capture (Model::record's inputs, src/model.rs:312-333): the f32
// rows a layer's projections take, for the AWQ search. Not on the decode path.
// ---------------------------------------------------------------------------

// rms_norm (src/kernels.rs:597-607) of residual rows: dot's eight lanes, each an
// fma chain over every eighth input in order, summed as hsum8 sums them
// (src/kernels.rs:191-213), then r = 1 / sqrt(ms + eps) and g * (x * r). One
// wave per row.
__global__ __launch_bounds__(64) void k_cap_norm(const float* __restrict__ x, int H, const float* __restrict__ g,
                                                 float eps, float* __restrict__ out, int ldo) {
    const int row = blockIdx.x, lane = threadIdx.x;
    const float* xr = x + (size_t)row * H;
    float acc = 0.0f;
    if (lane < 8)
        for (int i = lane; i < H; i += 8) acc = fmaf(xr[i], xr[i], acc);
    float l[8];
#pragma unroll
    for (int j = 0; j < 8; j++) l[j] = __shfl(acc, j);
    const float ss = ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
    const float r = 1.0f / sqrtf(ss / (float)H + eps);
    for (int i = lane; i < H; i += 64) out[(size_t)row * ldo + i] = g[i] * (xr[i] * r);
}

// The attention output rows in f32: k_merge_pieces' geometry and arithmetic
// (the same bits it splits into pieces), one lane of four writing each value.
template <int HD, int QM>
__global__ __launch_bounds__(64) void k_cap_merge(AttnArgs a, int m, float* __restrict__ out, int ldo) {
    const int kb = blockIdx.x, pass = blockIdx.y, lane = threadIdx.x;
    const int c = lane & 15, row = pass * 4 + (c >> 2), piece = c & 3;
    const int k0 = kb * 32 + (lane >> 4) * 8;
    if (row >= m || k0 >= a.nh * HD) return;
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    merge_spans<8>(a.part, *(const int4*)(a.mrec + (size_t)row * 4), a.nh, a.nkv, HD, QM, k0, piece, v);
    if (piece == 0)
#pragma unroll
        for (int s = 0; s < 8; s++) out[(size_t)row * ldo + k0 + s] = v[s];
}

void launch_cap_norm(hipStream_t st, const float* x, int m, int H, const float* g, float eps, float* out, int ldo) {
    if (m > 0) hipLaunchKernelGGL(k_cap_norm, dim3(m), dim3(64), 0, st, x, H, g, eps, out, ldo);
}

int launch_cap_merge(hipStream_t st, const AttnArgs& a, int m, float* out, int ldo) {
    if (m <= 0 || a.n_wi <= 0) return 0;
    const dim3 grid((a.nh * a.hd + 31) / 32, (m + 3) / 4);
    switch (a.hd) {
        case 16: hipLaunchKernelGGL((k_cap_merge<16, 64>), grid, dim3(64), 0, st, a, m, out, ldo); return 0;
        case 32: hipLaunchKernelGGL((k_cap_merge<32, 64>), grid, dim3(64), 0, st, a, m, out, ldo); return 0;
        case 64: hipLaunchKernelGGL((k_cap_merge<64, 32>), grid, dim3(64), 0, st, a, m, out, ldo); return 0;
        case 128: hipLaunchKernelGGL((k_cap_merge<128, 32>), grid, dim3(64), 0, st, a, m, out, ldo); return 0;
        default: return -1;
    }
}

// ---------------------------------------------------------------------------
// Output projection of a fused bf16 layer, split by query head: workgroup
// (n-tile, head h) merges head h's spans for the step's rows (SpanMerge, the
// merge kernel's arithmetic; the four lanes of a quad write the four bf16
// pieces of 8 merged values), multiplies them by the HD columns of W_o that
// belong to head h (HD / 32 k-blocks of its n-tile, bf16 MFMA), and adds the
// 16 outputs of each row into the accumulator a.acc_out (copy = workgroup %
// kAccCopiesB) as round(y * 2^kAccFrac). A workgroup reads one head's partials
// (about 4.6 KB per row for the 135M draft) instead of every head's, which is
// what an output projection that merges for itself must read per workgroup;
// a CU streams only about 27 GB/s, so that read was most of its time. The
// heads' contributions meet in the accumulator (integer sums: their order
// does not matter). Every launch also clears a.zero (the next stage's
// accumulator). 2 HD threads: an item (row slot, 8 dims, phase) per thread.
// ---------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(2 * HD) void k_o_heads(const GemvArgs a) {
    constexpr int KBH = HD / 32, SB = 5, IPR = HD / 2;  // k-blocks of a head, items per row
    __shared__ __align__(16) u16x8 xm[KBH * 64];
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const Stamp stamp(a.stamp);
    const int wg = (int)(blockIdx.x + gridDim.x * blockIdx.y);
    // this n-tile's columns of head h: wave w takes k-blocks w, w + 2, ... (requested first)
    constexpr int KW = (KBH + 1) / 2;
    bf16x8 wb[KW];
#pragma unroll
    for (int j = 0; j < KW; j++) {
        const int kb = min(wave + 2 * j, KBH - 1);
        wb[j] = ((const bf16x8*)a.W)[((size_t)t * a.KB + h * KBH + kb) * 64 + lane];
    }
    const int row = tid / IPR, rem = tid % IPR, k0 = (rem >> 2) * 8, phase = rem & 3;
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (row < a.m) {
        // the row's merge record (a vector load: the same address in every lane of the row)
        const int4 mr = ((const int4*)a.amrec)[row];
        SpanMerge<SB> sm;
        sm.init(a.apart, mr, a.anh, a.ankv, a.ahd, a.aqm, h * HD + k0);
        for (int s0 = phase; s0 < sm.ns; s0 += 4 * SB) {
            sm.load(s0);
            sm.fold(s0);
        }
        sm.finish(v);
    }
    u16x8 o;
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = (uint16_t)bf16_piece(v[e], phase);
    xm[(k0 >> 5) * 64 + ((k0 & 31) >> 3) * 16 + row * 4 + phase] = o;
    __syncthreads();
    // D of the 16 x 16 product: lane l holds the four pieces of row l / 16, column l % 16
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < KW; j++) {
        const int kb = wave + 2 * j;
        if (kb < KBH) {
            const u16x8 x = xm[kb * 64 + lane];
            bf16x8 ab;
            __builtin_memcpy(&ab, &x, sizeof(ab));
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, wb[j], acc, 0, 0, 0);
        }
    }
    // the two waves' k-blocks meet in LDS (wave 1 hands its product to wave 0)
    __shared__ f32x4 red[64];
    if (KBH > 1 && wave == 1) red[lane] = acc;
    __syncthreads();
    if (wave == 0) {
        if (KBH > 1) acc += red[lane];
        const int r = lane >> 4, n = t * 16 + (lane & 15);
        if (r < a.m && n < a.N) {
            const float y = ((acc[0] + acc[1]) + acc[2]) + acc[3];
            const double d = fmin(fmax((double)y * (double)(1ll << kAccFrac), -4.0e18), 4.0e18);
            __hip_atomic_fetch_add(a.acc_out + ((size_t)(wg % kAccCopiesB) * 4 + r) * a.acc_ld + n, (long long)rint(d),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // the next stage's accumulator starts at zero (stored last: loads and stores
    // retire in order, so earlier stores would hold up every wait on a load)
    if (a.zero)
        for (int i = wg * (int)blockDim.x + tid; i < a.zero_n; i += (int)(blockDim.x * gridDim.x * gridDim.y)) a.zero[i] = 0;
    stamp.end();
}

int launch_o_heads(hipStream_t st, const DMat& w, const GemvArgs& a, hipEvent_t e0, hipEvent_t e1) {
    if (a.m <= 0) return 0;
    const dim3 grid(w.n_tiles, a.anh);
    auto run = [&](auto kern, int threads) {
        if (e0 || e1)
            hipExtLaunchKernelGGL(kern, grid, dim3(threads), 0, st, e0, e1, 0, a);
        else
            hipLaunchKernelGGL(kern, grid, dim3(threads), 0, st, a);
    };
    switch (a.ahd) {
        case 64: run(k_o_heads<64>, 128); return 0;
        case 128: run(k_o_heads<128>, 256); return 0;
        default: return -1;
    }
}

#ifdef FERRO_STAMPS
__device__ unsigned long long g_stamps[kStampSlots][kStampWgs][2];
int stamps_read(uint64_t* out, int slots) {
    if (slots < 0 || slots > kStampSlots) return -1;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_stamps), (size_t)slots * kStampWgs * 2 * 8) == hipSuccess ? 0 : -1;
}
int stamps_clear() {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_stamps)) != hipSuccess) return -1;
    return hipMemset(p, 0, sizeof(g_stamps)) == hipSuccess ? 0 : -1;
}
#else
int stamps_read(uint64_t*, int) { return -1; }
int stamps_clear() { return -1; }
#endif

int launch_attention(hipStream_t st, const AttnArgs& a, int m, int consumer_kind, Pieces& out) {
    if (m <= 0 || a.n_wi <= 0) return 0;
    switch (a.hd) {
        case 16: attention_hd<16, 64, 64>(st, a, m, consumer_kind, out); return 0;
        case 32: attention_hd<32, 64, 64>(st, a, m, consumer_kind, out); return 0;
        case 64: attention_hd<64, 64, 32>(st, a, m, consumer_kind, out); return 0;
        case 128: attention_hd<128, 32, 32>(st, a, m, consumer_kind, out); return 0;
        default: return -1;  // no instance: nothing is launched
    }
}

// ---------------------------------------------------------------------------
// Argmax over the per-tile (max, index) pairs: first index of the maximum,
// NaN never wins (sampler::argmax, src/sampler.rs:41-51).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__global__ __launch_bounds__(256) void k_argmax_final(const float2* __restrict__ best, int tiles, int rows,
                                                      uint32_t* __restrict__ am, uint32_t* __restrict__ aux,
                                                      int aux_stride, int aux_off) {
    constexpr int UN = 8;  // partials per thread per pass, loaded before any is compared
    __shared__ float sv[4];
    __shared__ int si[4];
    const int r = blockIdx.x;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int t0 = threadIdx.x; t0 < tiles; t0 += 256 * UN) {
        float2 e[UN];
#pragma unroll
        for (int u = 0; u < UN; u++) {
            const int t = t0 + u * 256;
            e[u] = t < tiles ? best[(size_t)t * rows + r] : make_float2(-INFINITY, __int_as_float(0x7FFFFFFF));
        }
#pragma unroll
        for (int u = 0; u < UN; u++) {
            const int i = __float_as_int(e[u].y);
            if (better(e[u].x, i, bv, bi)) {
                bv = e[u].x;
                bi = i;
            }
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++)
            if (better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        const uint32_t t = bi == 0x7FFFFFFF ? 0u : (uint32_t)bi;
        if (am) am[r] = t;
        if (aux) aux[(size_t)r * aux_stride + aux_off] = t;
    }
}

void launch_argmax_final(hipStream_t st, const float2* best, int tiles, int rows, uint32_t* argmax_out,
                         uint32_t* aux, int aux_stride, int aux_off) {
    if (rows <= 0) return;
    hipLaunchKernelGGL(k_argmax_final, dim3(rows), dim3(256), 0, st, best, tiles, rows, argmax_out, aux, aux_stride,
                       aux_off);
}

// Greedy accept-prefix: proposals d_1..d_k against the target's argmax of
// rows 0..k; emits the accepted prefix and the target's own next token
// (src/engine.rs:563-610, greedy branch). verify_tokens holds each
// sequence's verify input [last, d_1..d_k].
__global__ void k_accept(const uint32_t* __restrict__ am, const uint32_t* __restrict__ verify_tokens, int n_seqs,
                         int k, uint32_t* __restrict__ out, int32_t* __restrict__ cnt, int32_t* __restrict__ acc) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n_seqs) return;
    const uint32_t* am_s = am + (size_t)s * (k + 1);
    const uint32_t* d = verify_tokens + (size_t)s * (k + 1) + 1;
    uint32_t* o = out + (size_t)s * (k + 1);
    int n = 0, ac = 0;
    for (int j = 0; j < k; j++) {
        if (am_s[j] == d[j]) {
            o[n++] = d[j];
            ac++;
        } else {
            o[n++] = am_s[j];
            break;
        }
    }
    if (ac == k) o[n++] = am_s[k];
    cnt[s] = n;
    acc[s] = ac;
}

void launch_accept(hipStream_t st, const uint32_t* argmax, const uint32_t* drafts, int n_seqs, int k,
                   uint32_t* out_tokens, int32_t* out_count, int32_t* out_accepted) {
    if (n_seqs <= 0) return;
    hipLaunchKernelGGL(k_accept, dim3((n_seqs + 63) / 64), dim3(64), 0, st, argmax, drafts, n_seqs, k, out_tokens,
                       out_count, out_accepted);
}

}  // namespace fg
