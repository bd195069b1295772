// HIP kernels for gfx950 (MI355X): the verify-path hot ops.
//
// Reference counterparts (Rust, /root/reference):
//   k_embed           Model::forward embedding gather      src/model.rs:295-298
//   k_residual_rms    kernels::add + rms_norm's mean square src/kernels.rs:597-607,665-669
//   k_pieces          rms_norm's scaling + operand prep    src/kernels.rs:597-607
//   k_gemv            kernels::matmul / quant::panels_of   src/kernels.rs:249-376, src/quant.rs:175-454
//   k_silu_pieces     kernels::silu_mul                    src/kernels.rs:650-663
//   k_rope_kv         rope + KvCache::write                src/model.rs:314-321,451-459; src/kv.rs:48-56
//   k_attn/_merge     Model::attention + kernels::attend   src/model.rs:395-432; src/kernels.rs:703-756
//   k_argmax1/2       sampler::argmax                      src/sampler.rs:41-51
//   k_accept          Engine::execute greedy accept        src/engine.rs:563-616
#include "internal.h"

#include <math.h>

namespace fg {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef int8_t i8x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
    uint32_t b = __float_as_uint(x);
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

// exp(x) by range reduction and the Cephes expf polynomial, the same
// sequence of operations as the reference's kernels::exp (src/kernels.rs:609-637).
__device__ __forceinline__ float dev_exp(float x) {
    x = fminf(fmaxf(x, -87.0f), 88.0f);
    float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(n, 2.1219444e-4f, fmaf(n, -0.6933594f, x));
    float p = 1.9875691e-4f;
    p = fmaf(p, r, 1.3982e-3f);
    p = fmaf(p, r, 8.333452e-3f);
    p = fmaf(p, r, 4.1665796e-2f);
    p = fmaf(p, r, 0.16666665f);
    p = fmaf(p, r, 0.5f);
    float y = fmaf(p, r * r, r) + 1.0f;
    return y * __int_as_float(((int)n + 127) << 23);
}

// Sum over a 256-thread block in a fixed order (deterministic).
__device__ __forceinline__ float block_sum256(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return t;
}

// ---------------------------------------------------------------------------
// Embedding gather: x[r] = embed[token[r]] as f32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_embed(const uint32_t* __restrict__ tok, int stride,
                                               const uint16_t* __restrict__ E, int H, float* __restrict__ x) {
    const int r = blockIdx.x;
    const uint16_t* e = E + (size_t)tok[(size_t)r * stride] * H;
    float* xr = x + (size_t)r * H;
    for (int i = threadIdx.x; i < H; i += 256) xr[i] = bf16_bits_to_f32(e[i]);
}

void launch_embed(hipStream_t st, const uint32_t* tokens, int stride, const uint16_t* embed, int m, int H, float* x) {
    if (m <= 0) return;
    hipLaunchKernelGGL(k_embed, dim3(m), dim3(256), 0, st, tokens, stride, embed, H, x);
}

// ---------------------------------------------------------------------------
// Residual add of a split GEMV's partial sums, then the RMSNorm factor
// rinv = 1/sqrt(mean(x^2) + eps) of the updated row. One block per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_residual_rms(float* __restrict__ x, const float* __restrict__ part,
                                                      int splits, int m, int H, float eps,
                                                      float* __restrict__ rinv) {
    __shared__ float red[4];
    const int r = blockIdx.x;
    float* xr = x + (size_t)r * H;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < H; i += 256) {
        float v = xr[i];
        if (part) {
            float p = 0.0f;
            for (int s = 0; s < splits; s++) p += part[((size_t)s * m + r) * H + i];
            v += p;
            xr[i] = v;
        }
        ss = fmaf(v, v, ss);
    }
    ss = block_sum256(ss, red);
    if (threadIdx.x == 0 && rinv) rinv[r] = 1.0f / sqrtf(ss / (float)H + eps);
}

void launch_residual_rms(hipStream_t st, float* x, const float* partials, int splits, int m, int H, float eps,
                         float* rinv) {
    if (m <= 0) return;
    hipLaunchKernelGGL(k_residual_rms, dim3(m), dim3(256), 0, st, x, partials, splits, m, H, eps, rinv);
}

// ---------------------------------------------------------------------------
// Activation pieces (see Pieces in internal.h). One wave per (k-block,
// pass); lane l covers (row, piece) = (4*pass + (l%16)/4, l%4) at inputs
// 8*(l/16)..+7 of the k-block.
// ---------------------------------------------------------------------------
template <int CK>
__device__ __forceinline__ void write_pieces(const float (&v)[8], int kb, int pass, int passes, int row, int piece,
                                             int lane, void* out, float* xs) {
    if (CK == BF16) {
        u16x8 o;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            float r = v[s];
            uint32_t h = 0;
            for (int p = 0; p <= piece; p++) {
                h = f32_to_bf16_bits(r);
                r = r - bf16_bits_to_f32(h);
            }
            o[s] = (uint16_t)h;
        }
        ((u16x8*)out)[((size_t)kb * passes + pass) * 64 + lane] = o;
    } else {
        float mx = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; s++) mx = fmaxf(mx, fabsf(v[s]));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        int e = 0;
        if (mx > 0.0f) {
            int fe;
            frexpf(mx, &fe);
            e = fe - 7;  // mx / 2^e in [64, 128)
            if (ldexpf(mx, -e) > 127.0f) e++;
        }
        i8x8 o;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            float r = ldexpf(v[s], -e);  // exact
            float a = rintf(r);
            for (int p = 0; p < piece; p++) {
                r = (r - a) * 128.0f;  // both exact
                a = rintf(r);
            }
            o[s] = (int8_t)(int)a;
        }
        ((i8x8*)out)[((size_t)kb * passes + pass) * 64 + lane] = o;
        if (lane < 16 && (lane & 3) == 0) xs[(size_t)kb * passes * 4 + row] = ldexpf(1.0f, e);
    }
}

template <int CK>
__global__ __launch_bounds__(64) void k_pieces(const float* __restrict__ x, int ldx, int m, int K,
                                               const float* __restrict__ g, const float* __restrict__ rinv,
                                               void* __restrict__ out, float* __restrict__ xs, int passes) {
    const int kb = blockIdx.x, pass = blockIdx.y, lane = threadIdx.x;
    const int c = lane & 15, row = pass * 4 + (c >> 2), piece = c & 3;
    const int k0 = kb * 32 + (lane >> 4) * 8;
    float v[8];
    const bool rv = row < m;
    const float ri = (rv && rinv) ? rinv[row] : 1.0f;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int k = k0 + s;
        float t = 0.0f;
        if (rv && k < K) {
            t = x[(size_t)row * ldx + k];
            if (g) t = g[k] * (t * ri);  // rms_norm's o = g * (v * r)
        }
        v[s] = t;
    }
    write_pieces<CK>(v, kb, pass, passes, row, piece, lane, out, xs);
}

void launch_pieces(hipStream_t st, int consumer_kind, const float* x, int ldx, int m, int K, const float* g,
                   const float* rinv, Pieces& out) {
    dim3 grid(out.kb, out.passes);
    if (consumer_kind == BF16)
        hipLaunchKernelGGL(k_pieces<BF16>, grid, dim3(64), 0, st, x, ldx, m, K, g, rinv, out.a, out.xs, out.passes);
    else
        hipLaunchKernelGGL(k_pieces<INT8>, grid, dim3(64), 0, st, x, ldx, m, K, g, rinv, out.a, out.xs, out.passes);
}

// SiLU(gate) * up from the gate/up GEMV's partial sums, straight into the
// down projection's pieces: o = g / (1 + exp(-g)) * u (src/kernels.rs:650-663).
template <int CK>
__global__ __launch_bounds__(64) void k_silu_pieces(const float* __restrict__ part, int splits, int m, int I,
                                                    void* __restrict__ out, float* __restrict__ xs, int passes,
                                                    float* __restrict__ act_out) {
    const int kb = blockIdx.x, pass = blockIdx.y, lane = threadIdx.x;
    const int c = lane & 15, row = pass * 4 + (c >> 2), piece = c & 3;
    const int k0 = kb * 32 + (lane >> 4) * 8;
    const size_t ld = (size_t)2 * I;
    float v[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int k = k0 + s;
        float t = 0.0f;
        if (row < m && k < I) {
            float gs = 0.0f, us = 0.0f;
            for (int sp = 0; sp < splits; sp++) {
                const float* pr = part + ((size_t)sp * m + row) * ld;
                gs += pr[k];
                us += pr[I + k];
            }
            t = gs / (1.0f + dev_exp(-gs)) * us;
            if (act_out && piece == 0) act_out[(size_t)row * I + k] = t;
        }
        v[s] = t;
    }
    write_pieces<CK>(v, kb, pass, passes, row, piece, lane, out, xs);
}

void launch_silu_pieces(hipStream_t st, const float* partials, int splits, int m, int I, Pieces& out,
                        float* act_out, int consumer_kind);

// ---------------------------------------------------------------------------
// GEMV / skinny GEMM: partial[split][row][n] = sum over the split's k-blocks
// of x[row] . W[n]. One wave per NT tiles of 16 outputs; the wave keeps the
// activation operand of a 4-k-block chunk in registers and streams the
// tiles' weights through the MFMA B-operand.
//   int4/int8: v_mfma_i32_16x16x32_i8, one MFMA per (tile, k-block, pass),
//     then the group's scale: acc += (D0 + D1/128 + D2/128^2 + D3/128^3) *
//     s_w[n][kb] * s_x[row][kb].
//   bf16: v_mfma_f32_16x16x32_bf16 accumulating over k; the four pieces
//     are summed at the end.
// D layout of a 16x16 MFMA: lane l holds rows 4*(l/16)+r (r = 0..3, the
// four pieces of activation row l/16 of the pass) of column l%16 (output n).
// ---------------------------------------------------------------------------
template <int KIND, int NT, int PASSES>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t* __restrict__ W, const float* __restrict__ S,
                                              const uint8_t* __restrict__ XA, const float* __restrict__ XS,
                                              float* __restrict__ out, int N, int KB, int n_tiles,
                                              int kb_per_split, int m, int p_total) {
    constexpr bool Q = KIND != BF16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tile0 = (blockIdx.x * 4 + wave) * NT;
    if (tile0 >= n_tiles) return;
    const int split = blockIdx.y;
    const int kb0 = split * kb_per_split;
    const int kb1 = min(kb0 + kb_per_split, KB);
    const int pass0 = blockIdx.z * PASSES;
    const int np = min(PASSES, p_total - pass0);
    const int KC = KB >> 2;

    float accq[NT][PASSES];
    f32x4 accb[NT][PASSES];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            accq[t][p] = 0.0f;
            accb[t][p] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
    const i32x4 izero = {0, 0, 0, 0};
    const float inv128 = 0.0078125f;

    for (int kb = kb0; kb < kb1; kb += 4) {
        long aq[4][PASSES];
        bf16x8 ab[4][PASSES];
        float sx[4][PASSES];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int p = 0; p < PASSES; p++) {
                if (p < np) {
                    const size_t idx = ((size_t)(kb + j) * p_total + pass0 + p) * 64 + lane;
                    if (Q) {
                        aq[j][p] = ((const long*)XA)[idx];
                        sx[j][p] = XS[(size_t)(kb + j) * p_total * 4 + (pass0 + p) * 4 + (lane >> 4)];
                    } else {
                        ab[j][p] = ((const bf16x8*)XA)[idx];
                    }
                }
            }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int tile = tile0 + t;
            if (tile >= n_tiles) break;
            if (KIND == INT4 || KIND == INT8) {
                const float4 sv = ((const float4*)S)[((size_t)tile * KC + (kb >> 2)) * 16 + (lane & 15)];
                const float svj[4] = {sv.x, sv.y, sv.z, sv.w};
                long bq[4];
                if (KIND == INT4) {
                    const u32x4 wv = ((const u32x4*)W)[((size_t)tile * KC + (kb >> 2)) * 64 + lane];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t w = wv[j];
                        const uint32_t lo = (w << 4) & 0xF0F0F0F0u, hi = w & 0xF0F0F0F0u;
                        bq[j] = (long)(((uint64_t)hi << 32) | lo);
                    }
                } else {
                    const u32x4 w01 = ((const u32x4*)W)[((size_t)tile * (KB >> 1) + (kb >> 1)) * 64 + lane];
                    const u32x4 w23 = ((const u32x4*)W)[((size_t)tile * (KB >> 1) + (kb >> 1) + 1) * 64 + lane];
                    bq[0] = (long)(((uint64_t)w01[1] << 32) | w01[0]);
                    bq[1] = (long)(((uint64_t)w01[3] << 32) | w01[2]);
                    bq[2] = (long)(((uint64_t)w23[1] << 32) | w23[0]);
                    bq[3] = (long)(((uint64_t)w23[3] << 32) | w23[2]);
                }
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int p = 0; p < PASSES; p++) {
                        if (p < np) {
                            const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aq[j][p], bq[j], izero, 0, 0, 0);
                            float comb = fmaf((float)d[3], inv128, (float)d[2]);
                            comb = fmaf(comb, inv128, (float)d[1]);
                            comb = fmaf(comb, inv128, (float)d[0]);
                            accq[t][p] = fmaf(comb, svj[j] * sx[j][p], accq[t][p]);
                        }
                    }
            } else {
                bf16x8 wb[4];
#pragma unroll
                for (int j = 0; j < 4; j++) wb[j] = ((const bf16x8*)W)[((size_t)tile * KB + kb + j) * 64 + lane];
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int p = 0; p < PASSES; p++)
                        if (p < np)
                            accb[t][p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab[j][p], wb[j], accb[t][p], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tile = tile0 + t;
        if (tile >= n_tiles) break;
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const int row = (pass0 + p) * 4 + (lane >> 4);
            if (p < np && row < m) {
                const float v = Q ? accq[t][p] : ((accb[t][p][0] + accb[t][p][1]) + accb[t][p][2]) + accb[t][p][3];
                out[((size_t)split * m + row) * N + tile * 16 + (lane & 15)] = v;
            }
        }
    }
}

static int nt_for(int kind) { return kind == INT4 ? 4 : 2; }

GemvPlan plan_gemv(const DMat& w, int m) {
    GemvPlan p;
    const int nt = nt_for(w.kind);
    const int p_total = (m + 3) / 4;
    const int pg = (p_total + 3) / 4;
    const int groups = (w.n_tiles + nt * 4 - 1) / (nt * 4);
    const int waves = groups * 4 * pg;
    const int chunks = w.kb / 4;
    const int want = 2048;
    int splits = want / (waves > 0 ? waves : 1);
    splits = splits < 1 ? 1 : splits;
    splits = splits > 16 ? 16 : splits;
    splits = splits > chunks ? chunks : splits;
    const int cps = (chunks + splits - 1) / splits;
    p.splits = (chunks + cps - 1) / cps;
    return p;
}

template <int KIND, int NT>
static void gemv_dispatch(hipStream_t st, const DMat& w, const Pieces& x, int m, int splits, float* out) {
    const int p_total = x.passes;
    const int chunks = w.kb / 4;
    const int cps = (chunks + splits - 1) / splits;
    const int groups = (w.n_tiles + NT * 4 - 1) / (NT * 4);
    const uint8_t* W = (const uint8_t*)w.w;
    const uint8_t* XA = (const uint8_t*)x.a;
    if (p_total == 1) {
        hipLaunchKernelGGL((k_gemv<KIND, NT, 1>), dim3(groups, splits, 1), dim3(256), 0, st, W, w.s, XA, x.xs, out,
                           w.rows, w.kb, w.n_tiles, cps * 4, m, p_total);
    } else if (p_total == 2) {
        hipLaunchKernelGGL((k_gemv<KIND, NT, 2>), dim3(groups, splits, 1), dim3(256), 0, st, W, w.s, XA, x.xs, out,
                           w.rows, w.kb, w.n_tiles, cps * 4, m, p_total);
    } else {
        hipLaunchKernelGGL((k_gemv<KIND, NT, 4>), dim3(groups, splits, (p_total + 3) / 4), dim3(256), 0, st, W, w.s,
                           XA, x.xs, out, w.rows, w.kb, w.n_tiles, cps * 4, m, p_total);
    }
}

void launch_gemv(hipStream_t st, const DMat& w, const Pieces& x, int m, const GemvPlan& plan, float* partials) {
    if (m <= 0) return;
    if (w.kind == INT4)
        gemv_dispatch<INT4, 4>(st, w, x, m, plan.splits, partials);
    else if (w.kind == INT8)
        gemv_dispatch<INT8, 2>(st, w, x, m, plan.splits, partials);
    else
        gemv_dispatch<BF16, 2>(st, w, x, m, plan.splits, partials);
}

void launch_silu_pieces(hipStream_t st, const float* partials, int splits, int m, int I, Pieces& out,
                        float* act_out, int consumer_kind) {
    dim3 grid(out.kb, out.passes);
    if (consumer_kind == BF16)
        hipLaunchKernelGGL(k_silu_pieces<BF16>, grid, dim3(64), 0, st, partials, splits, m, I, out.a, out.xs,
                           out.passes, act_out);
    else
        hipLaunchKernelGGL(k_silu_pieces<INT8>, grid, dim3(64), 0, st, partials, splits, m, I, out.a, out.xs,
                           out.passes, act_out);
}

// Sum of partials (+ bias, added after the product as the reference does,
// src/kernels.rs:268-274).
__global__ __launch_bounds__(256) void k_reduce(const float* __restrict__ part, int splits, int m, int N,
                                                const float* __restrict__ bias, float* __restrict__ y) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)m * N) return;
    float v = 0.0f;
    for (int s = 0; s < splits; s++) v += part[(size_t)s * m * N + i];
    if (bias) v += bias[i % N];
    y[i] = v;
}

void launch_reduce(hipStream_t st, const float* partials, int splits, int m, int N, const float* bias, float* y) {
    const size_t n = (size_t)m * N;
    if (!n) return;
    hipLaunchKernelGGL(k_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, partials, splits, m, N, bias, y);
}

// ---------------------------------------------------------------------------
// RoPE on q and k heads (rotate-half, src/model.rs:451-459) from the qkv
// GEMV's partials (+ bias), q to q_out, k and v into the paged cache slot
// (KvCache::write, src/kv.rs:48-56). Grid (rows, nh + 2*nkv), hd/2 threads.
// ---------------------------------------------------------------------------
__global__ void k_rope_kv(const float* __restrict__ part, int splits, int m, const float* __restrict__ bias,
                          const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_slot,
                          const float* __restrict__ cos_t, const float* __restrict__ sin_t, int nh, int nkv, int hd,
                          int bs, float* __restrict__ q_out, float* __restrict__ kc, float* __restrict__ vc) {
    const int r = blockIdx.x, h = blockIdx.y, i = threadIdx.x, half = hd >> 1;
    const int N = (nh + 2 * nkv) * hd;
    const int ca = h * hd + i, cb = ca + half;
    float a = 0.0f, b = 0.0f;
    for (int s = 0; s < splits; s++) {
        const float* pr = part + ((size_t)s * m + r) * N;
        a += pr[ca];
        b += pr[cb];
    }
    if (bias) {
        a += bias[ca];
        b += bias[cb];
    }
    if (h < nh + nkv) {
        const int pos = row_pos[r];
        const float c = cos_t[(size_t)pos * half + i], sn = sin_t[(size_t)pos * half + i];
        const float a2 = __fadd_rn(__fmul_rn(a, c), __fmul_rn(-b, sn));
        const float b2 = __fadd_rn(__fmul_rn(b, c), __fmul_rn(a, sn));
        a = a2;
        b = b2;
    }
    if (h < nh) {
        float* q = q_out + (size_t)r * nh * hd + (size_t)h * hd;
        q[i] = a;
        q[i + half] = b;
        return;
    }
    const int slot = row_slot[r];
    const int blk = slot / bs, o = slot % bs;
    const bool is_k = h < nh + nkv;
    const int kh = is_k ? h - nh : h - nh - nkv;
    float* dst = (is_k ? kc : vc) + (((size_t)blk * nkv + kh) * bs + o) * hd;
    dst[i] = a;
    dst[i + half] = b;
}

void launch_rope_kv(hipStream_t st, const float* partials, int splits, int m, const float* bias,
                    const int32_t* row_pos, const int32_t* row_slot, const float* cos_t, const float* sin_t, int nh,
                    int nkv, int hd, int bs, float* q_out, float* kc, float* vc) {
    if (m <= 0) return;
    hipLaunchKernelGGL(k_rope_kv, dim3(m, nh + 2 * nkv), dim3(hd / 2), 0, st, partials, splits, m, bias, row_pos,
                       row_slot, cos_t, sin_t, nh, nkv, hd, bs, q_out, kc, vc);
}

// ---------------------------------------------------------------------------
// Paged attention, split over the context (flash-decoding). A work item is
// (row group, split of split_pos positions) x kv head: the rows of a group
// are consecutive rows of one sequence (<= 16), their queries (rows x GQA
// group) share every K/V block the item reads, and each row is causally
// limited to positions <= its own. Partials (running max, sum, weighted
// values) are merged by k_attn_merge.
// ---------------------------------------------------------------------------
constexpr int ATT_QMAX = 64;

template <int HD>
__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
    constexpr int QPW = ATT_QMAX / 4;
    constexpr int DPL = (HD + 63) / 64;
    constexpr int HQ = HD / 4;
    __shared__ float qs[ATT_QMAX][HD];
    __shared__ float ks[16][HD + 1];
    __shared__ float vs[16][HD];
    __shared__ int lim[ATT_QMAX];

    const int wi = blockIdx.x, h = blockIdx.y;
    const int g = a.wi_group[wi], sidx = a.wi_split[wi];
    const int row0 = a.g_row0[g], nrows = a.g_nrows[g];
    const uint32_t* table = a.tables + a.g_table[g];
    const int G = a.nh / a.nkv;
    const int Q = nrows * G;
    const int Lmax = a.row_pos[row0 + nrows - 1] + 1;
    const int p0 = sidx * a.split_pos;
    const int p1 = min(p0 + a.split_pos, Lmax);

    for (int i = threadIdx.x; i < Q * HD; i += 256) {
        const int q = i / HD, d = i % HD, r = q / G, j = q % G;
        qs[q][d] = a.q[(size_t)(row0 + r) * a.nh * HD + (size_t)(h * G + j) * HD + d];
    }
    for (int q = threadIdx.x; q < Q; q += 256) lim[q] = a.row_pos[row0 + q / G];
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int pp = lane & 15, qq = lane >> 4;
    float mrun[QPW], lrun[QPW], o[QPW][DPL];
#pragma unroll
    for (int i = 0; i < QPW; i++) {
        mrun[i] = -INFINITY;
        lrun[i] = 0.0f;
#pragma unroll
        for (int d = 0; d < DPL; d++) o[i][d] = 0.0f;
    }

    for (int base = p0; base < p1; base += 16) {
        const uint32_t blk = table[base >> 4];
        const float4* kb = (const float4*)(a.kc + ((size_t)blk * a.nkv + h) * 16 * HD);
        const float4* vb = (const float4*)(a.vc + ((size_t)blk * a.nkv + h) * 16 * HD);
        for (int i = threadIdx.x; i < 16 * HD / 4; i += 256) {
            const float4 k4 = kb[i], v4 = vb[i];
            const int e = i * 4, row = e / HD, col = e % HD;
            ks[row][col] = k4.x;
            ks[row][col + 1] = k4.y;
            ks[row][col + 2] = k4.z;
            ks[row][col + 3] = k4.w;
            *(float4*)&vs[row][col] = v4;
        }
        __syncthreads();
#pragma unroll
        for (int qi = 0; qi < QPW; qi++) {
            const int q = wave + 4 * qi;
            if (q >= Q) break;
            float part = 0.0f;
#pragma unroll 8
            for (int e = 0; e < HQ; e++) part = fmaf(qs[q][qq * HQ + e], ks[pp][qq * HQ + e], part);
            part += __shfl_xor(part, 16);
            part += __shfl_xor(part, 32);
            float sc = part * a.scale;
            const int pos = base + pp;
            if (pos >= p1 || pos > lim[q]) sc = -INFINITY;
            float bm = sc;
            bm = fmaxf(bm, __shfl_xor(bm, 1));
            bm = fmaxf(bm, __shfl_xor(bm, 2));
            bm = fmaxf(bm, __shfl_xor(bm, 4));
            bm = fmaxf(bm, __shfl_xor(bm, 8));
            const float mnew = fmaxf(mrun[qi], bm);
            if (mnew == -INFINITY) continue;
            const float corr = mrun[qi] == -INFINITY ? 0.0f : dev_exp(mrun[qi] - mnew);
            const float pr = sc == -INFINITY ? 0.0f : dev_exp(sc - mnew);
            float bsum = pr;
            bsum += __shfl_xor(bsum, 1);
            bsum += __shfl_xor(bsum, 2);
            bsum += __shfl_xor(bsum, 4);
            bsum += __shfl_xor(bsum, 8);
            lrun[qi] = fmaf(lrun[qi], corr, bsum);
            float prj[16];
#pragma unroll
            for (int j = 0; j < 16; j++) prj[j] = __shfl(pr, j);
#pragma unroll
            for (int dd = 0; dd < DPL; dd++) {
                const int d = lane + 64 * dd;
                if (d < HD) {
                    float acc = o[qi][dd] * corr;
#pragma unroll
                    for (int j = 0; j < 16; j++) acc = fmaf(prj[j], vs[j][d], acc);
                    o[qi][dd] = acc;
                }
            }
            mrun[qi] = mnew;
        }
        __syncthreads();
    }
#pragma unroll
    for (int qi = 0; qi < QPW; qi++) {
        const int q = wave + 4 * qi;
        if (q >= Q) break;
        float* dst = a.part + (((size_t)wi * a.nkv + h) * ATT_QMAX + q) * (HD + 2);
        if (lane == 0) {
            dst[0] = mrun[qi];
            dst[1] = lrun[qi];
        }
#pragma unroll
        for (int dd = 0; dd < DPL; dd++)
            if (lane + 64 * dd < HD) dst[2 + lane + 64 * dd] = o[qi][dd];
    }
}

template <int HD>
__global__ void k_attn_merge(AttnArgs a) {
    const int row = blockIdx.x, hq = blockIdx.y, d = threadIdx.x;
    const int g = a.row_group[row];
    const int G = a.nh / a.nkv;
    const int h = hq / G, j = hq % G;
    const int q = (row - a.g_row0[g]) * G + j;
    const int wi0 = a.g_wi0[g], ns = a.g_nsplit[g];
    float M = -INFINITY;
    for (int s = 0; s < ns; s++) M = fmaxf(M, a.part[(((size_t)(wi0 + s) * a.nkv + h) * ATT_QMAX + q) * (HD + 2)]);
    float L = 0.0f, O = 0.0f;
    for (int s = 0; s < ns; s++) {
        const float* p = a.part + (((size_t)(wi0 + s) * a.nkv + h) * ATT_QMAX + q) * (HD + 2);
        const float ms = p[0];
        if (ms == -INFINITY) continue;
        const float w = dev_exp(ms - M);
        L = fmaf(p[1], w, L);
        O = fmaf(p[2 + d], w, O);
    }
    a.out[(size_t)row * a.nh * HD + (size_t)hq * HD + d] = O / L;
}

void launch_attention(hipStream_t st, const AttnArgs& a, int m) {
    if (m <= 0 || a.n_wi <= 0) return;
    switch (a.hd) {
        case 16:
            hipLaunchKernelGGL(k_attn<16>, dim3(a.n_wi, a.nkv), dim3(256), 0, st, a);
            hipLaunchKernelGGL(k_attn_merge<16>, dim3(m, a.nh), dim3(16), 0, st, a);
            break;
        case 32:
            hipLaunchKernelGGL(k_attn<32>, dim3(a.n_wi, a.nkv), dim3(256), 0, st, a);
            hipLaunchKernelGGL(k_attn_merge<32>, dim3(m, a.nh), dim3(32), 0, st, a);
            break;
        case 64:
            hipLaunchKernelGGL(k_attn<64>, dim3(a.n_wi, a.nkv), dim3(256), 0, st, a);
            hipLaunchKernelGGL(k_attn_merge<64>, dim3(m, a.nh), dim3(64), 0, st, a);
            break;
        case 128:
            hipLaunchKernelGGL(k_attn<128>, dim3(a.n_wi, a.nkv), dim3(256), 0, st, a);
            hipLaunchKernelGGL(k_attn_merge<128>, dim3(m, a.nh), dim3(128), 0, st, a);
            break;
    }
}

// ---------------------------------------------------------------------------
// Logits (sum of the lm_head GEMV's partials) and their argmax: first index
// of the maximum, NaN never wins (sampler::argmax, src/sampler.rs:41-51).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__global__ __launch_bounds__(256) void k_argmax1(const float* __restrict__ part, int splits, int rows, int V,
                                                 float* __restrict__ logits_out, float2* __restrict__ best,
                                                 int nblk) {
    __shared__ float sv[256];
    __shared__ int si[256];
    const int r = blockIdx.x, b = blockIdx.y;
    const int per = (V + nblk - 1) / nblk;
    const int i0 = b * per, i1 = min(i0 + per, V);
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = i0 + threadIdx.x; i < i1; i += 256) {
        float v = 0.0f;
        for (int s = 0; s < splits; s++) v += part[((size_t)s * rows + r) * V + i];
        if (logits_out) logits_out[(size_t)r * V + i] = v;
        if (v != v) v = -INFINITY;
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o && better(sv[threadIdx.x + o], si[threadIdx.x + o], sv[threadIdx.x], si[threadIdx.x])) {
            sv[threadIdx.x] = sv[threadIdx.x + o];
            si[threadIdx.x] = si[threadIdx.x + o];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) best[(size_t)r * nblk + b] = make_float2(sv[0], __int_as_float(si[0]));
}

__global__ __launch_bounds__(64) void k_argmax2(const float2* __restrict__ best, int nblk,
                                                uint32_t* __restrict__ am, uint32_t* __restrict__ aux,
                                                int aux_stride, int aux_off) {
    const int r = blockIdx.x;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int b = threadIdx.x; b < nblk; b += 64) {
        const float2 e = best[(size_t)r * nblk + b];
        const int i = __float_as_int(e.y);
        if (better(e.x, i, bv, bi)) {
            bv = e.x;
            bi = i;
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
    if (threadIdx.x == 0) {
        const uint32_t t = bi == 0x7FFFFFFF ? 0u : (uint32_t)bi;
        if (am) am[r] = t;
        if (aux) aux[(size_t)r * aux_stride + aux_off] = t;
    }
}

void launch_argmax(hipStream_t st, const float* partials, int splits, int rows, int V, float* logits_out,
                   float2* block_best, int nblk, uint32_t* argmax_out, uint32_t* aux, int aux_stride, int aux_off) {
    if (rows <= 0) return;
    hipLaunchKernelGGL(k_argmax1, dim3(rows, nblk), dim3(256), 0, st, partials, splits, rows, V, logits_out,
                       block_best, nblk);
    hipLaunchKernelGGL(k_argmax2, dim3(rows), dim3(64), 0, st, block_best, nblk, argmax_out, aux, aux_stride,
                       aux_off);
}

__global__ __launch_bounds__(256) void k_gather_rows(const float* __restrict__ x, const int32_t* __restrict__ rows,
                                                     int H, float* __restrict__ out) {
    const int i = blockIdx.x;
    const float* src = x + (size_t)rows[i] * H;
    for (int c = threadIdx.x; c < H; c += 256) out[(size_t)i * H + c] = src[c];
}

void launch_gather_rows(hipStream_t st, const float* x, const int32_t* rows, int n, int H, float* out) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_gather_rows, dim3(n), dim3(256), 0, st, x, rows, H, out);
}

// Greedy accept-prefix: proposals d_1..d_k against the target's argmax of
// rows 0..k; emits the accepted prefix and the target's own next token
// (src/engine.rs:563-610, greedy branch). verify_tokens holds each
// sequence's verify input [last, d_1..d_k].
__global__ void k_accept(const uint32_t* __restrict__ am, const uint32_t* __restrict__ verify_tokens, int n_seqs,
                         int k, uint32_t* __restrict__ out, int32_t* __restrict__ cnt, int32_t* __restrict__ acc) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n_seqs) return;
    const uint32_t* a = am + (size_t)s * (k + 1);
    const uint32_t* d = verify_tokens + (size_t)s * (k + 1) + 1;
    uint32_t* o = out + (size_t)s * (k + 1);
    int n = 0, ac = 0;
    for (int j = 0; j < k; j++) {
        if (a[j] == d[j]) {
            o[n++] = d[j];
            ac++;
        } else {
            o[n++] = a[j];
            break;
        }
    }
    if (ac == k) o[n++] = a[k];
    cnt[s] = n;
    acc[s] = ac;
}

void launch_accept(hipStream_t st, const uint32_t* argmax, const uint32_t* drafts, int n_seqs, int k,
                   uint32_t* out_tokens, int32_t* out_count, int32_t* out_accepted) {
    if (n_seqs <= 0) return;
    hipLaunchKernelGGL(k_accept, dim3((n_seqs + 63) / 64), dim3(64), 0, st, argmax, drafts, n_seqs, k, out_tokens,
                       out_count, out_accepted);
}

__global__ void k_copy_tokens(const uint32_t* __restrict__ src, int n, int ss, uint32_t* __restrict__ dst, int ds) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[(size_t)i * ds] = src[(size_t)i * ss];
}

void launch_copy_tokens(hipStream_t st, const uint32_t* src, int n, int src_stride, uint32_t* dst, int dst_stride) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_copy_tokens, dim3((n + 63) / 64), dim3(64), 0, st, src, n, src_stride, dst, dst_stride);
}

}  // namespace fg
