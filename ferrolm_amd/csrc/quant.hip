// Load-time quantization on the device: QMatrix::quantize (src/quant.rs:78-143)
// and the pieces of the AWQ alpha search (src/awq.rs:152-217): the column
// scaling, the reference's matmuls in their exact accumulation order, and the
// mean squared error summed in output order.
//
// Everything here reproduces the reference's bits. The quantizer's clip search
// is per (row, group) sequential arithmetic (f32 divide and round, f64 error),
// one lane per (row, group); the matmuls are one FMA chain per output, in k
// order, as src/kernels.rs:249-289 (bf16) and src/quant.rs:285-299 (per-group
// chains, then acc = fma(group sum, scale, acc)). Contraction is off for the
// whole build, so only the explicit fmaf calls fuse.
#include "internal.h"

namespace fg {

// f32::round then `as i32` (saturating, NaN to 0), then clamp(lo, hi)
__device__ __forceinline__ int clamp_code(float t, int lo, int hi) {
    if (!(t == t)) return 0;
    if (t >= (float)hi) return hi;
    if (t <= (float)lo) return lo;
    return (int)t;
}

// One wave per (32-row panel, two groups): lane l takes row 32 p + l % 32 of
// group 2 y + l / 32. Writes the reference's QMatrix layout: scales
// [panel][group][32]; codes per panel and input position, int8 one byte per
// row, int4 byte c = row c (low nibble) | row c + 16 (high nibble), each + 8.
// Groups whose every clip gives a non-finite error keep scale 0 and codes 0
// (the reference would keep the previous group's codes there).
template <bool Q8>
__global__ __launch_bounds__(64) void k_quantize(const float* __restrict__ w, const float* __restrict__ imp, int cols,
                                                 uint8_t* __restrict__ q, float* __restrict__ s) {
    constexpr int lo = Q8 ? -127 : -8, hi = Q8 ? 127 : 7, nclips = Q8 ? 6 : 11;
    const float clips8[6] = {1.0f, 0.98f, 0.96f, 0.94f, 0.92f, 0.9f};
    const float clips4[11] = {1.0f, 0.95f, 0.9f, 0.85f, 0.8f, 0.75f, 0.7f, 0.65f, 0.6f, 0.55f, 0.5f};
    const int lane = threadIdx.x, c = lane & 31, groups = cols >> 5;
    const int p = blockIdx.x, g = blockIdx.y * 2 + (lane >> 5);
    const bool live = g < groups;
    const int gc = live ? g : groups - 1;  // lanes past the last group work on a valid copy, write nothing
    const float* src = w + ((size_t)p * 32 + c) * cols + (size_t)gc * 32;
    float v[32], im[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 a = ((const float4*)src)[i];
        v[4 * i] = a.x;
        v[4 * i + 1] = a.y;
        v[4 * i + 2] = a.z;
        v[4 * i + 3] = a.w;
    }
#pragma unroll
    for (int i = 0; i < 32; i++) im[i] = imp ? imp[gc * 32 + i] : 1.0f;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    double best = INFINITY;
    float best_scale = 0.0f;
    if (amax > 0.0f) {
#pragma unroll
        for (int ci = 0; ci < nclips; ci++) {
            const float scale = (Q8 ? clips8[ci] : clips4[ci]) * amax / (float)hi;
            double err = 0.0;
#pragma unroll
            for (int i = 0; i < 32; i++) {
                const int code = clamp_code(roundf(v[i] / scale), lo, hi);
                const double d = (double)(v[i] - (float)code * scale);
                err = err + d * d * (double)im[i];
            }
            if (err < best) {
                best = err;
                best_scale = scale;
            }
        }
    }
    if (live) s[((size_t)p * groups + g) * 32 + c] = best_scale;
    // the chosen clip's codes (a function of the scale: recomputed)
    uint8_t* qp = q + ((size_t)p * cols + (size_t)gc * 32) * (Q8 ? 32 : 16);
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int code = best_scale > 0.0f ? clamp_code(roundf(v[i] / best_scale), lo, hi) : 0;
        if (Q8) {
            if (live) qp[i * 32 + c] = (uint8_t)(int8_t)code;
        } else {
            const int up = __shfl_down(code, 16, 32);  // row c + 16's code
            if (live && c < 16) qp[i * 16 + c] = (uint8_t)((code + 8) | ((up + 8) << 4));
        }
    }
}

// dst[r][c] = src[r][c] * s[c] (div = 0) or src[r][c] / s[c] (div = 1)
__global__ __launch_bounds__(256) void k_scale_cols(const float* __restrict__ src, int64_t n, int k,
                                                    const float* __restrict__ s, int div, float* __restrict__ dst) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float sc = s[i % k];
        dst[i] = div ? src[i] / sc : src[i] * sc;
    }
}

// y (m x rows) = x (m x K) W^T with the reference's accumulation order, one
// thread per output column j and 16 rows of x (blockIdx.y), the rows' 32
// inputs of each step staged in LDS.
//   BF: W is f32 rows x K, rounded to bf16 (Matrix::from_f32) as it is read;
//       acc = fma(x_k, w_jk, acc) for k = 0, 1, ...
//   else: W is a QMatrix (codes q, scales s); per group g a chain
//       gs = fma(x_k, code_jk, gs) over its 32 positions, then
//       acc = fma(gs, s_jg, acc).
template <bool BF, bool Q8>
__global__ __launch_bounds__(256) void k_mm_exact(const float* __restrict__ x, int m, int K,
                                                  const float* __restrict__ wf, const uint8_t* __restrict__ q,
                                                  const float* __restrict__ s, int rows, float* __restrict__ y) {
    __shared__ float xs[16][33];
    const int j = blockIdx.x * 256 + threadIdx.x, i0 = blockIdx.y * 16;
    const int jc = min(j, rows - 1);
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += 32) {
        __syncthreads();
        for (int e = threadIdx.x; e < 16 * 32; e += 256) {
            const int i = e >> 5, kk = e & 31;
            xs[i][kk] = i0 + i < m ? x[(size_t)(i0 + i) * K + k0 + kk] : 0.0f;
        }
        __syncthreads();
        if (BF) {
            const float* wr = wf + (size_t)jc * K + k0;
#pragma unroll
            for (int kk = 0; kk < 32; kk++) {
                const float wv = (float)(__bf16)wr[kk];
#pragma unroll
                for (int i = 0; i < 16; i++) acc[i] = fmaf(xs[i][kk], wv, acc[i]);
            }
        } else {
            const int p = jc >> 5, c = jc & 31, g = k0 >> 5, groups = K >> 5;
            float gs[16];
#pragma unroll
            for (int i = 0; i < 16; i++) gs[i] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 32; kk++) {
                float code;
                if (Q8) {
                    code = (float)(int8_t)q[((size_t)p * K + k0 + kk) * 32 + c];
                } else {
                    const uint8_t b = q[((size_t)p * K + k0 + kk) * 16 + (c & 15)];
                    code = (float)((int)(c < 16 ? (b & 0x0F) : (b >> 4)) - 8);
                }
#pragma unroll
                for (int i = 0; i < 16; i++) gs[i] = fmaf(xs[i][kk], code, gs[i]);
            }
            const float sc = s[((size_t)p * groups + g) * 32 + c];
#pragma unroll
            for (int i = 0; i < 16; i++) acc[i] = fmaf(gs[i], sc, acc[i]);
        }
    }
    if (j < rows)
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (i0 + i < m) y[(size_t)(i0 + i) * rows + j] = acc[i];
}

// err[b] = sum over t of (f64)(y_b[t] - yref[t])^2 in t order from 0, divided
// by n, for the sequences y_b = y + b * ystride (one workgroup each). The
// reference sums sequentially in f64 (each term is exact: the square of an f32
// difference), so one lane adds in order; the wave loads and squares the next
// 1024 terms into LDS while that lane adds the current ones, which leaves the
// f64 add chain as the only cost.
__global__ __launch_bounds__(64) void k_sq_err(const float* __restrict__ y, int64_t ystride,
                                               const float* __restrict__ yref, int64_t n, double* __restrict__ out) {
    constexpr int BATCH = 1024, PER = BATCH / 256;  // float4 loads per lane per batch
    __shared__ double buf[BATCH];
    const int lane = threadIdx.x;
    const float* yb = y + (size_t)blockIdx.x * ystride;
    float4 a[PER], b[PER];
    auto load = [&](int64_t t0) {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int64_t i = t0 + 4 * lane + 256 * u;  // n and t0 are multiples of 4: whole float4s
            const int64_t ic = i < n ? i : 0;
            a[u] = *(const float4*)(yb + ic);
            b[u] = *(const float4*)(yref + ic);
            if (i >= n) a[u] = b[u];  // past the end: a zero term (x + 0 = x)
        }
    };
    double err = 0.0;
    load(0);
    for (int64_t t0 = 0; t0 < n; t0 += BATCH) {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const double d0 = (double)(a[u].x - b[u].x), d1 = (double)(a[u].y - b[u].y);
            const double d2 = (double)(a[u].z - b[u].z), d3 = (double)(a[u].w - b[u].w);
            const int o = 4 * lane + 256 * u;
            buf[o] = d0 * d0;
            buf[o + 1] = d1 * d1;
            buf[o + 2] = d2 * d2;
            buf[o + 3] = d3 * d3;
        }
        __syncthreads();
        if (t0 + BATCH < n) load(t0 + BATCH);
        if (lane == 0)
#pragma unroll 16
            for (int i = 0; i < BATCH; i++) err = err + buf[i];
        __syncthreads();
    }
    if (lane == 0) out[blockIdx.x] = err / (double)n;
}

void launch_quantize(hipStream_t st, int kind, int rows, int cols, const float* w, const float* imp, uint8_t* q,
                     float* s) {
    const dim3 grid(rows / 32, (cols / 32 + 1) / 2);
    if (kind == INT8)
        hipLaunchKernelGGL(k_quantize<true>, grid, dim3(64), 0, st, w, imp, cols, q, s);
    else
        hipLaunchKernelGGL(k_quantize<false>, grid, dim3(64), 0, st, w, imp, cols, q, s);
}

void launch_scale_cols(hipStream_t st, const float* src, int64_t n, int k, const float* s, int div, float* dst) {
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_scale_cols, dim3((unsigned)blocks), dim3(256), 0, st, src, n, k, s, div, dst);
}

void launch_mm_exact(hipStream_t st, int kind, const float* x, int m, int K, const float* wf, const uint8_t* q,
                     const float* s, int rows, float* y) {
    const dim3 grid((rows + 255) / 256, (m + 15) / 16);
    if (kind == BF16)
        hipLaunchKernelGGL((k_mm_exact<true, false>), grid, dim3(256), 0, st, x, m, K, wf, q, s, rows, y);
    else if (kind == INT8)
        hipLaunchKernelGGL((k_mm_exact<false, true>), grid, dim3(256), 0, st, x, m, K, wf, q, s, rows, y);
    else
        hipLaunchKernelGGL((k_mm_exact<false, false>), grid, dim3(256), 0, st, x, m, K, wf, q, s, rows, y);
}

void launch_sq_err(hipStream_t st, const float* y, int64_t ystride, int count, const float* yref, int64_t n,
                   double* out) {
    hipLaunchKernelGGL(k_sq_err, dim3(count), dim3(64), 0, st, y, ystride, yref, n, out);
}

}  // namespace fg
