// Device helpers of the hot-path kernels (kernels.hip): vector
// types, non-temporal loads, bf16 conversion, the Cephes exp of the reference,
// cross-lane reductions and the activation-piece conversions. Not part of the
// public interface.
#pragma once
#include "internal.h"

#include <math.h>

namespace fg {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef int8_t i8x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef long long i64x2 __attribute__((ext_vector_type(2)));

// A load marked non-temporal (NT) or plain. Data read once per step (quantized
// weights and their scales, the lm_heads, the KV cache) is loaded
// non-temporally: such lines are not kept in the 256 MB memory-side cache,
// which then holds what a step reads again (a bf16 draft's layer weights,
// 212 MB at 135M, read by every draft round). Measured: a 200 MB buffer stays
// resident across a 1.2 GB non-temporal stream and is evicted by a plain one.
template <bool NT, typename T>
__device__ __forceinline__ T ld_nt(const T* p) {
    if constexpr (NT)
        return __builtin_nontemporal_load(p);
    else
        return *p;
}
__device__ __forceinline__ float4 ld_nt_f4(const float* p) {
    const f32x4 v = __builtin_nontemporal_load((const f32x4*)p);
    return make_float4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// In-kernel timeline (see stamps_read): declared at a kernel's entry, end()
// at each of its exits. Without FERRO_STAMPS it is empty and compiles away.
#ifdef FERRO_STAMPS
extern __device__ unsigned long long g_stamps[kStampSlots][kStampWgs][2];
struct Stamp {
    unsigned long long t0;
    int slot;
    __device__ explicit Stamp(int s) : t0(__builtin_amdgcn_s_memrealtime()), slot(s) {}
    __device__ void end() const {
        const int wg = (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
        if (threadIdx.x == 0 && slot >= 0 && slot < kStampSlots && wg < kStampWgs) {
            g_stamps[slot][wg][0] = t0;
            g_stamps[slot][wg][1] = __builtin_amdgcn_s_memrealtime();
        }
    }
};
#else
struct Stamp {
    __device__ explicit Stamp(int) {}
    __device__ void end() const {}
};
#endif

// round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }

__device__ __forceinline__ bf16x8 as_bf16x8(u16x8 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Four f32 values as two bf16 pieces each, hi = bf16(x) and lo = bf16(x - hi),
// stored as four consecutive bf16 at hi and at lo (8-byte aligned).
__device__ __forceinline__ void split4(const float (&v)[4], uint16_t* hi, uint16_t* lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        h[e] = f32_to_bf16_bits(v[e]);
        l[e] = f32_to_bf16_bits(v[e] - bf16_bits_to_f32(h[e]));
    }
    *(uint2*)hi = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    *(uint2*)lo = make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
}

// exp(x) by range reduction and the Cephes expf polynomial, the same
// sequence of operations as the reference's kernels::exp (src/kernels.rs:609-637).
__device__ __forceinline__ float dev_exp(float x) {
    x = fminf(fmaxf(x, -87.0f), 88.0f);
    const float n = rintf(x * 1.44269504088896341f);
    const float r = fmaf(n, 2.1219444e-4f, fmaf(n, -0.6933594f, x));
    float p = 1.9875691e-4f;
    p = fmaf(p, r, 1.3982e-3f);
    p = fmaf(p, r, 8.333452e-3f);
    p = fmaf(p, r, 4.1665796e-2f);
    p = fmaf(p, r, 0.16666665f);
    p = fmaf(p, r, 0.5f);
    const float y = fmaf(p, r * r, r) + 1.0f;
    return y * __int_as_float(((int)n + 127) << 23);
}

// ---------------------------------------------------------------------------
// Activation pieces (see Pieces in internal.h). Called by a whole wave: lane
// l holds v[0..7] = inputs 8*(l/16)..+7 of k-block kb for (row, piece) =
// (4*pass + (l%16)/4, l%4). The four lanes of a (row, inputs) pair must hold
// bit-identical v: each writes its own piece, and for int8 each derives the
// block scale itself. Producers that combine values across lanes therefore
// sum rounded values in a symmetric order (the library is built without
// floating-point contraction, so a shuffle sum is never fused with a product).
// ---------------------------------------------------------------------------
// Cross-lane reductions without the LDS crossbar (ds_bpermute). Within rows
// of 16 lanes: DPP quad swaps (partners l^1, l^2) and the row mirrors; across
// rows: the gfx950 row swaps, whose two results hold the even and the odd
// 16-lane rows (or 32-lane halves), so both lanes of a pair combine the same
// operands in the same order and end with the same bits. Every lane of the
// group must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_xor1(float v) { return dpp_f<0xB1>(v); }  // quad_perm [1,0,3,2]
__device__ __forceinline__ float lane_xor2(float v) { return dpp_f<0x4E>(v); }  // quad_perm [2,3,0,1]
template <bool MAX>
__device__ __forceinline__ float red_op(float x, float y) { return MAX ? fmaxf(x, y) : x + y; }
// over lanes l, l^16 (and l^32 when WIDE)
template <bool MAX, bool WIDE>
__device__ __forceinline__ float reduce_rows(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = red_op<MAX>(__uint_as_float(r[0]), __uint_as_float(r[1]));
    if (WIDE) {
        const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = red_op<MAX>(__uint_as_float(h[0]), __uint_as_float(h[1]));
    }
    return v;
}
// out[j] = v of lane (l % 16) + 16 j, for every lane l.
__device__ __forceinline__ void gather_rows(float v, float (&out)[4]) {
    const uint32_t x = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);  // rows (2r, 2r+1) of each half
    const auto e = __builtin_amdgcn_permlane32_swap(a[0], a[0], false, false);
    const auto o = __builtin_amdgcn_permlane32_swap(a[1], a[1], false, false);
    out[0] = __uint_as_float(e[0]);
    out[1] = __uint_as_float(o[0]);
    out[2] = __uint_as_float(e[1]);
    out[3] = __uint_as_float(o[1]);
}
// Max / sum over aligned groups of N lanes (4, 8, 16, 32 or 64).
template <int N, bool MAX>
__device__ __forceinline__ float group_reduce(float v) {
    static_assert(N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "4, 8, 16, 32 or 64 lanes");
    v = red_op<MAX>(v, lane_xor1(v));
    v = red_op<MAX>(v, lane_xor2(v));
    if (N >= 8) v = red_op<MAX>(v, dpp_f<0x141>(v));  // row_half_mirror: the other quad of the 8
    if (N >= 16) v = red_op<MAX>(v, dpp_f<0x140>(v));  // row_mirror: the other 8 of the row
    if (N >= 32) v = reduce_rows<MAX, N == 64>(v);
    return v;
}

// bf16 piece `piece` of x: four successive bf16 roundings of the remainder
// (all four are formed and one is selected, without branches).
__device__ __forceinline__ uint32_t bf16_piece(float x, int piece) {
    uint32_t h = f32_to_bf16_bits(x), sel = h;
#pragma unroll
    for (int p = 1; p < 4; p++) {
        x = x - bf16_bits_to_f32(h);
        h = f32_to_bf16_bits(x);
        sel = p == piece ? h : sel;
    }
    return sel;
}

// Exponent e of the int8 block scale 2^e shared by the four lanes of a row
// (l, l^16, l^32, l^48 hold its 32 inputs; mx is this lane's max |input|):
// the block maximum / 2^e lies in [64, 128) and never rounds past 127.
__device__ __forceinline__ int int8_block_exp(float mx) {
    mx = reduce_rows<true, true>(mx);
    int e = 0;
    if (mx > 0.0f) {
        int fe;
        frexpf(mx, &fe);
        e = fe - 7;
        if (ldexpf(mx, -e) > 127.0f) e++;
    }
    return e;
}

// int8 piece `piece` of x at block exponent e: x / 2^e = a0 + a1/128 + ...
__device__ __forceinline__ int int8_piece(float x, int e, int piece) {
    float r = ldexpf(x, -e);  // exact
    float a = rintf(r), sel = a;
#pragma unroll
    for (int p = 1; p < 4; p++) {
        r = (r - a) * 128.0f;  // both exact
        a = rintf(r);
        sel = p == piece ? a : sel;
    }
    return (int)sel;
}

}  // namespace fg
