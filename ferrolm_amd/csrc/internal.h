// Internal declarations shared by the device kernels (kernels.hip) and the
// host side of the C ABI (api.hip). Not part of the public interface.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fg {

// ---------------------------------------------------------------------------
// Device weight layout (repacked at upload from the reference's formats).
//
// A matrix of N output rows x K inputs is cut into tiles of 16 rows and
// k-blocks of 32 inputs (one quantization group). K is padded with zeros to
// a multiple of 128 (4 k-blocks). One tile x k-block is exactly one MFMA
// B-operand: lane l (0..63) holds row n = l % 16, inputs 8*(l/16) .. +7.
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
// Each (tile, 4 k-blocks) chunk is contiguous, so a wave's 16-byte loads
// cover 1 KB of consecutive memory.
// ---------------------------------------------------------------------------
enum { BF16 = 0, INT8 = 1, INT4 = 2 };

struct DMat {
    int kind = 0;
    int rows = 0, cols = 0;   // N, K (unpadded)
    int n_tiles = 0, kb = 0;  // rows/16, padded K/32 (multiple of 4)
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
struct Pieces {
    void* a = nullptr;
    float* xs = nullptr;
    int kb = 0, passes = 0;
};

struct GemvPlan {
    int splits = 1;
};

// Kernel launchers (kernels.hip).
void launch_embed(hipStream_t st, const uint32_t* tokens, int stride, const uint16_t* embed, int m, int H, float* x);
void launch_residual_rms(hipStream_t st, float* x, const float* partials, int splits, int m, int H, float eps,
                         float* rinv);
void launch_pieces(hipStream_t st, int consumer_kind, const float* x, int ldx, int m, int K, const float* g,
                   const float* rinv, Pieces& out);
void launch_silu_pieces(hipStream_t st, const float* partials, int splits, int m, int I, Pieces& out,
                        float* act_out, int consumer_kind);
GemvPlan plan_gemv(const DMat& w, int m);
void launch_gemv(hipStream_t st, const DMat& w, const Pieces& x, int m, const GemvPlan& plan, float* partials);
void launch_reduce(hipStream_t st, const float* partials, int splits, int m, int N, const float* bias, float* y);
void launch_rope_kv(hipStream_t st, const float* partials, int splits, int m, const float* bias,
                    const int32_t* row_pos, const int32_t* row_slot, const float* cos_t, const float* sin_t,
                    int nh, int nkv, int hd, int bs, float* q_out, float* kc, float* vc);

struct AttnArgs {
    const float* q;          // [m][nh*hd]
    const float* kc;         // layer K cache
    const float* vc;
    const int32_t* row_pos;  // [m]
    const int32_t* wi_group; // work item -> group
    const int32_t* wi_split; // work item -> split index within group
    const int32_t* g_row0;   // group -> first row
    const int32_t* g_nrows;
    const int32_t* g_table;  // group -> offset of its block table in tables[]
    const int32_t* g_wi0;    // group -> first work item
    const int32_t* g_nsplit;
    const uint32_t* tables;
    float* part;             // [wi][nkv][qmax][hd+2]
    float* out;              // [m][nh*hd]
    const int32_t* row_group;// [m] -> group
    int n_wi, nh, nkv, hd, bs, split_pos, qmax;
    float scale;
};
void launch_attention(hipStream_t st, const AttnArgs& a, int m);

void launch_argmax(hipStream_t st, const float* partials, int splits, int rows, int V, float* logits_out,
                   float2* block_best, int nblk, uint32_t* argmax_out, uint32_t* aux, int aux_stride,
                   int aux_off);
void launch_gather_rows(hipStream_t st, const float* x, const int32_t* rows, int n, int H, float* out);
void launch_accept(hipStream_t st, const uint32_t* argmax, const uint32_t* drafts, int n_seqs, int k,
                   uint32_t* out_tokens, int32_t* out_count, int32_t* out_accepted);
void launch_copy_tokens(hipStream_t st, const uint32_t* src, int n, int src_stride, uint32_t* dst,
                        int dst_stride);

}  // namespace fg
