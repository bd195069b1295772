// The persistent forward (pfwd.hip): arguments shared with the host side of
// the C ABI (api.hip). Not part of the public interface.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fg {

constexpr int kPfWaves = 8;                  // waves per workgroup
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfGroups = 256;               // workgroups: one per CU
constexpr int kPfMaxRows = 4;                // new rows per launch (one pass of pieces)
constexpr int kPfMaxGqa = 4;                 // query heads per kv head
constexpr int kPfMaxNtg = 8;                 // n-tiles of one work unit of a layer matrix
constexpr int kPfCounters = 32;              // counters per barrier: workgroup g arrives at counter g % 32
constexpr int kPfCounterWords = 256;         // words between two counters (1 KiB)
// control words (unsigned, 256 bytes apart): the launch epoch, the count of
// finished workgroups, the abort flag
constexpr int kPfCtlEpoch = 0, kPfCtlDone = 64, kPfCtlAbort = 128, kPfCtlWords = 192;
constexpr int kPfSpin = 1 << 20;             // polls a wait may take (about a second)
constexpr int kPfLdsMax = 160 * 1024;        // LDS of a CU

// One matrix in the device layout (internal.h) and its work units: (group of
// ntg n-tiles) x (ks slices of the chunks); unit u is group u / ks, slice u % ks.
struct PfMat {
    const void* w;
    const float* s;  // group scales (quantized kinds)
    int kb;          // padded k-blocks (a multiple of 4)
    int ntg, ks, units;
};

struct PfLayer {
    PfMat qkv, o, gu, down;
    const float* attn_norm;
    const float* mlp_norm;
    const float* bqkv;  // nullptr: no bias
};

// Offsets (floats) of one layer's exchange region; every buffer starts on a
// 256-byte boundary and no two share a cache line.
struct PfXch {
    // per layer: x_b, q/k/v partials, attention partials, the o projection's
    // input pieces and their int8 scales, o partials, x_a, the down
    // projection's input pieces and scales, down partials
    size_t xb, qkv, part, opa, oxs, o, xa, dpa, dxs, d, layer;
    size_t lmb;                                       // after the L layer regions: per-workgroup best (value, index) per row
    size_t total;
};

struct PfArgs {
    const PfLayer* layers;  // device array
    int L;
    float* kc;  // KV cache: layer l's keys at kc + l * layer_floats
    float* vc;
    size_t layer_floats;
    int H, I, nh, nkv, qd, kvd, V, il;
    float eps, scale;
    const uint16_t* embed;  // [V][H] bf16
    const void* lm;         // lm_head, bf16 tiles
    int lm_kb;
    const float* norm;
    const float* cos_t;
    const float* sin_t;
    int t;                   // new rows at positions *pos0 .. *pos0 + t - 1
    const int32_t* pos0;     // device word (a step graph replays with new positions)
    const uint32_t* tok;     // token of row r: tok[r * tok_stride]
    int tok_stride;
    const int32_t* blocks;   // the sequence's block table
    int logits_rows;         // the last logits_rows rows get an argmax
    int xk;                  // floats per row of the staged f32 input (LDS)
    int pkb;                 // k-blocks of the LDS pieces (in the layer matrices' format; also holds
                             // the lm_head's bf16 pieces)
    float* x;                // exchange buffer
    PfXch xo;
    unsigned* bar;           // barrier counters [barrier][kPfCounters][kPfCounterWords]
    unsigned* ctl;
    int spin;
    int gl;                  // workgroups that run the layers (0 .. gl - 1; every workgroup runs the lm_head)
    uint32_t* am;            // argmax of the selected rows
    uint32_t* aux;           // optional copy: aux[r * aux_stride + aux_off]
    int aux_stride, aux_off;
    // the greedy accept of a verify (k > 0): verify tokens [last, d_1 .. d_k]
    int k;
    const uint32_t* vtok;
    uint32_t* out;
    int32_t* cnt;
    int32_t* acc;
};

// Barriers of one launch of a model of L layers.
constexpr int pfwd_barriers(int L) { return 6 * L + 1; }
// Exchange offsets for a model of these sizes, work units and `items` attention
// work items at most.
PfXch pfwd_xch(int kind, int L, int H, int I, int qd, int qkvd, int nkv, int gq, int ks_qkv, int ks_o, int ks_d,
               int items, int groups);
size_t pfwd_lds_bytes(int kind, int xk, int pkb);
// Allows the kernels their dynamic LDS (once per process).
hipError_t pfwd_init();
// Workgroups one launch uses (all resident at once; 0 when fewer than kPfGroups fit).
int pfwd_groups(int kind, int xk, int pkb);
void launch_pfwd(hipStream_t st, int kind, int groups, const PfArgs& a);

}  // namespace fg
