// The persistent draft forward (pdraft.hip): arguments shared with the host
// side of the C ABI (api.hip). Not part of the public interface.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fg {

constexpr int kPdWaves = 8;     // waves per workgroup
constexpr int kPdGroups = 256;  // workgroups at most: one per CU
constexpr int kPdMaxRows = 4;   // new rows per launch
constexpr int kPdMaxGqa = 4;    // query heads per kv head
constexpr int kPdMaxKb = 48;    // k-blocks of 32 of any matrix (hidden, intermediate, q sizes <= 1536)
// control words (unsigned, 128-byte apart): the launch epoch, the count of
// finished workgroups, the abort flag
constexpr int kPdCtlEpoch = 0, kPdCtlDone = 32, kPdCtlAbort = 64, kPdCtlWords = 96;
constexpr int kPdSpin = 1 << 21;  // polls a wait may take (a few seconds)

// One layer's device weights: bf16 in the MFMA tile layout, K padded to kb * 32.
struct PdLayer {
    const void* wqkv;
    const void* wo;
    const void* wgu;  // gate/up interleaved in blocks of 16 rows
    const void* wd;
    int qkv_kb, o_kb, gu_kb, d_kb;
    const float* attn_norm;
    const float* mlp_norm;
    const float* bqkv;  // nullptr: no bias
};

struct PdArgs {
    const PdLayer* layers;  // device array
    float* kc;              // KV cache: layer l's keys at kc + l * layer_floats
    float* vc;
    size_t layer_floats;
    int L, H, I, nh, nkv, qd, kvd, V;
    float eps, scale;
    const uint16_t* embed;  // [V][H] bf16
    const void* lm;         // lm_head, tiles of 16 rows
    int lm_kb;
    const float* norm;
    const float* cos_t;
    const float* sin_t;
    int t;                  // new rows at positions *pos0 .. *pos0 + t - 1
    const int32_t* pos0;    // device word (a step graph replays with new positions)
    const uint32_t* tok;    // token of row r: tok[r * tok_stride]
    int tok_stride;
    const int32_t* blocks;  // the sequence's block table
    int logits_rows;        // the last logits_rows rows get logits and an argmax
    int ap_kb;              // k-blocks of the LDS activation operand (>= every matrix's kb)
    // tagged words (f32 bits | tag << 32)
    uint64_t *xa, *xb, *qkv, *att, *act, *part, *lmp;
    unsigned* ctl;
    int spin;               // polls a wait may take before it aborts the launch
    uint32_t* am;           // argmax of the selected rows
    uint32_t* aux;          // optional copy: aux[r * aux_stride + aux_off]
    int aux_stride, aux_off;
};

// Tagged words the exchange buffers need for a model of these sizes (t <= 4
// rows) and at most `spans` attention spans of 64 positions.
struct PdSizes {
    size_t xa, xb, qkv, att, act, part, lmp;
    size_t total() const { return xa + xb + qkv + att + act + part + lmp; }
};
PdSizes pdraft_sizes(int H, int I, int qd, int kvd, int nh, int nkv, int spans);
size_t pdraft_lds_bytes(int ap_kb);
// Allows the kernel its dynamic LDS (once per process).
hipError_t pdraft_init();
// Workgroups one launch may use so that all of them are resident at once (at
// most kPdGroups; 0 when the device cannot say).
int pdraft_groups(int ap_kb);
void launch_pdraft(hipStream_t st, int groups, const PdArgs& a);

}  // namespace fg
