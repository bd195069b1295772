// Host side of the C ABI declared in include/ferro_gpu.h: weight upload and
// repacking, the paged KV cache, the forward pass and the on-device greedy
// speculative step. Each entry point names the reference interface it
// replaces in the header.
#include "ferro_gpu.h"
#include "ferro_host.h"
#include "internal.h"

#include <algorithm>
#include <mutex>
#include <atomic>
#include <cstdlib>
#include <functional>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

using namespace fg;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define HIPCHK(x)                                                                                   \
    do {                                                                                            \
        hipError_t e_ = (x);                                                                        \
        if (e_ != hipSuccess) return fail(FG_E_DEVICE, std::string(#x) + ": " + hipGetErrorString(e_)); \
    } while (0)


template <class F>
void parallel_for(int n, F f) {
    int nt = (int)std::thread::hardware_concurrency();
    nt = std::max(1, std::min(nt, 16));
    nt = std::min(nt, std::max(1, n));
    if (nt == 1) {
        for (int i = 0; i < n; i++) f(i);
        return;
    }
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++)
        th.emplace_back([=, &f] {
            for (int i = t; i < n; i += nt) f(i);
        });
    for (auto& x : th) x.join();
}

int round_up(int a, int b) { return (a + b - 1) / b * b; }

// Carves aligned sub-buffers out of one allocation; with base == nullptr it
// only measures.
struct Carver {
    char* base;
    size_t off = 0;
    explicit Carver(void* b) : base((char*)b) {}
    template <class T>
    T* take(size_t n) {
        off = (off + 255) & ~(size_t)255;
        T* p = base ? (T*)(base + off) : nullptr;
        off += n * sizeof(T);
        return p;
    }
};

}  // namespace

// ---------------------------------------------------------------------------
// Handles
// ---------------------------------------------------------------------------
struct fg_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    // this device's copy of `scratch` (fg_matmul_device_noalloc), from
    // hipGetSymbolAddress at creation; nullptr when that failed
    uint8_t* scratch = nullptr;
    void* ws = nullptr;
    size_t ws_cap = 0;
    void* sbuf = nullptr;  // sampling: the distributions of a step's rows
    size_t sbuf_cap = 0;
    void* dmeta = nullptr;
    size_t dmeta_cap = 0;
    void* hmeta = nullptr;
    size_t hmeta_cap = 0;
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    float last_us[3] = {0, 0, 0};
    bool merge_in_o = true;  // small bf16 output projections merge the attention spans themselves
    bool mlp_fuse = true;    // bf16 layers of one pass run fused (mlp_fuse: split output projection, EPI_MLP)
    // in-kernel timeline (libraries built with stamps): the next launch's slot
    // (every fg_forward and speculative step starts over at 0, so a captured
    // graph bakes the same slots each time) and each slot's kernel label
    int stamp_seq = 0;
    std::vector<std::string> stamp_labels;
    // split-K GEMV meeting counters (GemvArgs::gcnt): zeroed once here, left at
    // zero by every launch's last workgroups
    unsigned* gcnt = nullptr;
    // GEMV launch profiling (fg_profile)
    bool prof = false;
    std::vector<hipEvent_t> pev;
    size_t pev_used = 0;
    struct Pending {
        int cls;
        double bytes, flops;
        size_t ev;
    };
    std::vector<Pending> pending;
    struct Rec {
        int64_t n = 0;
        double us = 0, bytes = 0, flops = 0;
    };
    Rec rec[12];
    // HIP graphs of the speculative step (draft rounds, verify pass), one
    // entry per launch signature, the least recently used replaced first.
    struct GraphSet {
        std::vector<int64_t> sig;
        hipGraphExec_t exec[2] = {nullptr, nullptr};
        uint64_t used = 0;
    };
    static constexpr int kGraphSets = 8;
    std::vector<GraphSet> gsets;
    bool capturing = false;  // a step is being captured: no per-launch events
    uint64_t gclock = 0;
    bool graphs = true;
};

static void drop_set(fg_ctx::GraphSet& g) {
    for (auto& e : g.exec)
        if (e) {
            (void)hipGraphExecDestroy(e);
            e = nullptr;
        }
    g.sig.clear();
}

static void drop_graphs(fg_ctx* c) {
    for (auto& g : c->gsets) drop_set(g);
    c->gsets.clear();
}

// Algorithmic bytes of one GEMV launch over m rows: codes + group scales
// (or bf16 weights), f32 activations in, f32 products out.
static double gemv_bytes(const DMat& d, int m) {
    const double nk = (double)d.rows * d.cols;
    double w = d.kind == BF16 ? nk * 2 : d.kind == INT8 ? nk + nk / 32 * 4 : nk / 2 + nk / 32 * 4;
    return w + (double)m * d.cols * 4 + (double)m * d.rows * 4;
}

static hipEvent_t prof_event(fg_ctx* c) {
    if (c->pev_used == c->pev.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        c->pev.push_back(e);
    }
    return c->pev[c->pev_used++];
}

// The timeline slot of the next launch, labelled (-1 in a library built without stamps).
static int next_stamp(fg_ctx* c, const std::string& label) {
#ifdef FERRO_STAMPS
    const int s = c->stamp_seq++;
    if (s >= kStampSlots) return -1;
    if ((int)c->stamp_labels.size() <= s) c->stamp_labels.resize(s + 1);
    c->stamp_labels[s] = label;
    return s;
#else
    (void)c;
    (void)label;
    return -1;
#endif
}

static std::string gemv_label(int epi, const DMat& w, const GemvArgs& a) {
    static const char* epis[] = {"store", "qkv", "resid", "silu", "lm_head", "mlp"};
    static const char* kinds[] = {"bf16", "int8", "int4"};
    std::string s = std::string(a.mm ? "gemm " : "gemv ") + kinds[w.kind] + " " + epis[epi];
    if (a.ax) s += " ax";
    if (a.am) s += " am";
    return s + " " + std::to_string(w.rows) + "x" + std::to_string(w.cols);
}

// launch_gemv, timed by its own dispatch while profiling (fg_profile). The
// speculative step launches directly (no graph) while profiling is on.
static void gemv(fg_ctx* c, int epi, const DMat& w, const GemvArgs& a0) {
    GemvArgs a = a0;
    a.stamp = next_stamp(c, gemv_label(epi, w, a));
    if (a.mm) a.gcnt = c->gcnt;  // a split GEMM of small tiles meets on these counters and finishes in place
    if (!c->prof || c->capturing) {
        launch_gemv(c->stream, epi, w, a);
        return;
    }
    const int pg = a.mm ? 3 : a.p_total == 1 ? 0 : a.p_total == 2 ? 1 : 2;
    const size_t i0 = c->pev_used;
    hipEvent_t e0 = prof_event(c), e1 = prof_event(c);
    if (!e0 || !e1) {
        launch_gemv(c->stream, epi, w, a);
        return;
    }
    launch_gemv(c->stream, epi, w, a, e0, e1);
    c->pending.push_back({w.kind * 4 + pg, gemv_bytes(w, a.m), 2.0 * a.m * w.rows * w.cols, i0});
}

struct DLayer {
    float* attn_norm = nullptr;
    DMat wqkv;
    float* bqkv = nullptr;
    DMat wo;
    float* mlp_norm = nullptr;
    DMat w_gate_up;
    DMat w_down;
};

// Every model and cache gets a process-wide serial number at creation; the
// step-graph cache keys on these, never on addresses that a later object
// could reuse.
static std::atomic<uint64_t> g_serial{1};

struct fg_model {
    uint64_t serial = g_serial++;
    fg_config cfg{};
    std::vector<DLayer> layers;
    uint16_t* embed = nullptr;
    DMat lm_head;
    float* norm = nullptr;
    float* cos_t = nullptr;
    float* sin_t = nullptr;
    int max_pos = 0;
    bool owns = true;
    std::vector<void*> allocs;
    int64_t ref_bytes = 0;
};

struct fg_kv {
    uint64_t serial = g_serial++;
    int layers = 0, kv_heads = 0, head_dim = 0, block_size = 0, blocks = 0;
    float* k = nullptr;  // [layer][blocks*bs*nkv*hd]
    float* v = nullptr;
    size_t layer_floats() const { return (size_t)blocks * block_size * kv_heads * head_dim; }
};

struct fg_mat {
    DMat m;
    int device = 0;
};

static int ensure(void** p, size_t* cap, size_t need, hipStream_t st, bool host) {
    if (need <= *cap && *p) return 0;
    if (st) HIPCHK(hipStreamSynchronize(st));
    size_t n = std::max(need + need / 4, (size_t)1 << 20);
    if (*p) {
        if (host)
            HIPCHK(hipHostFree(*p));
        else
            HIPCHK(hipFree(*p));
        *p = nullptr;
        *cap = 0;
    }
    if (host) {
        if (hipHostMalloc(p, n, hipHostMallocDefault) != hipSuccess) return fail(FG_E_NOMEM, "pinned host allocation failed");
    } else {
        if (hipMalloc(p, n) != hipSuccess) return fail(FG_E_NOMEM, "device allocation failed");
    }
    *cap = n;
    return 0;
}

// ---------------------------------------------------------------------------
// Repacking from the reference's formats to the device layout (internal.h).
// ---------------------------------------------------------------------------
static inline int qcode(const uint8_t* q, int kind, int K, int r, int k) {
    const int p = r / 32, c = r % 32;
    if (kind == INT8) return (int8_t)q[((size_t)p * K + k) * 32 + c];
    const uint8_t b = q[((size_t)p * K + k) * 16 + (c % 16)];
    return (c < 16 ? (b & 15) : (b >> 4)) - 8;
}

// Device row r of the gate/up matrix (interleaved in blocks of il rows, see
// internal.h) and the source row it holds.
static inline int src_row(int r, int inter, int il) {
    if (inter <= 0) return r;
    const int blk = r / (2 * il), within = r % (2 * il);
    return within < il ? blk * il + within : inter + blk * il + within - il;
}

static int repack(const fg_matrix& src, DMat& d, std::vector<uint8_t>& w, std::vector<float>& s, int inter, int il) {
    if (src.rows <= 0 || src.cols <= 0 || src.rows % 32 || (src.format != FG_BF16 && src.cols % 32))
        return fail(FG_E_SHAPE, "matrix rows must be a multiple of 32 (and cols of 32 when quantized)");
    if (src.format == FG_BF16 && !src.bf16) return fail(FG_E_ARG, "bf16 matrix without data");
    if (src.format != FG_BF16 && (!src.q || !src.s)) return fail(FG_E_ARG, "quantized matrix without codes/scales");
    if (src.format < 0 || src.format > 2) return fail(FG_E_ARG, "unknown matrix format");
    const int N = src.rows, K = src.cols;
    d.kind = src.format;
    d.rows = N;
    d.cols = K;
    d.n_tiles = N / 16;
    d.kb = round_up((K + 31) / 32, 4);
    const int KB = d.kb, KC = KB / 4;
    if (d.kind == BF16) {
        d.ref_bytes = (int64_t)N * K * 2;
        w.assign((size_t)d.n_tiles * KB * 64 * 16, 0);
        uint16_t* out = (uint16_t*)w.data();
        parallel_for(d.n_tiles, [&](int t) {
            for (int kb = 0; kb < KB; kb++)
                for (int l = 0; l < 64; l++) {
                    const int n = src_row(t * 16 + l % 16, inter, il), k0 = kb * 32 + 8 * (l / 16);
                    uint16_t* o = out + (((size_t)t * KB + kb) * 64 + l) * 8;
                    for (int sl = 0; sl < 8; sl++) o[sl] = k0 + sl < K ? src.bf16[(size_t)n * K + k0 + sl] : 0;
                }
        });
        s.clear();
        return 0;
    }
    const int G = K / 32;
    const bool q4 = d.kind == INT4;
    d.ref_bytes = (int64_t)N * K / (q4 ? 2 : 1) + (int64_t)N * G * 4;
    s.assign((size_t)d.n_tiles * KC * 16 * 4, 0.0f);
    parallel_for(d.n_tiles, [&](int t) {
        for (int kb = 0; kb < G; kb++)
            for (int r = 0; r < 16; r++) {
                const int n = src_row(t * 16 + r, inter, il), p = n / 32, c = n % 32;
                float v = src.s[((size_t)p * G + kb) * 32 + c];
                if (q4) v *= 0.0625f;
                s[(((size_t)t * KC + kb / 4) * 16 + r) * 4 + kb % 4] = v;
            }
    });
    if (q4) {
        w.assign((size_t)d.n_tiles * KC * 64 * 16, 0);
        uint32_t* out = (uint32_t*)w.data();
        parallel_for(d.n_tiles, [&](int t) {
            for (int kb = 0; kb < G; kb++)
                for (int l = 0; l < 64; l++) {
                    const int n = src_row(t * 16 + l % 16, inter, il), k0 = kb * 32 + 8 * (l / 16);
                    uint32_t word = 0;
                    for (int sl = 0; sl < 8; sl++) {
                        const int code = qcode(src.q, INT4, K, n, k0 + sl);
                        const int ni = sl < 4 ? 2 * sl : 2 * (sl - 4) + 1;
                        word |= (uint32_t)(code & 15) << (4 * ni);
                    }
                    out[(((size_t)t * KC + kb / 4) * 64 + l) * 4 + kb % 4] = word;
                }
        });
    } else {
        w.assign((size_t)d.n_tiles * (KB / 2) * 64 * 16, 0);
        int8_t* out = (int8_t*)w.data();
        parallel_for(d.n_tiles, [&](int t) {
            for (int kb = 0; kb < G; kb++)
                for (int l = 0; l < 64; l++) {
                    const int n = src_row(t * 16 + l % 16, inter, il), k0 = kb * 32 + 8 * (l / 16);
                    int8_t* o = out + (((size_t)t * (KB / 2) + kb / 2) * 64 + l) * 16 + (kb % 2) * 8;
                    for (int sl = 0; sl < 8; sl++) o[sl] = (int8_t)qcode(src.q, INT8, K, n, k0 + sl);
                }
        });
    }
    return 0;
}

static int upload_mat(const fg_matrix& src, DMat& d, std::vector<void*>* allocs, int inter = 0, int il = 32) {
    std::vector<uint8_t> w;
    std::vector<float> s;
    if (inter > 0 && (inter % 32 || src.rows != 2 * inter))
        return fail(FG_E_SHAPE, "intermediate size must be a multiple of 32");
    d.il = inter > 0 ? il : 0;
    int rc = repack(src, d, w, s, inter, il);
    if (rc) return rc;
    d.w_bytes = w.size();
    d.s_bytes = s.size() * 4;
    if (hipMalloc(&d.w, d.w_bytes) != hipSuccess) return fail(FG_E_NOMEM, "weight allocation failed");
    if (allocs) allocs->push_back(d.w);
    HIPCHK(hipMemcpy(d.w, w.data(), d.w_bytes, hipMemcpyHostToDevice));
    if (d.s_bytes) {
        if (hipMalloc((void**)&d.s, d.s_bytes) != hipSuccess) return fail(FG_E_NOMEM, "scale allocation failed");
        if (allocs) allocs->push_back(d.s);
        HIPCHK(hipMemcpy(d.s, s.data(), d.s_bytes, hipMemcpyHostToDevice));
    }
    return 0;
}

template <class T>
static int upload_vec(const T* src, size_t n, T** dst, std::vector<void*>& allocs) {
    if (hipMalloc((void**)dst, n * sizeof(T)) != hipSuccess) return fail(FG_E_NOMEM, "allocation failed");
    allocs.push_back(*dst);
    HIPCHK(hipMemcpy(*dst, src, n * sizeof(T), hipMemcpyHostToDevice));
    return 0;
}

// inv_freq and the cos/sin tables, in f32 with the C library's powf, cosf
// and sinf (src/model.rs:434-448, 461-492).
static void rope_tables(const fg_config& c, int max_pos, std::vector<float>& cs, std::vector<float>& sn) {
    const int dim = c.head_dim, half = dim / 2;
    std::vector<float> f(half);
    for (int i = 0; i < half; i++) f[i] = 1.0f / powf(c.rope_theta, (float)(2 * i) / (float)dim);
    if (c.rope_llama3) {
        const float old = (float)c.rope_orig_max_pos;
        const float low_wavelen = old / c.rope_low_freq, high_wavelen = old / c.rope_high_freq;
        for (int i = 0; i < half; i++) {
            const float fr = f[i];
            const float wavelen = 2.0f * 3.14159265358979323846f / fr;
            if (wavelen < high_wavelen) {
                f[i] = fr;
            } else if (wavelen > low_wavelen) {
                f[i] = fr / c.rope_factor;
            } else {
                const float smooth = (old / wavelen - c.rope_low_freq) / (c.rope_high_freq - c.rope_low_freq);
                const float a = (1.0f - smooth) * fr;
                const float b = smooth * fr;
                f[i] = a / c.rope_factor + b;
            }
        }
    }
    cs.resize((size_t)max_pos * half);
    sn.resize((size_t)max_pos * half);
    parallel_for(max_pos, [&](int p) {
        for (int i = 0; i < half; i++) {
            volatile float a = (float)p * f[i];
            cs[(size_t)p * half + i] = cosf(a);
            sn[(size_t)p * half + i] = sinf(a);
        }
    });
}

// ---------------------------------------------------------------------------
// Forward plan: row bookkeeping (src/model.rs:278-294), attention work items
// and the logits rows (src/model.rs:338-350), packed into one int32 upload.
// ---------------------------------------------------------------------------
struct ChunkIn {
    const uint32_t* tokens;  // host tokens, or nullptr when they come from device
    int n, pos;
    const uint32_t* blocks;
    int n_blocks, logits;
};

struct Plan {
    int t = 0, S = 0, W = 0;
    int ns = 1;  // attention sub-spans per work item (k_attn's NS)
    int Wc = 0;  // work items launched: W rounded up to 16, the extra records empty, so
                 // the launch shapes (and a captured step graph) last for 16 more spans
    int maxq = 0;  // queries of the largest attention row group (rows x GQA group)
    // wrec: one 16-word record per attention work item (a span of one row
    // group): row0, nrows, crow0, cpos0 (first row and position of the
    // group's chunk), p0, p1 (the span), 0, 0, then the physical ids of the
    // span's cache blocks. mrec: per row, the row's first query index within
    // its group, the group's first work item and its number of spans.
    std::vector<int32_t> wrec, mrec, sel;
    std::vector<uint32_t> tokens;
    // flash: the attention runs as k_attn_flash items (wrec holds one record per
    // item, W counts two partial slots per item); btab holds the block tables
    // of the chunks the items read
    bool flash = false;
    std::vector<int32_t> btab;
    // offsets (in int32 words) of each array inside the packed metadata
    size_t o_wrec, o_mrec, o_sel, o_tok, o_btab, words;
};


// one-span attention items from which decode-sized row groups at hd 64 take two sub-spans
static constexpr int64_t kTwoSubSpanItems = 4096;

static int build_plan(const fg_config& c, const fg_kv& kv, int max_pos, const ChunkIn* ch, int nch, Plan& P) {
    const int bs = kv.block_size;
    const int group = c.heads / c.kv_heads;
    // rows per attention row group: as many as the work item's queries allow, up
    // to 32 (each group re-reads the K/V of every span it sees; the 1.7B
    // shape's 1024-token prefill, MHA at hd 64, in groups of 32 rows rather
    // than 16: 16.6 against 17.5 ms)
    const int rg = std::max(1, std::min(32, attn_qmax(c.head_dim) / group));
    const int span1 = attn_span(c.head_dim);
    if (bs != 16 || span1 % bs || span1 / bs > 8) return fail(FG_E_SHAPE, "attention spans need 16-token blocks");
    P = Plan();
    // Work items of one span, or, when they would be more than 1024 workgroups
    // and a row group reaches kAttnMfmaQueries queries (GQA verify batches,
    // prefill chunks), of 128 positions: 2 or 4 sub-spans whose loads overlap
    // the scoring of the previous one. Otherwise one span per work item
    // (measured: fewer, longer items are slower for the few queries of a
    // decode step, cfg3 verify 3.02 against 2.73 ms; cfg4's 20-query items
    // gain, verify 11.2 to 10.0 ms).
    int64_t w1 = 0;
    int maxq = 0;
    for (int ci = 0; ci < nch; ci++)
        for (int r0 = 0; r0 < ch[ci].n; r0 += rg) {
            const int nr = std::min(rg, ch[ci].n - r0);
            const int64_t L = (int64_t)ch[ci].pos + r0 + nr;
            w1 += (L + span1 - 1) / span1;
            maxq = std::max(maxq, nr * group);
        }
    P.ns = w1 * c.kv_heads > 1024 && maxq >= kAttnMfmaQueries ? 128 / span1 : 1;
    // Decode-sized row groups at hd 64 take two sub-spans per item once the
    // launch holds at least kTwoSubSpanItems one-span items (on the MFMA path,
    // the queries padded to a 16-row tile): the second sub-span's loads fly
    // while the first is scored. cfg3 at 32 sequences (16,896 items): verify
    // 6105-6111 against 5867 us; 32-position spans instead: 6182 us. At 8
    // sequences (about 4,400 items) verify 2595-2599 against 2546-2549 us; the
    // 135M draft at 32 sequences (1,584 items) is slower with them (draft
    // 5594-5601 against 5456-5458 us), so the bar sits between. Groups of at
    // most 4 queries stay on one-span items, which large launches run with the
    // keys and values in registers (k_attn_dec): cfg4's 1B draft (about 4,600
    // items of 4 queries) 6358 -> 6152 us per step and 1079 -> 1094 tok/s, where
    // cfg3's target (5 queries) went 5547-5607 -> 6101 us the same way.
    if (c.head_dim == 64 && w1 * c.kv_heads >= kTwoSubSpanItems && maxq > 4) P.ns = 128 / span1;
    P.maxq = maxq;
    const int span = span1 * P.ns;
    // Long chunks at hd 64 and 128 take the flash items (rf rows each, split into
    // parts of at most kFlashPart positions: on the 1.7B shape's 1024-token
    // prefill 15.7 ms unsplit, 15.5 at 512, 15.3 at 256) when there are at least
    // 256 rows and enough parts to spread over the CUs.
    const int rf = 2 * (attn_qmax(c.head_dim) / group);
    const int fblk = kFlashBlock(c.head_dim);
    auto flash_parts = [&](int L) {
        const int nb = (L + fblk - 1) / fblk, per = kFlashPart / fblk;
        return (nb + per - 1) / per;
    };
    {
        int64_t parts = 0, rows = 0;
        for (int ci = 0; ci < nch; ci++)
            if (ch[ci].n > 0) {
                rows += ch[ci].n;
                if (rf >= 2)
                    for (int r0 = 0; r0 < ch[ci].n; r0 += rf)
                        parts += flash_parts(ch[ci].pos + r0 + std::min(rf, ch[ci].n - r0));
            }
        P.flash = (c.head_dim == 64 || c.head_dim == 128) && rf >= 2 && rows >= 256 && parts * c.kv_heads >= 256;
        if (P.flash) P.ns = 1;
    }
    for (int ci = 0; ci < nch; ci++) {
        const ChunkIn& k = ch[ci];
        if (k.n < 0 || k.pos < 0) return fail(FG_E_ARG, "negative chunk length or position");
        if (k.n == 0) continue;
        if ((int64_t)k.n_blocks * bs < (int64_t)k.pos + k.n)
            return fail(FG_E_SHAPE, "chunk overruns its cache blocks");
        if (k.pos + k.n > max_pos) return fail(FG_E_SHAPE, "position beyond max_position");
        if (!k.blocks) return fail(FG_E_ARG, "chunk without a block table");
        const int used = (k.pos + k.n + bs - 1) / bs;
        for (int b = 0; b < used; b++)
            if (k.blocks[b] >= (uint32_t)kv.blocks) return fail(FG_E_ARG, "block id beyond the cache");
        const int row_base = P.t;
        for (int i = 0; i < k.n; i++) {
            if (k.tokens) {
                if (k.tokens[i] >= (uint32_t)c.vocab) return fail(FG_E_ARG, "token outside the vocabulary");
                P.tokens.push_back(k.tokens[i]);
            } else {
                P.tokens.push_back(0);
            }
        }
        if (P.flash) {
            const int boff = (int)P.btab.size();
            for (int b = 0; b < used; b++) P.btab.push_back((int32_t)k.blocks[b]);
            for (int r0 = 0; r0 < k.n; r0 += rf) {
                // an item whose rows see more than kFlashBlocks blocks of 64 positions
                // is split into parts of even length, each writing its own partials
                // (the merge combines them as spans)
                const int nr = std::min(rf, k.n - r0), L = k.pos + r0 + nr, nb = (L + fblk - 1) / fblk;
                const int parts = flash_parts(L), per = (nb + parts - 1) / parts;
                const int base = P.W;
                for (int sp = 0; sp < parts; sp++) {
                    const int p0 = sp * per * fblk, p1 = std::min(L, (sp + 1) * per * fblk);
                    const int32_t rec[16] = {row_base + r0, nr,   row_base, k.pos, p0, p1, boff, base + sp,
                                             base + parts + sp, 0, 0, 0, 0, 0, 0, 0};
                    P.wrec.insert(P.wrec.end(), rec, rec + 16);
                }
                for (int i = 0; i < nr; i++) {
                    const int half = i >= rf / 2 ? 1 : 0;
                    const int32_t mr[4] = {(i - half * (rf / 2)) * group, base + half * parts, parts, 0};
                    P.mrec.insert(P.mrec.end(), mr, mr + 4);
                }
                P.W += 2 * parts;
            }
        } else
        for (int r0 = 0; r0 < k.n; r0 += rg) {
            const int nr = std::min(rg, k.n - r0);
            const int wi0 = P.W;
            const int L = k.pos + r0 + nr;  // positions the group's last row sees
            const int ns = (L + span - 1) / span;
            for (int sp = 0; sp < ns; sp++) {
                const int p0 = sp * span, p1 = std::min(p0 + span, L);
                const int32_t rec[8] = {row_base + r0, nr, row_base, k.pos, p0, p1, 0, 0};
                P.wrec.insert(P.wrec.end(), rec, rec + 8);
                for (int j = 0; j < 8; j++)
                    P.wrec.push_back(p0 + bs * j < p1 ? (int32_t)k.blocks[p0 / bs + j] : 0);
                P.W++;
            }
            for (int i = 0; i < nr; i++) {
                const int32_t rec[4] = {i * group, wi0, ns, 0};
                P.mrec.insert(P.mrec.end(), rec, rec + 4);
            }
        }
        if (k.logits == FG_LOGITS_LAST) P.sel.push_back(row_base + k.n - 1);
        if (k.logits == FG_LOGITS_ALL)
            for (int i = 0; i < k.n; i++) P.sel.push_back(row_base + i);
        P.t += k.n;
    }
    P.S = (int)P.sel.size();
    // launch capacity (unused slots exit at once): a multiple of 16 work items,
    // or of a power of two near W/16 for large launches, so that a step graph
    // keyed on it outlives the context growth of many sequences (at 32 of them
    // a launch gains an item every two or four steps, and each new capacity
    // captures the step's graphs again: cfg3 at 32 sequences, 48 steps,
    // 2627-2649 -> 2716-2723 tok/s with this rounding)
    int wstep = 16;
    while (wstep * 16 <= P.W) wstep *= 2;
    P.Wc = std::max(16, (P.W + wstep - 1) / wstep * wstep);
    P.wrec.resize((size_t)P.Wc * 16, 0);
    size_t o = 0;
    auto place = [&](size_t n) {
        size_t r = o;
        o += (n + 63) / 64 * 64;
        return r;
    };
    P.o_wrec = place(P.wrec.size());
    P.o_mrec = place(P.mrec.size());
    P.o_sel = place(P.S);
    P.o_tok = place(P.t);
    P.o_btab = place(P.btab.size());
    P.words = o;
    return 0;
}

static void pack_plan(const Plan& P, int32_t* h) {
    auto cp = [&](size_t off, const std::vector<int32_t>& v) {
        if (!v.empty()) memcpy(h + off, v.data(), v.size() * 4);
    };
    cp(P.o_wrec, P.wrec);
    cp(P.o_mrec, P.mrec);
    cp(P.o_sel, P.sel);
    if (!P.tokens.empty()) memcpy(h + P.o_tok, P.tokens.data(), P.tokens.size() * 4);
    cp(P.o_btab, P.btab);
}

// Workspace of one forward pass over a plan.
struct Work {
    float *x, *ss, *qkv, *apart, *logits;
    float* x2;  // the fused MLP's layer input x + acc (formed by the next q/k/v, read by its o projection)
    float* kpart;  // GEMM split-K partial tiles (steps of more than kGemvRows rows)
    size_t kpart_cap;
    float* gpart;  // GEMV split-K partial tiles (decode steps of one pass)
    long long* acc;   // fused layers' accumulators (steps of one pass), [copies][4][hidden]:
    long long* acc2;  // A (acc) the MLP's output, B (acc2) the output projection's
    void* pa[2];   // activation pieces, ping-pong: each kernel reads one and writes the other
    float* pxs[2];
    float2* best;
    uint32_t* am;
    int passes, lm_passes;
};

static int kind_of(const DMat& m) { return m.kind; }

// Steps with more rows than this run their projections as GEMMs (k_gemm on
// MM pieces); up to this many rows, as GEMVs on BF16/INT8 pieces. A model
// narrower than kGemmMinHidden keeps the GEMV below kNarrowGemmRows rows:
// its small projections finish sooner on the GEMV (measured on the 135M
// shape, one forward: 16 rows 1.18 against 1.39 ms, 128 rows 1.71 against
// 1.98), while from 256 rows the GEMM wins (2.07 against 2.20 ms; a
// 1024-token prompt 4.51 against 6.11). The lm_head, a large product either
// way, switches at kGemvRows for every model. At exactly 16 rows a
// 2048-wide bf16 model is faster on the GEMM (measured: cfg4's 1B draft
// rounds of 16 sequences, 7.15 against 6.85 ms per step), so 16-row steps
// take the GEMM.
static constexpr int kGemvRows = 15;
static constexpr int kGemvSplitGroups = 1024;  // output groups a split-K GEMV may have (counters per context)
static constexpr int kGemmMinHidden = 1024;
static constexpr int kNarrowGemmRows = 256;
// Floats of the GEMM split-K partial tiles ([split][row][column]) in a plan's
// workspace: 32 MiB. At 4 MiB the split of the 80-row products into 4096
// outputs stopped at two (80 x 4096 x 4 floats do not fit); four splits take
// the 4096 x 14336 int4 down from 56.4 to 38.7 us and the 4096 x 4096 o from
// 24.9 to 19.7 us (single-matrix products, event-timed).
static constexpr size_t kKpartFloats = (size_t)1 << 23;
static bool step_gemm(int t, int H) { return t > kGemvRows && (H >= kGemmMinHidden || t >= kNarrowGemmRows); }

// n-tiles per workgroup of a bf16 projection with fewer than 256 tiles: one, so
// that it spreads over twice the CUs (a CU streams only about 22 GB/s), unless
// it finishes int8 pieces, whose per-block scale needs a whole 32-column
// k-block. Quantized projections keep two (their 16-wave two-tile variant
// streams faster per CU).
static int narrow_nt(const DMat& w, bool int8_pieces) {
    return w.kind == BF16 && w.n_tiles < 256 && !int8_pieces ? 1 : 2;
}

// Split K of a residual projection (o, down) in a decode step: a quantized
// projection whose output groups (two n-tiles, the 32 columns of an int8
// k-block of its consumer) cannot fill the CUs splits K among up to
// kGemvSplitMax workgroups per group, to at most 256 workgroups, while each
// share keeps at least 16 chunks of four k-blocks. A CU streams only about
// 20 GB/s of weights, so 64 busy CUs cap a projection near 1.3 TB/s; the
// last workgroup of a group to finish sums the partials (k_gemv), which
// costs about 1.5 us. Measured on the 1.7B shape (graph, cold weights):
// down (64 groups, 64 chunks) 10.2 us unsplit, 7.1 us in four; o (16
// chunks) 5.3 us unsplit, 5.6 to 6.1 us split, so it stays whole.
static constexpr int kGemvSplitMax = 8;
static int gemv_split(const DMat& d, int nt, int passes, bool mm) {
    if (mm || passes != 1 || d.kind == BF16) return 1;
    const int groups = d.n_tiles / nt, kc = d.kb / 4;
    if (groups > kGemvSplitGroups) return 1;
    int s = 1;
    while (s < kGemvSplitMax && groups * s * 2 <= 256 && kc >= s * 2 * 16) s *= 2;
    return s;
}
static int qkv_dim(const fg_config& c) { return (c.heads + 2 * c.kv_heads) * c.head_dim; }

// Whether the output projection merges the attention spans itself (one launch
// less per layer): a bf16 projection of one pass of rows over at most 1024
// inputs, when the partials each workgroup re-reads stay small (every
// workgroup merges every head; the 135M draft reads about 40 KB per row).
static bool merge_in_o(const fg_config& c, const Plan& P, const DMat& wo, bool mm) {
    if (mm || wo.kind != BF16 || P.t > 4 || wo.kb > 32 || c.heads * c.head_dim > 1024) return false;
    const size_t part_bytes = (size_t)P.t * c.heads * P.Wc * (c.head_dim + 4) * 4;  // bound: every row sees Wc spans
    return part_bytes <= 160 * 1024;
}

// Whether the layers of a forward run fused (all but the last): the output
// projection split by head (k_o_heads: each workgroup merges one head's
// attention spans) adds into a fixed-point accumulator, and gate/up, SiLU and
// down run as one launch (EPI_MLP: each workgroup multiplies its channels'
// activations by their columns of the down projection) whose prologue forms x +
// that accumulator and its norm (AX) and whose output goes into a second
// accumulator, which the next layer's q/k/v reads the same way. Four launches
// per layer instead of five, and no workgroup reads every head's partials.
// For bf16 layers of one pass of at most 4 rows on the GEMV path, at most 1024
// wide, head dim 64 or 128, without hidden-state or calibration taps (x is
// complete only inside the next layer's first launch): the 135M draft's rounds.
static bool mlp_fuse(const fg_ctx* ctx, const fg_model* m, const Plan& P, bool mm) {
    const fg_config& c = m->cfg;
    if (!ctx->mlp_fuse || mm || P.t < 1 || P.t > 4 || c.hidden > 1024 || c.hidden % 8 || m->layers.size() < 2 ||
        (c.head_dim != 64 && c.head_dim != 128))
        return false;
    for (const DLayer& l : m->layers) {
        if (l.wqkv.kind != BF16 || l.wo.kind != BF16 || l.w_gate_up.kind != BF16 || l.w_down.kind != BF16 ||
            l.w_gate_up.il != 16 || l.w_down.rows != c.hidden || l.w_down.cols != c.intermediate ||
            l.wo.rows != c.hidden)
            return false;
        // the down columns of a gate/up group: 32 items per n-tile, at most four per thread
        const int wv = std::max(1, std::min(8, l.w_gate_up.kb / 4));
        if ((l.w_down.rows / 16) * 32 > 4 * 64 * wv || l.wqkv.kb > 32) return false;
    }
    return true;
}

static size_t layout_work(const fg_model* m, const Plan& P, Work& w, void* base) {
    const fg_config& c = m->cfg;
    const int t = P.t, H = c.hidden, S = std::max(P.S, 1);
    Carver cv(base);
    int kb_max = m->lm_head.kb;
    for (const DLayer& l : m->layers)
        for (const DMat* d : {&l.wqkv, &l.wo, &l.w_gate_up, &l.w_down}) kb_max = std::max(kb_max, d->kb);
    w.passes = (t + 3) / 4;
    w.lm_passes = (S + 3) / 4;
    const int passes = std::max(w.passes, w.lm_passes);
    w.x = cv.take<float>((size_t)t * H);
    w.ss = cv.take<float>((size_t)(H / 16) * t);
    for (int i = 0; i < 2; i++) {
        w.pa[i] = cv.take<uint8_t>((size_t)kb_max * passes * 64 * 16);
        w.pxs[i] = cv.take<float>((size_t)kb_max * passes * 4);
    }
    w.qkv = cv.take<float>((size_t)t * qkv_dim(c));
    w.apart = cv.take<float>((size_t)std::max(P.Wc, 1) * c.kv_heads * attn_qmax(c.head_dim) * (c.head_dim + 4));
    w.logits = cv.take<float>((size_t)S * c.vocab);
    w.best = cv.take<float2>((size_t)(c.vocab / 32) * S);
    w.am = cv.take<uint32_t>(S);
    // the split rule keeps splits x rows x N within 64 x 256 x 64 floats
    w.kpart_cap = step_gemm(t, H) || S > kGemvRows ? kKpartFloats : 0;
    w.kpart = w.kpart_cap ? cv.take<float>(w.kpart_cap) : nullptr;
    // GEMV split K: [group][split][16 rows][group columns] over the hidden columns
    w.gpart = w.passes == 1 ? cv.take<float>((size_t)kGemvSplitMax * 16 * H) : nullptr;
    w.acc = w.passes == 1 ? cv.take<long long>((size_t)kAccCopies * 4 * H) : nullptr;
    w.acc2 = w.passes == 1 ? cv.take<long long>((size_t)kAccCopiesB * 4 * H) : nullptr;
    w.x2 = w.passes == 1 ? cv.take<float>((size_t)4 * H) : nullptr;
    return cv.off + 256;
}

static Pieces pieces(const Work& w, int i, int kb, int passes) {
    Pieces p;
    p.a = w.pa[i];
    p.xs = w.pxs[i];
    p.kb = kb;
    p.passes = passes;
    return p;
}

static GemvArgs gemv_args(const DMat& d, const Pieces& in, int m, const Work& w) {
    GemvArgs a;
    a.kpart = w.kpart;
    a.kpart_cap = w.kpart_cap;
    a.W = (const uint8_t*)d.w;
    a.S = d.s;
    a.kind = d.kind;
    a.N = d.rows;
    a.KB = d.kb;
    a.XA = (const uint8_t*)in.a;
    a.XS = in.xs;
    a.m = m;
    a.p_total = in.passes;
    return a;
}

// Runs one forward pass. `meta` is the device copy of the plan's packed
// metadata; tokens come from tok_dev with stride tok_stride. Outputs:
// logits rows to logits_dev (may be null), argmax to am_out (or the
// workspace), optional aux copy of the argmax (for chaining draft rounds),
// and the hidden-state taps to host.
static int run_forward(fg_ctx* ctx, const fg_model* m, fg_kv* kv, const Plan& P, const int32_t* meta,
                       const uint32_t* tok_dev, int tok_stride, Work& w, float* logits_dev, uint32_t* am_out,
                       uint32_t* aux, int aux_stride, int aux_off, float* hidden_host,
                       float* cap = nullptr) {
    const fg_config& c = m->cfg;
    hipStream_t st = ctx->stream;
    const int t = P.t, H = c.hidden, hd = c.head_dim, nh = c.heads, nkv = c.kv_heads;
    const int L = (int)m->layers.size();
    if (t == 0) return 0;
    const int passes = w.passes;
    int cur = 0;  // pieces buffer the next GEMV reads
    // 16 rows or more (of a wide enough model): every projection runs as a GEMM on MM pieces
    const bool mm = step_gemm(t, H);
    auto ck = [&](const DMat& d) { return mm ? (int)MM : kind_of(d); };

    if (L > 0) {
        Pieces p0 = pieces(w, cur, m->layers[0].wqkv.kb, passes);
        launch_embed(st, tok_dev, tok_stride, m->embed, t, H, m->layers[0].attn_norm, w.x, w.ss,
                     ck(m->layers[0].wqkv), p0);
    } else {
        Pieces p0 = pieces(w, cur, m->lm_head.kb, passes);
        launch_embed(st, tok_dev, tok_stride, m->embed, t, H, nullptr, w.x, w.ss, BF16, p0);
    }
    if (hidden_host) HIPCHK(hipMemcpyAsync(hidden_host, w.x, (size_t)t * H * 4, hipMemcpyDeviceToHost, st));

    AttnArgs aa{};
    aa.qkv = w.qkv;
    aa.ld = qkv_dim(c);
    aa.cos_t = m->cos_t;
    aa.sin_t = m->sin_t;
    aa.wrec = meta + P.o_wrec;
    aa.mrec = meta + P.o_mrec;
    aa.flash = P.flash ? 1 : 0;
    aa.btab = meta + P.o_btab;
    aa.part = w.apart;
    aa.n_wi = P.Wc;
    aa.maxq = P.maxq;
    aa.ns = P.ns;
    aa.nh = nh;
    aa.nkv = nkv;
    aa.hd = hd;
    aa.bs = kv->block_size;
    aa.scale = 1.0f / sqrtf((float)hd);

    // When every row's logits are selected, in order (draft rounds, verify
    // steps), the last layer's down projection writes the lm_head's pieces of
    // norm * x itself, the same product k_pieces forms, so that launch is saved.
    const bool lm_mm = P.S > kGemvRows;
    bool sel_all = P.S == t;
    for (int i = 0; sel_all && i < P.S; i++) sel_all = P.sel[i] == i;
    int ss_cols = 32;  // columns per sum-of-squares partial in w.ss (the embedding writes one per k-block)
    // Fused layers (all but the last; mlp_fuse): the residual rows alternate
    // between xb[0] and xb[1] (a stage that forms x + acc reads one and writes the
    // other); accumulator B (w.acc2) takes the output projection, A (w.acc) the
    // MLP. Each is cleared by the launch before the one that adds into it: B by
    // the q/k/v, A by the output projection.
    const bool fuse = w.acc && !hidden_host && !cap && mlp_fuse(ctx, m, P, mm);
    float* xb[2] = {w.x, w.x2};
    int xc = 0;
    const int acc_n = kAccCopies * 4 * H;
    // calibration capture: per layer the four projection inputs [t][H], [t][qd], [t][H], [t][inter]
    const int qd = nh * hd;
    const size_t cap_layer = (size_t)t * (2 * H + qd + c.intermediate);
    for (int li = 0; li < L; li++) {
        const DLayer& l = m->layers[li];
        float* capl = cap ? cap + li * cap_layer : nullptr;
        if (cap) launch_cap_norm(st, w.x, t, H, l.attn_norm, c.rms_eps, capl, H);
        // q/k/v of the normed rows: rinv from the sum-of-squares partials
        GemvArgs g = gemv_args(l.wqkv, pieces(w, cur, l.wqkv.kb, passes), t, w);
        g.out = w.qkv;
        g.ldo = qkv_dim(c);
        g.bias = l.bqkv;
        g.ss_in = w.ss;
        g.ss_tiles = (H + ss_cols - 1) / ss_cols;
        g.ss_m = t;
        g.hidden = H;
        g.eps = c.rms_eps;
        g.nt = narrow_nt(l.wqkv, false);
        g.mm = mm;
        const bool fuse_l = fuse && li + 1 < L;
        if (fuse && li > 0) {
            // the previous layer's MLP left its output in accumulator A
            g.ax = true;
            g.acc = w.acc;
            g.acc_ld = H;
            g.g_in = l.attn_norm;
            g.x = xb[xc];
            g.x_alt = xb[xc ^ 1];
            g.ldx = H;
            xc ^= 1;
        }
        if (fuse_l) {
            g.zero = w.acc2;
            g.zero_n = kAccCopiesB * 4 * H;
        }
        gemv(ctx, EPI_QKV, l.wqkv, g);
        // attention (RoPE, cache write) and the merge into wo's pieces
        aa.kc = kv->k + li * kv->layer_floats();
        aa.vc = kv->v + li * kv->layer_floats();
        Pieces po = pieces(w, cur ^ 1, l.wo.kb, passes);
        const bool am = fuse_l || (ctx->merge_in_o && merge_in_o(c, P, l.wo, mm));
        aa.stamp = next_stamp(ctx, "attention");
        if (!am && aa.stamp >= 0) next_stamp(ctx, "merge");  // the merge launch takes the next slot
        if (launch_attention(st, aa, t, am ? -1 : ck(l.wo), po))
            return fail(FG_E_SHAPE, "no attention kernel for head_dim " + std::to_string(hd));
        if (cap && launch_cap_merge(st, aa, t, capl + (size_t)t * H, qd))
            return fail(FG_E_SHAPE, "no attention kernel for head_dim " + std::to_string(hd));
        cur ^= 1;
        if (fuse_l) {
            // the output projection by head, into accumulator B (A cleared for the MLP)
            g = gemv_args(l.wo, pieces(w, cur, l.wo.kb, passes), t, w);
            g.apart = w.apart;
            g.amrec = aa.mrec;
            g.anh = nh;
            g.ankv = nkv;
            g.ahd = hd;
            g.aqm = attn_qmax(hd);
            g.acc_out = w.acc2;
            g.acc_ld = H;
            g.zero = w.acc;
            g.zero_n = acc_n;
            g.stamp = next_stamp(ctx, "o by head bf16 " + std::to_string(l.wo.rows) + "x" + std::to_string(l.wo.cols));
            if (launch_o_heads(st, l.wo, g))
                return fail(FG_E_SHAPE, "no split output projection for head_dim " + std::to_string(hd));
            cur ^= 1;
            // gate/up, SiLU and down in one launch: input x + B, output into A
            g = gemv_args(l.w_gate_up, pieces(w, cur, l.w_gate_up.kb, passes), t, w);
            g.ax = true;
            g.acc = w.acc2;
            g.acc_ld = H;
            g.g_in = l.mlp_norm;
            g.x = xb[xc];
            g.x_alt = xb[xc ^ 1];
            g.ldx = H;
            xc ^= 1;
            g.hidden = H;
            g.eps = c.rms_eps;
            g.il = l.w_gate_up.il;
            g.acc_out = w.acc;
            g.W2 = (const uint8_t*)l.w_down.w;
            g.N2 = l.w_down.rows;
            g.KB2 = l.w_down.kb;
            gemv(ctx, EPI_MLP, l.w_gate_up, g);
            cur ^= 1;
            cur ^= 1;
            continue;
        }
        // o projection + residual; pieces of mlp_norm * x for gate/up
        g = gemv_args(l.wo, pieces(w, cur, l.wo.kb, passes), t, w);
        if (am) {
            g.am = true;
            g.apart = w.apart;
            g.amrec = aa.mrec;
            g.anh = nh;
            g.ankv = nkv;
            g.ahd = hd;
            g.aqm = attn_qmax(hd);
        }
        g.x = w.x;
        if (xb[xc] != w.x) g.x_alt = xb[xc];  // the layer input x + acc, formed by this layer's q/k/v
        xc = 0;
        g.ldx = H;
        g.ss_out = w.ss;
        g.ss_m = t;
        g.g_next = l.mlp_norm;
        g.pa = w.pa[cur ^ 1];
        g.pxs = w.pxs[cur ^ 1];
        g.pa_kind = ck(l.w_gate_up);
        g.pa_passes = passes;
        g.pa_kb = l.w_gate_up.kb;
        g.nt = narrow_nt(l.wo, g.pa_kind == INT8 || g.pa_kind == INT4);
        g.mm = mm;
        if (!am) {
            g.gsplit = gemv_split(l.wo, g.nt, passes, mm);
            g.gpart = w.gpart;
            g.gcnt = ctx->gcnt;
        }
        ss_cols = mm ? 64 : 16 * g.nt;
        gemv(ctx, EPI_RESID, l.wo, g);
        if (cap) launch_cap_norm(st, w.x, t, H, l.mlp_norm, c.rms_eps, capl + (size_t)t * (H + qd), H);
        cur ^= 1;
        // gate/up with SiLU; pieces of the activation for down
        g = gemv_args(l.w_gate_up, pieces(w, cur, l.w_gate_up.kb, passes), t, w);
        g.ss_in = w.ss;
        g.ss_tiles = (H + ss_cols - 1) / ss_cols;
        g.ss_m = t;
        g.hidden = H;
        g.eps = c.rms_eps;
        g.pa = w.pa[cur ^ 1];
        g.pxs = w.pxs[cur ^ 1];
        g.pa_kind = ck(l.w_down);
        g.pa_passes = passes;
        g.pa_kb = l.w_down.kb;
        g.il = l.w_gate_up.il;
        g.mm = mm;
        if (cap) {
            g.cap = capl + (size_t)t * (2 * H + qd);
            g.ldcap = c.intermediate;
        }
        gemv(ctx, EPI_SILU, l.w_gate_up, g);
        cur ^= 1;
        // down projection + residual; pieces of the next layer's attn_norm * x
        g = gemv_args(l.w_down, pieces(w, cur, l.w_down.kb, passes), t, w);
        g.x = w.x;
        g.ldx = H;
        g.ss_out = w.ss;
        g.ss_m = t;
        if (li + 1 < L) {
            const DLayer& nl = m->layers[li + 1];
            g.g_next = nl.attn_norm;
            g.pa = w.pa[cur ^ 1];
            g.pxs = w.pxs[cur ^ 1];
            g.pa_kind = ck(nl.wqkv);
            g.pa_passes = passes;
            g.pa_kb = nl.wqkv.kb;
        } else if (sel_all) {
            g.g_next = m->norm;
            g.pa = w.pa[cur ^ 1];
            g.pxs = w.pxs[cur ^ 1];
            g.pa_kind = lm_mm ? (int)MM : kind_of(m->lm_head);
            g.pa_passes = w.lm_passes;
            g.pa_kb = m->lm_head.kb;
        }
        g.nt = narrow_nt(l.w_down, g.pa && (g.pa_kind == INT8 || g.pa_kind == INT4));
        g.mm = mm;
        g.gsplit = gemv_split(l.w_down, g.nt, passes, mm);
        g.gpart = w.gpart;
        g.gcnt = ctx->gcnt;
        ss_cols = mm ? 64 : 16 * g.nt;
        gemv(ctx, EPI_RESID, l.w_down, g);
        cur ^= 1;
        if (hidden_host)
            HIPCHK(hipMemcpyAsync(hidden_host + (li + 1) * (size_t)t * H, w.x, (size_t)t * H * 4,
                                  hipMemcpyDeviceToHost, st));
    }
    HIPCHK(hipGetLastError());
    if (P.S == 0) return 0;
    // final norm of the selected rows (weight now, 1/rms in the epilogue), lm_head, argmax
    const int32_t* sel = meta + P.o_sel;
    Pieces pl = pieces(w, cur, m->lm_head.kb, w.lm_passes);
    if (!(sel_all && L > 0))
        launch_pieces(st, lm_mm ? (int)MM : kind_of(m->lm_head), w.x, H, P.S, H, m->norm, sel, pl);
    GemvArgs g = gemv_args(m->lm_head, pl, P.S, w);
    g.mm = lm_mm;
    g.ss_in = w.ss;
    g.ss_tiles = (H + ss_cols - 1) / ss_cols;
    g.ss_m = t;
    g.hidden = H;
    g.eps = c.rms_eps;
    g.rows_src = sel;
    g.logits = logits_dev;
    g.best = w.best;
    gemv(ctx, EPI_ARGMAX, m->lm_head, g);
    launch_argmax_final(st, w.best, c.vocab / 32, P.S, am_out ? am_out : w.am, aux, aux_stride, aux_off);
    HIPCHK(hipGetLastError());
    return 0;
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

const char* fg_last_error(void) { return g_err.c_str(); }

// The device scratch of fg_matmul_device_noalloc: the activation pieces and
// their block scales of one product. Each GPU holds its own copy for the
// life of the process; host code uses only the address hipGetSymbolAddress
// gives for the current device (kept per device below), never the array's
// name. Calls that overlap on one GPU share it and race.
static constexpr size_t kScratchBytes = (size_t)2 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_at[kMaxDevices];

// This device's scratch address (the device is current), looked up once.
static uint8_t* scratch_address(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_at[device]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        g_scratch_at[device] = (uint8_t*)ptr;
    }
    return g_scratch_at[device];
}

int fg_ctx_create(int device, fg_ctx** out) {
    if (!out) return fail(FG_E_ARG, "null out");
    int n = 0;
    HIPCHK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(FG_E_ARG, "no such device");
    HIPCHK(hipSetDevice(device));
    fg_ctx* c = new fg_ctx();
    c->device = device;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return fail(FG_E_DEVICE, "stream creation failed");
    }
    for (auto& e : c->ev) HIPCHK(hipEventCreate(&e));
    if (hipMalloc((void**)&c->gcnt, kGemvSplitGroups * 32 * sizeof(unsigned)) != hipSuccess) {
        fg_ctx_destroy(c);
        return fail(FG_E_NOMEM, "counter allocation failed");
    }
    HIPCHK(hipMemset(c->gcnt, 0, kGemvSplitGroups * 32 * sizeof(unsigned)));
    c->scratch = scratch_address(device);
    const char* ng = std::getenv("FERRO_NO_GRAPH");
    c->graphs = !(ng && ng[0] == '1');
    const char* sm = std::getenv("FERRO_SEPARATE_MERGE");
    c->merge_in_o = !(sm && sm[0] == '1');
    const char* nf = std::getenv("FERRO_NO_MLP_FUSE");
    c->mlp_fuse = !(nf && nf[0] == '1');
    *out = c;
    return 0;
}

void fg_ctx_destroy(fg_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    drop_graphs(c);
    if (c->ws) (void)hipFree(c->ws);
    if (c->sbuf) (void)hipFree(c->sbuf);
    if (c->dmeta) (void)hipFree(c->dmeta);
    if (c->hmeta) (void)hipHostFree(c->hmeta);
    if (c->gcnt) (void)hipFree(c->gcnt);
    for (auto& e : c->ev)
        if (e) (void)hipEventDestroy(e);
    for (auto& e : c->pev) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(c->stream);
    delete c;
}

int fg_ctx_sync(fg_ctx* c) {
    if (!c) return fail(FG_E_ARG, "null ctx");
    HIPCHK(hipStreamSynchronize(c->stream));
    return 0;
}

// Head dims with an attention kernel instance (launch_attention).
static bool head_dim_supported(int hd) { return hd == 16 || hd == 32 || hd == 64 || hd == 128; }

int fg_config_check(const fg_config* cfg) {
    if (!cfg) return fail(FG_E_ARG, "null config");
    const fg_config& c = *cfg;
    if (c.heads <= 0 || c.kv_heads <= 0 || c.heads % c.kv_heads || c.head_dim % 16 || c.hidden % 16 ||
        c.vocab <= 0 || c.layers < 0 || c.max_position <= 0)
        return fail(FG_E_SHAPE, "unsupported model shape");  // src/config.rs:70-74
    if (!head_dim_supported(c.head_dim))
        return fail(FG_E_SHAPE, "head_dim " + std::to_string(c.head_dim) +
                                    " has no device attention kernel (supported: 16, 32, 64, 128)");
    if (c.heads / c.kv_heads > attn_qmax(c.head_dim)) return fail(FG_E_SHAPE, "GQA group too large");
    if (c.hidden % 32 || c.intermediate % 32 || (c.heads * c.head_dim) % 32 || c.vocab % 32)
        return fail(FG_E_SHAPE, "hidden, intermediate, q and vocab sizes must be multiples of 32");
    return 0;
}

int fg_model_upload(fg_ctx* ctx, const fg_config* cfg, const fg_layer* layers, const uint16_t* embed,
                    const float* norm, const uint16_t* lm_head, fg_model** out) {
    if (!ctx || !cfg || (!layers && cfg->layers > 0) || !embed || !norm || !out) return fail(FG_E_ARG, "null argument");
    const fg_config& c = *cfg;
    if (int rc = fg_config_check(cfg)) return rc;
    HIPCHK(hipSetDevice(ctx->device));
    fg_model* m = new fg_model();
    m->cfg = c;
    const int H = c.hidden, qkv = (c.heads + 2 * c.kv_heads) * c.head_dim;
    auto bad = [&](int rc) {
        fg_model_destroy(m);
        return rc;
    };
    m->layers.resize(c.layers);
    int64_t ref = 0;
    for (int i = 0; i < c.layers; i++) {
        const fg_layer& s = layers[i];
        DLayer& d = m->layers[i];
        if (!s.attn_norm || !s.mlp_norm || (c.qkv_bias && !s.bqkv)) return bad(fail(FG_E_ARG, "layer missing a vector"));
        if (s.wqkv.rows != qkv || s.wqkv.cols != H || s.wo.rows != H || s.wo.cols != c.heads * c.head_dim ||
            s.w_gate_up.rows != 2 * c.intermediate || s.w_gate_up.cols != H || s.w_down.rows != H ||
            s.w_down.cols != c.intermediate)
            return bad(fail(FG_E_SHAPE, "weight shapes do not match the config"));  // src/model.rs:243-261
        int rc;
        if ((rc = upload_vec(s.attn_norm, H, &d.attn_norm, m->allocs))) return bad(rc);
        if ((rc = upload_vec(s.mlp_norm, H, &d.mlp_norm, m->allocs))) return bad(rc);
        if (c.qkv_bias && (rc = upload_vec(s.bqkv, qkv, &d.bqkv, m->allocs))) return bad(rc);
        if ((rc = upload_mat(s.wqkv, d.wqkv, &m->allocs))) return bad(rc);
        if ((rc = upload_mat(s.wo, d.wo, &m->allocs))) return bad(rc);
        // bf16 gate/up feeding a bf16 down: 16-row blocks, so a 32-row output group
        // finishes 16 channels (bf16 pieces carry no per-block scale)
        const int il = s.w_gate_up.format == FG_BF16 && s.w_down.format == FG_BF16 ? 16 : 32;
        if ((rc = upload_mat(s.w_gate_up, d.w_gate_up, &m->allocs, c.intermediate, il))) return bad(rc);
        if ((rc = upload_mat(s.w_down, d.w_down, &m->allocs))) return bad(rc);
        ref += d.wqkv.ref_bytes + d.wo.ref_bytes + d.w_gate_up.ref_bytes + d.w_down.ref_bytes;
    }
    int rc;
    if ((rc = upload_vec(embed, (size_t)c.vocab * H, &m->embed, m->allocs))) return bad(rc);
    fg_matrix lm{FG_BF16, c.vocab, H, 0, (lm_head && !c.tie_embeddings) ? lm_head : embed, nullptr, nullptr};
    if ((rc = upload_mat(lm, m->lm_head, &m->allocs))) return bad(rc);
    ref += (int64_t)c.vocab * H * 2 * ((lm_head && !c.tie_embeddings) ? 2 : 1);
    if ((rc = upload_vec(norm, H, &m->norm, m->allocs))) return bad(rc);
    m->max_pos = c.max_position;
    std::vector<float> cs, sn;
    rope_tables(c, m->max_pos, cs, sn);
    if ((rc = upload_vec(cs.data(), cs.size(), &m->cos_t, m->allocs))) return bad(rc);
    if ((rc = upload_vec(sn.data(), sn.size(), &m->sin_t, m->allocs))) return bad(rc);
    m->ref_bytes = ref;
    *out = m;
    return 0;
}

int fg_model_truncated(fg_ctx* ctx, const fg_model* base, int32_t layers, fg_model** out) {
    if (!ctx || !base || !out || layers < 0) return fail(FG_E_ARG, "bad argument");
    fg_model* m = new fg_model();
    m->cfg = base->cfg;
    m->layers.assign(base->layers.begin(), base->layers.begin() + std::min<size_t>(layers, base->layers.size()));
    m->cfg.layers = (int)m->layers.size();
    m->embed = base->embed;
    m->lm_head = base->lm_head;
    m->norm = base->norm;
    m->cos_t = base->cos_t;
    m->sin_t = base->sin_t;
    m->max_pos = base->max_pos;
    m->owns = false;
    int64_t ref = (int64_t)m->cfg.vocab * m->cfg.hidden * 2;
    for (const DLayer& d : m->layers) ref += d.wqkv.ref_bytes + d.wo.ref_bytes + d.w_gate_up.ref_bytes + d.w_down.ref_bytes;
    m->ref_bytes = ref;
    *out = m;
    return 0;
}

void fg_model_destroy(fg_model* m) {
    if (!m) return;
    if (m->owns)
        for (void* p : m->allocs) (void)hipFree(p);
    delete m;
}

int64_t fg_model_weight_bytes(const fg_model* m) { return m ? m->ref_bytes : 0; }

int fg_kv_create(fg_ctx* ctx, int32_t layers, int32_t kv_heads, int32_t head_dim, int32_t block_size, int32_t blocks,
                 fg_kv** out) {
    if (!ctx || !out || layers <= 0 || kv_heads <= 0 || head_dim <= 0 || block_size != 16 || blocks <= 0)
        return fail(FG_E_ARG, "bad cache shape (block_size must be 16)");
    if (!head_dim_supported(head_dim))
        return fail(FG_E_SHAPE, "head_dim " + std::to_string(head_dim) +
                                    " has no device attention kernel (supported: 16, 32, 64, 128)");
    HIPCHK(hipSetDevice(ctx->device));
    fg_kv* kv = new fg_kv();
    kv->layers = layers;
    kv->kv_heads = kv_heads;
    kv->head_dim = head_dim;
    kv->block_size = block_size;
    kv->blocks = blocks;
    const size_t bytes = kv->layer_floats() * layers * 4;
    if (hipMalloc((void**)&kv->k, bytes) != hipSuccess || hipMalloc((void**)&kv->v, bytes) != hipSuccess) {
        fg_kv_destroy(kv);
        return fail(FG_E_NOMEM, "cache allocation failed");
    }
    HIPCHK(hipMemset(kv->k, 0, bytes));
    HIPCHK(hipMemset(kv->v, 0, bytes));
    *out = kv;
    return 0;
}

void fg_kv_destroy(fg_kv* kv) {
    if (!kv) return;
    if (kv->k) (void)hipFree(kv->k);
    if (kv->v) (void)hipFree(kv->v);
    delete kv;
}

int fg_kv_read(fg_ctx* ctx, const fg_kv* kv, int32_t layer, float* k_out, float* v_out) {
    if (!ctx || !kv || layer < 0 || layer >= kv->layers || !k_out || !v_out) return fail(FG_E_ARG, "bad argument");
    const size_t n = kv->layer_floats();
    HIPCHK(hipMemcpyAsync(k_out, kv->k + layer * n, n * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(hipMemcpyAsync(v_out, kv->v + layer * n, n * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}

int fg_kv_write(fg_ctx* ctx, fg_kv* kv, int32_t layer, const float* k, const float* v) {
    if (!ctx || !kv || layer < 0 || layer >= kv->layers || !k || !v) return fail(FG_E_ARG, "bad argument");
    const size_t n = kv->layer_floats();
    HIPCHK(hipMemcpyAsync(kv->k + layer * n, k, n * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(hipMemcpyAsync(kv->v + layer * n, v, n * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}

static int check_model_kv(const fg_model* m, const fg_kv* kv) {
    if (kv->layers < (int)m->layers.size() || kv->kv_heads != m->cfg.kv_heads || kv->head_dim != m->cfg.head_dim)
        return fail(FG_E_SHAPE, "cache does not match the model");
    return 0;
}

int fg_forward(fg_ctx* ctx, const fg_model* m, fg_kv* kv, const fg_chunk* chunks, int32_t n_chunks, float* logits_out,
               uint32_t* argmax_out, int32_t* rows_out, float* hidden_out) {
    if (!ctx || !m || !kv || (!chunks && n_chunks > 0) || n_chunks < 0) return fail(FG_E_ARG, "null argument");
    int rc = check_model_kv(m, kv);
    if (rc) return rc;
    HIPCHK(hipSetDevice(ctx->device));
    ctx->stamp_seq = 0;
    std::vector<ChunkIn> in(n_chunks);
    for (int i = 0; i < n_chunks; i++) {
        if (chunks[i].n > 0 && !chunks[i].tokens) return fail(FG_E_ARG, "chunk without tokens");
        in[i] = ChunkIn{chunks[i].tokens, chunks[i].n, chunks[i].pos, chunks[i].blocks, chunks[i].n_blocks,
                        chunks[i].logits};
    }
    Plan P;
    if ((rc = build_plan(m->cfg, *kv, m->max_pos, in.data(), n_chunks, P))) return rc;
    if (rows_out) *rows_out = P.S;
    if (P.t == 0) return 0;
    if ((rc = ensure(&ctx->hmeta, &ctx->hmeta_cap, P.words * 4, ctx->stream, true))) return rc;
    if ((rc = ensure(&ctx->dmeta, &ctx->dmeta_cap, P.words * 4, ctx->stream, false))) return rc;
    pack_plan(P, (int32_t*)ctx->hmeta);
    HIPCHK(hipMemcpyAsync(ctx->dmeta, ctx->hmeta, P.words * 4, hipMemcpyHostToDevice, ctx->stream));
    Work w{};
    const size_t need = layout_work(m, P, w, nullptr);
    if ((rc = ensure(&ctx->ws, &ctx->ws_cap, need, ctx->stream, false))) return rc;
    layout_work(m, P, w, ctx->ws);
    const int32_t* meta = (const int32_t*)ctx->dmeta;
    rc = run_forward(ctx, m, kv, P, meta, (const uint32_t*)(meta + P.o_tok), 1, w, logits_out ? w.logits : nullptr,
                     nullptr, nullptr, 0, 0, hidden_out);
    if (rc) return rc;
    if (P.S > 0 && logits_out)
        HIPCHK(hipMemcpyAsync(logits_out, w.logits, (size_t)P.S * m->cfg.vocab * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (P.S > 0 && argmax_out)
        HIPCHK(hipMemcpyAsync(argmax_out, w.am, (size_t)P.S * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}

int fg_forward_capture(fg_ctx* ctx, const fg_model* m, fg_kv* kv, const fg_chunk* chunks, int32_t n_chunks,
                       float* inputs_out) {
    if (!ctx || !m || !kv || !inputs_out || (!chunks && n_chunks > 0) || n_chunks < 0)
        return fail(FG_E_ARG, "null argument");
    int rc = check_model_kv(m, kv);
    if (rc) return rc;
    HIPCHK(hipSetDevice(ctx->device));
    std::vector<ChunkIn> in(n_chunks);
    for (int i = 0; i < n_chunks; i++) {
        if (chunks[i].n > 0 && !chunks[i].tokens) return fail(FG_E_ARG, "chunk without tokens");
        // only the projection inputs are wanted: no logits rows (Logits::None)
        in[i] = ChunkIn{chunks[i].tokens, chunks[i].n, chunks[i].pos, chunks[i].blocks, chunks[i].n_blocks,
                        FG_LOGITS_NONE};
    }
    Plan P;
    if ((rc = build_plan(m->cfg, *kv, m->max_pos, in.data(), n_chunks, P))) return rc;
    if (P.t == 0 || m->layers.empty()) return 0;
    const fg_config& c = m->cfg;
    const size_t floats =
        m->layers.size() * (size_t)P.t * (2 * (size_t)c.hidden + (size_t)c.heads * c.head_dim + c.intermediate);
    if ((rc = ensure(&ctx->hmeta, &ctx->hmeta_cap, P.words * 4, ctx->stream, true))) return rc;
    if ((rc = ensure(&ctx->dmeta, &ctx->dmeta_cap, P.words * 4, ctx->stream, false))) return rc;
    pack_plan(P, (int32_t*)ctx->hmeta);
    HIPCHK(hipMemcpyAsync(ctx->dmeta, ctx->hmeta, P.words * 4, hipMemcpyHostToDevice, ctx->stream));
    Work w{};
    const size_t need = layout_work(m, P, w, nullptr);
    if ((rc = ensure(&ctx->ws, &ctx->ws_cap, need, ctx->stream, false))) return rc;
    layout_work(m, P, w, ctx->ws);
    float* cap = nullptr;
    if (hipMalloc((void**)&cap, floats * 4) != hipSuccess) {
        (void)hipGetLastError();
        return fail(FG_E_NOMEM, "capture buffer of " + std::to_string(floats * 4) + " bytes");
    }
    const int32_t* meta = (const int32_t*)ctx->dmeta;
    rc = run_forward(ctx, m, kv, P, meta, (const uint32_t*)(meta + P.o_tok), 1, w, nullptr, nullptr, nullptr, 0, 0,
                     nullptr, cap);
    if (!rc && hipMemcpyAsync(inputs_out, cap, floats * 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess)
        rc = fail(FG_E_DEVICE, "capture copy");
    if (!rc && hipStreamSynchronize(ctx->stream) != hipSuccess) rc = fail(FG_E_DEVICE, "capture synchronize");
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(cap);
    return rc;
}

// Distributions of rows carved from the context's sampling buffer starting at
// row `first` (the buffer holds `total` rows of `cap` pairs): tok, pr, tok_id,
// pr_id [total][cap], n [total]; with wide rows also dense [total][cap] and
// the sort scratch [total][4 cap].
static size_t sample_cap(bool wide, int vocab) { return wide ? (size_t)vocab : (size_t)kSampleCap; }
static SampleRows sample_rows(void* buf, int total, int first, bool wide, int vocab) {
    const size_t cap = sample_cap(wide, vocab), tc = (size_t)total * cap;
    uint8_t* b = (uint8_t*)buf;
    SampleRows r;
    r.tok = (uint32_t*)b + (size_t)first * cap;
    r.pr = (float*)(b + tc * 4) + (size_t)first * cap;
    r.tok_id = (uint32_t*)(b + tc * 8) + (size_t)first * cap;
    r.pr_id = (float*)(b + tc * 12) + (size_t)first * cap;
    const size_t o_n = tc * 16, o_dense = o_n + ((size_t)total * 4 + 255) / 256 * 256;
    r.n = (int*)(b + o_n) + first;
    r.cap = (int)cap;
    r.vocab = vocab;
    r.dense = wide ? (float*)(b + o_dense) + (size_t)first * cap : nullptr;
    r.scratch = wide ? (uint32_t*)(b + o_dense + tc * 4) + (size_t)first * cap * 4 : nullptr;
    return r;
}
static size_t sample_bytes(int total, bool wide, int vocab) {
    const size_t tc = (size_t)total * sample_cap(wide, vocab);
    return tc * 16 + ((size_t)total * 4 + 255) / 256 * 256 + (wide ? tc * 20 : 0);
}
static_assert(sizeof(SampleParams) == sizeof(fg_sampling), "fg_sampling is copied to the device as SampleParams");

// Sets *wide when a sampled row has top_k 0 (no limit) or above kSampleCap.
static int check_sampling(const fg_sampling* p, int n, bool* wide) {
    *wide = false;
    for (int i = 0; i < n; i++) {
        if (p[i].temperature > 0.0f && p[i].top_k < 0) return fail(FG_E_ARG, "top_k must be 0 (no limit) or positive");
        *wide |= sample_wide(*(const SampleParams*)&p[i]);
    }
    return 0;
}

// chunks (n_chunks, greedy only): other sequences' prefill chunks and plain
// rows, carried by the verify forward after the verify rows (Engine::execute's
// one target pass); chunk_am gets the argmax of their FG_LOGITS_LAST rows.
static int spec_step(fg_ctx* ctx, const fg_model* target, fg_kv* tkv, const fg_model* draft, fg_kv* dkv,
                     const fg_spec_seq* seqs, int32_t n_seqs, int32_t k, const fg_sampling* params, uint64_t* rng,
                     uint32_t* out_tokens, int32_t* out_count, int32_t* out_accepted, const fg_chunk* chunks = nullptr,
                     int32_t n_chunks = 0, uint32_t* chunk_am = nullptr) {
    if (!ctx || !target || !tkv || !draft || !dkv || !seqs || n_seqs <= 0 || k <= 0 || !out_tokens || !out_count ||
        !out_accepted || (params && !rng) || n_chunks < 0 || (n_chunks > 0 && !chunks))
        return fail(FG_E_ARG, "bad argument");
    const bool sampling = params != nullptr;
    if (sampling && n_chunks > 0) return fail(FG_E_ARG, "chunks ride only with greedy steps");
    ctx->stamp_seq = 0;
    int c_last = 0;  // FG_LOGITS_LAST rows of the chunks
    for (int c = 0; c < n_chunks; c++) {
        if (chunks[c].n > 0 && !chunks[c].tokens) return fail(FG_E_ARG, "chunk without tokens");
        if (chunks[c].logits == FG_LOGITS_ALL) return fail(FG_E_ARG, "chunks take FG_LOGITS_NONE or FG_LOGITS_LAST");
        c_last += chunks[c].logits == FG_LOGITS_LAST && chunks[c].n > 0;
    }
    if (c_last > 0 && !chunk_am) return fail(FG_E_ARG, "bad argument");
    bool wide = false;  // a sampled sequence with top_k 0 or above kSampleCap
    for (int i = 0; sampling && i < n_seqs; i++) wide |= sample_wide(*(const SampleParams*)&params[i]);
    if (wide && draft->cfg.vocab != target->cfg.vocab)
        return fail(FG_E_SHAPE, "draft and target must share a vocabulary");
    if (draft->cfg.vocab != target->cfg.vocab) return fail(FG_E_SHAPE, "draft and target must share a vocabulary");
    int rc;
    if ((rc = check_model_kv(target, tkv)) || (rc = check_model_kv(draft, dkv))) return rc;
    HIPCHK(hipSetDevice(ctx->device));
    const int K1 = k + 1;
    // Plans: draft rounds 0..k-1, then the verify pass.
    std::vector<Plan> plans(k + 1);
    std::vector<ChunkIn> in(n_seqs);
    for (int s = 0; s < n_seqs; s++) {
        const fg_spec_seq& q = seqs[s];
        if (!q.tail || q.n_tail < 1) return fail(FG_E_ARG, "empty tail");
        if (q.draft_pos + q.n_tail != q.pos + 1) return fail(FG_E_ARG, "tail must end at the last token");
        in[s] = ChunkIn{q.tail, q.n_tail, q.draft_pos, q.draft_blocks, q.n_draft_blocks, FG_LOGITS_LAST};
    }
    if ((rc = build_plan(draft->cfg, *dkv, draft->max_pos, in.data(), n_seqs, plans[0]))) return rc;
    static const uint32_t zero_tok[64] = {0};
    for (int r = 1; r < k; r++) {
        for (int s = 0; s < n_seqs; s++)
            in[s] = ChunkIn{nullptr, 1, seqs[s].pos + r, seqs[s].draft_blocks, seqs[s].n_draft_blocks, FG_LOGITS_LAST};
        if ((rc = build_plan(draft->cfg, *dkv, draft->max_pos, in.data(), n_seqs, plans[r]))) return rc;
    }
    // the verify rows (device tokens), then the chunks (host tokens, checked and
    // packed by build_plan; copied after the verify tokens for the launch)
    std::vector<ChunkIn> vin(n_seqs + n_chunks);
    for (int s = 0; s < n_seqs; s++)
        vin[s] = ChunkIn{nullptr, K1, seqs[s].pos, seqs[s].blocks, seqs[s].n_blocks, FG_LOGITS_ALL};
    for (int c = 0; c < n_chunks; c++)
        vin[n_seqs + c] = ChunkIn{chunks[c].tokens, chunks[c].n, chunks[c].pos, chunks[c].blocks,
                                  chunks[c].n_blocks, chunks[c].logits};
    if ((rc = build_plan(target->cfg, *tkv, target->max_pos, vin.data(), n_seqs + n_chunks, plans[k]))) return rc;
    const int c_rows = plans[k].t - n_seqs * K1;  // the chunks' rows
    (void)zero_tok;
    // One packed upload: every plan, then the verify token rows and outputs.
    std::vector<size_t> base(k + 1);
    size_t words = 0;
    for (int r = 0; r <= k; r++) {
        base[r] = words;
        words += plans[r].words;
    }
    const size_t o_vtok = words;
    words += (size_t)n_seqs * K1 + c_rows + 64;
    // sampling: parameters and generator states (uploaded with the plans; the
    // states come back with the outputs)
    words = (words + 15) / 16 * 16;  // 64-byte aligned parameters and states
    const size_t o_prm = words;
    if (sampling) words += (size_t)n_seqs * 4 + 64;
    const size_t o_rng = words;
    if (sampling) words += (size_t)n_seqs * 2 + 64;
    const size_t o_out = words;
    words += (size_t)n_seqs * K1 + 64;
    const size_t o_cnt = words;
    words += (size_t)n_seqs + 64;
    const size_t o_acc = words;
    words += (size_t)n_seqs + 64;
    const size_t o_am = words;
    words += (size_t)n_seqs * K1 + c_last + 64;
    if ((rc = ensure(&ctx->hmeta, &ctx->hmeta_cap, words * 4, ctx->stream, true))) return rc;
    if ((rc = ensure(&ctx->dmeta, &ctx->dmeta_cap, words * 4, ctx->stream, false))) return rc;
    int32_t* h = (int32_t*)ctx->hmeta;
    for (int r = 0; r <= k; r++) pack_plan(plans[r], h + base[r]);
    uint32_t* hv = (uint32_t*)(h + o_vtok);
    for (int s = 0; s < n_seqs; s++) {
        hv[s * K1] = seqs[s].tail[seqs[s].n_tail - 1];
        for (int j = 1; j < K1; j++) hv[s * K1 + j] = 0;
    }
    for (int r = n_seqs * K1; r < plans[k].t; r++) hv[r] = plans[k].tokens[r];
    if (sampling) {
        memcpy(h + o_prm, params, (size_t)n_seqs * sizeof(SampleParams));
        memcpy(h + o_rng, rng, (size_t)n_seqs * 8);
    }
    HIPCHK(hipMemcpyAsync(ctx->dmeta, ctx->hmeta, o_out * 4, hipMemcpyHostToDevice, ctx->stream));
    size_t need = 0;
    Work w{};
    const fg_model* models[2] = {draft, target};
    for (int r = 0; r <= k; r++) need = std::max(need, layout_work(models[r == k], plans[r], w, nullptr));
    if ((rc = ensure(&ctx->ws, &ctx->ws_cap, need, ctx->stream, false))) return rc;
    // sampling rows: the target's n_seqs*(k+1) verify rows, then k draft rounds of n_seqs
    const int srows = n_seqs * K1 + k * n_seqs;
    const int vocab = target->cfg.vocab;
    if (sampling && (rc = ensure(&ctx->sbuf, &ctx->sbuf_cap, sample_bytes(srows, wide, vocab), ctx->stream, false)))
        return rc;
    int32_t* dm = (int32_t*)ctx->dmeta;
    uint32_t* vtok = (uint32_t*)(dm + o_vtok);
    const SampleParams* dprm = (const SampleParams*)(dm + o_prm);
    uint64_t* drng = (uint64_t*)(dm + o_rng);
    // The two phases as launch sequences (captured into graphs when enabled).
    auto draft_phase = [&]() -> int {
        for (int r = 0; r < k; r++) {
            layout_work(draft, plans[r], w, ctx->ws);
            const int32_t* meta = dm + base[r];
            const uint32_t* tok = r == 0 ? (const uint32_t*)(meta + plans[r].o_tok) : vtok + r;
            const int stride = r == 0 ? 1 : K1;
            // the draft's proposal d_{r+1} goes to verify row s, column r+1: the
            // greedy argmax, replaced by a draw for sampled sequences
            int e = run_forward(ctx, draft, dkv, plans[r], meta, tok, stride, w, sampling ? w.logits : nullptr,
                                (uint32_t*)(dm + o_am), vtok, K1, r + 1, nullptr);
            if (e) return e;
            if (sampling) {
                SampleRows q = sample_rows(ctx->sbuf, srows, n_seqs * K1 + r * n_seqs, wide, vocab);
                launch_dist(ctx->stream, w.logits, n_seqs, draft->cfg.vocab, 1, dprm, q);
                launch_draw(ctx->stream, n_seqs, dprm, q, drng, vtok, K1, r + 1);
            }
        }
        return 0;
    };
    auto verify_phase = [&]() -> int {
        layout_work(target, plans[k], w, ctx->ws);
        int e = run_forward(ctx, target, tkv, plans[k], dm + base[k], vtok, 1, w, sampling ? w.logits : nullptr,
                            (uint32_t*)(dm + o_am), nullptr, 0, 0, nullptr);
        if (e) return e;
        if (sampling) {
            SampleRows p = sample_rows(ctx->sbuf, srows, 0, wide, vocab);
            launch_dist(ctx->stream, w.logits, n_seqs * K1, target->cfg.vocab, K1, dprm, p);
            SampleRows q = sample_rows(ctx->sbuf, srows, n_seqs * K1, wide, vocab);
            launch_accept_sampled(ctx->stream, n_seqs, k, dprm, vtok, (const uint32_t*)(dm + o_am), p, q, drng,
                                  (uint32_t*)(dm + o_out), dm + o_cnt, dm + o_acc);
        } else {
            launch_accept(ctx->stream, (const uint32_t*)(dm + o_am), vtok, n_seqs, k, (uint32_t*)(dm + o_out),
                          dm + o_cnt, dm + o_acc);
        }
        return 0;
    };
    // steps that carry chunks launch directly (their plans vary step to step)
    bool use_graph = ctx->graphs && !ctx->prof && n_chunks == 0;
    fg_ctx::GraphSet* gset = nullptr;
    if (use_graph) {
        // everything the captured launches bake in: object identities, the
        // workspace and metadata allocations, and each plan's shapes
        std::vector<int64_t> sig = {n_seqs, k, (int64_t)target->serial, (int64_t)draft->serial,
                                    (int64_t)tkv->serial, (int64_t)dkv->serial, (int64_t)(uintptr_t)ctx->ws,
                                    (int64_t)ctx->ws_cap, (int64_t)(uintptr_t)ctx->dmeta, (int64_t)ctx->dmeta_cap,
                                    (int64_t)sampling, (int64_t)wide, (int64_t)(uintptr_t)ctx->sbuf,
                                    (int64_t)ctx->sbuf_cap, (int64_t)o_out};
        for (int r = 0; r <= k; r++) {
            const Plan& P = plans[r];
            for (int64_t v : {(int64_t)P.t, (int64_t)P.S, (int64_t)P.Wc, (int64_t)P.words, (int64_t)P.ns,
                              (int64_t)P.flash, (int64_t)P.maxq})
                sig.push_back(v);
        }
        for (auto& g : ctx->gsets)
            if (g.sig == sig) gset = &g;
        if (!gset) {
            if ((int)ctx->gsets.size() < fg_ctx::kGraphSets) {
                ctx->gsets.emplace_back();
                gset = &ctx->gsets.back();
            } else {
                gset = &ctx->gsets[0];
                for (auto& g : ctx->gsets)
                    if (g.used < gset->used) gset = &g;
                drop_set(*gset);
            }
            std::function<int()> phases[2] = {draft_phase, verify_phase};
            for (int g = 0; g < 2 && use_graph; g++) {
                HIPCHK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
                ctx->capturing = true;
                const int e = phases[g]();
                ctx->capturing = false;
                hipGraph_t graph = nullptr;
                const hipError_t ce = hipStreamEndCapture(ctx->stream, &graph);
                if (e) {
                    if (graph) (void)hipGraphDestroy(graph);
                    drop_set(*gset);
                    return e;
                }
                if (ce != hipSuccess || !graph ||
                    hipGraphInstantiate(&gset->exec[g], graph, nullptr, nullptr, 0) != hipSuccess) {
                    if (graph) (void)hipGraphDestroy(graph);
                    (void)hipGetLastError();
                    drop_set(*gset);
                    use_graph = false;  // launch directly this time
                    break;
                }
                (void)hipGraphDestroy(graph);
            }
            if (use_graph) gset->sig = sig;
        }
        if (use_graph) gset->used = ++ctx->gclock;
    }
    HIPCHK(hipEventRecord(ctx->ev[0], ctx->stream));
    if (use_graph)
        HIPCHK(hipGraphLaunch(gset->exec[0], ctx->stream));
    else if ((rc = draft_phase()))
        return rc;
    HIPCHK(hipEventRecord(ctx->ev[1], ctx->stream));
    if (use_graph)
        HIPCHK(hipGraphLaunch(gset->exec[1], ctx->stream));
    else if ((rc = verify_phase()))
        return rc;
    HIPCHK(hipGetLastError());
    HIPCHK(hipEventRecord(ctx->ev[2], ctx->stream));
    HIPCHK(hipMemcpyAsync(h + o_rng, dm + o_rng, (words - o_rng) * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    if (sampling) memcpy(rng, h + o_rng, (size_t)n_seqs * 8);
    memcpy(out_tokens, h + o_out, (size_t)n_seqs * K1 * 4);
    memcpy(out_count, h + o_cnt, (size_t)n_seqs * 4);
    memcpy(out_accepted, h + o_acc, (size_t)n_seqs * 4);
    if (c_last > 0) memcpy(chunk_am, h + o_am + (size_t)n_seqs * K1, (size_t)c_last * 4);
    float a = 0, b = 0;
    HIPCHK(hipEventElapsedTime(&a, ctx->ev[0], ctx->ev[1]));
    HIPCHK(hipEventElapsedTime(&b, ctx->ev[1], ctx->ev[2]));
    ctx->last_us[0] = a * 1000.0f;
    ctx->last_us[1] = b * 1000.0f;
    ctx->last_us[2] = (a + b) * 1000.0f;
    return 0;
}

int fg_forward_sampled(fg_ctx* ctx, const fg_model* m, fg_kv* kv, const fg_chunk* chunks, int32_t n_chunks,
                       const fg_sampling* params, uint64_t* rng, uint32_t* tokens_out, int32_t* rows_out) {
    if (!ctx || !m || !kv || (!chunks && n_chunks > 0) || n_chunks < 0 || !tokens_out)
        return fail(FG_E_ARG, "null argument");
    int rc = check_model_kv(m, kv);
    if (rc) return rc;
    HIPCHK(hipSetDevice(ctx->device));
    std::vector<ChunkIn> in(n_chunks);
    for (int i = 0; i < n_chunks; i++) {
        if (chunks[i].n > 0 && !chunks[i].tokens) return fail(FG_E_ARG, "chunk without tokens");
        in[i] = ChunkIn{chunks[i].tokens, chunks[i].n, chunks[i].pos, chunks[i].blocks, chunks[i].n_blocks,
                        chunks[i].logits};
    }
    Plan P;
    if ((rc = build_plan(m->cfg, *kv, m->max_pos, in.data(), n_chunks, P))) return rc;
    if (rows_out) *rows_out = P.S;
    if (P.t == 0) return 0;
    if (P.S > 0 && (!params || !rng)) return fail(FG_E_ARG, "sampling parameters and generator states required");
    bool wide = false;
    if (P.S > 0 && (rc = check_sampling(params, P.S, &wide))) return rc;
    // the plan, then the selected rows' parameters and generator states
    const size_t o_prm = P.words, o_rng = o_prm + (size_t)P.S * 4 + 64, words = o_rng + (size_t)P.S * 2 + 64;
    if ((rc = ensure(&ctx->hmeta, &ctx->hmeta_cap, words * 4, ctx->stream, true))) return rc;
    if ((rc = ensure(&ctx->dmeta, &ctx->dmeta_cap, words * 4, ctx->stream, false))) return rc;
    int32_t* h = (int32_t*)ctx->hmeta;
    pack_plan(P, h);
    if (P.S > 0) {
        memcpy(h + o_prm, params, (size_t)P.S * sizeof(SampleParams));
        memcpy(h + o_rng, rng, (size_t)P.S * 8);
    }
    HIPCHK(hipMemcpyAsync(ctx->dmeta, ctx->hmeta, words * 4, hipMemcpyHostToDevice, ctx->stream));
    Work w{};
    const size_t need = layout_work(m, P, w, nullptr);
    if ((rc = ensure(&ctx->ws, &ctx->ws_cap, need, ctx->stream, false))) return rc;
    if (P.S > 0 &&
        (rc = ensure(&ctx->sbuf, &ctx->sbuf_cap, sample_bytes(P.S, wide, m->cfg.vocab), ctx->stream, false)))
        return rc;
    layout_work(m, P, w, ctx->ws);
    int32_t* dm = (int32_t*)ctx->dmeta;
    rc = run_forward(ctx, m, kv, P, dm, (const uint32_t*)(dm + P.o_tok), 1, w, w.logits, nullptr, nullptr, 0, 0,
                     nullptr);
    if (rc) return rc;
    if (P.S > 0) {
        // greedy rows keep the argmax in w.am; sampled rows are drawn over it
        SampleRows d = sample_rows(ctx->sbuf, P.S, 0, wide, m->cfg.vocab);
        const SampleParams* dprm = (const SampleParams*)(dm + o_prm);
        launch_dist(ctx->stream, w.logits, P.S, m->cfg.vocab, 1, dprm, d);
        launch_draw(ctx->stream, P.S, dprm, d, (uint64_t*)(dm + o_rng), w.am, 1, 0);
        HIPCHK(hipGetLastError());
        HIPCHK(hipMemcpyAsync(tokens_out, w.am, (size_t)P.S * 4, hipMemcpyDeviceToHost, ctx->stream));
        HIPCHK(hipMemcpyAsync(h + o_rng, dm + o_rng, (size_t)P.S * 8, hipMemcpyDeviceToHost, ctx->stream));
    }
    HIPCHK(hipStreamSynchronize(ctx->stream));
    if (P.S > 0) memcpy(rng, h + o_rng, (size_t)P.S * 8);
    return 0;
}

int fg_spec_step(fg_ctx* ctx, const fg_model* target, fg_kv* tkv, const fg_model* draft, fg_kv* dkv,
                 const fg_spec_seq* seqs, int32_t n_seqs, int32_t k, uint32_t* out_tokens, int32_t* out_count,
                 int32_t* out_accepted) {
    return spec_step(ctx, target, tkv, draft, dkv, seqs, n_seqs, k, nullptr, nullptr, out_tokens, out_count,
                     out_accepted);
}

int fg_spec_step_mixed(fg_ctx* ctx, const fg_model* target, fg_kv* tkv, const fg_model* draft, fg_kv* dkv,
                       const fg_spec_seq* seqs, int32_t n_seqs, int32_t k, const fg_chunk* chunks, int32_t n_chunks,
                       uint32_t* out_tokens, int32_t* out_count, int32_t* out_accepted, uint32_t* chunk_argmax_out) {
    return spec_step(ctx, target, tkv, draft, dkv, seqs, n_seqs, k, nullptr, nullptr, out_tokens, out_count,
                     out_accepted, chunks, n_chunks, chunk_argmax_out);
}

int fg_spec_step_sampled(fg_ctx* ctx, const fg_model* target, fg_kv* tkv, const fg_model* draft, fg_kv* dkv,
                         const fg_spec_seq* seqs, int32_t n_seqs, int32_t k, const fg_sampling* params, uint64_t* rng,
                         uint32_t* out_tokens, int32_t* out_count, int32_t* out_accepted) {
    if (!params || !rng || n_seqs <= 0) return fail(FG_E_ARG, "sampling parameters and generator states required");
    bool wide = false;
    int rc = check_sampling(params, n_seqs, &wide);
    if (rc) return rc;
    return spec_step(ctx, target, tkv, draft, dkv, seqs, n_seqs, k, params, rng, out_tokens, out_count,
                     out_accepted);
}

int fg_last_step_times(const fg_ctx* ctx, float* us3) {
    if (!ctx || !us3) return fail(FG_E_ARG, "null argument");
    memcpy(us3, ctx->last_us, sizeof(ctx->last_us));
    return 0;
}

int fg_stamps_reset(fg_ctx* ctx) {
    if (!ctx) return fail(FG_E_ARG, "null ctx");
    HIPCHK(hipSetDevice(ctx->device));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    if (stamps_clear()) return fail(FG_E_ARG, "this library was built without stamps (python -m ferrolm_amd.build --stamps)");
    return 0;
}

int fg_stamps_read(fg_ctx* ctx, int32_t slots, uint64_t* ticks, char* labels, int32_t label_cap) {
    if (!ctx || slots < 0 || (slots > 0 && !ticks) || (label_cap > 0 && !labels)) return fail(FG_E_ARG, "bad argument");
    HIPCHK(hipSetDevice(ctx->device));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    const int used = (int)ctx->stamp_labels.size();
    if (stamps_read(ticks, std::min(slots, kStampSlots)))
        return fail(FG_E_ARG, "this library was built without stamps (python -m ferrolm_amd.build --stamps)");
    std::string all;
    for (const auto& l : ctx->stamp_labels) all += l + "\n";
    if (label_cap > 0) {
        const size_t n = std::min(all.size(), (size_t)label_cap - 1);
        memcpy(labels, all.data(), n);
        labels[n] = 0;
    }
    return used;
}

int fg_profile(fg_ctx* ctx, int32_t on) {
    if (!ctx) return fail(FG_E_ARG, "null ctx");
    ctx->prof = on != 0;
    return 0;
}

int fg_profile_read(fg_ctx* ctx, int32_t cap, int32_t* cls, int64_t* launches, double* us, double* bytes,
                    double* flops, int32_t reset) {
    if (!ctx || cap < 0 || (cap > 0 && (!cls || !launches || !us || !bytes || !flops)))
        return fail(FG_E_ARG, "bad argument");
    HIPCHK(hipStreamSynchronize(ctx->stream));
    for (const auto& p : ctx->pending) {
        float ms = 0;
        HIPCHK(hipEventElapsedTime(&ms, ctx->pev[p.ev], ctx->pev[p.ev + 1]));
        auto& r = ctx->rec[p.cls];
        r.n++;
        r.us += ms * 1000.0;
        r.bytes += p.bytes;
        r.flops += p.flops;
    }
    ctx->pending.clear();
    ctx->pev_used = 0;
    int n = 0;
    for (int i = 0; i < 12; i++) {
        if (!ctx->rec[i].n) continue;
        if (n < cap) {
            cls[n] = i;
            launches[n] = ctx->rec[i].n;
            us[n] = ctx->rec[i].us;
            bytes[n] = ctx->rec[i].bytes;
            flops[n] = ctx->rec[i].flops;
        }
        n++;
    }
    if (reset)
        for (auto& r : ctx->rec) r = fg_ctx::Rec();
    return n;
}

int fg_mat_upload(fg_ctx* ctx, const fg_matrix* w, fg_mat** out) {
    if (!ctx || !w || !out) return fail(FG_E_ARG, "null argument");
    HIPCHK(hipSetDevice(ctx->device));
    fg_mat* m = new fg_mat();
    m->device = ctx->device;
    int rc = upload_mat(*w, m->m, nullptr);
    if (rc) {
        fg_mat_destroy(m);
        return rc;
    }
    *out = m;
    return 0;
}

void fg_mat_destroy(fg_mat* m) {
    if (!m) return;
    if (m->m.w) (void)hipFree(m->m.w);
    if (m->m.s) (void)hipFree(m->m.s);
    delete m;
}

// Workspace for a lone product: pieces, staged x and y, GEMM split-K partials.
static size_t layout_mat(const DMat& d, int m, Pieces& p, float** xbuf, float** ybuf, float** bbuf, Work& w,
                         void* base) {
    Carver cv(base);
    p.kb = d.kb;
    p.passes = (m + 3) / 4;
    p.a = cv.take<uint8_t>((size_t)d.kb * p.passes * 64 * 16);
    p.xs = cv.take<float>((size_t)d.kb * p.passes * 4);
    *xbuf = cv.take<float>((size_t)m * d.cols);
    *ybuf = cv.take<float>((size_t)m * d.rows);
    *bbuf = cv.take<float>((size_t)d.rows);
    w.kpart_cap = m > kGemvRows ? kKpartFloats : 0;
    w.kpart = w.kpart_cap ? cv.take<float>(w.kpart_cap) : nullptr;
    return cv.off + 256;
}

// y = x W^T (+ bias): a GEMV on BF16/INT8 pieces up to kGemvRows rows, a GEMM
// on MM pieces beyond, as in the forward pass.
static void matmul_launch(fg_ctx* ctx, const DMat& d, Pieces& p, const Work& w, const float* x, int m,
                          const float* bias, float* y) {
    const bool mm = m > kGemvRows;
    launch_pieces(ctx->stream, mm ? (int)MM : d.kind, x, d.cols, m, d.cols, nullptr, nullptr, p);
    GemvArgs g = gemv_args(d, p, m, w);
    g.mm = mm;
    g.out = y;
    g.ldo = d.rows;
    g.bias = bias;
    gemv(ctx, EPI_STORE, d, g);
}

int fg_matmul(fg_ctx* ctx, const fg_mat* w, const float* x, int32_t m, const float* bias, float* y) {
    if (!ctx || !w || !x || !y || m <= 0) return fail(FG_E_ARG, "bad argument");
    HIPCHK(hipSetDevice(ctx->device));
    const DMat& d = w->m;
    Pieces p;
    Work wk{};
    float *xb, *yb, *bb;
    int rc;
    if ((rc = ensure(&ctx->ws, &ctx->ws_cap, layout_mat(d, m, p, &xb, &yb, &bb, wk, nullptr), ctx->stream, false)))
        return rc;
    layout_mat(d, m, p, &xb, &yb, &bb, wk, ctx->ws);
    if (bias) HIPCHK(hipMemcpyAsync(bb, bias, (size_t)d.rows * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(hipMemcpyAsync(xb, x, (size_t)m * d.cols * 4, hipMemcpyHostToDevice, ctx->stream));
    matmul_launch(ctx, d, p, wk, xb, m, bias ? bb : nullptr, yb);
    HIPCHK(hipGetLastError());
    HIPCHK(hipMemcpyAsync(y, yb, (size_t)m * d.rows * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}

int fg_matmul_device(fg_ctx* ctx, const fg_mat* w, const float* x_dev, int32_t m, float* y_dev) {
    if (!ctx || !w || !x_dev || !y_dev || m <= 0) return fail(FG_E_ARG, "bad argument");
    const DMat& d = w->m;
    Pieces p;
    Work wk{};
    float *xb, *yb, *bb;
    int rc;
    if ((rc = ensure(&ctx->ws, &ctx->ws_cap, layout_mat(d, m, p, &xb, &yb, &bb, wk, nullptr), ctx->stream, false)))
        return rc;
    layout_mat(d, m, p, &xb, &yb, &bb, wk, ctx->ws);
    matmul_launch(ctx, d, p, wk, x_dev, m, nullptr, y_dev);
    HIPCHK(hipGetLastError());
    return 0;
}

int fg_matmul_device_noalloc(fg_ctx* ctx, const fg_mat* w, const float* x_dev, int32_t m, float* y_dev) {
    if (!ctx || !w || !x_dev || !y_dev || m <= 0) return fail(FG_E_ARG, "bad argument");
    if (!ctx->scratch) return fail(FG_E_DEVICE, "no scratch address on this device");
    if (m > kGemvRows) return fail(FG_E_SHAPE, "at most 15 rows without allocating (the GEMV path)");
    const DMat& d = w->m;
    // pieces, then their block scales, in the scratch (no byte of it is read
    // before this call's k_pieces writes it: nothing to clear)
    Pieces p;
    p.kb = d.kb;
    p.passes = (m + 3) / 4;
    const size_t a_bytes = (size_t)d.kb * p.passes * 64 * 16;
    const size_t xs_off = (a_bytes + 255) / 256 * 256;
    if (xs_off + (size_t)d.kb * p.passes * 4 * sizeof(float) > kScratchBytes)
        return fail(FG_E_SHAPE, "the product's pieces exceed the 2 MiB scratch (at most 504 k-blocks at 15 rows)");
    p.a = ctx->scratch;
    p.xs = (float*)(ctx->scratch + xs_off);
    launch_pieces(ctx->stream, d.kind, x_dev, d.cols, m, d.cols, nullptr, nullptr, p);
    Work wk{};
    GemvArgs g = gemv_args(d, p, m, wk);
    g.out = y_dev;
    g.ldo = d.rows;
    launch_gemv(ctx->stream, EPI_STORE, d, g);  // no timing events: nothing is created
    HIPCHK(hipGetLastError());
    return 0;
}

// ---- load-time quantization on the device --------------------------------

namespace {
// A device allocation freed when it leaves scope (hipFree waits for the
// device, so queued work that uses it has finished).
struct DevBuf {
    void* p = nullptr;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    float* f() const { return (float*)p; }
    uint8_t* u8() const { return (uint8_t*)p; }
};
}  // namespace

static int dev_alloc(DevBuf& b, size_t bytes) {
    if (hipMalloc(&b.p, std::max<size_t>(bytes, 256)) != hipSuccess) {
        b.p = nullptr;
        (void)hipGetLastError();
        return fail(FG_E_NOMEM, "device allocation failed");
    }
    return 0;
}

static int quant_shape(int32_t kind, int32_t rows, int32_t cols) {
    if (kind != FG_INT8 && kind != FG_INT4) return fail(FG_E_ARG, "format must be FG_INT8 or FG_INT4");
    if (rows <= 0 || cols <= 0) return fail(FG_E_ARG, "empty matrix");
    if (rows % 32 || cols % 32) return fail(FG_E_SHAPE, "quantized matrices need rows and cols that are multiples of 32");
    return 0;
}

int fg_quantize(fg_ctx* ctx, int32_t kind, int32_t rows, int32_t cols, const float* w, const float* importance,
                uint8_t* q, float* s) {
    if (!ctx || !w || !q || !s) return fail(FG_E_ARG, "null pointer");
    int rc;
    if ((rc = quant_shape(kind, rows, cols))) return rc;
    HIPCHK(hipSetDevice(ctx->device));
    hipStream_t st = ctx->stream;
    const size_t n = (size_t)rows * cols, qb = kind == FG_INT8 ? n : n / 2, sn = n / 32;
    DevBuf dw, di, dq, ds;
    if ((rc = dev_alloc(dw, n * 4)) || (rc = dev_alloc(di, (size_t)cols * 4)) || (rc = dev_alloc(dq, qb)) ||
        (rc = dev_alloc(ds, sn * 4)))
        return rc;
    HIPCHK(hipMemcpyAsync(dw.p, w, n * 4, hipMemcpyHostToDevice, st));
    if (importance) HIPCHK(hipMemcpyAsync(di.p, importance, (size_t)cols * 4, hipMemcpyHostToDevice, st));
    launch_quantize(st, kind, rows, cols, dw.f(), importance ? di.f() : nullptr, dq.u8(), ds.f());
    HIPCHK(hipGetLastError());
    HIPCHK(hipMemcpyAsync(q, dq.p, qb, hipMemcpyDeviceToHost, st));
    HIPCHK(hipMemcpyAsync(s, ds.p, sn * 4, hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    return 0;
}

int fg_awq_search(fg_ctx* ctx, int32_t kind, int32_t rows, int32_t k, const float* w, int32_t m, const float* cal,
                  float* scales, fg_awq_choice* choice, uint8_t* q, float* s) {
    if (!ctx || !w || !cal || !scales || !choice || !q || !s) return fail(FG_E_ARG, "null pointer");
    int rc;
    if ((rc = quant_shape(kind, rows, k))) return rc;
    if (m <= 0) return fail(FG_E_ARG, "no calibration rows");
    HIPCHK(hipSetDevice(ctx->device));
    hipStream_t st = ctx->stream;
    const size_t rk = (size_t)rows * k, mk = (size_t)m * k, ny = (size_t)m * rows;
    const size_t qb = kind == FG_INT8 ? rk : rk / 2, sn = rk / 32;
    // channel statistics on the host (f64 sums in row order)
    std::vector<float> am(k), sq(k), sc(k), imp(k), best_s(k);
    fh_awq_stats(cal, m, k, am.data(), sq.data());
    constexpr int kSteps = 11;  // alpha = 0, 0.1, ..., 1
    DevBuf dw, dws, dx, dxs, dyref, dy, dsc, dimp, dq, ds, derr;
    if ((rc = dev_alloc(dw, rk * 4)) || (rc = dev_alloc(dws, rk * 4)) || (rc = dev_alloc(dx, mk * 4)) ||
        (rc = dev_alloc(dxs, mk * 4)) || (rc = dev_alloc(dyref, ny * 4)) || (rc = dev_alloc(dy, kSteps * ny * 4)) ||
        (rc = dev_alloc(dsc, (size_t)k * 4)) || (rc = dev_alloc(dimp, (size_t)k * 4)) || (rc = dev_alloc(dq, qb)) ||
        (rc = dev_alloc(ds, sn * 4)) || (rc = dev_alloc(derr, kSteps * 8)))
        return rc;
    HIPCHK(hipMemcpyAsync(dw.p, w, rk * 4, hipMemcpyHostToDevice, st));
    HIPCHK(hipMemcpyAsync(dx.p, cal, mk * 4, hipMemcpyHostToDevice, st));
    // the reference output, with the unquantized weights as bf16 (Matrix::from_f32)
    launch_mm_exact(st, BF16, dx.f(), m, k, dw.f(), nullptr, nullptr, rows, dyref.f());
    HIPCHK(hipGetLastError());
    // imp = sq / s^2 + 1e-8 and the scaled operands, then the quantizer (apply, src/awq.rs:152-165)
    auto apply = [&](const float* sv) -> int {
        for (int32_t c = 0; c < k; c++) imp[c] = sq[c] / (sv[c] * sv[c]) + 1e-8f;
        HIPCHK(hipMemcpyAsync(dsc.p, sv, (size_t)k * 4, hipMemcpyHostToDevice, st));
        HIPCHK(hipMemcpyAsync(dimp.p, imp.data(), (size_t)k * 4, hipMemcpyHostToDevice, st));
        launch_scale_cols(st, dw.f(), (int64_t)rk, k, dsc.f(), 0, dws.f());
        launch_quantize(st, kind, rows, k, dws.f(), dimp.f(), dq.u8(), ds.f());
        HIPCHK(hipGetLastError());
        return 0;
    };
    // every alpha's product first, then their error sums side by side
    std::vector<std::vector<float>> scs(kSteps);
    for (int step = 0; step < kSteps; step++) {
        scs[step].resize(k);
        fh_awq_scales(am.data(), k, (float)step / 10.0f, scs[step].data());
        if ((rc = apply(scs[step].data()))) return rc;
        launch_scale_cols(st, dx.f(), (int64_t)mk, k, dsc.f(), 1, dxs.f());
        launch_mm_exact(st, kind, dxs.f(), m, k, nullptr, dq.u8(), ds.f(), rows, dy.f() + (size_t)step * ny);
        HIPCHK(hipGetLastError());
        // the scales and importance buffers are rewritten by the next step's copies
        HIPCHK(hipStreamSynchronize(st));
    }
    launch_sq_err(st, dy.f(), (int64_t)ny, kSteps, dyref.f(), (int64_t)ny, (double*)derr.p);
    HIPCHK(hipGetLastError());
    double errs[kSteps];
    HIPCHK(hipMemcpyAsync(errs, derr.p, sizeof(errs), hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    double best = INFINITY, plain = errs[0];
    float best_alpha = 0.0f;
    bool have = false;
    for (int step = 0; step < kSteps; step++)
        if (!have || errs[step] < best) {  // the first minimum, as the reference's search
            have = true;
            best = errs[step];
            best_alpha = (float)step / 10.0f;
            best_s = scs[step];
        }
    if ((rc = apply(best_s.data()))) return rc;
    HIPCHK(hipMemcpyAsync(q, dq.p, qb, hipMemcpyDeviceToHost, st));
    HIPCHK(hipMemcpyAsync(s, ds.p, sn * 4, hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    std::memcpy(scales, best_s.data(), (size_t)k * 4);
    choice->alpha = best_alpha;
    choice->_pad = 0;
    choice->error_plain = plain;
    choice->error_awq = best;
    return 0;
}

}  // extern "C"
