// Persistent forward of a small bf16 model over t <= 4 new rows of one
// sequence: the draft rounds of a speculative step (Engine::propose,
// src/engine.rs:658-717; each round is Model::forward with Logits::Last,
// src/model.rs:269-362, then sampler::argmax, src/sampler.rs:42-51).
//
// A draft round is about 150 dependent steps (six per layer), each only a few
// microseconds of work. As separate kernels every step pays a launch boundary
// (about 1.5 us in a graph) plus its own load round trips; here one launch of
// one workgroup per CU runs them all. The steps ("stages") hand their outputs
// on through tagged words: each f32 is stored together with a 32-bit tag
// (launch epoch << 8 | stage) in one 64-bit store that bypasses the caches,
// and a consumer polls its inputs until every tag is the stage's. There is no
// grid barrier: a workgroup only ever waits for the inputs of its own work,
// and it issues the loads that do not depend on them (its weight operands, the
// cached keys and values of its attention span) before it starts waiting.
//
// Stages (s = 1 + 6 l for layer l; a tag's low byte is the stage number):
//   0        embed: x_b = embed[token]
//   s        q/k/v = ((attn_norm (.) x_b) W_qkv^T) * rinv(x_b) (+ bias)
//   s + 1    attention, items (kv head, span of 64 positions): RoPE of the
//            queries and of the new keys, the new keys/values into their cache
//            slots, then per query the span's max score, sum of exponentials
//            and weighted values
//   s + 2    the spans merged per (row, query head): the attention output
//   s + 3    x_a = x_b + att W_o^T
//   s + 4    act = silu(g rinv(x_a)) * (u rinv(x_a)), [g u] = (mlp_norm (.) x_a) W_gu^T
//   s + 5    x_b = x_a + act W_down^T
//   1 + 6 L  logits of the selected rows (final norm, lm_head); each workgroup
//            publishes its (max, first index) per row
//   2 + 6 L  the argmax over the workgroups (first index of the maximum)
// Every wait is bounded: past a.spin polls a workgroup sets the launch's
// abort flag, which every wait also watches; an aborted launch runs to the
// end without further waiting and the host reports it as an error. The last
// workgroup to finish advances the epoch for the next launch.
#include "devutil.h"
#include "pdraft.h"

namespace fg {

namespace {

constexpr int HD = 64, HALF = HD / 2;
constexpr int NW = kPdWaves, NTHR = 64 * NW;
// a partial: the weighted values, then max score and sum of exponentials,
// padded to whole 128-byte lines (no line is shared between writers)
constexpr int PSZ = HD + 16;
constexpr int LINE = 16;        // tagged words per 128-byte line
constexpr int PST = HD + 4;     // LDS row stride of keys, values, queries
constexpr int MAXB = 6;         // weight operands per wave per round (layer stages)
constexpr int LMB = 16;         // the same for the lm_head (four tiles at a time)
constexpr int YTS = 64;
constexpr int MSP = 4;          // spans per wave per round of the merge         // LDS row stride of finished products (four tiles)

__device__ __forceinline__ unsigned make_tag(unsigned epoch, int stage) { return (epoch << 8) | (unsigned)stage; }

__device__ __forceinline__ void ll_put(uint64_t* p, float v, unsigned tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ll_get(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool ll_ready(uint64_t w, unsigned tag) { return (unsigned)(w >> 32) == tag; }
__device__ __forceinline__ float ll_val(uint64_t w) { return __uint_as_float((unsigned)w); }

// threadIdx.x, opaque to the compiler: the addresses a stage derives from it
// are then not hoisted out of the layer loop (where they would all stay live
// at once).
__device__ __forceinline__ int fresh_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

struct Sh {
    uint16_t* ap; // [kb][64 lanes][8] the fetched rows' bf16 pieces as MFMA A operands
    float* ks;    // [64][PST] keys of a span
    float* vs;    // [64][PST] values of a span
    float* qs;    // [16][PST] queries of an attention item
    float* kn;    // [4][HD] new keys (before RoPE)
    float* vn;    // [4][HD] new values
    float* red;   // [NW][2][64] cross-wave products; [4][NTHR] row sums
    float* yt;    // [4][YTS] finished products of a tile group
    float* rs;    // [8]: row sums of squares, then 1/rms
    int* flag;    // [2]
};

// One more poll of a wait: false (after raising the launch's abort flag)
// once the wait has taken `spin` polls, or when another wait raised it.
__device__ __forceinline__ bool keep_waiting(int& spins, int spin, unsigned* ctl) {
    if (++spins > spin) {
        __hip_atomic_store(ctl + kPdCtlAbort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    if ((spins & 63) == 0 && __hip_atomic_load(ctl + kPdCtlAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
        return false;
    __builtin_amdgcn_s_sleep(1);
    return true;
}

// Polls one tagged word until it carries `tag` (bounded; watches the abort flag).
__device__ __forceinline__ bool poll1(const uint64_t* p, unsigned tag, unsigned* ctl, int spin, uint64_t& w) {
    int spins = 0;
    while (true) {
        w = ll_get(p);
        if (ll_ready(w, tag)) return true;
        if (!keep_waiting(spins, spin, ctl)) return false;
    }
}

// Polls the tagged words src[at(i)] of this thread's slots i = tid + u NTHR
// (u < FM, i < n) until each carries `tag`; their values go to v[u]. Every
// pending slot's load of a round is in flight at once. False when the launch
// was aborted (this thread's view).
template <int FM, class At>
__device__ __forceinline__ bool poll_words(int n, const uint64_t* __restrict__ src, At at, unsigned tag, unsigned* ctl,
                                           int spin, float (&v)[FM]) {
    const int tid = fresh_tid();
    unsigned pending = 0;
#pragma unroll
    for (int u = 0; u < FM; u++)
        if (tid + u * NTHR < n) pending |= 1u << u;
    int spins = 0;
    while (pending) {
#pragma unroll
        for (int u = 0; u < FM; u++)
            if ((pending >> u) & 1u) {
                const uint64_t w = ll_get(src + at(tid + u * NTHR));
                if (ll_ready(w, tag)) {
                    v[u] = ll_val(w);
                    pending &= ~(1u << u);
                }
            }
        if (!pending) break;
        if (!keep_waiting(spins, spin, ctl)) return false;
    }
    return true;
}

// Words of a fetched input per thread: t x K <= 4 x 1536 (the host admits
// models whose hidden, intermediate and q sizes are at most 1536).
constexpr int FETCH_SLOTS = kPdMaxRows * 1536 / NTHR;

// The four bf16 pieces of x: successive round-to-nearest-even bf16 roundings
// of the remainder (x = p0 + p1 + p2 + p3 up to the last piece's rounding).
__device__ __forceinline__ void bf16_pieces(float x, uint16_t* h) {
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t b = f32_to_bf16_bits(x);
        h[p] = (uint16_t)b;
        x = x - bf16_bits_to_f32(b);
    }
}

// A-operand slot of row r, piece p, column k: k-block k / 32, lane
// (4 r + p) + 16 ((k % 32) / 8), element k % 8.
__device__ __forceinline__ int ap_at(int r, int p, int k) {
    return ((k >> 5) * 64 + (r * 4 + p) + 16 * ((k & 31) >> 3)) * 8 + (k & 7);
}

// All threads: the t x K tagged words of src (row-major, rows of K), times
// g[k] (when g), as bf16 pieces into the A operands ap (k-blocks 0 .. KB-1;
// zero past K and for rows >= t); the rows' sums of squares of the raw
// values, summed in a fixed order, into rs[0..t-1] and 1 / rms (the mean over
// K plus eps) into rs[4..7] (when g). False (in every thread) when the launch
// was aborted.
__device__ __forceinline__ bool fetch(const uint64_t* __restrict__ src, int t, int K, int KB, unsigned tag,
                                      const float* __restrict__ g, float eps, unsigned* ctl, int spin, Sh& sh) {
    const int tid = fresh_tid();
    if (tid == 0) sh.flag[0] = 0;
    float vals[FETCH_SLOTS];
    const int n = t * K;
    // slot u is element tid + u NTHR = (row r, column k), stepped without division
    const int r_0 = tid / K, k_0 = tid - r_0 * K;
    const bool good = poll_words<FETCH_SLOTS>(n, src, [](int i) { return i; }, tag, ctl, spin, vals);
    float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (good) {
        int r = r_0, k = k_0;
#pragma unroll
        for (int u = 0; u < FETCH_SLOTS; u++) {
            if (tid + u * NTHR < n) {
                const float v = vals[u];
                uint16_t h[4];
                bf16_pieces(g ? g[k] * v : v, h);
#pragma unroll
                for (int p = 0; p < 4; p++) sh.ap[ap_at(r, p, k)] = h[p];
#pragma unroll
                for (int rr = 0; rr < 4; rr++)
                    if (rr == r) part[rr] = fmaf(v, v, part[rr]);
            }
            k += NTHR;
            while (k >= K) {
                k -= K;
                r++;
            }
        }
    }
    // zeros: every piece of rows >= t (16-byte slots), columns K .. 32 KB - 1 of live rows
    for (int i = tid; i < KB * 64; i += NTHR) {
        const int ln = i & 63, r = (ln & 15) >> 2;
        if (r >= t) *(uint4*)&sh.ap[i * 8] = make_uint4(0u, 0u, 0u, 0u);
    }
    const int kpad = KB * 32 - K;
    for (int i = tid; i < t * 4 * kpad; i += NTHR) {
        const int rp = i / kpad, k = K + i - rp * kpad;
        sh.ap[ap_at(rp >> 2, rp & 3, k)] = 0;
    }
    if (g) {
#pragma unroll
        for (int r = 0; r < 4; r++) sh.red[r * NTHR + tid] = part[r];
    }
    __syncthreads();
    if (!good) sh.flag[0] = 1;
    if (g && (tid >> 6) < 4) {
        // row r in wave r: each lane sums its slots in order, then a fixed tree
        // across the wave; rs[4 + r] = 1 / rms (0 for rows >= t)
        const int r = tid >> 6, lane = tid & 63;
        float v = 0.0f;
        for (int j = 0; j < NW; j++) v += sh.red[r * NTHR + j * 64 + lane];
        v = group_reduce<64, false>(v);
        if (lane == 0) {
            sh.rs[r] = v;
            sh.rs[4 + r] = r < t ? 1.0f / sqrtf(v / (float)K + eps) : 0.0f;
        }
    }
    __syncthreads();
    return sh.flag[0] == 0;
}

// The weight operands of a wave for NTL (1 or 2) tiles starting at tile0 of
// a bf16 matrix in the MFMA tile layout ([tile][kb][lane][8 x bf16]): the
// wave's k-blocks kb0 .. kb1 - 1, NB / NTL of them per round, the tiles of
// one k-block side by side (b[m NTL + tt]).
template <int NB>
struct Ops {
    bf16x8 b[NB];
};

__device__ __forceinline__ void wave_kb(int KB, int& kb0, int& kb1) {
    const int wave = threadIdx.x >> 6;
    kb0 = wave * KB / NW;
    kb1 = (wave + 1) * KB / NW;
}

template <bool NT, int NTL, int NB>
__device__ __forceinline__ void load_ops(const bf16x8* __restrict__ W, int KB, int tile0, int round, Ops<NB>& o) {
    constexpr int PER = NB / NTL;
    const int lane = fresh_tid() & 63;
    int kb0, kb1;
    wave_kb(KB, kb0, kb1);
#pragma unroll
    for (int m = 0; m < PER; m++) {
        const int kb = kb0 + round * PER + m;
        if (kb < kb1) {
#pragma unroll
            for (int tt = 0; tt < NTL; tt++) {
                const bf16x8* src = W + ((size_t)(tile0 + tt) * KB + kb) * 64 + lane;
                o.b[m * NTL + tt] = NT ? __builtin_nontemporal_load(src) : *src;
            }
        }
    }
}

// Products of the NTL (1, 2 or 4) tiles with the fetched input rows, through the MFMA:
// A = the four bf16 pieces of each live row (from ap, one read per k-block),
// B = the weights; the waves' sums go through LDS in wave order into
// yt[r][16 tt + n]. `o` holds the wave's first round of operands (loaded
// before the input was fetched).
template <bool NT, int NTL, int NB>
__device__ __forceinline__ void products(const bf16x8* __restrict__ W, int KB, int tile0, Sh& sh, Ops<NB>& o) {
    constexpr int PER = NB / NTL;
    const int tid = fresh_tid(), wave = tid >> 6, lane = tid & 63;
    int kb0, kb1;
    wave_kb(KB, kb0, kb1);
    f32x4 acc[NTL];
#pragma unroll
    for (int tt = 0; tt < NTL; tt++) acc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int round = 0; kb0 + round * PER < kb1; round++) {
        if (round > 0) load_ops<NT, NTL, NB>(W, KB, tile0, round, o);
#pragma unroll
        for (int m = 0; m < PER; m++) {
            const int kb = kb0 + round * PER + m;
            if (kb < kb1) {
                const bf16x8 a = *(const bf16x8*)&sh.ap[(kb * 64 + lane) * 8];
#pragma unroll
                for (int tt = 0; tt < NTL; tt++)
                    acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, o.b[m * NTL + tt], acc[tt], 0, 0, 0);
            }
        }
    }
    // D: lane l holds rows 4 (l / 16) + r, the four pieces of activation row l / 16, column l % 16
#pragma unroll
    for (int tt = 0; tt < NTL; tt++)
        sh.red[(wave * NTL + tt) * 64 + lane] = ((acc[tt][0] + acc[tt][1]) + acc[tt][2]) + acc[tt][3];
    __syncthreads();
    if (tid < NTL * 64) {
        const int tt = tid >> 6;
        float v = 0.0f;
        for (int w = 0; w < NW; w++) v += sh.red[(w * NTL + tt) * 64 + lane];
        sh.yt[(lane >> 4) * YTS + tt * 16 + (lane & 15)] = v;
    }
    __syncthreads();
}

}  // namespace

__global__ __launch_bounds__(NTHR) void k_pdraft(const PdArgs a) {
    extern __shared__ __align__(16) float lds[];
    Sh sh;
    sh.ap = (uint16_t*)lds;
    sh.ks = lds + a.ap_kb * 64 * 8 / 2;
    sh.vs = sh.ks + 64 * PST;
    sh.qs = sh.vs + 64 * PST;
    sh.kn = sh.qs + 16 * PST;
    sh.vn = sh.kn + 4 * HD;
    sh.red = sh.vn + 4 * HD;
    sh.yt = sh.red + 4 * NTHR;
    sh.rs = sh.yt + 4 * YTS;
    sh.flag = (int*)(sh.rs + 8);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = gridDim.x, wg = blockIdx.x;
    const int t = a.t, H = a.H, I = a.I, qd = a.qd, kvd = a.kvd, nh = a.nh, nkv = a.nkv, GQ = nh / nkv;
    const int qkvd = qd + 2 * kvd;
    unsigned* ctl = a.ctl;
    const int spin = a.spin;
    const unsigned epoch = __hip_atomic_load(ctl + kPdCtlEpoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int pos0 = *a.pos0;
    bool ok = __hip_atomic_load(ctl + kPdCtlAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u;

    // ---- stage 0: embedding, by hidden tiles. The residual stream of this
    // workgroup's own tile (wg < H / 16), row tid / 16, column 16 wg + tid % 16,
    // stays in xres: the o projection and the down projection of that tile both
    // run here; other workgroups read the copy in x_b / x_a.
    float xres = 0.0f;
    if (wg < H / 16 && tid < 16 * t) {
        const int r = tid >> 4, n = wg * 16 + (tid & 15);
        const uint32_t tok = a.tok[(size_t)r * a.tok_stride];
        xres = bf16_bits_to_f32(a.embed[(size_t)tok * H + n]);
        ll_put(a.xb + (size_t)r * H + n, xres, make_tag(epoch, 0));
    }
    const int S = (pos0 + t + 63) / 64;  // spans of 64 positions the new rows see
    for (int l = 0; l < a.L && ok; l++) {
        const int tid = fresh_tid(), lane = tid & 63, wave = tid >> 6;
        const PdLayer& Ly = a.layers[l];
        float* const kc = a.kc + (size_t)l * a.layer_floats;
        float* const vc = a.vc + (size_t)l * a.layer_floats;
        const int s0 = 1 + 6 * l;
        // ---- q/k/v projection: tiles wg, wg + G, ...
        {
            const bf16x8* W = (const bf16x8*)Ly.wqkv;
            const int KB = Ly.qkv_kb, ntile = qkvd / 16;
            const unsigned tout = make_tag(epoch, s0);
            for (int tile = wg; tile < ntile && ok; tile += G) {
                Ops<MAXB> o;
                load_ops<false, 1, MAXB>(W, KB, tile, 0, o);
                const float bias = Ly.bqkv && tid < 16 * t ? Ly.bqkv[tile * 16 + (tid & 15)] : 0.0f;
                if (tile == wg) {
                    ok = fetch(a.xb, t, H, KB, make_tag(epoch, s0 - 1), Ly.attn_norm, a.eps, ctl, spin, sh);
                    if (!ok) break;
                }
                products<false, 1, MAXB>(W, KB, tile, sh, o);
                if (tid < 16 * t) {
                    const int r = tid >> 4, n = tile * 16 + (tid & 15);
                    float v = sh.yt[r * YTS + (tid & 15)] * sh.rs[4 + r];
                    if (Ly.bqkv) v += bias;
                    ll_put(a.qkv + (size_t)r * qkvd + n, v, tout);
                }
                __syncthreads();
            }
        }
        if (!ok) break;
        // ---- attention: items (kv head h, span sp), item = h S + sp
        {
            const unsigned tin = make_tag(epoch, s0), tout = make_tag(epoch, s0 + 1);
            const int Q = t * GQ;
            for (int item = wg; item < nkv * S && ok; item += G) {
                const int h = item / S, sp = item - h * S, p0 = sp * 64, p1 = min(p0 + 64, pos0 + t);
                const int np = p1 - p0, pc1 = min(pos0, p1);  // cached positions p0 .. pc1 - 1
                // the span's cached keys and values, requested before waiting on the new rows
                float4 kk[2], vv[2];
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int i = tid + u * NTHR, o = i >> 4, d = (i & 15) * 4;
                    const int p = min(p0 + o, max(p0, pc1 - 1));
                    const size_t at = (((size_t)(uint32_t)a.blocks[p >> 4] * nkv + h) * 16 + (p & 15)) * HD + d;
                    kk[u] = ld_nt_f4(kc + at);
                    vv[u] = ld_nt_f4(vc + at);
                }
                // the rotation of this thread's query pair and new-key pair (Q HALF and
                // t HALF <= NTHR pairs), also requested before the wait
                float rq_c = 0.0f, rq_s = 0.0f, rk_c = 0.0f, rk_s = 0.0f;
                if (tid < Q * HALF) {
                    const int q = tid / HALF, d = tid - q * HALF, pos = pos0 + q / GQ;
                    rq_c = a.cos_t[(size_t)pos * HALF + d];
                    rq_s = a.sin_t[(size_t)pos * HALF + d];
                }
                if (tid < t * HALF) {
                    const int r = tid / HALF, d = tid - r * HALF, pos = pos0 + r;
                    rk_c = a.cos_t[(size_t)pos * HALF + d];
                    rk_s = a.sin_t[(size_t)pos * HALF + d];
                }
                // the rows' queries of this kv head's group, new keys and values (tagged)
                if (tid == 0) sh.flag[0] = 0;
                __syncthreads();
                {
                    // element i = (row r, j): j < GQ HD a query, then the key, then the value
                    constexpr int FM = kPdMaxRows * (kPdMaxGqa + 2) * HD / NTHR;
                    const int per = GQ * HD + 2 * HD;
                    auto at = [&](int i) {
                        const int r = i / per, j = i - r * per;
                        size_t o = (size_t)r * qkvd;
                        if (j < GQ * HD) o += (size_t)h * GQ * HD + j;
                        else if (j < GQ * HD + HD) o += qd + (size_t)h * HD + (j - GQ * HD);
                        else o += qd + kvd + (size_t)h * HD + (j - GQ * HD - HD);
                        return o;
                    };
                    float vals[FM];
                    const bool good = poll_words<FM>(t * per, a.qkv, at, tin, ctl, spin, vals);
                    if (good) {
#pragma unroll
                        for (int u = 0; u < FM; u++) {
                            const int i = tid + u * NTHR;
                            if (i < t * per) {
                                const int r = i / per, j = i - r * per;
                                if (j < GQ * HD) sh.qs[(r * GQ + j / HD) * PST + j % HD] = vals[u];
                                else if (j < GQ * HD + HD) sh.kn[r * HD + (j - GQ * HD)] = vals[u];
                                else sh.vn[r * HD + (j - GQ * HD - HD)] = vals[u];
                            }
                        }
                    } else {
                        sh.flag[0] = 1;
                    }
                }
                // the cached keys and values into LDS (zero past the cached positions)
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int i = tid + u * NTHR, o = i >> 4, d = (i & 15) * 4;
                    float4 kx = kk[u], vx = vv[u];
                    if (p0 + o >= pc1) kx = vx = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    *(float4*)&sh.ks[o * PST + d] = kx;
                    *(float4*)&sh.vs[o * PST + d] = vx;
                }
                __syncthreads();
                if (sh.flag[0]) {
                    ok = false;
                    break;
                }
                // RoPE (rotate-half, src/model.rs:451-459) of the queries at their row's position
                if (tid < Q * HALF) {
                    const int q = tid / HALF, d = tid - q * HALF;
                    const float x1 = sh.qs[q * PST + d], x2 = sh.qs[q * PST + d + HALF];
                    sh.qs[q * PST + d] = __fadd_rn(__fmul_rn(x1, rq_c), __fmul_rn(-x2, rq_s));
                    sh.qs[q * PST + d + HALF] = __fadd_rn(__fmul_rn(x2, rq_c), __fmul_rn(x1, rq_s));
                }
                // new rows inside this span: the rotated key and the value into LDS and
                // into their cache slot (KvCache::write, src/kv.rs:48-56)
                if (tid < t * HALF) {
                    const int r = tid / HALF, d = tid - r * HALF, pos = pos0 + r;
                    const float c = rk_c, sn = rk_s;
                    if (pos >= p0 && pos < p1) {
                    const float x1 = sh.kn[r * HD + d], x2 = sh.kn[r * HD + d + HALF];
                    const float k1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(-x2, sn));
                    const float k2 = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, sn));
                    const float v1 = sh.vn[r * HD + d], v2 = sh.vn[r * HD + d + HALF];
                    const int o = pos - p0;
                    sh.ks[o * PST + d] = k1;
                    sh.ks[o * PST + d + HALF] = k2;
                    sh.vs[o * PST + d] = v1;
                    sh.vs[o * PST + d + HALF] = v2;
                    const size_t at = (((size_t)(uint32_t)a.blocks[pos >> 4] * nkv + h) * 16 + (pos & 15)) * HD;
                    kc[at + d] = k1;
                    kc[at + d + HALF] = k2;
                    vc[at + d] = v1;
                    vc[at + d + HALF] = v2;
                    }
                }
                __syncthreads();
                // one query per wave pass: position p0 + lane in lane `lane`, scores,
                // their max and sum of exponentials, then the weighted values (dim = lane)
                for (int q = wave; q < Q; q += NW) {
                    const int r = q / GQ, lim = pos0 + r;
                    float sc = -INFINITY;
                    if (lane < np && p0 + lane <= lim) {
                        const float4* kr = (const float4*)&sh.ks[lane * PST];
                        const float4* qr = (const float4*)&sh.qs[q * PST];
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
                    const float mx = group_reduce<64, true>(sc);
                    const float e = sc == -INFINITY ? 0.0f : dev_exp(sc - mx);
                    const float sum = group_reduce<64, false>(e);
                    // the weights through this wave's LDS row (read back as broadcasts)
                    float* ew = sh.red + wave * 64;
                    ew[lane] = e;
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    // all 64 rows: weights past np are 0 and those value rows are zeroed
                    float ov = 0.0f;
#pragma unroll
                    for (int p4 = 0; p4 < 16; p4++) {
                        const float4 w4 = *(const float4*)&ew[p4 * 4];
                        ov = fmaf(w4.x, sh.vs[(p4 * 4 + 0) * PST + lane], ov);
                        ov = fmaf(w4.y, sh.vs[(p4 * 4 + 1) * PST + lane], ov);
                        ov = fmaf(w4.z, sh.vs[(p4 * 4 + 2) * PST + lane], ov);
                        ov = fmaf(w4.w, sh.vs[(p4 * 4 + 3) * PST + lane], ov);
                    }
                    uint64_t* dst = a.part + (((size_t)item * kPdMaxRows + r) * GQ + (q - r * GQ)) * PSZ;
                    ll_put(dst + lane, ov, tout);
                    if (lane == 0) {
                        ll_put(dst + HD, mx, tout);
                        ll_put(dst + HD + 1, sum, tout);
                    }
                }
                __syncthreads();
            }
        }
        if (!ok) break;
        // ---- merge: items (row r, query head qh), one per workgroup; wave w takes
        // the spans w, w + 8, ... (all their words in flight at once), the waves'
        // results are merged in wave order
        {
            const unsigned tin = make_tag(epoch, s0 + 1), tout = make_tag(epoch, s0 + 2);
            for (int it = wg; it < t * nh && ok; it += G) {
                const int r = it / nh, qh = it - r * nh, h = qh / GQ, j = qh - h * GQ;
                float M = -INFINITY, L = 0.0f, O = 0.0f;
                bool wok = true;
                for (int sp0 = wave; sp0 < S && wok; sp0 += NW * MSP) {
                    uint64_t wm[MSP], wl[MSP], wo[MSP];
                    const int n = min(MSP, (S - sp0 + NW - 1) / NW);
                    int spins = 0;
                    while (true) {
                        bool ready = true;
#pragma unroll
                        for (int u = 0; u < MSP; u++)
                            if (u < n) {
                                const uint64_t* src =
                                    a.part + (((size_t)(h * S + sp0 + u * NW) * kPdMaxRows + r) * GQ + j) * PSZ;
                                wm[u] = ll_get(src + HD);
                                wl[u] = ll_get(src + HD + 1);
                                wo[u] = ll_get(src + lane);
                                ready &= ll_ready(wm[u], tin) && ll_ready(wl[u], tin) && ll_ready(wo[u], tin);
                            }
                        if (__all(ready)) break;
                        if (!keep_waiting(spins, spin, ctl)) {
                            wok = false;
                            break;
                        }
                    }
#pragma unroll
                    for (int u = 0; u < MSP; u++) {
                        if (!wok || u >= n) break;
                        const float m = ll_val(wm[u]);
                        if (m == -INFINITY) continue;  // a span this row does not reach
                        const float nM = fmaxf(M, m);
                        const float fo = M == -INFINITY ? 0.0f : dev_exp(M - nM), fn = dev_exp(m - nM);
                        L = fmaf(ll_val(wl[u]), fn, L * fo);
                        O = fmaf(ll_val(wo[u]), fn, O * fo);
                        M = nM;
                    }
                }
                // the waves' (M, L, O) through LDS, merged by wave 0 in wave order
                if (tid == 0) sh.flag[1] = 0;
                sh.red[wave * (HD + 2) + 2 + lane] = O;
                if (lane == 0) {
                    sh.red[wave * (HD + 2)] = M;
                    sh.red[wave * (HD + 2) + 1] = L;
                }
                __syncthreads();
                if (!wok && lane == 0) sh.flag[1] = 1;
                __syncthreads();
                if (sh.flag[1]) {
                    ok = false;
                    break;
                }
                if (wave == 0) {
                    float M2 = -INFINITY, L2 = 0.0f, O2 = 0.0f;
                    for (int w = 0; w < NW; w++) {
                        const float m = sh.red[w * (HD + 2)];
                        if (m == -INFINITY) continue;
                        const float nM = fmaxf(M2, m);
                        const float fo = M2 == -INFINITY ? 0.0f : dev_exp(M2 - nM), fn = dev_exp(m - nM);
                        L2 = fmaf(sh.red[w * (HD + 2) + 1], fn, L2 * fo);
                        O2 = fmaf(sh.red[w * (HD + 2) + 2 + lane], fn, O2 * fo);
                        M2 = nM;
                    }
                    ll_put(a.att + (size_t)r * qd + qh * HD + lane, O2 / L2, tout);
                }
                __syncthreads();
            }
        }
        if (!ok) break;
        // ---- o projection and residual: x_a = x_b + att W_o^T (tile wg; x_b of
        // the tile is this workgroup's own, in xres)
        if (wg < H / 16) {
            const bf16x8* W = (const bf16x8*)Ly.wo;
            const int KB = Ly.o_kb, tile = wg;
            Ops<MAXB> o;
            load_ops<false, 1, MAXB>(W, KB, tile, 0, o);
            ok = fetch(a.att, t, qd, KB, make_tag(epoch, s0 + 2), nullptr, 0.0f, ctl, spin, sh);
            if (ok) {
                products<false, 1, MAXB>(W, KB, tile, sh, o);
                if (tid < 16 * t) {
                    xres = xres + sh.yt[(tid >> 4) * YTS + (tid & 15)];
                    ll_put(a.xa + (size_t)(tid >> 4) * H + tile * 16 + (tid & 15), xres, make_tag(epoch, s0 + 3));
                }
                __syncthreads();
            }
        }
        if (!ok) break;
        // ---- gate/up and SiLU: groups of two tiles [gate 16 channels | up 16 channels]
        {
            const bf16x8* W = (const bf16x8*)Ly.wgu;
            const int KB = Ly.gu_kb, ngroup = I / 16;
            const unsigned tin = make_tag(epoch, s0 + 3), tout = make_tag(epoch, s0 + 4);
            for (int gi = wg; gi < ngroup && ok; gi += G) {
                Ops<MAXB> o;
                load_ops<false, 2, MAXB>(W, KB, 2 * gi, 0, o);
                if (gi == wg) {
                    ok = fetch(a.xa, t, H, KB, tin, Ly.mlp_norm, a.eps, ctl, spin, sh);
                    if (!ok) break;
                }
                products<false, 2, MAXB>(W, KB, 2 * gi, sh, o);
                if (tid < 16 * t) {
                    const int r = tid >> 4, c = tid & 15;
                    const float gt = sh.yt[r * YTS + c] * sh.rs[4 + r], up = sh.yt[r * YTS + 16 + c] * sh.rs[4 + r];
                    ll_put(a.act + (size_t)r * I + gi * 16 + c, gt / (1.0f + dev_exp(-gt)) * up, tout);
                }
                __syncthreads();
            }
        }
        if (!ok) break;
        // ---- down projection and residual: x_b = x_a + act W_down^T (tile wg, as
        // the o projection: x_a of the tile is in xres)
        if (wg < H / 16) {
            const bf16x8* W = (const bf16x8*)Ly.wd;
            const int KB = Ly.d_kb, tile = wg;
            Ops<MAXB> o;
            load_ops<false, 1, MAXB>(W, KB, tile, 0, o);
            ok = fetch(a.act, t, I, KB, make_tag(epoch, s0 + 4), nullptr, 0.0f, ctl, spin, sh);
            if (ok) {
                products<false, 1, MAXB>(W, KB, tile, sh, o);
                if (tid < 16 * t) {
                    xres = xres + sh.yt[(tid >> 4) * YTS + (tid & 15)];
                    ll_put(a.xb + (size_t)(tid >> 4) * H + tile * 16 + (tid & 15), xres, make_tag(epoch, s0 + 5));
                }
                __syncthreads();
            }
        }
    }
    // ---- logits of the selected rows r0 .. t-1: final norm, lm_head tiles
    // 4 wg .. 4 wg + 3, then 4 (wg + G) ...; each workgroup's (max, first index) per row
    const int sl = 1 + 6 * a.L, r0 = t - a.logits_rows;
    if (ok) {
        const bf16x8* W = (const bf16x8*)a.lm;
        const int KB = a.lm_kb, ntile = a.V / 16;  // a multiple of 4 (the host admits V % 64 == 0)
        float bv = -INFINITY;  // wave r (< 4) keeps row r's best
        int bi = 0x7fffffff;
        bool fetched = false;
        for (int tile = 4 * wg; tile < ntile && ok; tile += 4 * G) {
            Ops<LMB> o;
            load_ops<true, 4, LMB>(W, KB, tile, 0, o);
            if (!fetched) {
                ok = fetch(a.xb, t, H, KB, make_tag(epoch, sl - 1), a.norm, a.eps, ctl, spin, sh);
                if (!ok) break;
                fetched = true;
            }
            products<true, 4, LMB>(W, KB, tile, sh, o);
            if (wave >= r0 && wave < t) {
                const int r = wave;
                float v = -INFINITY;
                int idx = 0x7fffffff;
                {
                    const float y = sh.yt[r * YTS + lane] * sh.rs[4 + r];
                    v = y != y ? -INFINITY : y;  // NaN never wins
                    idx = tile * 16 + lane;
                }
                for (int off = 32; off >= 1; off >>= 1) {
                    const float ov = __shfl_xor(v, off);
                    const int oi = __shfl_xor(idx, off);
                    if (ov > v || (ov == v && oi < idx)) {
                        v = ov;
                        idx = oi;
                    }
                }
                if (v > bv || (v == bv && idx < bi)) {
                    bv = v;
                    bi = idx;
                }
            }
            __syncthreads();
        }
        // every workgroup publishes, with or without columns of its own
        if (ok && wave >= r0 && wave < t && lane == 0) {
            const unsigned tag = make_tag(epoch, sl);
            uint64_t* dst = a.lmp + ((size_t)wg * kPdMaxRows + wave) * LINE;
            ll_put(dst, bv, tag);
            ll_put(dst + 1, __int_as_float(bi), tag);
        }
    }
    // ---- argmax over the workgroups (workgroup 0): row r in wave r, workgroups in lanes
    if (ok && wg == 0 && wave >= r0 && wave < t) {
        const int r = wave;
        const unsigned tag = make_tag(epoch, sl);
        float v = -INFINITY;
        int idx = 0x7fffffff;
        bool wok = true;
        for (int g0 = 0; g0 < G && wok; g0 += 64) {
            // lanes past the last workgroup read workgroup 0's words (ready when it is)
            const int gg = g0 + lane < G ? g0 + lane : 0;
            const uint64_t* src = a.lmp + ((size_t)gg * kPdMaxRows + r) * LINE;
            uint64_t wv, wi;
            int spins = 0;
            while (true) {
                wv = ll_get(src);
                wi = ll_get(src + 1);
                if (__all(ll_ready(wv, tag) && ll_ready(wi, tag))) break;
                if (!keep_waiting(spins, spin, ctl)) {
                    wok = false;
                    break;
                }
            }
            if (!wok) break;
            const float ov = ll_val(wv);
            const int oi = __float_as_int(ll_val(wi));
            if (ov > v || (ov == v && oi < idx)) {
                v = ov;
                idx = oi;
            }
        }
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(v, off);
            const int oi = __shfl_xor(idx, off);
            if (ov > v || (ov == v && oi < idx)) {
                v = ov;
                idx = oi;
            }
        }
        if (wok && lane == 0) {
            const uint32_t tok = idx == 0x7fffffff ? 0u : (uint32_t)idx;  // all NaN: index 0, as sampler::argmax
            a.am[r - r0] = tok;
            if (a.aux) a.aux[(size_t)(r - r0) * a.aux_stride + a.aux_off] = tok;
        }
    }
    // ---- the last workgroup to finish advances the epoch for the next launch
    __syncthreads();
    if (tid == 0) {
        const unsigned done = __hip_atomic_fetch_add(ctl + kPdCtlDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == (unsigned)G - 1) {
            __hip_atomic_store(ctl + kPdCtlDone, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctl + kPdCtlEpoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

PdSizes pdraft_sizes(int H, int I, int qd, int kvd, int nh, int nkv, int spans) {
    PdSizes s;
    const int R = kPdMaxRows;
    s.xa = (size_t)R * H;
    s.xb = (size_t)R * H;
    s.qkv = (size_t)R * (qd + 2 * kvd);
    s.att = (size_t)R * qd;
    s.act = (size_t)R * I;
    s.part = (size_t)nkv * spans * R * (nh / nkv) * PSZ;
    s.lmp = (size_t)kPdGroups * R * LINE;
    return s;
}

size_t pdraft_lds_bytes(int ap_kb) {
    return (size_t)ap_kb * 64 * 8 * sizeof(uint16_t) +
           ((size_t)2 * 64 * PST + 16 * PST + 2 * 4 * HD + 4 * NTHR + 4 * YTS + 8) * sizeof(float) + 4 * sizeof(int);
}

hipError_t pdraft_init() {
    const hipError_t e = hipFuncSetAttribute((const void*)k_pdraft, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)pdraft_lds_bytes(kPdMaxKb));
    if (e != hipSuccess) (void)hipGetLastError();  // not left behind for an unrelated call to report
    return e;
}

int pdraft_groups(int ap_kb) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_pdraft, NTHR, pdraft_lds_bytes(ap_kb)) != hipSuccess)
        return 0;
    return std::min(kPdGroups, cus * per);
}

void launch_pdraft(hipStream_t st, int groups, const PdArgs& a) {
    hipLaunchKernelGGL(k_pdraft, dim3(groups), dim3(NTHR), pdraft_lds_bytes(a.ap_kb), st, a);
}

}  // namespace fg
