// Sampling on the device (sampler::distribution / draw, src/sampler.rs:52-103)
// and the speculative step's sampling acceptance (Engine::execute,
// src/engine.rs:575-610): min(1, p/q) acceptance, residual resampling from
// max(0, p - q), the bonus draw; each sequence draws from its own generator
// (Rng, src/rng.rs), in the reference's order.
//
// A distribution of top_k 1..kSampleCap is at most kSampleCap (token,
// probability) pairs, stored twice per row: in the reference's order (value
// descending, token ascending; draws scan this order) and in token order (for
// lookups and the residual, which the reference builds in token order). A
// wide one (top_k 0, no limit, or above kSampleCap) keeps up to the whole
// vocabulary in the reference's order plus a dense by-token copy; its kernels
// (k_dist_wide, k_draw_wide, k_accept_wide) run after the small ones, each
// kind skipping the other's rows.
#include "internal.h"

#include <math.h>

namespace fg {

// f32::total_cmp as unsigned order
__device__ __forceinline__ uint32_t total_key(float x) {
    const uint32_t b = __float_as_uint(x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// exp rounded to f32 from a double-precision evaluation (within a few double
// ulps): the correctly rounded expf except when exp(x) lies within about
// 1e-9 relative of a rounding boundary
__device__ __forceinline__ float expf_rounded(float x) { return (float)exp((double)x); }

// Rng (src/rng.rs:12-34): xorshift64*, uniform with 53 bits
__device__ __forceinline__ uint64_t rng_next(uint64_t& s) {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1DULL;
}
__device__ __forceinline__ double rng_uniform(uint64_t& s) {
    return (double)(rng_next(s) >> 11) / 9007199254740992.0;
}

// In-place bitonic sort of n = 1024 64-bit keys in LDS, descending; every
// thread of the 1024-thread workgroup takes part.
__device__ void bitonic_desc(uint64_t* v) {
    const int i = threadIdx.x;
    for (int size = 2; size <= kSampleCap; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const int j = i ^ stride;
            if (j > i) {
                const bool desc = (i & size) == 0;
                const uint64_t a = v[i], b = v[j];
                if (desc ? a < b : a > b) {
                    v[i] = b;
                    v[j] = a;
                }
            }
            __syncthreads();
        }
}

// One workgroup of kSampleCap threads per logits row: the row's distribution
// (sampler::distribution). Rows of greedy sequences get n = 0.
__global__ __launch_bounds__(kSampleCap) void k_dist(const float* __restrict__ logits, int vocab, int rows_per_seq,
                                                     const SampleParams* __restrict__ prm, uint32_t* __restrict__ tok,
                                                     float* __restrict__ pr, uint32_t* __restrict__ tok_id,
                                                     float* __restrict__ pr_id, int* __restrict__ n_out, int cap) {
    __shared__ uint32_t hist[256];
    __shared__ int sel[2];
    __shared__ int scan[kSampleCap];
    __shared__ uint64_t ck[kSampleCap];
    __shared__ float ev[kSampleCap];
    __shared__ int cgt;
    __shared__ double dsum;
    __shared__ int keep_s;
    __shared__ float ssum;
    const int row = blockIdx.x, tid = threadIdx.x;
    const SampleParams p = prm[row / rows_per_seq];
    if (p.temperature <= 0.0f) {
        if (tid == 0) n_out[row] = 0;
        return;
    }
    if (sample_wide(p)) return;  // k_dist_wide
    const float* lg = logits + (size_t)row * vocab;
    const float t = p.temperature > 1e-5f ? p.temperature : 1e-5f;
    const int K = min(p.top_k, vocab);
    // (1) the K-th largest key, eight bits at a time
    uint32_t prefix = 0, mask = 0;
    int need = K;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (int i = tid; i < vocab; i += kSampleCap) {
            const uint32_t key = total_key(lg[i] / t);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            int cum = 0, d = 255;
            for (; d > 0; d--) {
                if (cum + (int)hist[d] >= need) break;
                cum += (int)hist[d];
            }
            sel[0] = d;
            sel[1] = cum;
        }
        __syncthreads();
        need -= sel[1];
        prefix |= (uint32_t)sel[0] << shift;
        mask |= 255u << shift;
        __syncthreads();
    }
    const uint32_t kth = prefix;  // need = elements equal to kth that make the top K
    // (2) gather: keys above kth in any order, then the first `need` equal
    // keys by token index (each thread scans a contiguous range; a block scan
    // ranks the ties)
    const int per = (vocab + kSampleCap - 1) / kSampleCap, i0 = tid * per, i1 = min(vocab, i0 + per);
    int ties = 0;
    for (int i = i0; i < i1; i++) ties += total_key(lg[i] / t) == kth;
    scan[tid] = ties;
    if (tid == 0) cgt = 0;
    ck[tid] = 0;
    __syncthreads();
    for (int off = 1; off < kSampleCap; off <<= 1) {
        const int v = tid >= off ? scan[tid - off] : 0;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    int rank = scan[tid] - ties;
    for (int i = i0; i < i1; i++) {
        const uint32_t key = total_key(lg[i] / t);
        // composite: value descending, then token ascending
        const uint64_t c = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)i;
        if (key > kth) {
            ck[atomicAdd(&cgt, 1)] = c;
        } else if (key == kth) {
            if (rank < need) ck[K - need + rank] = c;
            rank++;
        }
    }
    __syncthreads();
    // (3) the reference's order
    bitonic_desc(ck);
    // (4) exp(v - max) in f32, their f64 sum in order, probabilities
    const float mx = key_value((uint32_t)(ck[0] >> 32));
    if (tid < K) ev[tid] = expf_rounded(key_value((uint32_t)(ck[tid] >> 32)) - mx);
    __syncthreads();
    if (tid == 0) {
        double s = 0.0;
        for (int i = 0; i < K; i++) s += (double)ev[i];
        dsum = s;
    }
    __syncthreads();
    float pv = tid < K ? (float)((double)ev[tid] / dsum) : 0.0f;
    int n = K;
    if (p.top_p < 1.0f) {
        __syncthreads();
        if (tid < K) ev[tid] = pv;
        __syncthreads();
        if (tid == 0) {
            float acc = 0.0f;
            int keep = K;
            for (int i = 0; i < K; i++) {
                acc += ev[i];
                if (acc >= p.top_p) {
                    keep = i + 1;
                    break;
                }
            }
            float s2 = 0.0f;
            for (int i = 0; i < keep; i++) s2 += ev[i];
            keep_s = keep;
            ssum = s2;
        }
        __syncthreads();
        n = keep_s;
        pv = pv / ssum;
    }
    const size_t base = (size_t)row * cap;
    const uint32_t tk = ~(uint32_t)ck[tid];
    if (tid < n) {
        tok[base + tid] = tk;
        pr[base + tid] = pv;
    }
    if (tid == 0) n_out[row] = n;
    // (5) the same pairs in token order
    __syncthreads();
    ck[tid] = tid < n ? ((uint64_t)(0xFFFFFFFFu - tk) << 32) | __float_as_uint(pv) : 0;
    __syncthreads();
    bitonic_desc(ck);
    if (tid < n) {
        tok_id[base + tid] = 0xFFFFFFFFu - (uint32_t)(ck[tid] >> 32);
        pr_id[base + tid] = __uint_as_float((uint32_t)ck[tid]);
    }
}

// sampler::draw over n pairs (src/sampler.rs:93-103)
__device__ uint32_t draw_pairs(const uint32_t* tok, const float* pr, int n, uint64_t& rng) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += pr[i];
    float u = (float)rng_uniform(rng) * s;
    for (int i = 0; i < n; i++) {
        if (u < pr[i]) return tok[i];
        u -= pr[i];
    }
    return n > 0 ? tok[n - 1] : 0;
}

// probability of token t in a row's token-ordered pairs (0 if absent)
__device__ float lookup(const uint32_t* tok_id, const float* pr_id, int n, uint32_t t) {
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (tok_id[mid] < t)
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo < n && tok_id[lo] == t ? pr_id[lo] : 0.0f;
}

// One thread per row: sampler::sample of each sampled row's distribution
// into out[row * out_stride + out_off]; greedy rows keep what the argmax
// wrote there.
__global__ void k_draw(int rows, const SampleParams* __restrict__ prm, const uint32_t* __restrict__ tok,
                       const float* __restrict__ pr, const int* __restrict__ n, uint64_t* __restrict__ rng,
                       uint32_t* __restrict__ out, int out_stride, int out_off, int cap) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows || prm[r].temperature <= 0.0f || sample_wide(prm[r])) return;
    uint64_t s = rng[r];
    out[(size_t)r * out_stride + out_off] = draw_pairs(tok + (size_t)r * cap, pr + (size_t)r * cap, n[r], s);
    rng[r] = s;
}

// One thread per sequence: Engine::execute's verify of proposals d1..dk
// (vtok[s*(k+1) + 1 + j]) against target rows s*(k+1) + j, for sampled
// sequences (src/engine.rs:575-610) and greedy ones (:570-574, with the
// argmax of each verify row in am).
__global__ void k_accept_sampled(int n_seqs, int k, const SampleParams* __restrict__ prm,
                                 const uint32_t* __restrict__ vtok, const uint32_t* __restrict__ am,
                                 const uint32_t* __restrict__ p_tok, const float* __restrict__ p_pr,
                                 const uint32_t* __restrict__ p_tok_id, const float* __restrict__ p_pr_id,
                                 const int* __restrict__ p_n, const uint32_t* __restrict__ q_tok_id,
                                 const float* __restrict__ q_pr_id, const int* __restrict__ q_n,
                                 uint64_t* __restrict__ rng, uint32_t* __restrict__ out_tokens,
                                 int32_t* __restrict__ out_count, int32_t* __restrict__ out_accepted, int cap) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n_seqs || sample_wide(prm[s])) return;  // k_accept_wide
    const int K1 = k + 1;
    const bool greedy = prm[s].temperature <= 0.0f;
    uint64_t st = rng[s];
    int ne = 0, accepted = 0;
    uint32_t* out = out_tokens + (size_t)s * K1;
    for (int j = 0; j < k; j++) {
        const int row = s * K1 + j;
        const uint32_t d = vtok[(size_t)s * K1 + 1 + j];
        bool take_d;
        uint32_t t = 0;
        if (greedy) {
            t = am[row];
            take_d = t == d;
        } else {
            const size_t pb = (size_t)row * cap, qb = ((size_t)j * n_seqs + s) * cap;
            const int pn = p_n[row], qn = q_n[j * n_seqs + s];
            const float px = lookup(p_tok_id + pb, p_pr_id + pb, pn, d);
            const float qx = lookup(q_tok_id + qb, q_pr_id + qb, qn, d);
            take_d = qx > 0.0f && rng_uniform(st) < (double)fminf(px / qx, 1.0f);
            if (!take_d) {
                // the part of p that q under-covers, in token order
                float rs = 0.0f;
                int rc = 0;
                for (int i = 0; i < pn; i++) {
                    const float a = p_pr_id[pb + i], b = lookup(q_tok_id + qb, q_pr_id + qb, qn, p_tok_id[pb + i]);
                    if (a > b) {
                        rs += a - b;
                        rc++;
                    }
                }
                if (rc > 0) {
                    float u = (float)rng_uniform(st) * rs;
                    bool done = false;
                    for (int i = 0; i < pn && !done; i++) {
                        const float a = p_pr_id[pb + i], b = lookup(q_tok_id + qb, q_pr_id + qb, qn, p_tok_id[pb + i]);
                        if (a > b) {
                            t = p_tok_id[pb + i];  // the last residual token if u never falls below
                            if (u < a - b)
                                done = true;
                            else
                                u -= a - b;
                        }
                    }
                } else {
                    // dense_pairs(p): its positive entries in token order
                    float ps = 0.0f;
                    for (int i = 0; i < pn; i++)
                        if (p_pr_id[pb + i] > 0.0f) ps += p_pr_id[pb + i];
                    float u = (float)rng_uniform(st) * ps;
                    bool done = false;
                    for (int i = 0; i < pn && !done; i++) {
                        const float a = p_pr_id[pb + i];
                        if (a > 0.0f) {
                            t = p_tok_id[pb + i];
                            if (u < a)
                                done = true;
                            else
                                u -= a;
                        }
                    }
                }
            }
        }
        if (take_d) {
            out[ne++] = d;
            accepted++;
        } else {
            out[ne++] = t;
            break;
        }
    }
    if (accepted == k) {
        const int row = s * K1 + k;
        if (greedy) {
            out[ne++] = am[row];
        } else {
            const size_t pb = (size_t)row * cap;
            out[ne++] = draw_pairs(p_tok + pb, p_pr + pb, p_n[row], st);
        }
    }
    out_count[s] = ne;
    out_accepted[s] = accepted;
    rng[s] = st;
}

// ---------------------------------------------------------------------------
// Wide distributions: top_k = 0 (no limit) or above kSampleCap. A row holds up
// to `cap` (the vocabulary) pairs, in the reference's order, plus a dense
// token-indexed copy of the probabilities (0 where a token is not kept) for
// the acceptance's lookups and residual. One workgroup per row or sequence.
// The reference's sums and walks are sequential (f64 softmax sum, f32 top-p
// prefix, f32 draw sums): one thread runs them in order over values the
// whole workgroup stages in LDS, BATCH at a time.
// ---------------------------------------------------------------------------
constexpr int kWideThreads = 1024;

// Stable LSD radix sort of n (key, value) pairs, ascending by key, four 8-bit
// passes through global ping-pong buffers (k0/v0 -> k1/v1 -> k0/v0 ...; the
// result ends in k0/v0). Each 1024-element tile ranks its elements by digit
// with wave ballots (equal digits keep element order), then scatters after
// the digit's running offset.
__device__ void radix_sort_wide(uint32_t* k0, uint32_t* v0, uint32_t* k1, uint32_t* v1, int n) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t wcnt[kWideThreads / 64][256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t below = (1ull << lane) - 1;
    for (int i = tid; i < (kWideThreads / 64) * 256; i += kWideThreads) (&wcnt[0][0])[i] = 0;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 8 * pass;
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += kWideThreads) atomicAdd(&hist[(k0[i] >> shift) & 255u], 1u);
        __syncthreads();
        if (tid == 0) {
            uint32_t run = 0;
            for (int d = 0; d < 256; d++) {
                const uint32_t c = hist[d];
                hist[d] = run;
                run += c;
            }
        }
        __syncthreads();
        for (int t0 = 0; t0 < n; t0 += kWideThreads) {
            const int i = t0 + tid;
            const bool valid = i < n;
            const uint32_t key = valid ? k0[i] : 0u, val = valid ? v0[i] : 0u;
            const uint32_t d = (key >> shift) & 255u;
            uint64_t m = __ballot(valid);
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const uint64_t bb = __ballot((d >> b) & 1u);
                m &= ((d >> b) & 1u) ? bb : ~bb;
            }
            const int rank = __popcll(m & below);
            if (valid && rank == 0) wcnt[wave][d] = __popcll(m);
            __syncthreads();
            if (tid < 256) {
                uint32_t run = hist[tid];
                for (int w = 0; w < kWideThreads / 64; w++) {
                    const uint32_t c = wcnt[w][tid];
                    wcnt[w][tid] = run;
                    run += c;
                }
                hist[tid] = run;
            }
            __syncthreads();
            if (valid) {
                const uint32_t dst = wcnt[wave][d] + rank;
                k1[dst] = key;
                v1[dst] = val;
            }
            __syncthreads();
            for (int z = tid; z < (kWideThreads / 64) * 256; z += kWideThreads) (&wcnt[0][0])[z] = 0;
            __syncthreads();
        }
        uint32_t* tk = k0;
        k0 = k1;
        k1 = tk;
        uint32_t* tv = v0;
        v0 = v1;
        v1 = tv;
    }
}

// Thread 0 visits v(i) for i = 0, 1, ... < n in order: the workgroup stages
// BATCH values at a time in LDS (`stage`); visit(i, value) returns true to
// stop. Every thread of the workgroup must call it.
template <int BATCH, class Value, class Visit>
__device__ void ordered_scan(int n, float* stage, Value value, Visit visit) {
    __shared__ int stop;
    if (threadIdx.x == 0) stop = 0;
    for (int i0 = 0; i0 < n; i0 += BATCH) {
        __syncthreads();
        for (int i = threadIdx.x; i < BATCH; i += blockDim.x) stage[i] = i0 + i < n ? value(i0 + i) : 0.0f;
        __syncthreads();
        if (threadIdx.x == 0)
            for (int i = 0; i < BATCH && i0 + i < n; i++)
                if (visit(i0 + i, stage[i])) {
                    stop = 1;
                    break;
                }
        __syncthreads();
        if (stop) break;
    }
    __syncthreads();
}

// sampler::distribution for rows whose top_k is 0 or above kSampleCap (other
// rows are k_dist's): the keys sorted by value descending and token ascending
// (a stable ascending sort of the complemented keys in token order), exp(v -
// max) for the top K, their f64 sum in that order, probabilities, the top-p
// prefix; the pairs in that order (tok, pr) and the dense copy.
__global__ __launch_bounds__(kWideThreads) void k_dist_wide(const float* __restrict__ logits, int vocab,
                                                            int rows_per_seq, const SampleParams* __restrict__ prm,
                                                            SampleRows d) {
    __shared__ float stage[kWideThreads];
    __shared__ double dsum_s;
    __shared__ int keep_s;
    __shared__ float s2_s;
    const int row = blockIdx.x, tid = threadIdx.x;
    const SampleParams p = prm[row / rows_per_seq];
    if (!sample_wide(p)) return;  // greedy rows and small top_k rows: k_dist
    const size_t base = (size_t)row * d.cap;
    const float* lg = logits + (size_t)row * vocab;
    const float t = p.temperature > 1e-5f ? p.temperature : 1e-5f;
    const int K = p.top_k == 0 ? vocab : min(p.top_k, vocab);
    uint32_t* k0 = d.scratch + (size_t)row * d.cap * 4;
    uint32_t *v0 = k0 + d.cap, *k1 = v0 + d.cap, *v1 = k1 + d.cap;
    for (int i = tid; i < vocab; i += kWideThreads) {
        k0[i] = ~total_key(lg[i] / t);
        v0[i] = (uint32_t)i;
    }
    __syncthreads();
    radix_sort_wide(k0, v0, k1, v1, vocab);
    float* pr = d.pr + base;
    uint32_t* tok = d.tok + base;
    const float mx = key_value(~k0[0]);
    for (int i = tid; i < K; i += kWideThreads) pr[i] = expf_rounded(key_value(~k0[i]) - mx);
    __syncthreads();
    // the f64 sum in the reference's order
    {
        double sum = 0.0;
        ordered_scan<kWideThreads>(K, stage, [&](int i) { return pr[i]; }, [&](int, float e) {
            sum += (double)e;
            return false;
        });
        if (tid == 0) dsum_s = sum;
        __syncthreads();
    }
    const double dsum = dsum_s;
    for (int i = tid; i < K; i += kWideThreads) pr[i] = (float)((double)pr[i] / dsum);
    __syncthreads();
    int n = K;
    if (p.top_p < 1.0f) {
        int keep = K;
        float acc = 0.0f;
        ordered_scan<kWideThreads>(K, stage, [&](int i) { return pr[i]; }, [&](int i, float v) {
            acc += v;
            if (acc >= p.top_p) {
                keep = i + 1;
                return true;
            }
            return false;
        });
        if (tid == 0) keep_s = keep;
        __syncthreads();
        n = keep_s;
        float s2 = 0.0f;
        ordered_scan<kWideThreads>(n, stage, [&](int i) { return pr[i]; }, [&](int, float v) {
            s2 += v;
            return false;
        });
        if (tid == 0) s2_s = s2;
        __syncthreads();
        const float ss = s2_s;
        for (int i = tid; i < n; i += kWideThreads) pr[i] = pr[i] / ss;
    }
    float* dense = d.dense + base;
    for (int i = tid; i < vocab; i += kWideThreads) dense[i] = 0.0f;
    __syncthreads();
    for (int i = tid; i < n; i += kWideThreads) {
        tok[i] = v0[i];
        dense[v0[i]] = pr[i];
    }
    if (tid == 0) d.n[row] = n;
}

// sampler::draw over a wide row's n pairs, on the workgroup; thread 0 holds
// the generator. Returns the token on thread 0.
__device__ uint32_t draw_wide(const uint32_t* tok, const float* pr, int n, uint64_t& rng, float* stage) {
    float s = 0.0f;
    ordered_scan<256>(n, stage, [&](int i) { return pr[i]; }, [&](int, float v) {
        s += v;
        return false;
    });
    uint32_t out = n > 0 ? tok[n - 1] : 0;
    if (threadIdx.x == 0) {
        float u = (float)rng_uniform(rng) * s;
        // the walk: thread 0 keeps u; staged like the sum
        stage[256] = u;
    }
    float u = 0.0f;
    if (threadIdx.x == 0) u = stage[256];
    ordered_scan<256>(n, stage, [&](int i) { return pr[i]; }, [&](int i, float v) {
        if (u < v) {
            out = tok[i];
            return true;
        }
        u -= v;
        return false;
    });
    return out;
}

// One workgroup per row: sampler::sample of each wide sampled row into
// out[row * out_stride + out_off].
__global__ __launch_bounds__(256) void k_draw_wide(int rows, const SampleParams* __restrict__ prm, SampleRows d,
                                                   uint64_t* __restrict__ rng, uint32_t* __restrict__ out,
                                                   int out_stride, int out_off) {
    __shared__ float stage[257];
    const int r = blockIdx.x;
    const SampleParams p = prm[r];
    if (!sample_wide(p)) return;
    uint64_t s = rng[r];
    const size_t base = (size_t)r * d.cap;
    const uint32_t t = draw_wide(d.tok + base, d.pr + base, d.n[r], s, stage);
    if (threadIdx.x == 0) {
        out[(size_t)r * out_stride + out_off] = t;
        rng[r] = s;
    }
}

// One workgroup per sequence: k_accept_sampled's rule for sequences whose
// distributions are wide (dense lookups; the residual max(0, p - q) and the
// dense pairs of p in token order over the whole vocabulary).
__global__ __launch_bounds__(256) void k_accept_wide(int n_seqs, int k, int vocab, const SampleParams* __restrict__ prm,
                                                     const uint32_t* __restrict__ vtok,
                                                     const uint32_t* __restrict__ am, SampleRows p, SampleRows q,
                                                     uint64_t* __restrict__ rng, uint32_t* __restrict__ out_tokens,
                                                     int32_t* __restrict__ out_count,
                                                     int32_t* __restrict__ out_accepted) {
    __shared__ float stage[257];
    __shared__ int take_s;
    const int sq = blockIdx.x;
    const SampleParams pp = prm[sq];
    if (!sample_wide(pp)) return;
    const int K1 = k + 1;
    uint64_t st = rng[sq];
    int ne = 0, accepted = 0;
    uint32_t* out = out_tokens + (size_t)sq * K1;
    for (int j = 0; j < k; j++) {
        const int row = sq * K1 + j;
        const uint32_t dtok = vtok[(size_t)sq * K1 + 1 + j];
        const float* pd = p.dense + (size_t)row * p.cap;
        const float* qd = q.dense + ((size_t)j * n_seqs + sq) * q.cap;
        if (threadIdx.x == 0) {
            const float px = pd[dtok], qx = qd[dtok];
            take_s = qx > 0.0f && rng_uniform(st) < (double)fminf(px / qx, 1.0f);
        }
        __syncthreads();
        const bool take = take_s;
        __syncthreads();
        if (take) {
            if (threadIdx.x == 0) out[ne] = dtok;
            ne++;
            accepted++;
            continue;
        }
        // the part of p that q under-covers, in token order
        float rs = 0.0f;
        int rc = 0;
        ordered_scan<256>(vocab, stage, [&](int i) { return pd[i] > qd[i] ? pd[i] - qd[i] : 0.0f; },
                          [&](int i, float v) {
                              if (pd[i] > qd[i]) {
                                  rs += v;
                                  rc++;
                              }
                              return false;
                          });
        if (threadIdx.x == 0) stage[256] = (float)rc;
        __syncthreads();
        const bool any = stage[256] > 0.0f;
        __syncthreads();
        uint32_t t = 0;
        float u = 0.0f;
        if (any) {
            if (threadIdx.x == 0) u = (float)rng_uniform(st) * rs;
            ordered_scan<256>(vocab, stage, [&](int i) { return pd[i] > qd[i] ? pd[i] - qd[i] : 0.0f; },
                              [&](int i, float v) {
                                  if (pd[i] > qd[i]) {
                                      t = (uint32_t)i;  // the last residual token if u never falls below
                                      if (u < v) return true;
                                      u -= v;
                                  }
                                  return false;
                              });
        } else {
            // dense_pairs(p): its positive entries in token order
            float ps = 0.0f;
            ordered_scan<256>(vocab, stage, [&](int i) { return pd[i]; }, [&](int, float v) {
                if (v > 0.0f) ps += v;
                return false;
            });
            if (threadIdx.x == 0) u = (float)rng_uniform(st) * ps;
            ordered_scan<256>(vocab, stage, [&](int i) { return pd[i]; }, [&](int i, float v) {
                if (v > 0.0f) {
                    t = (uint32_t)i;
                    if (u < v) return true;
                    u -= v;
                }
                return false;
            });
        }
        if (threadIdx.x == 0) out[ne] = t;
        ne++;
        break;
    }
    if (accepted == k) {
        const int row = sq * K1 + k;
        const size_t pb = (size_t)row * p.cap;
        const uint32_t t = draw_wide(p.tok + pb, p.pr + pb, p.n[row], st, stage);
        if (threadIdx.x == 0) out[ne] = t;
        ne++;
    }
    if (threadIdx.x == 0) {
        out_count[sq] = ne;
        out_accepted[sq] = accepted;
        rng[sq] = st;
    }
}

void launch_dist(hipStream_t st, const float* logits, int rows, int vocab, int rows_per_seq, const SampleParams* prm,
                 SampleRows& out) {
    if (rows <= 0) return;
    hipLaunchKernelGGL(k_dist, dim3(rows), dim3(kSampleCap), 0, st, logits, vocab, rows_per_seq, prm, out.tok, out.pr,
                       out.tok_id, out.pr_id, out.n, out.cap);
    if (out.dense) hipLaunchKernelGGL(k_dist_wide, dim3(rows), dim3(kWideThreads), 0, st, logits, vocab, rows_per_seq,
                                      prm, out);
}

void launch_draw(hipStream_t st, int rows, const SampleParams* prm, const SampleRows& d, uint64_t* rng, uint32_t* out,
                 int out_stride, int out_off) {
    if (rows <= 0) return;
    hipLaunchKernelGGL(k_draw, dim3((rows + 63) / 64), dim3(64), 0, st, rows, prm, d.tok, d.pr, d.n, rng, out,
                       out_stride, out_off, d.cap);
    if (d.dense) hipLaunchKernelGGL(k_draw_wide, dim3(rows), dim3(256), 0, st, rows, prm, d, rng, out, out_stride, out_off);
}

void launch_accept_sampled(hipStream_t st, int n_seqs, int k, const SampleParams* prm, const uint32_t* vtok,
                           const uint32_t* am, const SampleRows& p, const SampleRows& q, uint64_t* rng,
                           uint32_t* out_tokens, int32_t* out_count, int32_t* out_accepted) {
    hipLaunchKernelGGL(k_accept_sampled, dim3((n_seqs + 63) / 64), dim3(64), 0, st, n_seqs, k, prm, vtok, am, p.tok,
                       p.pr, p.tok_id, p.pr_id, p.n, q.tok_id, q.pr_id, q.n, rng, out_tokens, out_count,
                       out_accepted, p.cap);
    if (p.dense)
        hipLaunchKernelGGL(k_accept_wide, dim3(n_seqs), dim3(256), 0, st, n_seqs, k, p.vocab, prm, vtok, am, p, q, rng,
                           out_tokens, out_count, out_accepted);
}

}  // namespace fg
