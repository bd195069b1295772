/*
 * CPU oracle for the ferrolm speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the
 * timed CPU baseline. Not linked into, loaded by or called from the
 * product library. See ferro_oracle.h for the contract.
 *
 * A restatement of the reference's CPU algorithm (Rust). Each definition
 * names the reference function it follows as file:line in
 * /root/reference. Compile with -ffp-contract=off: every fused
 * multiply-add below is an explicit fmaf(), exactly where the reference
 * uses mul_add or an FMA intrinsic, and nothing else is contracted.
 *
 * Storage differs from the reference where it does not change a single
 * rounding: bf16 matrices are packed in 32-row panels in natural column
 * order (the reference permutes columns inside a panel only so its SIMD
 * unpack lands in order, src/kernels.rs:27-36); quantized matrices keep
 * the reference's QMatrix layout byte for byte (src/quant.rs:70-76).
 */
#include "ferro_oracle.h"

#include <float.h>
#include <math.h>
#include <omp.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define PANEL 32
#define GROUP 32

#if defined(__x86_64__)
#define HOT __attribute__((target_clones("avx512f", "arch=haswell", "default")))
#else
#define HOT
#endif

/* ------------------------------------------------------------------ */
/* rng: src/rng.rs:8-44 (xorshift64*, Box-Muller)                      */
/* ------------------------------------------------------------------ */
uint64_t or_rng_new(uint64_t seed) { return (seed * 0x9E3779B97F4A7C15ULL) | 1ULL; }

uint64_t or_rng_next(uint64_t* s) {
    *s ^= *s >> 12;
    *s ^= *s << 25;
    *s ^= *s >> 27;
    return *s * 0x2545F4914F6CDD1DULL;
}

double or_rng_uniform(uint64_t* s) {
    return (double)(or_rng_next(s) >> 11) / (double)(1ULL << 53);
}

double or_rng_normal(uint64_t* s) {
    double u = 1.0 - or_rng_uniform(s);
    double v = or_rng_uniform(s);
    return sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v);
}

/* ------------------------------------------------------------------ */
/* bf16: src/safetensors.rs:166-178                                    */
/* ------------------------------------------------------------------ */
static inline float bf16f(uint16_t x) {
    uint32_t b = (uint32_t)x << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

float or_bf16_to_f32(uint16_t x) { return bf16f(x); }

uint16_t or_f32_to_bf16(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    if (isnan(x)) return (uint16_t)((b >> 16) | 0x40);
    uint32_t round = 0x7FFF + ((b >> 16) & 1);
    return (uint16_t)((b + round) >> 16);
}

/* n > 0: use n threads; n <= 0: all available processors. */
void or_set_threads(int32_t n) { omp_set_num_threads(n > 0 ? n : omp_get_num_procs()); }

/* ------------------------------------------------------------------ */
/* dot / hsum8: src/kernels.rs:191-213 (8 lanes, fixed lane sum)       */
/* ------------------------------------------------------------------ */
static inline float hsum8(const float* l) {
    return ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
}

float or_dot(const float* a, const float* b, int32_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int32_t i = 0; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    return hsum8(acc);
}

/* rms_norm: src/kernels.rs:597-607 */
void or_rms_norm(const float* x, const float* w, int32_t dim, int32_t rows, float eps, float* out) {
    for (int32_t r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * dim;
        float* o = out + (size_t)r * dim;
        float ms = or_dot(xr, xr, dim) / (float)dim;
        float rr = 1.0f / sqrtf(ms + eps);
        for (int32_t i = 0; i < dim; i++) o[i] = w[i] * (xr[i] * rr);
    }
}

/* exp: src/kernels.rs:609-637 (range reduction + Cephes polynomial) */
static const float LOG2E = 1.44269504088896340736f;
static const float LN2_HI = 0.6933594f;
static const float LN2_LO = -2.1219444e-4f;
static const float EXP_C[6] = {1.9875691e-4f, 1.3982e-3f, 8.333452e-3f,
                               4.1665796e-2f, 0.16666665f, 0.5f};

float or_exp(float x) {
    /* f32::clamp: NaN passes through */
    if (x < -87.0f) x = -87.0f;
    if (x > 88.0f) x = 88.0f;
    float n = rintf(x * LOG2E); /* round_ties_even in the default mode */
    float r = fmaf(n, -LN2_LO, fmaf(n, -LN2_HI, x));
    float p = EXP_C[0];
    for (int i = 1; i < 6; i++) p = fmaf(p, r, EXP_C[i]);
    float y = fmaf(p, r * r, r) + 1.0f;
    int32_t e = ((int32_t)n + 127) << 23;
    float scale;
    memcpy(&scale, &e, 4);
    return y * scale;
}

/* silu_mul: src/kernels.rs:650-663 */
void or_silu_mul(const float* gate_up, int32_t inter, int32_t rows, float* out) {
    for (int32_t r = 0; r < rows; r++) {
        const float* g = gate_up + (size_t)r * 2 * inter;
        const float* u = g + inter;
        float* o = out + (size_t)r * inter;
        for (int32_t i = 0; i < inter; i++) {
            float e = or_exp(-g[i]);
            o[i] = g[i] / (1.0f + e) * u[i];
        }
    }
}

/* argmax: src/sampler.rs:41-51 (first index of the maximum; NaN never wins) */
uint32_t or_argmax(const float* v, int32_t n) {
    int32_t best = 0;
    for (int32_t i = 0; i < n; i++)
        if (v[i] > v[best]) best = i;
    return (uint32_t)best;
}

/* Sampling (src/sampler.rs:52-103). Keys of f32::total_cmp: the float's bits
 * mapped so that unsigned order is the total order (NaNs at the ends). */
static inline uint32_t total_key(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
typedef struct {
    uint32_t t;
    float v;
} tok_val;
/* value descending by total_cmp, then token ascending (src/sampler.rs:58) */
static int cmp_desc(const void* a, const void* b) {
    const tok_val *x = (const tok_val*)a, *y = (const tok_val*)b;
    const uint32_t kx = total_key(x->v), ky = total_key(y->v);
    if (kx != ky) return kx > ky ? -1 : 1;
    return x->t < y->t ? -1 : (x->t > y->t);
}

/* sampler::distribution (src/sampler.rs:54-90): temperature, sort, top-k,
 * exp(v - max) in f32 summed in f64, normalise in f64 then round to f32;
 * top-p keeps the shortest prefix whose f32 running sum reaches top_p and
 * renormalises it by its f32 sum. Returns the pair count. */
int32_t or_distribution(const float* logits, int32_t vocab, float temperature, float top_p, int32_t top_k,
                        uint32_t* tok_out, float* p_out) {
    const float t = temperature > 1e-5f ? temperature : 1e-5f;
    tok_val* v = (tok_val*)malloc((size_t)vocab * sizeof(tok_val));
    for (int32_t i = 0; i < vocab; i++) {
        v[i].t = (uint32_t)i;
        v[i].v = logits[i] / t;
    }
    qsort(v, (size_t)vocab, sizeof(tok_val), cmp_desc);
    int32_t n = vocab;
    if (top_k > 0 && top_k < n) n = top_k;
    const float mx = v[0].v;
    double sum = 0.0;
    for (int32_t i = 0; i < n; i++) {
        v[i].v = expf(v[i].v - mx);
        sum += (double)v[i].v;
    }
    for (int32_t i = 0; i < n; i++) v[i].v = (float)((double)v[i].v / sum);
    if (top_p < 1.0f) {
        float acc = 0.0f;
        int32_t keep = n;
        for (int32_t i = 0; i < n; i++) {
            acc += v[i].v;
            if (acc >= top_p) {
                keep = i + 1;
                break;
            }
        }
        n = keep;
        float s2 = 0.0f;
        for (int32_t i = 0; i < n; i++) s2 += v[i].v;
        for (int32_t i = 0; i < n; i++) v[i].v /= s2;
    }
    for (int32_t i = 0; i < n; i++) {
        tok_out[i] = v[i].t;
        p_out[i] = v[i].v;
    }
    free(v);
    return n;
}

/* sampler::draw (src/sampler.rs:93-103): u in [0, f32 sum) scanned in order. */
uint32_t or_draw(const uint32_t* tok, const float* p, int32_t n, uint64_t* rng) {
    float s = 0.0f;
    for (int32_t i = 0; i < n; i++) s += p[i];
    float u = (float)or_rng_uniform(rng) * s;
    for (int32_t i = 0; i < n; i++) {
        if (u < p[i]) return tok[i];
        u -= p[i];
    }
    return n > 0 ? tok[n - 1] : 0;
}

/* ------------------------------------------------------------------ */
/* Matrices                                                            */
/* ------------------------------------------------------------------ */
typedef struct {
    int32_t kind, rows, cols;
    uint16_t* packed; /* bf16: [panel][k][32] */
    uint8_t* q;       /* QMatrix codes, reference layout */
    float* s;         /* QMatrix scales [panel][group][32] */
    int owns;
} omat;

static int32_t bytes_per_k(int32_t kind) { return kind == OR_INT8 ? PANEL : PANEL / 2; }

static int omat_init(omat* m, const or_matrix_desc* d) {
    memset(m, 0, sizeof(*m));
    m->kind = d->kind;
    m->rows = d->rows;
    m->cols = d->cols;
    m->owns = 1;
    if (d->rows % PANEL) return -1;
    size_t rc = (size_t)d->rows * d->cols;
    if (d->kind == OR_BF16) {
        m->packed = (uint16_t*)malloc(rc * 2);
        if (!m->packed) return -1;
        int32_t K = d->cols;
#pragma omp parallel for schedule(static)
        for (int32_t r = 0; r < d->rows; r++) {
            int32_t p = r / PANEL, c = r % PANEL;
            const uint16_t* row = d->bf16 + (size_t)r * K;
            uint16_t* dst = m->packed + (size_t)p * K * PANEL + c;
            for (int32_t k = 0; k < K; k++) dst[(size_t)k * PANEL] = row[k];
        }
    } else {
        if (d->cols % GROUP) return -1;
        size_t qb = (size_t)d->rows / PANEL * d->cols * bytes_per_k(d->kind);
        size_t sn = (size_t)d->rows / PANEL * (d->cols / GROUP) * PANEL;
        m->q = (uint8_t*)malloc(qb);
        m->s = (float*)malloc(sn * 4);
        if (!m->q || !m->s) return -1;
        memcpy(m->q, d->q, qb);
        memcpy(m->s, d->s, sn * 4);
    }
    return 0;
}

static void omat_free(omat* m) {
    if (!m->owns) return;
    free(m->packed);
    free(m->q);
    free(m->s);
    memset(m, 0, sizeof(*m));
}

/* Matrix::row_f32 / QMatrix::row_f32 (src/kernels.rs:121-130, src/quant.rs:145-168) */
static int32_t qcode(const uint8_t* q, int32_t kind, int32_t cols, int32_t r, int32_t k) {
    int32_t p = r / PANEL, c = r % PANEL;
    size_t base = ((size_t)p * cols + k) * bytes_per_k(kind);
    if (kind == OR_INT8) return (int32_t)(int8_t)q[base + c];
    uint8_t b = q[base + c % 16];
    return (int32_t)(c < 16 ? (b & 0x0F) : (b >> 4)) - 8;
}

static void omat_row_f32(const omat* m, int32_t r, float* out) {
    if (m->kind == OR_BF16) {
        int32_t p = r / PANEL, c = r % PANEL;
        const uint16_t* panel = m->packed + (size_t)p * m->cols * PANEL;
        for (int32_t k = 0; k < m->cols; k++) out[k] = bf16f(panel[(size_t)k * PANEL + c]);
    } else {
        int32_t G = m->cols / GROUP, p = r / PANEL, c = r % PANEL;
        for (int32_t k = 0; k < m->cols; k++)
            out[k] = (float)qcode(m->q, m->kind, m->cols, r, k) * m->s[((size_t)p * G + k / GROUP) * PANEL + c];
    }
}

void or_dequantize(int32_t kind, int32_t rows, int32_t cols, const uint8_t* q, const float* s, float* out) {
    int32_t G = cols / GROUP;
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) {
        int32_t p = r / PANEL, c = r % PANEL;
        for (int32_t k = 0; k < cols; k++)
            out[(size_t)r * cols + k] = (float)qcode(q, kind, cols, r, k) * s[((size_t)p * G + k / GROUP) * PANEL + c];
    }
}

/* QMatrix::quantize: src/quant.rs:78-143 */
static const float CLIPS8[6] = {1.0f, 0.98f, 0.96f, 0.94f, 0.92f, 0.9f};
static const float CLIPS4[11] = {1.0f, 0.95f, 0.9f, 0.85f, 0.8f, 0.75f, 0.7f, 0.65f, 0.6f, 0.55f, 0.5f};

int32_t or_quantize(int32_t kind, int32_t rows, int32_t cols, const float* w, const float* importance,
                    uint8_t* q, float* s) {
    if (kind == OR_BF16 || rows % PANEL || cols % GROUP) return -1;
    int32_t groups = cols / GROUP, bpk = bytes_per_k(kind);
    int32_t lo = kind == OR_INT8 ? -127 : -8, hi = kind == OR_INT8 ? 127 : 7;
    const float* clips = kind == OR_INT8 ? CLIPS8 : CLIPS4;
    int32_t nclips = kind == OR_INT8 ? 6 : 11;
    memset(q, 0, (size_t)rows / PANEL * cols * bpk);
    /* Panels are independent: each owns its bytes and scales. */
#pragma omp parallel for schedule(dynamic)
    for (int32_t p = 0; p < rows / PANEL; p++) {
        int32_t codes[GROUP], best_codes[GROUP];
        for (int32_t c = 0; c < PANEL; c++) {
            int32_t r = p * PANEL + c;
            for (int32_t g = 0; g < groups; g++) {
                const float* vals = w + (size_t)r * cols + (size_t)g * GROUP;
                const float* imp = importance ? importance + (size_t)g * GROUP : NULL;
                float amax = 0.0f;
                for (int i = 0; i < GROUP; i++) {
                    float a = fabsf(vals[i]);
                    amax = a > amax ? a : amax; /* f32::max, NaN ignored */
                }
                double best_err = INFINITY;
                float best_scale = 0.0f;
                if (amax > 0.0f) {
                    for (int32_t ci = 0; ci < nclips; ci++) {
                        float scale = clips[ci] * amax / (float)hi;
                        double err = 0.0;
                        for (int kk = 0; kk < GROUP; kk++) {
                            float v = vals[kk];
                            float t = roundf(v / scale); /* f32::round: half away from zero */
                            int32_t code = (int32_t)t;   /* in range: |v/scale| <= 1/0.5*7 */
                            if (code < lo) code = lo;
                            if (code > hi) code = hi;
                            codes[kk] = code;
                            double d = (double)(v - (float)code * scale);
                            err += d * d * (imp ? (double)imp[kk] : 1.0);
                        }
                        if (err < best_err) {
                            best_err = err;
                            best_scale = scale;
                            memcpy(best_codes, codes, sizeof(codes));
                        }
                    }
                } else {
                    memset(best_codes, 0, sizeof(best_codes));
                }
                s[((size_t)p * groups + g) * PANEL + c] = best_scale;
                for (int kk = 0; kk < GROUP; kk++) {
                    int32_t k = g * GROUP + kk, code = best_codes[kk];
                    size_t base = ((size_t)p * cols + k) * bpk;
                    if (kind == OR_INT8) {
                        q[base + c] = (uint8_t)(int8_t)code;
                    } else {
                        uint8_t nib = (uint8_t)(code + 8);
                        if (c < 16)
                            q[base + c] = (uint8_t)((q[base + c] & 0xF0) | nib);
                        else
                            q[base + c - 16] = (uint8_t)((q[base + c - 16] & 0x0F) | (nib << 4));
                    }
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* matmul: src/kernels.rs:244-376 (bf16) and src/quant.rs:175-304      */
/* Every output is one chain from zero, in order over k (bf16), or per */
/* group a chain over its 32 positions then fmaf(gs, scale, acc).      */
/* ------------------------------------------------------------------ */
HOT static void mm_bf16_panel(const float* x, int32_t m, int32_t K, const uint16_t* panel, float* y,
                              int32_t n, int32_t p) {
    int32_t i = 0;
    for (; i + 4 <= m; i += 4) {
        float a0[PANEL] = {0}, a1[PANEL] = {0}, a2[PANEL] = {0}, a3[PANEL] = {0};
        const float *x0 = x + (size_t)i * K, *x1 = x0 + K, *x2 = x1 + K, *x3 = x2 + K;
        for (int32_t k = 0; k < K; k++) {
            const uint16_t* w = panel + (size_t)k * PANEL;
            float wf[PANEL];
            for (int c = 0; c < PANEL; c++) wf[c] = bf16f(w[c]);
            float v0 = x0[k], v1 = x1[k], v2 = x2[k], v3 = x3[k];
            for (int c = 0; c < PANEL; c++) {
                a0[c] = fmaf(v0, wf[c], a0[c]);
                a1[c] = fmaf(v1, wf[c], a1[c]);
                a2[c] = fmaf(v2, wf[c], a2[c]);
                a3[c] = fmaf(v3, wf[c], a3[c]);
            }
        }
        memcpy(y + (size_t)(i + 0) * n + (size_t)p * PANEL, a0, sizeof(a0));
        memcpy(y + (size_t)(i + 1) * n + (size_t)p * PANEL, a1, sizeof(a1));
        memcpy(y + (size_t)(i + 2) * n + (size_t)p * PANEL, a2, sizeof(a2));
        memcpy(y + (size_t)(i + 3) * n + (size_t)p * PANEL, a3, sizeof(a3));
    }
    for (; i < m; i++) {
        float a0[PANEL] = {0};
        const float* x0 = x + (size_t)i * K;
        for (int32_t k = 0; k < K; k++) {
            const uint16_t* w = panel + (size_t)k * PANEL;
            float v0 = x0[k];
            for (int c = 0; c < PANEL; c++) a0[c] = fmaf(v0, bf16f(w[c]), a0[c]);
        }
        memcpy(y + (size_t)i * n + (size_t)p * PANEL, a0, sizeof(a0));
    }
}

static inline void load_codes(const uint8_t* q, int32_t kind, float* cf) {
    if (kind == OR_INT8) {
        for (int c = 0; c < PANEL; c++) cf[c] = (float)(int8_t)q[c];
    } else {
        for (int c = 0; c < 16; c++) {
            cf[c] = (float)((int32_t)(q[c] & 0x0F) - 8);
            cf[c + 16] = (float)((int32_t)(q[c] >> 4) - 8);
        }
    }
}

HOT static void mm_q_panel(const float* x, int32_t m, int32_t K, const uint8_t* qp, const float* sp,
                           int32_t kind, float* y, int32_t n, int32_t p) {
    int32_t bpk = bytes_per_k(kind), G = K / GROUP;
    int32_t i = 0;
    for (; i + 4 <= m; i += 4) {
        float a0[PANEL] = {0}, a1[PANEL] = {0}, a2[PANEL] = {0}, a3[PANEL] = {0};
        const float *x0 = x + (size_t)i * K, *x1 = x0 + K, *x2 = x1 + K, *x3 = x2 + K;
        for (int32_t g = 0; g < G; g++) {
            float g0[PANEL] = {0}, g1[PANEL] = {0}, g2[PANEL] = {0}, g3[PANEL] = {0};
            for (int32_t kk = g * GROUP; kk < (g + 1) * GROUP; kk++) {
                float cf[PANEL];
                load_codes(qp + (size_t)kk * bpk, kind, cf);
                float v0 = x0[kk], v1 = x1[kk], v2 = x2[kk], v3 = x3[kk];
                for (int c = 0; c < PANEL; c++) {
                    g0[c] = fmaf(v0, cf[c], g0[c]);
                    g1[c] = fmaf(v1, cf[c], g1[c]);
                    g2[c] = fmaf(v2, cf[c], g2[c]);
                    g3[c] = fmaf(v3, cf[c], g3[c]);
                }
            }
            const float* sc = sp + (size_t)g * PANEL;
            for (int c = 0; c < PANEL; c++) {
                a0[c] = fmaf(g0[c], sc[c], a0[c]);
                a1[c] = fmaf(g1[c], sc[c], a1[c]);
                a2[c] = fmaf(g2[c], sc[c], a2[c]);
                a3[c] = fmaf(g3[c], sc[c], a3[c]);
            }
        }
        memcpy(y + (size_t)(i + 0) * n + (size_t)p * PANEL, a0, sizeof(a0));
        memcpy(y + (size_t)(i + 1) * n + (size_t)p * PANEL, a1, sizeof(a1));
        memcpy(y + (size_t)(i + 2) * n + (size_t)p * PANEL, a2, sizeof(a2));
        memcpy(y + (size_t)(i + 3) * n + (size_t)p * PANEL, a3, sizeof(a3));
    }
    for (; i < m; i++) {
        float a0[PANEL] = {0};
        const float* x0 = x + (size_t)i * K;
        for (int32_t g = 0; g < G; g++) {
            float g0[PANEL] = {0};
            for (int32_t kk = g * GROUP; kk < (g + 1) * GROUP; kk++) {
                float cf[PANEL];
                load_codes(qp + (size_t)kk * bpk, kind, cf);
                float v0 = x0[kk];
                for (int c = 0; c < PANEL; c++) g0[c] = fmaf(v0, cf[c], g0[c]);
            }
            const float* sc = sp + (size_t)g * PANEL;
            for (int c = 0; c < PANEL; c++) a0[c] = fmaf(g0[c], sc[c], a0[c]);
        }
        memcpy(y + (size_t)i * n + (size_t)p * PANEL, a0, sizeof(a0));
    }
    (void)G;
}

/* ------------------------------------------------------------------ */
/* The CPU baseline's fast path (or_set_fast): the reference's register */
/* tiles (src/kernels.rs:279-289; AVX-512 tiles src/kernels.rs:378-430  */
/* and src/quant.rs:306-374) dispatched in panel ranges on a spinning   */
/* thread pool (src/pool.rs). Each output is the same chain of fused    */
/* multiply-adds as in the portable loops above, in the same order, so  */
/* the two agree bit for bit (tests/test_oracle.py holds them equal, as */
/* the reference's ISA-invariance test does, src/quant.rs:471-506).     */
/* ------------------------------------------------------------------ */
static int g_fast = 0;
static int32_t g_fast_threads = 0;

/* Pool: src/pool.rs:40-152. run(n, f) calls f(0..n) on the workers and the
 * calling thread; tasks are handed out from a shared counter, each writes a
 * fixed part of the output. Workers spin between jobs (a decode step
 * issues hundreds of small ones), then sleep on a condition variable. */
#define POOL_SPINS (1 << 16)
#define POOL_MAX 256
typedef void (*task_fn)(void* arg, int32_t task);
typedef struct {
    int32_t workers;
    pthread_t th[POOL_MAX];
    _Atomic uint64_t generation;
    task_fn fn;
    void* arg;
    _Atomic int32_t tasks, next, pending, shutdown;
    pthread_mutex_t lock;
    pthread_cond_t wake;
} spool;
static spool* g_pool = NULL;

static inline void cpu_relax(void) {
#if defined(__x86_64__)
    _mm_pause();
#endif
}

static void pool_drain(spool* s, task_fn fn, void* arg) {
    int32_t n = atomic_load_explicit(&s->tasks, memory_order_relaxed);
    for (;;) {
        int32_t i = atomic_fetch_add_explicit(&s->next, 1, memory_order_relaxed);
        if (i >= n) break;
        fn(arg, i);
    }
}

static void* pool_worker(void* p) {
    spool* s = (spool*)p;
    uint64_t seen = 0;
    for (;;) {
        int32_t spins = 0;
        while (atomic_load_explicit(&s->generation, memory_order_acquire) == seen &&
               !atomic_load_explicit(&s->shutdown, memory_order_relaxed)) {
            if (++spins < POOL_SPINS) {
                cpu_relax();
                continue;
            }
            pthread_mutex_lock(&s->lock);
            while (atomic_load_explicit(&s->generation, memory_order_acquire) == seen &&
                   !atomic_load_explicit(&s->shutdown, memory_order_relaxed))
                pthread_cond_wait(&s->wake, &s->lock);
            pthread_mutex_unlock(&s->lock);
        }
        if (atomic_load_explicit(&s->shutdown, memory_order_relaxed)) return NULL;
        seen = atomic_load_explicit(&s->generation, memory_order_acquire);
        pool_drain(s, s->fn, s->arg);
        atomic_fetch_sub_explicit(&s->pending, 1, memory_order_release);
    }
}

static void pool_stop(void) {
    if (!g_pool) return;
    spool* s = g_pool;
    atomic_store(&s->shutdown, 1);
    pthread_mutex_lock(&s->lock);
    pthread_cond_broadcast(&s->wake);
    pthread_mutex_unlock(&s->lock);
    for (int32_t i = 0; i < s->workers; i++) pthread_join(s->th[i], NULL);
    pthread_mutex_destroy(&s->lock);
    pthread_cond_destroy(&s->wake);
    free(s);
    g_pool = NULL;
}

/* A pool of `threads` threads in all, the caller included. */
static int pool_start(int32_t threads) {
    pool_stop();
    spool* s = (spool*)calloc(1, sizeof(spool));
    if (!s) return -1;
    pthread_mutex_init(&s->lock, NULL);
    pthread_cond_init(&s->wake, NULL);
    int32_t want = threads - 1 < POOL_MAX ? threads - 1 : POOL_MAX;
    for (int32_t i = 0; i < want; i++) {
        if (pthread_create(&s->th[i], NULL, pool_worker, s)) break;
        s->workers++;
    }
    g_pool = s;
    return 0;
}

static void pool_run(int32_t tasks, task_fn fn, void* arg) {
    if (tasks <= 0) return;
    spool* s = g_pool;
    if (tasks == 1 || !s || s->workers == 0) {
        for (int32_t i = 0; i < tasks; i++) fn(arg, i);
        return;
    }
    s->fn = fn;
    s->arg = arg;
    atomic_store_explicit(&s->tasks, tasks, memory_order_relaxed);
    atomic_store_explicit(&s->next, 0, memory_order_relaxed);
    atomic_store_explicit(&s->pending, s->workers, memory_order_relaxed);
    atomic_fetch_add_explicit(&s->generation, 1, memory_order_release);
    pthread_mutex_lock(&s->lock);
    pthread_cond_broadcast(&s->wake);
    pthread_mutex_unlock(&s->lock);
    pool_drain(s, fn, arg);
    int32_t spins = 0;
    while (atomic_load_explicit(&s->pending, memory_order_acquire) != 0) {
        if (++spins < POOL_SPINS)
            cpu_relax();
        else
            sched_yield();
    }
}

#if defined(__x86_64__)
#define AVX512 __attribute__((target("avx512f,avx512bw")))
#define AVX2 __attribute__((target("avx2,fma")))

/* One register tile of `mr` rows x `np` panels over kc inner positions,
 * starting from zero (init) or from the partial sums already in y. */
typedef struct {
    const float* x;
    int32_t xs;
    const uint16_t* w; /* bf16 panel data at (p0, k0) */
    const uint8_t* q;  /* quantized codes at (p0, k0) */
    const float* s;    /* group scales at (p0, k0 / GROUP) */
    size_t ws, qs, ss; /* strides between panels */
    int32_t kc, q4, init;
    float* y;
    int32_t ys;
} mtile;

/* bf16 tile: per output one chain over k from zero (src/kernels.rs:344-356). */
#define DEF_BTILE(MR, NP)                                                                      \
    AVX512 static void btile_##MR##_##NP(const mtile* t) {                                     \
        __m512 acc[MR][NP][2];                                                                 \
        for (int i = 0; i < MR; i++)                                                           \
            for (int p = 0; p < NP; p++) {                                                     \
                float* yy = t->y + (size_t)i * t->ys + p * PANEL;                              \
                acc[i][p][0] = t->init ? _mm512_setzero_ps() : _mm512_loadu_ps(yy);            \
                acc[i][p][1] = t->init ? _mm512_setzero_ps() : _mm512_loadu_ps(yy + 16);       \
            }                                                                                  \
        for (int32_t kk = 0; kk < t->kc; kk++) {                                               \
            __m512 xb[MR];                                                                     \
            for (int i = 0; i < MR; i++) xb[i] = _mm512_set1_ps(t->x[(size_t)i * t->xs + kk]); \
            for (int p = 0; p < NP; p++) {                                                     \
                const uint16_t* wp = t->w + p * t->ws + (size_t)kk * PANEL;                    \
                __m512i lo = _mm512_cvtepu16_epi32(_mm256_loadu_si256((const __m256i*)wp));   \
                __m512i hi = _mm512_cvtepu16_epi32(_mm256_loadu_si256((const __m256i*)(wp + 16))); \
                __m512 w0 = _mm512_castsi512_ps(_mm512_slli_epi32(lo, 16));                    \
                __m512 w1 = _mm512_castsi512_ps(_mm512_slli_epi32(hi, 16));                    \
                for (int i = 0; i < MR; i++) {                                                 \
                    acc[i][p][0] = _mm512_fmadd_ps(xb[i], w0, acc[i][p][0]);                   \
                    acc[i][p][1] = _mm512_fmadd_ps(xb[i], w1, acc[i][p][1]);                   \
                }                                                                              \
            }                                                                                  \
        }                                                                                      \
        for (int i = 0; i < MR; i++)                                                           \
            for (int p = 0; p < NP; p++) {                                                     \
                float* yy = t->y + (size_t)i * t->ys + p * PANEL;                              \
                _mm512_storeu_ps(yy, acc[i][p][0]);                                            \
                _mm512_storeu_ps(yy + 16, acc[i][p][1]);                                       \
            }                                                                                  \
    }

/* Columns 0-15 and 16-31 of one panel at one position, as f32: int8 codes,
 * or int4 nibbles (low: columns 0-15, high: 16-31) minus 8. */
AVX512 static inline void q_codes(const uint8_t* p, int32_t q4, __m512* w0, __m512* w1) {
    if (q4) {
        __m512i b = _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i*)p));
        __m512i eight = _mm512_set1_epi32(8);
        *w0 = _mm512_cvtepi32_ps(_mm512_sub_epi32(_mm512_and_si512(b, _mm512_set1_epi32(0x0F)), eight));
        *w1 = _mm512_cvtepi32_ps(_mm512_sub_epi32(_mm512_srli_epi32(b, 4), eight));
    } else {
        *w0 = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i*)p)));
        *w1 = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i*)(p + 16))));
    }
}

/* Quantized tile: per group a chain over its 32 positions from zero, then
 * y = fma(group sum, scale, y) (src/quant.rs:318-370). */
#define DEF_QTILE(MR, NP)                                                                      \
    AVX512 static void qtile_##MR##_##NP(const mtile* t) {                                     \
        const int32_t bpk = t->q4 ? PANEL / 2 : PANEL;                                         \
        if (t->init)                                                                           \
            for (int i = 0; i < MR; i++)                                                       \
                for (int p = 0; p < NP; p++) {                                                 \
                    float* yy = t->y + (size_t)i * t->ys + p * PANEL;                          \
                    _mm512_storeu_ps(yy, _mm512_setzero_ps());                                 \
                    _mm512_storeu_ps(yy + 16, _mm512_setzero_ps());                            \
                }                                                                              \
        for (int32_t g = 0; g < t->kc / GROUP; g++) {                                          \
            __m512 gs[MR][NP][2];                                                              \
            for (int i = 0; i < MR; i++)                                                       \
                for (int p = 0; p < NP; p++) gs[i][p][0] = gs[i][p][1] = _mm512_setzero_ps();  \
            for (int32_t kk = g * GROUP; kk < (g + 1) * GROUP; kk++) {                         \
                __m512 xb[MR];                                                                 \
                for (int i = 0; i < MR; i++) xb[i] = _mm512_set1_ps(t->x[(size_t)i * t->xs + kk]); \
                for (int p = 0; p < NP; p++) {                                                 \
                    __m512 w0, w1;                                                             \
                    q_codes(t->q + p * t->qs + (size_t)kk * bpk, t->q4, &w0, &w1);             \
                    for (int i = 0; i < MR; i++) {                                             \
                        gs[i][p][0] = _mm512_fmadd_ps(xb[i], w0, gs[i][p][0]);                 \
                        gs[i][p][1] = _mm512_fmadd_ps(xb[i], w1, gs[i][p][1]);                 \
                    }                                                                          \
                }                                                                              \
            }                                                                                  \
            for (int p = 0; p < NP; p++) {                                                     \
                const float* sp = t->s + p * t->ss + (size_t)g * PANEL;                        \
                __m512 s0 = _mm512_loadu_ps(sp), s1 = _mm512_loadu_ps(sp + 16);                \
                for (int i = 0; i < MR; i++) {                                                 \
                    float* yy = t->y + (size_t)i * t->ys + p * PANEL;                          \
                    _mm512_storeu_ps(yy, _mm512_fmadd_ps(gs[i][p][0], s0, _mm512_loadu_ps(yy)));         \
                    _mm512_storeu_ps(yy + 16, _mm512_fmadd_ps(gs[i][p][1], s1, _mm512_loadu_ps(yy + 16))); \
                }                                                                              \
            }                                                                                  \
        }                                                                                      \
    }

DEF_BTILE(1, 1)
DEF_BTILE(1, 2)
DEF_BTILE(1, 3)
DEF_BTILE(1, 4)
DEF_BTILE(2, 1)
DEF_BTILE(2, 2)
DEF_BTILE(4, 1)
DEF_BTILE(4, 2)
DEF_BTILE(8, 1)
DEF_QTILE(1, 1)
DEF_QTILE(1, 2)
DEF_QTILE(1, 3)
DEF_QTILE(1, 4)
DEF_QTILE(2, 1)
DEF_QTILE(2, 2)
DEF_QTILE(4, 1)
DEF_QTILE(4, 2)
DEF_QTILE(8, 1)

static void run_tile(const mtile* t, int32_t bf, int32_t mr, int32_t np) {
#define TCASE(MR, NP)                                   \
    if (mr == MR && np == NP) {                         \
        bf ? btile_##MR##_##NP(t) : qtile_##MR##_##NP(t); \
        return;                                         \
    }
    TCASE(1, 1) TCASE(1, 2) TCASE(1, 3) TCASE(1, 4) TCASE(2, 1) TCASE(2, 2) TCASE(4, 1) TCASE(4, 2) TCASE(8, 1)
#undef TCASE
    abort();
}

/* The AVX-512 tile shapes by the rows left in a block (src/kernels.rs:281-289). */
static void tile_shape(int32_t rows, int32_t* mr, int32_t* np) {
    if (rows == 1) *mr = 1, *np = 4;
    else if (rows <= 3) *mr = 2, *np = 2;
    else if (rows <= 7) *mr = 4, *np = 2;
    else *mr = 8, *np = 1;
}

/* Rows of x per cache block, inner positions per block (a multiple of GROUP). */
#define MC 60
#define KC 256

typedef struct {
    const omat* w;
    const float* x;
    float* y;
    int32_t m, per_task, panels;
} mm_job;

/* Output panels of one task for every row (src/kernels.rs:293-322, src/quant.rs:180-217). */
static void mm_task(void* arg, int32_t task) {
    const mm_job* j = (const mm_job*)arg;
    const omat* w = j->w;
    int32_t n = w->rows, K = w->cols, bf = w->kind == OR_BF16, G = K / GROUP;
    int32_t bpk = bf ? 0 : bytes_per_k(w->kind);
    int32_t p0 = task * j->per_task, p1 = p0 + j->per_task < j->panels ? p0 + j->per_task : j->panels;
    for (int32_t m0 = 0; m0 < j->m; m0 += MC) {
        int32_t m1 = m0 + MC < j->m ? m0 + MC : j->m;
        for (int32_t k0 = 0; k0 < K; k0 += KC) {
            int32_t kc = KC < K - k0 ? KC : K - k0;
            for (int32_t i = m0; i < m1;) {
                int32_t mr, np;
                tile_shape(m1 - i, &mr, &np);
                for (int32_t p = p0; p < p1;) {
                    int32_t npp = np < p1 - p ? np : p1 - p;
                    mtile t;
                    memset(&t, 0, sizeof(t));
                    t.x = j->x + (size_t)i * K + k0;
                    t.xs = K;
                    if (bf) {
                        t.w = w->packed + ((size_t)p * K + k0) * PANEL;
                        t.ws = (size_t)K * PANEL;
                    } else {
                        t.q = w->q + ((size_t)p * K + k0) * bpk;
                        t.qs = (size_t)K * bpk;
                        t.s = w->s + ((size_t)p * G + k0 / GROUP) * PANEL;
                        t.ss = (size_t)G * PANEL;
                        t.q4 = w->kind == OR_INT4;
                    }
                    t.kc = kc;
                    t.init = k0 == 0;
                    t.y = j->y + (size_t)i * n + (size_t)p * PANEL;
                    t.ys = n;
                    run_tile(&t, bf, mr, npp);
                    p += npp;
                }
                i += mr;
            }
        }
    }
}

/* kernels::matmul's dispatch (src/kernels.rs:250-268): enough tasks to
 * balance the threads, in whole panels. */
static void fast_matmul(const omat* w, const float* x, int32_t m, float* y) {
    int32_t panels = w->rows / PANEL, threads = g_pool ? g_pool->workers + 1 : 1;
    int32_t per = panels / (threads * 6);
    per = per < 1 ? 1 : per > 64 ? 64 : per;
    mm_job j = {w, x, y, m, per, panels};
    pool_run((panels + per - 1) / per, mm_task, &j);
}

/* dot's lane order (src/kernels.rs:193-214) on eight-wide vectors: lane l
 * sums products l, l + 8, ..., then the fixed pairwise sum of the lanes. */
AVX2 static float dot8(const float* a, const float* b, int32_t n) {
    __m256 acc = _mm256_setzero_ps();
    for (int32_t i = 0; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
    float l[8];
    _mm256_storeu_ps(l, acc);
    return hsum8(l);
}

/* out[d] = fma(w, v[d], out[d]) for every d: the weighted values' in-order chain. */
AVX512 static void axpy16(float* out, float w, const float* v, int32_t n) {
    __m512 ww = _mm512_set1_ps(w);
    int32_t d = 0;
    for (; d + 16 <= n; d += 16)
        _mm512_storeu_ps(out + d, _mm512_fmadd_ps(ww, _mm512_loadu_ps(v + d), _mm512_loadu_ps(out + d)));
    for (; d < n; d++) out[d] = fmaf(w, v[d], out[d]);
}
#else
static void fast_matmul(const omat* w, const float* x, int32_t m, float* y) {
    (void)w, (void)x, (void)m, (void)y;
    abort();
}
static float dot8(const float* a, const float* b, int32_t n) { return or_dot(a, b, n); }
static void axpy16(float* out, float w, const float* v, int32_t n) {
    for (int32_t d = 0; d < n; d++) out[d] = fmaf(w, v[d], out[d]);
}
#endif

/* The fast path on (threads in all, caller included) when the CPU has
 * AVX-512 F/BW; 0 when it is on, -1 when this CPU cannot take it. */
int32_t or_set_fast(int32_t on, int32_t threads) {
    pool_stop();
    g_fast = 0;
    if (!on) return 0;
#if defined(__x86_64__)
    __builtin_cpu_init();
    if (!__builtin_cpu_supports("avx512f") || !__builtin_cpu_supports("avx512bw") || !__builtin_cpu_supports("avx2") ||
        !__builtin_cpu_supports("fma"))
        return -1;
    if (pool_start(threads > 0 ? threads : omp_get_num_procs())) return -1;
    g_fast = 1;
    g_fast_threads = threads;
    return 0;
#else
    (void)threads;
    return -1;
#endif
}

/* kernels::matmul: src/kernels.rs:249-275 (bias added after the chains) */
static void omat_matmul(const omat* w, const float* x, int32_t m, const float* bias, float* y) {
    int32_t n = w->rows, K = w->cols, panels = n / PANEL;
    if (m == 0) return;
    if (g_fast) {
        fast_matmul(w, x, m, y);
    } else {
#pragma omp parallel for schedule(dynamic, 1)
        for (int32_t p = 0; p < panels; p++) {
            if (w->kind == OR_BF16)
                mm_bf16_panel(x, m, K, w->packed + (size_t)p * K * PANEL, y, n, p);
            else
                mm_q_panel(x, m, K, w->q + (size_t)p * K * bytes_per_k(w->kind),
                           w->s + (size_t)p * (K / GROUP) * PANEL, w->kind, y, n, p);
        }
    }
    if (bias)
        for (int32_t i = 0; i < m; i++)
            for (int32_t j = 0; j < n; j++) y[(size_t)i * n + j] += bias[j];
}

int32_t or_matmul(const or_matrix_desc* d, const float* x, int32_t m, const float* bias, float* y) {
    omat w;
    if (omat_init(&w, d)) {
        omat_free(&w);
        return -1;
    }
    omat_matmul(&w, x, m, bias, y);
    omat_free(&w);
    return 0;
}

/* ------------------------------------------------------------------ */
/* AWQ: src/awq.rs:128-217                                              */
/* ------------------------------------------------------------------ */

/* stats (src/awq.rs:128-142): mean |x| and mean x^2 per input channel, f64
 * sums taken in row order, divided by max(rows, 1), rounded to f32. */
void or_awq_stats(const float* cal, int32_t m, int32_t k, float* abs_mean, float* sq_mean) {
    double* a = (double*)calloc((size_t)k, sizeof(double));
    double* q = (double*)calloc((size_t)k, sizeof(double));
    for (int32_t i = 0; i < m; i++)
        for (int32_t c = 0; c < k; c++) {
            const float v = cal[(size_t)i * k + c];
            a[c] += (double)fabsf(v);
            q[c] += (double)v * (double)v;
        }
    const double n = (double)(m > 1 ? m : 1);
    for (int32_t c = 0; c < k; c++) {
        abs_mean[c] = (float)(a[c] / n);
        sq_mean[c] = (float)(q[c] / n);
    }
    free(a);
    free(q);
}

/* scales (src/awq.rs:144-150): max(a, 1e-5)^alpha (f32 powf), divided by
 * max(sqrt(max * min), 1e-8), floored at 1e-4. */
void or_awq_scales(const float* abs_mean, int32_t k, float alpha, float* s) {
    float mx = 0.0f, mn = FLT_MAX;
    for (int32_t c = 0; c < k; c++) {
        const float v = powf(fmaxf(abs_mean[c], 1e-5f), alpha);
        s[c] = v;
        mx = fmaxf(mx, v);
        mn = fminf(mn, v);
    }
    const float norm = fmaxf(sqrtf(mx * mn), 1e-8f);
    for (int32_t c = 0; c < k; c++) s[c] = fmaxf(s[c] / norm, 1e-4f);
}

/* apply (src/awq.rs:152-165): quantize w (rows x k) with its columns times
 * s, importance sq / s^2 + 1e-8. */
static int32_t awq_apply(int32_t kind, int32_t rows, int32_t k, const float* w, const float* s, const float* sq,
                         float* ws, float* imp, uint8_t* q, float* sc) {
    for (int32_t r = 0; r < rows; r++)
        for (int32_t c = 0; c < k; c++) ws[(size_t)r * k + c] = w[(size_t)r * k + c] * s[c];
    for (int32_t c = 0; c < k; c++) imp[c] = sq[c] / (s[c] * s[c]) + 1e-8f;
    return or_quantize(kind, rows, k, ws, imp, q, sc);
}

/* search + apply (src/awq.rs:167-217): alpha in 0, 0.1, ..., 1; per alpha
 * the quantized projection of the scaled calibration rows against the
 * unquantized (bf16) projection, mean squared error summed in f64 in output
 * order; the first minimum wins. Writes the chosen scales (k), alpha,
 * errs[0] = error at alpha 0 (plain), errs[1] = chosen error, and the
 * quantized matrix in the QMatrix layout. */
int32_t or_awq_search(int32_t kind, int32_t rows, int32_t k, const float* w, int32_t m, const float* cal,
                      float* scales_out, float* alpha_out, double* errs, uint8_t* q, float* s) {
    if (kind == OR_BF16 || rows <= 0 || k <= 0 || m <= 0 || rows % PANEL || k % GROUP) return -1;
    const size_t rk = (size_t)rows * k, qb = (size_t)rows / PANEL * k * bytes_per_k(kind);
    const size_t sn = (size_t)rows / PANEL * (k / GROUP) * PANEL, ny = (size_t)m * rows;
    float *am = (float*)malloc((size_t)k * 4), *sq = (float*)malloc((size_t)k * 4);
    float *sc = (float*)malloc((size_t)k * 4), *best_s = (float*)malloc((size_t)k * 4);
    float *imp = (float*)malloc((size_t)k * 4), *ws = (float*)malloc(rk * 4);
    float *xs = (float*)malloc((size_t)m * k * 4), *yref = (float*)malloc(ny * 4), *y = (float*)malloc(ny * 4);
    uint16_t* wb = (uint16_t*)malloc(rk * 2);
    uint8_t* qt = (uint8_t*)malloc(qb);
    float* st = (float*)malloc(sn * 4);
    or_awq_stats(cal, m, k, am, sq);
    /* the reference output, with the unquantized weights (Matrix::from_f32: bf16) */
    for (size_t i = 0; i < rk; i++) wb[i] = or_f32_to_bf16(w[i]);
    or_matrix_desc dref = {OR_BF16, rows, k, 0, wb, NULL, NULL};
    or_matmul(&dref, cal, m, NULL, yref);
    double best = INFINITY, plain = 0.0;
    float best_alpha = 0.0f;
    int have = 0;
    for (int32_t step = 0; step <= 10; step++) {
        const float alpha = (float)step / 10.0f;
        or_awq_scales(am, k, alpha, sc);
        awq_apply(kind, rows, k, w, sc, sq, ws, imp, qt, st);
        for (int32_t i = 0; i < m; i++)
            for (int32_t c = 0; c < k; c++) xs[(size_t)i * k + c] = cal[(size_t)i * k + c] / sc[c];
        or_matrix_desc dq = {kind, rows, k, 0, NULL, qt, st};
        or_matmul(&dq, xs, m, NULL, y);
        double err = 0.0;
        for (size_t i = 0; i < ny; i++) {
            const double d = (double)(y[i] - yref[i]);
            err += d * d;
        }
        err /= (double)ny;
        if (step == 0) plain = err;
        if (!have || err < best) {
            have = 1;
            best = err;
            best_alpha = alpha;
            memcpy(best_s, sc, (size_t)k * 4);
        }
    }
    awq_apply(kind, rows, k, w, best_s, sq, ws, imp, q, s);
    memcpy(scales_out, best_s, (size_t)k * 4);
    *alpha_out = best_alpha;
    errs[0] = plain;
    errs[1] = best;
    free(am); free(sq); free(sc); free(best_s); free(imp); free(ws); free(xs); free(yref); free(y); free(wb);
    free(qt); free(st);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Model                                                                */
/* ------------------------------------------------------------------ */
typedef struct {
    float* attn_norm;
    omat wqkv;
    float* bqkv;
    omat wo;
    float* mlp_norm;
    omat w_gate_up;
    omat w_down;
} olayer;

struct or_model {
    or_config cfg;
    olayer* layers;
    int32_t n_layers;
    omat embed;
    omat lm_head; /* kind -1 when tied */
    float* norm;
    float* inv_freq;
    int owns;
};

static float* dup_f32(const float* p, size_t n) {
    if (!p) return NULL;
    float* d = (float*)malloc(n * 4);
    memcpy(d, p, n * 4);
    return d;
}

/* inv_freq: src/model.rs:461-492 (f32, powf, Llama 3 scaling) */
static float* make_inv_freq(const or_config* c) {
    int32_t dim = c->head_dim;
    float* f = (float*)malloc((size_t)(dim / 2) * 4);
    for (int32_t i = 0; i < dim / 2; i++) f[i] = 1.0f / powf(c->rope_theta, (float)(2 * i) / (float)dim);
    if (c->rope_llama3) {
        float old = (float)c->rope_orig_max_pos;
        float low_wavelen = old / c->rope_low_freq;
        float high_wavelen = old / c->rope_high_freq;
        for (int32_t i = 0; i < dim / 2; i++) {
            float fr = f[i];
            float wavelen = 2.0f * 3.14159265358979323846f / fr;
            if (wavelen < high_wavelen) {
                f[i] = fr;
            } else if (wavelen > low_wavelen) {
                f[i] = fr / c->rope_factor;
            } else {
                float smooth = (old / wavelen - c->rope_low_freq) / (c->rope_high_freq - c->rope_low_freq);
                f[i] = (1.0f - smooth) * fr / c->rope_factor + smooth * fr;
            }
        }
    }
    return f;
}

or_model* or_model_create(const or_config* cfg, const or_layer_desc* layers, const uint16_t* embed,
                          const float* norm, const uint16_t* lm_head) {
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    m->cfg = *cfg;
    m->owns = 1;
    int32_t H = cfg->hidden, qkv = (cfg->heads + 2 * cfg->kv_heads) * cfg->head_dim;
    m->n_layers = cfg->layers;
    m->layers = (olayer*)calloc((size_t)cfg->layers, sizeof(olayer));
    int bad = 0;
    for (int32_t i = 0; i < cfg->layers; i++) {
        const or_layer_desc* d = &layers[i];
        olayer* l = &m->layers[i];
        l->attn_norm = dup_f32(d->attn_norm, H);
        l->mlp_norm = dup_f32(d->mlp_norm, H);
        l->bqkv = cfg->qkv_bias ? dup_f32(d->bqkv, qkv) : NULL;
        bad |= omat_init(&l->wqkv, &d->wqkv);
        bad |= omat_init(&l->wo, &d->wo);
        bad |= omat_init(&l->w_gate_up, &d->w_gate_up);
        bad |= omat_init(&l->w_down, &d->w_down);
        /* check_shapes: src/model.rs:243-261 */
        bad |= l->wqkv.rows != qkv || l->wqkv.cols != H || l->wo.rows != H ||
               l->wo.cols != cfg->heads * cfg->head_dim || l->w_gate_up.rows != 2 * cfg->intermediate ||
               l->w_gate_up.cols != H || l->w_down.rows != H || l->w_down.cols != cfg->intermediate;
    }
    or_matrix_desc ed = {OR_BF16, cfg->vocab, H, 0, embed, NULL, NULL};
    bad |= omat_init(&m->embed, &ed);
    if (lm_head && !cfg->tie_embeddings) {
        or_matrix_desc ld = {OR_BF16, cfg->vocab, H, 0, lm_head, NULL, NULL};
        bad |= omat_init(&m->lm_head, &ld);
    } else {
        m->lm_head.kind = -1;
    }
    m->norm = dup_f32(norm, H);
    m->inv_freq = make_inv_freq(cfg);
    if (bad) {
        or_model_destroy(m);
        return NULL;
    }
    return m;
}

or_model* or_model_truncated(const or_model* base, int32_t layers) {
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    *m = *base;
    m->owns = 0;
    if (layers < m->n_layers) m->n_layers = layers;
    m->cfg.layers = m->n_layers;
    return m;
}

void or_model_destroy(or_model* m) {
    if (!m) return;
    if (m->owns) {
        for (int32_t i = 0; i < m->cfg.layers; i++) {
            olayer* l = &m->layers[i];
            free(l->attn_norm);
            free(l->mlp_norm);
            free(l->bqkv);
            omat_free(&l->wqkv);
            omat_free(&l->wo);
            omat_free(&l->w_gate_up);
            omat_free(&l->w_down);
        }
        free(m->layers);
        omat_free(&m->embed);
        if (m->lm_head.kind >= 0) omat_free(&m->lm_head);
        free(m->norm);
        free(m->inv_freq);
    }
    free(m);
}

/* ------------------------------------------------------------------ */
/* KvCache: src/kv.rs:23-71 ([layer][block][kv_head][offset][dim], f32) */
/* ------------------------------------------------------------------ */
struct or_kv {
    int32_t layers, kv_heads, head_dim, block_size, blocks;
    float** k;
    float** v;
};

or_kv* or_kv_create(int32_t layers, int32_t kv_heads, int32_t head_dim, int32_t block_size, int32_t blocks) {
    or_kv* kv = (or_kv*)calloc(1, sizeof(or_kv));
    kv->layers = layers;
    kv->kv_heads = kv_heads;
    kv->head_dim = head_dim;
    kv->block_size = block_size;
    kv->blocks = blocks;
    size_t n = (size_t)blocks * block_size * kv_heads * head_dim;
    kv->k = (float**)calloc((size_t)layers, sizeof(float*));
    kv->v = (float**)calloc((size_t)layers, sizeof(float*));
    for (int32_t l = 0; l < layers; l++) {
        kv->k[l] = (float*)calloc(n, 4);
        kv->v[l] = (float*)calloc(n, 4);
    }
    return kv;
}

void or_kv_destroy(or_kv* kv) {
    if (!kv) return;
    for (int32_t l = 0; l < kv->layers; l++) {
        free(kv->k[l]);
        free(kv->v[l]);
    }
    free(kv->k);
    free(kv->v);
    free(kv);
}

static size_t kv_layer_floats(const or_kv* kv) {
    return (size_t)kv->blocks * kv->block_size * kv->kv_heads * kv->head_dim;
}

int32_t or_kv_read(const or_kv* kv, int32_t layer, float* k_out, float* v_out) {
    if (layer < 0 || layer >= kv->layers) return -1;
    memcpy(k_out, kv->k[layer], kv_layer_floats(kv) * 4);
    memcpy(v_out, kv->v[layer], kv_layer_floats(kv) * 4);
    return 0;
}

int32_t or_kv_write_layer(or_kv* kv, int32_t layer, const float* k, const float* v) {
    if (layer < 0 || layer >= kv->layers) return -1;
    memcpy(kv->k[layer], k, kv_layer_floats(kv) * 4);
    memcpy(kv->v[layer], v, kv_layer_floats(kv) * 4);
    return 0;
}

/* KvCache::write: src/kv.rs:46-56 */
static void kv_write(or_kv* kv, int32_t layer, size_t slot, const float* k, const float* v) {
    int32_t bs = kv->block_size, hd = kv->head_dim, nkv = kv->kv_heads;
    size_t b = slot / bs, o = slot % bs;
    for (int32_t h = 0; h < nkv; h++) {
        size_t at = ((b * nkv + h) * bs + o) * hd;
        memcpy(kv->k[layer] + at, k + (size_t)h * hd, (size_t)hd * 4);
        memcpy(kv->v[layer] + at, v + (size_t)h * hd, (size_t)hd * 4);
    }
}

/* attend: src/kernels.rs:703-756 (scores by dot, softmax in position
 * order, weighted values as an in-order fma chain) for the `heads` query
 * heads sharing one kv head. */
static void attend(const float* q, int32_t heads, int32_t hd, int32_t n, float scale, const float* K,
                   const float* V, const uint32_t* blocks, int32_t bs, size_t block_stride, size_t head_off,
                   float* scores, float* out) {
    int32_t p = 0;
    for (int32_t bi = 0; p < n; bi++) {
        size_t base = (size_t)blocks[bi] * block_stride + head_off;
        for (int32_t o = 0; o < bs && p < n; o++, p++) {
            const float* kp = K + base + (size_t)o * hd;
            for (int32_t j = 0; j < heads; j++)
                scores[(size_t)j * n + p] = (g_fast ? dot8(q + (size_t)j * hd, kp, hd) : or_dot(q + (size_t)j * hd, kp, hd)) * scale;
        }
    }
    for (int32_t j = 0; j < heads; j++) {
        float* s = scores + (size_t)j * n;
        float mx = -INFINITY;
        for (int32_t i = 0; i < n; i++) mx = s[i] > mx ? s[i] : mx;
        for (int32_t i = 0; i < n; i++) s[i] -= mx;
        for (int32_t i = 0; i < n; i++) s[i] = or_exp(s[i]);
        float sum = -0.0f;
        for (int32_t i = 0; i < n; i++) sum += s[i];
        for (int32_t i = 0; i < n; i++) s[i] /= sum;
    }
    memset(out, 0, (size_t)heads * hd * 4);
    p = 0;
    for (int32_t bi = 0; p < n; bi++) {
        size_t base = (size_t)blocks[bi] * block_stride + head_off;
        for (int32_t o = 0; o < bs && p < n; o++, p++) {
            const float* vp = V + base + (size_t)o * hd;
            for (int32_t j = 0; j < heads; j++) {
                float w = scores[(size_t)j * n + p];
                float* oj = out + (size_t)j * hd;
                if (g_fast)
                    axpy16(oj, w, vp, hd);
                else
                    for (int32_t d = 0; d < hd; d++) oj[d] = fmaf(w, vp[d], oj[d]);
            }
        }
    }
}

/* rope: src/model.rs:451-459 */
static void rope(float* x, const float* cs, const float* sn, int32_t hd) {
    int32_t half = hd / 2;
    for (int32_t i = 0; i < half; i++) {
        float a = x[i], b = x[i + half];
        x[i] = a * cs[i] + -b * sn[i];
        x[i + half] = b * cs[i] + a * sn[i];
    }
}

/* silu_mul on the fast path: the same element formula, in pool tasks of
 * 1024 elements. */
typedef struct {
    const float* gate_up;
    float* out;
    int32_t inter, n;
} silu_job;

static void silu_task(void* arg, int32_t task) {
    const silu_job* j = (const silu_job*)arg;
    int32_t i1 = (task + 1) * 1024 < j->n ? (task + 1) * 1024 : j->n;
    for (int32_t idx = task * 1024; idx < i1; idx++) {
        int32_t r = idx / j->inter, i = idx % j->inter;
        const float* g = j->gate_up + (size_t)r * 2 * j->inter;
        float e = or_exp(-g[i]);
        j->out[idx] = g[i] / (1.0f + e) * g[j->inter + i];
    }
}

/* One (row, kv head) attention task of the fast path (the pool's tasks). */
typedef struct {
    const or_chunk* chunks;
    const int32_t *owner, *pos;
    const float* qkv;
    float* att;
    const float *K, *V;
    int32_t group, hd, nkv, bs, qkv_dim, q_dim, maxn;
    float scale;
    size_t block_stride;
} attn_job;

static void attn_task(void* arg, int32_t task) {
    const attn_job* j = (const attn_job*)arg;
    int32_t rr = task / j->nkv, g = task % j->nkv;
    const or_chunk* ch = &j->chunks[j->owner[rr]];
    float* scores = (float*)malloc((size_t)j->group * j->maxn * 4);
    attend(j->qkv + (size_t)rr * j->qkv_dim + (size_t)g * j->group * j->hd, j->group, j->hd, j->pos[rr] + 1, j->scale,
           j->K, j->V, ch->blocks, j->bs, j->block_stride, (size_t)g * j->bs * j->hd, scores,
           j->att + (size_t)rr * j->q_dim + (size_t)g * j->group * j->hd);
    free(scores);
}

/* Model::forward: src/model.rs:267-362 */
int32_t or_forward(const or_model* m, or_kv* kv, const or_chunk* chunks, int32_t n_chunks, float* logits_out,
                   float* hidden_out) {
    return or_forward_taps(m, kv, chunks, n_chunks, logits_out, hidden_out, NULL);
}

int32_t or_forward_taps(const or_model* m, or_kv* kv, const or_chunk* chunks, int32_t n_chunks, float* logits_out,
                        float* hidden_out, float* proj_out) {
    const or_config* c = &m->cfg;
    int32_t H = c->hidden, hd = c->head_dim, nh = c->heads, nkv = c->kv_heads, I = c->intermediate;
    int32_t q_dim = nh * hd, qkv_dim = (nh + 2 * nkv) * hd, half = hd / 2;
    int32_t bs = kv->block_size;
    int32_t t = 0;
    for (int32_t ci = 0; ci < n_chunks; ci++) t += chunks[ci].n;
    if (t == 0) return 0;
    int32_t* pos = (int32_t*)malloc((size_t)t * 4);
    size_t* slot = (size_t*)malloc((size_t)t * sizeof(size_t));
    int32_t* owner = (int32_t*)malloc((size_t)t * 4);
    int32_t r = 0;
    for (int32_t ci = 0; ci < n_chunks; ci++) {
        const or_chunk* ch = &chunks[ci];
        if ((int64_t)ch->n_blocks * bs < (int64_t)ch->pos + ch->n) {
            free(pos);
            free(slot);
            free(owner);
            return -1; /* "chunk overruns its cache blocks" */
        }
        for (int32_t i = 0; i < ch->n; i++, r++) {
            int32_t p = ch->pos + i;
            pos[r] = p;
            slot[r] = (size_t)ch->blocks[p / bs] * bs + p % bs;
            owner[r] = ci;
        }
    }
    float* x = (float*)malloc((size_t)t * H * 4);
    r = 0;
    for (int32_t ci = 0; ci < n_chunks; ci++)
        for (int32_t i = 0; i < chunks[ci].n; i++, r++) {
            uint32_t tok = chunks[ci].tokens[i];
            if ((int32_t)tok >= c->vocab) tok = 0; /* callers validate ids */
            omat_row_f32(&m->embed, (int32_t)tok, x + (size_t)r * H);
        }
    if (hidden_out) memcpy(hidden_out, x, (size_t)t * H * 4);
    /* rope_tables: src/model.rs:434-448 */
    float* cs = (float*)malloc((size_t)t * half * 4);
    float* sn = (float*)malloc((size_t)t * half * 4);
    for (r = 0; r < t; r++)
        for (int32_t i = 0; i < half; i++) {
            float a = (float)pos[r] * m->inv_freq[i];
            cs[(size_t)r * half + i] = cosf(a);
            sn[(size_t)r * half + i] = sinf(a);
        }
    float* xn = (float*)malloc((size_t)t * H * 4);
    float* qkv = (float*)malloc((size_t)t * qkv_dim * 4);
    float* att = (float*)malloc((size_t)t * q_dim * 4);
    float* proj = (float*)malloc((size_t)t * H * 4);
    float* gate_up = (float*)malloc((size_t)t * 2 * I * 4);
    float* act = (float*)malloc((size_t)t * I * 4);
    int32_t group = nh / nkv;
    float scale = 1.0f / sqrtf((float)hd);
    size_t block_stride = (size_t)nkv * hd * bs;
    int32_t maxn = 0;
    for (r = 0; r < t; r++) maxn = pos[r] + 1 > maxn ? pos[r] + 1 : maxn;

    for (int32_t li = 0; li < m->n_layers; li++) {
        const olayer* l = &m->layers[li];
        /* Model::record's four projection inputs (src/model.rs:312,323,329,333) */
        float* tap = proj_out ? proj_out + (size_t)li * t * (2 * H + q_dim + I) : NULL;
        or_rms_norm(x, l->attn_norm, H, t, c->rms_eps, xn);
        if (tap) memcpy(tap, xn, (size_t)t * H * 4);
        omat_matmul(&l->wqkv, xn, t, l->bqkv, qkv);
        for (r = 0; r < t; r++) {
            float* row = qkv + (size_t)r * qkv_dim;
            for (int32_t h = 0; h < nh + nkv; h++) rope(row + (size_t)h * hd, cs + (size_t)r * half, sn + (size_t)r * half, hd);
            kv_write(kv, li, slot[r], row + q_dim, row + q_dim + nkv * hd);
        }
        /* Model::attention: src/model.rs:394-432, one task per (row, kv head) */
        if (g_fast) {
            attn_job aj = {chunks, owner, pos, qkv, att, kv->k[li], kv->v[li], group, hd, nkv, bs, qkv_dim, q_dim,
                           maxn, scale, block_stride};
            pool_run(t * nkv, attn_task, &aj);
        } else
#pragma omp parallel
        {
            float* scores = (float*)malloc((size_t)group * maxn * 4);
#pragma omp for schedule(dynamic, 1)
            for (int32_t task = 0; task < t * nkv; task++) {
                int32_t rr = task / nkv, g = task % nkv;
                const or_chunk* ch = &chunks[owner[rr]];
                attend(qkv + (size_t)rr * qkv_dim + (size_t)g * group * hd, group, hd, pos[rr] + 1, scale, kv->k[li],
                       kv->v[li], ch->blocks, bs, block_stride, (size_t)g * bs * hd,
                       scores, att + (size_t)rr * q_dim + (size_t)g * group * hd);
            }
            free(scores);
        }
        if (tap) memcpy(tap + (size_t)t * H, att, (size_t)t * q_dim * 4);
        omat_matmul(&l->wo, att, t, NULL, proj);
        for (size_t i = 0; i < (size_t)t * H; i++) x[i] += proj[i];
        or_rms_norm(x, l->mlp_norm, H, t, c->rms_eps, xn);
        if (tap) memcpy(tap + (size_t)t * (H + q_dim), xn, (size_t)t * H * 4);
        omat_matmul(&l->w_gate_up, xn, t, NULL, gate_up);
        if (g_fast) {
            silu_job sj = {gate_up, act, I, t * I};
            pool_run((t * I + 1023) / 1024, silu_task, &sj);
        } else {
            or_silu_mul(gate_up, I, t, act);
        }
        if (tap) memcpy(tap + (size_t)t * (2 * H + q_dim), act, (size_t)t * I * 4);
        omat_matmul(&l->w_down, act, t, NULL, proj);
        for (size_t i = 0; i < (size_t)t * H; i++) x[i] += proj[i];
        if (hidden_out) memcpy(hidden_out + (size_t)(li + 1) * t * H, x, (size_t)t * H * 4);
    }

    /* Only the requested rows go through the head: src/model.rs:338-361 */
    int32_t* rows = (int32_t*)malloc((size_t)t * 4);
    int32_t nr = 0;
    r = 0;
    for (int32_t ci = 0; ci < n_chunks; ci++) {
        int32_t n = chunks[ci].n;
        if (chunks[ci].logits == OR_LOGITS_LAST && n > 0) rows[nr++] = r + n - 1;
        if (chunks[ci].logits == OR_LOGITS_ALL)
            for (int32_t i = 0; i < n; i++) rows[nr++] = r + i;
        r += n;
    }
    if (nr > 0 && logits_out) {
        float* hsel = (float*)malloc((size_t)nr * H * 4);
        for (int32_t i = 0; i < nr; i++)
            or_rms_norm(x + (size_t)rows[i] * H, m->norm, H, 1, c->rms_eps, hsel + (size_t)i * H);
        omat_matmul(m->lm_head.kind >= 0 ? &m->lm_head : &m->embed, hsel, nr, NULL, logits_out);
        free(hsel);
    }
    free(rows);
    free(pos);
    free(slot);
    free(owner);
    free(x);
    free(cs);
    free(sn);
    free(xn);
    free(qkv);
    free(att);
    free(proj);
    free(gate_up);
    free(act);
    return nr;
}

/* ------------------------------------------------------------------ */
/* Greedy speculative decoding for one sequence                         */
/* ------------------------------------------------------------------ */

/* The target pass and greedy accept of Engine::execute
 * (src/engine.rs:511-616, Logits::All branch, greedy). */
int32_t or_verify(const or_model* target, or_kv* kv, const uint32_t* blocks, int32_t n_blocks, int32_t pos,
                  uint32_t last, const uint32_t* drafts, int32_t k, uint32_t* out, int32_t* accepted,
                  float* logits_out) {
    int32_t V = target->cfg.vocab;
    uint32_t* in = (uint32_t*)malloc((size_t)(k + 1) * 4);
    in[0] = last;
    for (int32_t j = 0; j < k; j++) in[j + 1] = drafts[j];
    or_chunk ch = {in, k + 1, pos, blocks, n_blocks, OR_LOGITS_ALL};
    float* logits = logits_out ? logits_out : (float*)malloc((size_t)(k + 1) * V * 4);
    int32_t nr = or_forward(target, kv, &ch, 1, logits, NULL);
    free(in);
    if (nr != k + 1) {
        if (!logits_out) free(logits);
        return -1;
    }
    int32_t acc = 0, n = 0;
    for (int32_t j = 0; j < k; j++) {
        uint32_t tk = or_argmax(logits + (size_t)j * V, V);
        if (tk == drafts[j]) {
            out[n++] = drafts[j];
            acc++;
        } else {
            out[n++] = tk;
            break;
        }
    }
    if (acc == k) out[n++] = or_argmax(logits + (size_t)k * V, V);
    if (accepted) *accepted = acc;
    if (!logits_out) free(logits);
    return n;
}

int32_t or_spec_step(const or_model* target, or_kv* tkv, const or_model* draft, or_kv* dkv, const uint32_t* tokens,
                     int32_t len, int32_t* computed, int32_t* draft_computed, const uint32_t* blocks, int32_t n_blocks,
                     const uint32_t* draft_blocks, int32_t n_draft_blocks, int32_t k, uint32_t* out,
                     int32_t* accepted) {
    int32_t V = target->cfg.vocab;
    if (k <= 0 || *computed != len - 1 || *draft_computed > len - 1) return -1;
    float* logits = (float*)malloc((size_t)V * 4);
    uint32_t* drafts = (uint32_t*)malloc((size_t)k * 4);
    int32_t dc = *draft_computed;
    /* propose: src/engine.rs:656-717 */
    for (int32_t round = 0; round < k; round++) {
        or_chunk ch;
        uint32_t one;
        if (round == 0) {
            ch = (or_chunk){tokens + dc, len - dc, dc, draft_blocks, n_draft_blocks, OR_LOGITS_LAST};
        } else {
            one = drafts[round - 1];
            ch = (or_chunk){&one, 1, len + round - 1, draft_blocks, n_draft_blocks, OR_LOGITS_LAST};
        }
        if (or_forward(draft, dkv, &ch, 1, logits, NULL) != 1) {
            free(logits);
            free(drafts);
            return -1;
        }
        if (round == 0) dc = len;
        drafts[round] = or_argmax(logits, V);
    }
    free(logits);
    dc = len + k - 1;
    int32_t acc = 0;
    int32_t ne = or_verify(target, tkv, blocks, n_blocks, *computed, tokens[*computed], drafts, k, out, &acc, NULL);
    free(drafts);
    if (ne < 0) return -1;
    /* rollback: src/engine.rs:613-615 */
    *computed = len + acc;
    *draft_computed = dc < len + acc ? dc : len + acc;
    if (accepted) *accepted = acc;
    return ne;
}

typedef struct {
    uint32_t* ids;
    int32_t n, cap;
} blist;

static int blist_grow_to(blist* b, int32_t tokens, int32_t bs, int32_t* next_free, int32_t limit) {
    while ((int64_t)b->n * bs < tokens) {
        if (*next_free >= limit) return -1;
        if (b->n == b->cap) {
            b->cap = b->cap ? b->cap * 2 : 64;
            b->ids = (uint32_t*)realloc(b->ids, (size_t)b->cap * 4);
        }
        b->ids[b->n++] = (uint32_t)(*next_free)++;
    }
    return 0;
}

int32_t or_generate(const or_model* target, const or_model* draft, const uint32_t* prompt, int32_t n_prompt,
                    int32_t max_tokens, int32_t k, int32_t kv_blocks, int32_t max_batch_tokens, uint32_t* out,
                    int32_t* accepted_out, int64_t* stats) {
    const int32_t bs = 16, max_seqs = 64;
    const or_config* c = &target->cfg;
    if (!draft) k = 0;
    int32_t max_len = c->max_position < kv_blocks * bs ? c->max_position : kv_blocks * bs;
    if (n_prompt == 0 || n_prompt >= max_len) return -1; /* src/engine.rs:273-281 */
    int32_t V = c->vocab;
    int32_t cap = n_prompt + max_tokens + k + 2;
    uint32_t* tokens = (uint32_t*)malloc((size_t)cap * 4);
    memcpy(tokens, prompt, (size_t)n_prompt * 4);
    int32_t len = n_prompt, computed = 0, draft_computed = 0, generated = 0, nsteps = 0;
    int64_t proposed = 0, acc_total = 0, spec_steps = 0;
    blist tb = {0}, db = {0};
    int32_t t_free = 0, d_free = 0;
    or_kv* tkv = or_kv_create(c->layers, c->kv_heads, c->head_dim, bs, kv_blocks);
    or_kv* dkv = draft ? or_kv_create(draft->cfg.layers, draft->cfg.kv_heads, draft->cfg.head_dim, bs,
                                      kv_blocks + max_seqs)
                       : NULL;
    float* logits = (float*)malloc((size_t)V * 4);
    uint32_t emit[64];
    int32_t rc = 0, done = 0;
    while (!done) {
        /* schedule: src/engine.rs:395-426 */
        int32_t budget = max_batch_tokens;
        int32_t left = len - computed;
        int32_t decoding = left == 1;
        int32_t spec = decoding && k > 0 && len + k < max_len && budget > k;
        int32_t n = spec ? k + 1 : (left < budget ? left : budget);
        if (blist_grow_to(&tb, computed + n, bs, &t_free, kv_blocks) ||
            (spec && blist_grow_to(&db, len + k - 1, bs, &d_free, kv_blocks + max_seqs))) {
            rc = -1; /* the single sequence cannot be preempted in favour of anything */
            break;
        }
        int32_t ne = 0;
        if (spec) {
            int32_t accepted = 0;
            ne = or_spec_step(target, tkv, draft, dkv, tokens, len, &computed, &draft_computed, tb.ids, tb.n,
                              db.ids, db.n, k, emit, &accepted);
            if (ne < 0) {
                rc = -1;
                break;
            }
            proposed += k;
            acc_total += accepted;
            if (accepted_out && spec_steps < max_tokens) accepted_out[spec_steps] = accepted;
            spec_steps++;
        } else {
            int32_t last = computed + n == len;
            or_chunk ch = {tokens + computed, n, computed, tb.ids, tb.n, last ? OR_LOGITS_LAST : OR_LOGITS_NONE};
            int32_t nr = or_forward(target, tkv, &ch, 1, logits, NULL);
            if (nr < 0) {
                rc = -1;
                break;
            }
            computed += n;
            if (last) emit[ne++] = or_argmax(logits, V);
        }
        /* token delivery: src/engine.rs:618-637 (ignore_eos, no stop ids) */
        for (int32_t i = 0; i < ne; i++) {
            tokens[len++] = emit[i];
            out[generated++] = emit[i];
            if (generated >= max_tokens || len >= max_len) {
                done = 1;
                break;
            }
        }
        nsteps++;
    }
    if (stats) {
        stats[0] = proposed;
        stats[1] = acc_total;
        stats[2] = spec_steps;
    }
    free(tokens);
    free(tb.ids);
    free(db.ids);
    or_kv_destroy(tkv);
    or_kv_destroy(dkv);
    free(logits);
    (void)nsteps;
    return rc ? -1 : generated;
}
