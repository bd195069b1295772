// Load-time host routines (include/ferro_host.h): the synthetic weight
// draw and the group-32 quantizer. CPU code, run once per model.
#include "ferro_host.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "ferro_gpu.h"

namespace {

// Rng (src/rng.rs:8-44): xorshift64*, Box-Muller in f64.
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ULL | 1ULL) {}
    uint64_t next() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return s * 0x2545F4914F6CDD1DULL;
    }
    double uniform() { return (double)(next() >> 11) / (double)(1ULL << 53); }
    double normal() {
        const double u = 1.0 - uniform();
        const double v = uniform();
        return std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v);
    }
};

uint16_t to_bf16(float x) {
    uint32_t b;
    std::memcpy(&b, &x, 4);
    if (std::isnan(x)) return (uint16_t)((b >> 16) | 0x40);
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

template <class F>
void for_each_parallel(int64_t n, F f) {
    int nt = (int)std::thread::hardware_concurrency();
    nt = (int)std::max<int64_t>(1, std::min<int64_t>({(int64_t)nt, (int64_t)16, n}));
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++)
        th.emplace_back([=, &f] {
            for (int64_t i = t; i < n; i += nt) f(i);
        });
    for (auto& x : th) x.join();
}

uint64_t splitmix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

}  // namespace

extern "C" {

uint64_t fh_stream_seed(uint64_t seed, uint64_t tensor, uint64_t block) {
    return splitmix(splitmix(splitmix(seed) ^ tensor) ^ block);
}

int fh_random_bf16(uint64_t seed, uint64_t tensor, int64_t rows, int64_t cols, float std, uint16_t* out) {
    if (rows < 0 || cols < 0 || !out) return FG_E_ARG;
    const int64_t blocks = (rows + 63) / 64;
    const double scale = std;
    for_each_parallel(blocks, [&](int64_t b) {
        Rng rng(fh_stream_seed(seed, tensor, (uint64_t)b));
        const int64_t r1 = std::min(rows, (b + 1) * 64);
        for (int64_t i = b * 64 * cols; i < r1 * cols; i++) out[i] = to_bf16((float)(rng.normal() * scale));
    });
    return 0;
}

// One (row, group) of QMatrix::quantize: the clip with the smallest
// importance-weighted squared error, the first on ties; an all-zero group
// gets scale 0 and codes 0.
static float quantize_group(const float* v, const float* imp, int lo, int hi, const float* clips, int nclips,
                            int* codes) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(v[i]));
    if (!(amax > 0.0f)) {
        std::fill(codes, codes + 32, 0);
        return 0.0f;
    }
    double best = INFINITY;
    float best_scale = 0.0f;
    int trial[32];
    for (int ci = 0; ci < nclips; ci++) {
        const float scale = clips[ci] * amax / (float)hi;
        double err = 0.0;
        for (int i = 0; i < 32; i++) {
            int c = (int)std::round(v[i] / scale);  // half away from zero, as f32::round
            c = std::min(hi, std::max(lo, c));
            trial[i] = c;
            const float q = (float)c * scale;
            const double d = (double)(v[i] - q);
            err += d * d * (imp ? (double)imp[i] : 1.0);
        }
        if (err < best) {
            best = err;
            best_scale = scale;
            std::memcpy(codes, trial, sizeof(trial));
        }
    }
    return best_scale;
}

int fh_quantize(int32_t kind, int32_t rows, int32_t cols, const float* w, const float* importance, uint8_t* q,
                float* s) {
    if ((kind != FG_INT8 && kind != FG_INT4) || rows <= 0 || cols <= 0 || rows % 32 || cols % 32 || !w || !q || !s)
        return FG_E_ARG;
    static const float c8[] = {1.0f, 0.98f, 0.96f, 0.94f, 0.92f, 0.9f};
    static const float c4[] = {1.0f, 0.95f, 0.9f, 0.85f, 0.8f, 0.75f, 0.7f, 0.65f, 0.6f, 0.55f, 0.5f};
    const bool q8 = kind == FG_INT8;
    const int lo = q8 ? -127 : -8, hi = q8 ? 127 : 7;
    const int groups = cols / 32, bpk = q8 ? 32 : 16;
    // Panel p owns bytes [p*cols*bpk, (p+1)*cols*bpk) and its scales.
    for_each_parallel(rows / 32, [&](int64_t p) {
        uint8_t* qp = q + (size_t)p * cols * bpk;
        std::memset(qp, 0, (size_t)cols * bpk);
        int codes[32];
        for (int c = 0; c < 32; c++) {
            const int64_t r = p * 32 + c;
            for (int g = 0; g < groups; g++) {
                const float scale = quantize_group(w + r * cols + (int64_t)g * 32,
                                                   importance ? importance + g * 32 : nullptr, lo, hi,
                                                   q8 ? c8 : c4, q8 ? 6 : 11, codes);
                s[((size_t)p * groups + g) * 32 + c] = scale;
                for (int i = 0; i < 32; i++) {
                    uint8_t* at = qp + (size_t)(g * 32 + i) * bpk;
                    if (q8) {
                        at[c] = (uint8_t)(int8_t)codes[i];
                    } else {
                        const uint8_t nib = (uint8_t)(codes[i] + 8);
                        if (c < 16)
                            at[c] = (uint8_t)((at[c] & 0xF0) | nib);
                        else
                            at[c - 16] = (uint8_t)((at[c - 16] & 0x0F) | (nib << 4));
                    }
                }
            }
        }
    });
    return 0;
}

// stats (src/awq.rs:128-142): f64 sums in row order, divided by max(m, 1).
int fh_awq_stats(const float* cal, int32_t m, int32_t k, float* abs_mean, float* sq_mean) {
    if (!cal || !abs_mean || !sq_mean || m < 0 || k <= 0) return FG_E_ARG;
    std::vector<double> a((size_t)k, 0.0), q((size_t)k, 0.0);
    for (int32_t i = 0; i < m; i++)
        for (int32_t c = 0; c < k; c++) {
            const float v = cal[(size_t)i * k + c];
            a[c] += (double)std::fabs(v);
            q[c] += (double)v * (double)v;
        }
    const double n = (double)std::max(m, 1);
    for (int32_t c = 0; c < k; c++) {
        abs_mean[c] = (float)(a[c] / n);
        sq_mean[c] = (float)(q[c] / n);
    }
    return 0;
}

// scales (src/awq.rs:144-150): f32 powf (libm, as f32::powf), f32::max/min
// fold, normalised by max(sqrt(max * min), 1e-8), floored at 1e-4.
int fh_awq_scales(const float* abs_mean, int32_t k, float alpha, float* s) {
    if (!abs_mean || !s || k <= 0) return FG_E_ARG;
    float mx = 0.0f, mn = 3.40282347e38f;
    for (int32_t c = 0; c < k; c++) {
        const float v = powf(std::fmax(abs_mean[c], 1e-5f), alpha);
        s[c] = v;
        mx = std::fmax(mx, v);
        mn = std::fmin(mn, v);
    }
    const float norm = std::fmax(std::sqrt(mx * mn), 1e-8f);
    for (int32_t c = 0; c < k; c++) s[c] = std::fmax(s[c] / norm, 1e-4f);
    return 0;
}

}  // extern "C"
