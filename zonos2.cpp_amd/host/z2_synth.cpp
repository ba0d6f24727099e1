// z2_synth.cpp — synthetic weight / KV generation and GGUF-format quantizers (host, C ABI).
//
// The benchmark configurations are random-init models (N(0, sigma) matrices quantized to a GGUF
// block type), in the style of the reference's dummy-model generator
// (scripts/make-dummy-model.py:53-142, tensor names/shapes mirrored there). Values are a pure
// function of (seed, stream, element index): a splitmix64 counter feeds an inverse-CDF transform, so any slice
// of any tensor can be regenerated independently and in parallel. Normal deviates come from the
// inverse CDF of a 53-bit uniform.
//
// The quantizers are this project's own simple min/max fits. Parity is defined on the same
// quantized bytes for the CPU oracle and the device, so they need not match ggml's quantizer.
#include "z2_formats.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

using namespace z2;

namespace {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Standard normal by inversion of the CDF: P. J. Acklam's rational approximation (2003;
// relative error < 1.2e-9), which needs a log/sqrt only in the 2 x 2.425% tails.
inline double inv_norm_cdf(double p) {
    static const double a[6] = {-3.969683028665376e+01, 2.209460984245205e+02, -2.759285104469687e+02,
                                1.383577518672690e+02, -3.066479806614716e+01, 2.506628277459239e+00};
    static const double b[5] = {-5.447609879822406e+01, 1.615858368580409e+02, -1.556989798598866e+02,
                                6.680131188771972e+01, -1.328068155288572e+01};
    static const double c[6] = {-7.784894002430293e-03, -3.223964580411365e-01, -2.400758277161838e+00,
                                -2.549732539343734e+00, 4.374664141464968e+00, 2.938163982698783e+00};
    static const double d[4] = {7.784695709041462e-03, 3.224671290700398e-01, 2.445134137142996e+00,
                                3.754408661907416e+00};
    const double plow = 0.02425;
    if (p < plow || p > 1.0 - plow) {
        const double q = std::sqrt(-2.0 * std::log(p < plow ? p : 1.0 - p));
        const double x = (((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5]) /
                         ((((d[0] * q + d[1]) * q + d[2]) * q + d[3]) * q + 1.0);
        return p < plow ? x : -x;
    }
    const double q = p - 0.5, r = q * q;
    return (((((a[0] * r + a[1]) * r + a[2]) * r + a[3]) * r + a[4]) * r + a[5]) * q /
           (((((b[0] * r + b[1]) * r + b[2]) * r + b[3]) * r + b[4]) * r + 1.0);
}

// kind: 0 normal(a, b) | 1 b*|normal(0,1)| | 2 constant a | 3 uniform integer in [a, b]
inline float gen_value(uint64_t key, int64_t i, int kind, float a, float b) {
    if (kind == 2) return a;
    const uint64_t x = splitmix64(key + (uint64_t) i);
    if (kind == 3) {
        const int64_t lo = (int64_t) a, hi = (int64_t) b;
        return (float) (lo + (int64_t) (x % (uint64_t) (hi - lo + 1)));
    }
    const double u = ((double) (x >> 11) + 0.5) * (1.0 / 9007199254740992.0);   // (0, 1)
    const float z = (float) inv_norm_cdf(u);
    if (kind == 1) return b * std::fabs(z);
    return a + b * z;
}

inline int nint(float x) { return (int) std::nearbyint(x); }

void quant_q8_0_row(const float * x, blk_q8_0 * y, int64_t n) {
    for (int64_t b = 0; b < n / QK8_0; ++b) {
        const float * v = x + b * QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; ++j) amax = std::max(amax, std::fabs(v[j]));
        const uint16_t dh = f32_to_f16(amax / 127.0f);
        const float d = f16_to_f32(dh);
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        y[b].d = dh;
        for (int j = 0; j < QK8_0; ++j) y[b].qs[j] = (int8_t) std::clamp(nint(v[j] * id), -127, 127);
    }
}

void quant_q4_k_row(const float * x, blk_q4_k * y, int64_t n) {
    for (int64_t b = 0; b < n / QK_K; ++b) {
        const float * v = x + b * QK_K;
        float scale[8], minv[8];
        for (int j = 0; j < 8; ++j) {
            float lo = 0.0f, hi = -INFINITY;
            for (int l = 0; l < 32; ++l) { lo = std::min(lo, v[32 * j + l]); hi = std::max(hi, v[32 * j + l]); }
            hi = std::max(hi, lo);
            scale[j] = (hi - lo) / 15.0f;
            minv[j]  = -lo;
        }
        const float ms = *std::max_element(scale, scale + 8), mm = *std::max_element(minv, minv + 8);
        const uint16_t dh = f32_to_f16(ms / 63.0f), mh = f32_to_f16(mm / 63.0f);
        const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
        int sc[8], m[8];
        for (int j = 0; j < 8; ++j) {
            sc[j] = d > 0.0f ? std::clamp(nint(scale[j] / d), 0, 63) : 0;
            m[j]  = dmin > 0.0f ? std::clamp(nint(minv[j] / dmin), 0, 63) : 0;
        }
        blk_q4_k & o = y[b];
        o.d = dh; o.dmin = mh;
        for (int i = 0; i < 4; ++i) {
            o.scales[i]     = (uint8_t) ((sc[i] & 63) | ((sc[i + 4] >> 4) << 6));
            o.scales[i + 4] = (uint8_t) ((m[i] & 63)  | ((m[i + 4] >> 4) << 6));
            o.scales[i + 8] = (uint8_t) ((sc[i + 4] & 15) | ((m[i + 4] & 15) << 4));
        }
        uint8_t q[QK_K];
        for (int j = 0; j < 8; ++j) {
            const float es = d * (float) sc[j], em = dmin * (float) m[j];
            for (int l = 0; l < 32; ++l)
                q[32 * j + l] = (uint8_t) (es > 0.0f ? std::clamp(nint((v[32 * j + l] + em) / es), 0, 15) : 0);
        }
        for (int p = 0; p < 4; ++p)
            for (int l = 0; l < 32; ++l)
                o.qs[32 * p + l] = (uint8_t) (q[64 * p + l] | (q[64 * p + 32 + l] << 4));
    }
}

void quant_q6_k_row(const float * x, blk_q6_k * y, int64_t n) {
    for (int64_t b = 0; b < n / QK_K; ++b) {
        const float * v = x + b * QK_K;
        float gs[16];
        for (int g = 0; g < 16; ++g) {
            float amax = 0.0f;
            for (int l = 0; l < 16; ++l) amax = std::max(amax, std::fabs(v[16 * g + l]));
            gs[g] = amax / 31.0f;
        }
        const float mx = *std::max_element(gs, gs + 16);
        const uint16_t dh = f32_to_f16(mx / 127.0f);
        const float d = f16_to_f32(dh);
        blk_q6_k & o = y[b];
        o.d = dh;
        uint8_t u[QK_K];
        for (int g = 0; g < 16; ++g) {
            const int sc = d > 0.0f ? std::clamp(nint(gs[g] / d), -128, 127) : 0;
            o.scales[g] = (int8_t) sc;
            const float es = d * (float) sc;
            for (int l = 0; l < 16; ++l) {
                const int q = es != 0.0f ? std::clamp(nint(v[16 * g + l] / es), -32, 31) : 0;
                u[16 * g + l] = (uint8_t) (q + 32);
            }
        }
        for (int h = 0; h < 2; ++h) {
            const uint8_t * uh = u + 128 * h;
            uint8_t * ql = o.ql + 64 * h;
            uint8_t * qh = o.qh + 32 * h;
            for (int l = 0; l < 32; ++l) {
                ql[l]      = (uint8_t) ((uh[l] & 15)      | ((uh[l + 64] & 15) << 4));
                ql[l + 32] = (uint8_t) ((uh[l + 32] & 15) | ((uh[l + 96] & 15) << 4));
                qh[l] = (uint8_t) ((uh[l] >> 4) | ((uh[l + 32] >> 4) << 2) |
                                   ((uh[l + 64] >> 4) << 4) | ((uh[l + 96] >> 4) << 6));
            }
        }
    }
}

bool quant_row(int type, const float * x, void * dst, int64_t n) {
    switch (type) {
        case T_F32: std::memcpy(dst, x, (size_t) n * 4); return true;
        case T_F16: {
            uint16_t * h = (uint16_t *) dst;
            for (int64_t i = 0; i < n; ++i) h[i] = f32_to_f16(x[i]);
            return true;
        }
        case T_Q8_0: quant_q8_0_row(x, (blk_q8_0 *) dst, n); return true;
        case T_Q4_K: quant_q4_k_row(x, (blk_q4_k *) dst, n); return true;
        case T_Q6_K: quant_q6_k_row(x, (blk_q6_k *) dst, n); return true;
        default: return false;
    }
}

template <class F>
void parallel_rows(int64_t nrows, int n_threads, F && fn) {
    n_threads = std::max(1, std::min<int>(n_threads, (int) std::min<int64_t>(nrows, 256)));
    if (n_threads == 1) { fn(0, nrows); return; }
    std::vector<std::thread> th;
    const int64_t per = (nrows + n_threads - 1) / n_threads;
    for (int t = 0; t < n_threads; ++t) {
        const int64_t r0 = t * per, r1 = std::min(nrows, r0 + per);
        if (r0 >= r1) break;
        th.emplace_back([&, r0, r1] { fn(r0, r1); });
    }
    for (auto & t : th) t.join();
}

} // namespace

extern "C" {

int64_t z2s_row_bytes(int type, int64_t n_per_row) {
    if (!type_known(type) || n_per_row % type_block(type)) return -1;
    return row_bytes(type, n_per_row);
}

uint64_t z2s_stream_id(const char * name) {                 // FNV-1a of the tensor name
    uint64_t h = 1469598103934665603ull;
    for (const char * p = name; *p; ++p) { h ^= (uint8_t) *p; h *= 1099511628211ull; }
    return h;
}

// Generate nrows x n_per_row values (element index = row * n_per_row + col) and store them as
// `type`. Returns 0 on success.
int z2s_generate(uint64_t seed, uint64_t stream, int kind, float a, float b, int type,
                 int64_t nrows, int64_t n_per_row, void * dst, int n_threads) {
    if (!type_known(type) || n_per_row % type_block(type) || !dst) return 1;
    const uint64_t key = splitmix64(seed ^ splitmix64(stream));
    const int64_t rb = row_bytes(type, n_per_row);
    parallel_rows(nrows, n_threads, [&](int64_t r0, int64_t r1) {
        std::vector<float> buf((size_t) n_per_row);
        for (int64_t r = r0; r < r1; ++r) {
            for (int64_t c = 0; c < n_per_row; ++c) buf[c] = gen_value(key, r * n_per_row + c, kind, a, b);
            quant_row(type, buf.data(), (uint8_t *) dst + r * rb, n_per_row);
        }
    });
    return 0;
}

// Quantize caller-provided fp32 rows to `type`.
int z2s_quantize(int type, const float * src, void * dst, int64_t nrows, int64_t n_per_row, int n_threads) {
    if (!type_known(type) || n_per_row % type_block(type) || !src || !dst) return 1;
    const int64_t rb = row_bytes(type, n_per_row);
    parallel_rows(nrows, n_threads, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r)
            quant_row(type, src + r * n_per_row, (uint8_t *) dst + r * rb, n_per_row);
    });
    return 0;
}

int z2s_f32_to_f16(const float * src, uint16_t * dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = f32_to_f16(src[i]);
    return 0;
}

int z2s_f16_to_f32(const uint16_t * src, float * dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = f16_to_f32(src[i]);
    return 0;
}

} // extern "C"
