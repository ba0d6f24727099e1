// oracle.cpp — CPU restatement of the reference's ggml CPU decode path.
//
// TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline ("C++ restatement of
// the ggml CPU path"; ggml itself is absent from the reference tree, so this is not ggml).
//
// Numerics contract (shared with the device kernels; compiled with -ffp-contract=off, no fast-math):
//  * Quantized matmuls follow ggml's CPU scheme: the fp32 activation row is first encoded in the
//    weight type's dot type (Q8_K per 256 for Q4_K/Q6_K, Q8_0 per 32 for Q8_0, f16 for F16), the
//    block dot is exact integer arithmetic, and each block's value is combined in fp32 as written
//    in dot_block() / dot_row(). ggml's own SIMD summation order is not known here, so the order is
//    fixed to the device matmuls' (dot_row), which makes every Q4_K / Q6_K / Q8_0 matmul output
//    bit-identical on the CPU and the device for identical inputs. F16 matmuls run on the device's
//    matrix cores, whose internal order is the hardware's: those agree within the tolerance only.
//  * The rest of a decode step is specified the same way (rms_norm, qk_norm, z_sincos for RoPE,
//    attention_fwd's 64-row chunks and their merge, z_softcap), so that a whole decode step of a
//    Q4_K / Q6_K / Q8_0 model gives bit-identical hidden states, routing and logits.
//  * The router (src/zonos2-graph.cpp:199-220) is specified exactly, including reduction order
//    and the exp/erf implementations, so that identical router inputs give bit-identical logits,
//    probabilities, top-k indices and weights on the CPU and on the device:
//      - n_embd-long dots: 64 lane partials (lane l sums i = l, l+64, ... with fmaf, ascending),
//        then a xor butterfly (32,16,8,4,2,1) of fp32 adds;
//      - router_dim-long dots (MLP layers): 8 fmaf partial chains over contiguous eighths + xor
//        butterfly (4,2,1);
//      - RMSNorm sum of squares in double: 64 lane partials + xor butterfly;
//      - softmax: max, exp via orc_expf, double sum with the same butterfly, p = e * (float)(1/sum);
//      - top-k: score descending, ties to the lower expert index.
//  * orc_expf / orc_erff are this project's own: Cody-Waite reduction + degree-7 Taylor
//    polynomial, and Abramowitz & Stegun 7.1.26 for erf.
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_err;
int g_threads = 0;

int fail(const std::string & msg) { g_err = msg; return 1; }

int n_threads() {
    if (g_threads > 0) return g_threads;
    const unsigned hc = std::thread::hardware_concurrency();
    return hc ? (int) hc : 1;
}

template <class F>
void parallel_for(int64_t n, F && fn) {
    const int nt = (int) std::max<int64_t>(1, std::min<int64_t>(n, n_threads()));
    if (nt == 1) { for (int64_t i = 0; i < n; ++i) fn(i); return; }
    std::atomic<int64_t> next(0);
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t)
        th.emplace_back([&] {
            for (int64_t i = next.fetch_add(1); i < n; i = next.fetch_add(1)) fn(i);
        });
    for (auto & t : th) t.join();
}

// ------------------------------------------------------------------ fp16
uint16_t to_f16(float f) {
    uint32_t x; std::memcpy(&x, &f, 4);
    const uint32_t s = (x >> 16) & 0x8000u, a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t) (s | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) return (uint16_t) (s | 0x7c00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return (uint16_t) s;
        const uint32_t e = a >> 23, m = (a & 0x7fffffu) | 0x800000u, sh = 126 - e;
        uint32_t r = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t) (s | r);
    }
    uint32_t r = (a - 0x38000000u) >> 13;
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t) (s | r);
}

float from_f16_calc(uint16_t h) {
    const uint32_t s = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu;
    float f;
    if (e == 0) f = std::ldexp((float) m, -24);
    else if (e == 31) { uint32_t x = s | 0x7f800000u | (m << 13); std::memcpy(&f, &x, 4); return f; }
    else f = std::ldexp((float) (m | 0x400u), (int) e - 25);
    return s ? -f : f;
}

// every f16 value's float, computed once (the F16 matmuls convert two values per product)
struct f16_table {
    float v[65536];
    f16_table() { for (uint32_t h = 0; h < 65536; ++h) v[h] = from_f16_calc((uint16_t) h); }
};
const f16_table g_f16;
inline float from_f16(uint16_t h) { return g_f16.v[h]; }

// ------------------------------------------------------------------ exact elementwise functions
float z_expf(float x) {
    if (x > 88.72283f) return INFINITY;
    if (x < -103.97208f) return 0.0f;
    const float n = std::rint(x * 1.44269504088896341f);
    float r = std::fma(n, -0.693145751953125f, x);          // ln2 high part (exact product)
    r = std::fma(n, -1.428606765330187e-06f, r);             // ln2 low part
    float p = 1.98412698e-4f;                                // 1/7!
    p = std::fma(p, r, 1.38888889e-3f);                      // 1/6!
    p = std::fma(p, r, 8.33333333e-3f);                      // 1/5!
    p = std::fma(p, r, 4.16666667e-2f);                      // 1/4!
    p = std::fma(p, r, 1.66666667e-1f);                      // 1/3!
    p = std::fma(p, r, 0.5f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    return std::ldexp(p, (int) n);
}

float z_erff(float x) {                                       // Abramowitz & Stegun 7.1.26
    const float ax = std::fabs(x);
    const float t = 1.0f / (1.0f + 0.3275911f * ax);
    float p = std::fma(1.061405429f, t, -1.453152027f);
    p = std::fma(p, t, 1.421413741f);
    p = std::fma(p, t, -0.284496736f);
    p = std::fma(p, t, 0.254829592f);
    p = p * t;
    const float y = 1.0f - p * z_expf(-(ax * ax));
    return std::copysign(y, x);
}

float z_gelu(float x) { return (0.5f * x) * (1.0f + z_erff(x * 0.70710678118654752f)); }
float z_silu(float x) { return x / (1.0f + z_expf(-x)); }
float z_sigmoid(float x) { return 1.0f / (1.0f + z_expf(-x)); }

// exp in double: x = n ln2 + r (ln2 in two parts, Cody-Waite), exp(r) by the degree-13 Taylor
// polynomial in Horner form with fma, times 2^n.
double exp_d(double x) {
    if (x < -745.0) return 0.0;
    const double n = std::rint(x * 0x1.71547652b82fep+0);
    double r = std::fma(-n, 0x1.62e42fee00000p-1, x);
    r = std::fma(-n, 0x1.a39ef35793c76p-33, r);
    static const double c[14] = {0x1.6124613a86d09p-33, 0x1.1eed8eff8d898p-29, 0x1.ae64567f544e4p-26, 0x1.27e4fb7789f5cp-22,
                                 0x1.71de3a556c734p-19, 0x1.a01a01a01a01ap-16, 0x1.a01a01a01a01ap-13, 0x1.6c16c16c16c17p-10,
                                 0x1.1111111111111p-7, 0x1.5555555555555p-5, 0x1.5555555555555p-3, 0.5, 1.0, 1.0};
    double p = c[0];
    for (int i = 1; i < 14; ++i) p = std::fma(p, r, c[i]);
    return std::ldexp(p, (int) n);
}

// Logit softcap cap * tanh(x / cap) (graph.cpp:359-362). y = x * (1/cap) in fp32; tanh(|y|) in
// double: below 2^-10 its Taylor series to y^5 (next term < 2^-60 relative), above it
// 1 - 2 / (exp(2|y|) + 1); rounded to fp32, the sign restored, times cap.
float z_softcap(float x, float cap) {
    const float y = x * (1.0f / cap);
    const double a = std::fabs((double) y);
    double t;
    if (a < 0x1p-10) {
        const double a2 = a * a;
        t = a + (a * a2) * (-1.0 / 3.0 + a2 * (2.0 / 15.0));
    } else {
        t = 1.0 - 2.0 / (exp_d(2.0 * a) + 1.0);
    }
    return std::copysign((float) t, y) * cap;
}

// sin and cos of a RoPE angle (0 <= x < 2^24): reduced modulo 2 pi in double, then by quadrant to
// [-pi/4, pi/4] (rounded to fp32 there), degree-9 / degree-8 Taylor polynomials in fp32 with fma.
void z_sincos(float x, float & s, float & c) {
    const double xd = (double) x;
    const double k2 = std::rint(xd * 0.15915494309189533577);
    const double rd = std::fma(-k2, 6.28318530717958647692, xd);
    const double q = std::rint(rd * 0.63661977236758134308);
    const float r = (float) std::fma(-q, 1.57079632679489661923, rd);
    const float r2 = r * r;
    float sp = 2.75573192e-6f;
    sp = std::fma(sp, r2, -1.98412698e-4f);
    sp = std::fma(sp, r2, 8.33333333e-3f);
    sp = std::fma(sp, r2, -1.66666667e-1f);
    const float sr = std::fma(sp * r2, r, r);
    float cp = 2.48015873e-5f;
    cp = std::fma(cp, r2, -1.38888889e-3f);
    cp = std::fma(cp, r2, 4.16666667e-2f);
    cp = std::fma(cp, r2, -0.5f);
    const float cr = std::fma(cp, r2, 1.0f);
    const int qi = ((int) q) & 3;
    s = qi == 0 ? sr : qi == 1 ? cr : qi == 2 ? -sr : -cr;
    c = qi == 0 ? cr : qi == 1 ? -sr : qi == 2 ? -cr : sr;
}

// ------------------------------------------------------------------ tensors
struct tensor {
    int type = -1;
    int64_t ne[4] = {1, 1, 1, 1};
    const uint8_t * data = nullptr;
    bool ok() const { return data != nullptr; }
};

int64_t blk_elems(int t) { return t == 0 || t == 1 ? 1 : (t == 8 ? 32 : 256); }
int64_t blk_bytes(int t) {
    switch (t) { case 0: return 4; case 1: return 2; case 8: return 34; case 12: return 144; case 14: return 210; }
    return -1;
}
int64_t row_nbytes(int t, int64_t n) { return n / blk_elems(t) * blk_bytes(t); }

void q4k_scale_min(const uint8_t * sc, int j, int & s, int & m) {
    if (j < 4) { s = sc[j] & 63; m = sc[j + 4] & 63; }
    else {
        s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

uint16_t rd16(const uint8_t * p) { uint16_t v; std::memcpy(&v, p, 2); return v; }

// ggml dequantize_row_* semantics (get_rows on quantized tables, and dequantized router weights)
void dequant_row(int type, const uint8_t * src, float * y, int64_t n) {
    switch (type) {
        case 0: std::memcpy(y, src, (size_t) n * 4); break;
        case 1: for (int64_t i = 0; i < n; ++i) y[i] = from_f16(rd16(src + 2 * i)); break;
        case 8:
            for (int64_t b = 0; b < n / 32; ++b) {
                const uint8_t * blk = src + 34 * b;
                const float d = from_f16(rd16(blk));
                for (int j = 0; j < 32; ++j) y[32 * b + j] = (float) (int8_t) blk[2 + j] * d;
            }
            break;
        case 12:
            for (int64_t b = 0; b < n / 256; ++b) {
                const uint8_t * blk = src + 144 * b;
                const float d = from_f16(rd16(blk)), dmin = from_f16(rd16(blk + 2));
                const uint8_t * sc = blk + 4, * qs = blk + 16;
                for (int p = 0; p < 4; ++p) {
                    int s0, m0, s1, m1;
                    q4k_scale_min(sc, 2 * p, s0, m0);
                    q4k_scale_min(sc, 2 * p + 1, s1, m1);
                    const float d0 = d * (float) s0, n0 = dmin * (float) m0;
                    const float d1 = d * (float) s1, n1 = dmin * (float) m1;
                    for (int l = 0; l < 32; ++l) {
                        y[256 * b + 64 * p + l]      = d0 * (float) (qs[32 * p + l] & 15) - n0;
                        y[256 * b + 64 * p + 32 + l] = d1 * (float) (qs[32 * p + l] >> 4) - n1;
                    }
                }
            }
            break;
        case 14:
            for (int64_t b = 0; b < n / 256; ++b) {
                const uint8_t * blk = src + 210 * b;
                const float d = from_f16(rd16(blk + 208));
                const int8_t * sc = (const int8_t *) (blk + 192);
                for (int h = 0; h < 2; ++h) {
                    const uint8_t * ql = blk + 64 * h, * qh = blk + 128 + 32 * h;
                    float * yy = y + 256 * b + 128 * h;
                    for (int l = 0; l < 32; ++l) {
                        const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        yy[l]      = d * (float) sc[8 * h + l / 16 + 0] * (float) q1;
                        yy[l + 32] = d * (float) sc[8 * h + l / 16 + 2] * (float) q2;
                        yy[l + 64] = d * (float) sc[8 * h + l / 16 + 4] * (float) q3;
                        yy[l + 96] = d * (float) sc[8 * h + l / 16 + 6] * (float) q4;
                    }
                }
            }
            break;
    }
}

// ------------------------------------------------------------------ activation encodings
struct qact {
    int kind = ORC_ACT_F32;
    int64_t n = 0;
    std::vector<int8_t> q;       // Q8_0 / Q8_K values
    std::vector<float> d;        // per block scale (Q8_0: the f16-rounded scale as float)
    std::vector<int16_t> bsum;   // Q8_K sums per 16
    std::vector<uint16_t> h;     // F16
    std::vector<float> f;        // F32
};

int act_kind_for(int wtype) {
    switch (wtype) { case 12: case 14: return ORC_ACT_Q8_K; case 8: return ORC_ACT_Q8_0; case 1: return ORC_ACT_F16; }
    return ORC_ACT_F32;
}

// Q8_K: per 256 the element of largest |x| (first occurrence) fixes iscale = -127/x; q =
// min(127, rint(iscale*x)); d = 1/iscale; bsum per 16. Q8_0: per 32, d = amax/127, q =
// rint(x*127/amax), the scale used in dots is f16(d). F16: round-to-nearest-even.
void quantize_act(int kind, const float * x, int64_t n, qact & a) {
    a.kind = kind; a.n = n;
    if (kind == ORC_ACT_F32) { a.f.assign(x, x + n); return; }
    if (kind == ORC_ACT_F16) { a.h.resize(n); for (int64_t i = 0; i < n; ++i) a.h[i] = to_f16(x[i]); return; }
    a.q.resize(n);
    if (kind == ORC_ACT_Q8_0) {
        a.d.resize(n / 32);
        for (int64_t b = 0; b < n / 32; ++b) {
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[32 * b + j]));
            const float d = amax / 127.0f, id = amax != 0.0f ? 127.0f / amax : 0.0f;
            a.d[b] = from_f16(to_f16(d));
            for (int j = 0; j < 32; ++j) a.q[32 * b + j] = (int8_t) (int) std::rint(x[32 * b + j] * id);
        }
        return;
    }
    a.d.resize(n / 256); a.bsum.resize(n / 16);
    for (int64_t b = 0; b < n / 256; ++b) {
        const float * v = x + 256 * b;
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 256; ++j) { const float ax = std::fabs(v[j]); if (ax > amax) { amax = ax; mx = v[j]; } }
        if (amax == 0.0f) {
            a.d[b] = 0.0f;
            for (int j = 0; j < 256; ++j) a.q[256 * b + j] = 0;
            for (int g = 0; g < 16; ++g) a.bsum[16 * b + g] = 0;
            continue;
        }
        const float iscale = -127.0f / mx;
        for (int j = 0; j < 256; ++j) a.q[256 * b + j] = (int8_t) std::min(127, (int) std::rint(iscale * v[j]));
        for (int g = 0; g < 16; ++g) {
            int s = 0;
            for (int l = 0; l < 16; ++l) s += a.q[256 * b + 16 * g + l];
            a.bsum[16 * b + g] = (int16_t) s;
        }
        a.d[b] = 1.0f / iscale;
    }
}

// value of one weight block (block index b of the row) against the encoded activation
float dot_block(int type, const uint8_t * blk, const qact & a, int64_t b) {
    switch (type) {
        case 8: {
            int isum = 0;
            const int8_t * q = a.q.data() + 32 * b;
            for (int j = 0; j < 32; ++j) isum += (int) (int8_t) blk[2 + j] * q[j];
            return (from_f16(rd16(blk)) * a.d[b]) * (float) isum;
        }
        case 12: {
            const uint8_t * sc = blk + 4, * qs = blk + 16;
            const int8_t * q = a.q.data() + 256 * b;
            int sumi = 0, summ = 0;
            for (int j = 0; j < 8; ++j) {
                int s, m; q4k_scale_min(sc, j, s, m);
                const int p = j / 2, hi = j % 2;
                int isum = 0;
                for (int l = 0; l < 32; ++l) {
                    const int w = hi ? (qs[32 * p + l] >> 4) : (qs[32 * p + l] & 15);
                    isum += w * q[32 * j + l];
                }
                sumi += s * isum;
                summ += m * (a.bsum[16 * b + 2 * j] + a.bsum[16 * b + 2 * j + 1]);
            }
            // the superblock's value before the activation scale: d * sumi - dmin * summ with one
            // rounding of the product sum (dot_row folds it with the activation scale)
            const float d = from_f16(rd16(blk)), dmin = from_f16(rd16(blk + 2));
            return std::fma(d, (float) sumi, -(dmin * (float) summ));
        }
        case 14: {
            const int8_t * sc = (const int8_t *) (blk + 192);
            const int8_t * q = a.q.data() + 256 * b;
            int sumi = 0;
            for (int h = 0; h < 2; ++h) {
                const uint8_t * ql = blk + 64 * h, * qh = blk + 128 + 32 * h;
                int isum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int l = 0; l < 32; ++l) {
                    const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    const int8_t * qq = q + 128 * h;
                    isum[l / 16 + 0] += q1 * qq[l];
                    isum[l / 16 + 2] += q2 * qq[l + 32];
                    isum[l / 16 + 4] += q3 * qq[l + 64];
                    isum[l / 16 + 6] += q4 * qq[l + 96];
                }
                for (int g = 0; g < 8; ++g) sumi += sc[8 * h + g] * isum[g];
            }
            return (from_f16(rd16(blk + 208)) * a.d[b]) * (float) sumi;
        }
        case 1: {                                              // 256-element chunk b
            float s = 0.0f;
            for (int j = 0; j < 256; ++j) s += from_f16(rd16(blk + 2 * j)) * from_f16(a.h[256 * b + j]);
            return s;
        }
        case 0: {
            const float * w = (const float *) blk;
            float s = 0.0f;
            for (int j = 0; j < 256; ++j) s = std::fma(w[j], a.f[256 * b + j], s);
            return s;
        }
    }
    return NAN;
}

// One output element. The summation order of the block values is the device matmuls' (every
// quantized matmul, any batch width): Q4_K folds each superblock value x (dot_block) with the
// activation's superblock scale dx as s = fma(dx, x, s) in superblock order; Q8_0 adds the block
// products of each 256-column unit (8 blocks) in order from zero, then adds the unit sums in order;
// Q6_K adds the superblock values in order; F16 / F32 add 256-column chunk values in order.
float dot_row(int type, const uint8_t * row, const qact & a) {
    const int64_t n = a.n;
    if (type == 0 || type == 1) {
        const int64_t nb = n / 256;
        const int64_t es = type == 0 ? 4 : 2;
        float s = 0.0f;
        for (int64_t b = 0; b < nb; ++b) s += dot_block(type, row + 256 * es * b, a, b);
        for (int64_t j = nb * 256; j < n; ++j)                 // tail (n not a multiple of 256)
            s += type == 0 ? ((const float *) row)[j] * a.f[j] : from_f16(rd16(row + 2 * j)) * from_f16(a.h[j]);
        return s;
    }
    const int64_t be = blk_elems(type), bb = blk_bytes(type), nb = n / be;
    float s = 0.0f;
    if (type == 12) {
        for (int64_t b = 0; b < nb; ++b) s = std::fma(a.d[b], dot_block(type, row + bb * b, a, b), s);
    } else if (type == 8) {
        for (int64_t g = 0; g < nb; g += 8) {
            float u = 0.0f;
            for (int64_t b = g; b < std::min(nb, g + 8); ++b) u += dot_block(type, row + bb * b, a, b);
            s = s + u;
        }
    } else {
        for (int64_t b = 0; b < nb; ++b) s += dot_block(type, row + bb * b, a, b);
    }
    return s;
}

// y[t][o] = W[o] . x[t]   (ggml_mul_mat(W, x): W [n_in, n_out], x [n_in, T])
void matmul(const tensor & w, int64_t expert, int T, const float * x, float * y) {
    const int64_t n_in = w.ne[0], n_out = w.ne[1];
    const int64_t rb = row_nbytes(w.type, n_in);
    const uint8_t * base = w.data + expert * n_out * rb;
    std::vector<qact> acts(T);
    for (int t = 0; t < T; ++t) quantize_act(act_kind_for(w.type), x + (int64_t) t * n_in, n_in, acts[t]);
    const int64_t chunk = 16;
    parallel_for((n_out + chunk - 1) / chunk, [&](int64_t c) {
        for (int64_t o = c * chunk; o < std::min(n_out, (c + 1) * chunk); ++o)
            for (int t = 0; t < T; ++t) y[(int64_t) t * n_out + o] = dot_row(w.type, base + o * rb, acts[t]);
    });
}

// ggml rms_norm: x / sqrt(mean(x^2) + eps), then the optional weight mul (graph.cpp:92-95). The sum of
// squares is in double (as ggml's CPU sums it); its order is the device norm kernels': a 256-thread
// block in which thread tid owns the 4-element groups i0 = 4 (tid + 256 j), j = 0, 1, ... (i0 < n) and
// adds (((x0^2 + x1^2) + x2^2) + x3^2) per group in j order (squares rounded to fp32, sums in double);
// each wave's 64 partials go through the xor butterfly and the four wave sums add left to right.
double tree64d(double * p);
double block_sumsq(const float * x, int64_t n) {
    double ws[4];
    for (int wv = 0; wv < 4; ++wv) {
        double p[64];
        for (int l = 0; l < 64; ++l) {
            const int64_t tid = 64 * wv + l;
            double ss = 0.0;
            for (int64_t i0 = 4 * tid; i0 < n; i0 += 1024) {
                double g = (double) (x[i0] * x[i0]);
                for (int e = 1; e < 4; ++e) g = g + (i0 + e < n ? (double) (x[i0 + e] * x[i0 + e]) : 0.0);
                ss += g;
            }
            p[l] = ss;
        }
        ws[wv] = tree64d(p);
    }
    return ((ws[0] + ws[1]) + ws[2]) + ws[3];
}
void rms_norm(const float * x, const float * w, int64_t n, float eps, float * y) {
    const double s = block_sumsq(x, n);
    const float mean = (float) (s / (double) n);
    const float scale = 1.0f / std::sqrt(mean + eps);
    for (int64_t i = 0; i < n; ++i) y[i] = w ? (x[i] * scale) * w[i] : x[i] * scale;
}

// Per-head QK RMSNorm (graph.cpp:113-116) times mul (|temp| for queries, 1 for keys), in the device's
// order: lane l of one wave holds the dim pair (x[2l], x[2l+1]) (lanes past hd/2 hold zeros) and adds
// its two squares in double; the 64 lanes go through the xor butterfly.
void qk_norm(float * x, int hd, float eps, float mul) {
    double p[64];
    for (int l = 0; l < 64; ++l)
        p[l] = 2 * l + 1 < hd ? (double) (x[2 * l] * x[2 * l]) + (double) (x[2 * l + 1] * x[2 * l + 1]) : 0.0;
    const double ss = tree64d(p);
    const float sc = 1.0f / std::sqrt((float) (ss / (double) hd) + eps);
    for (int i = 0; i < hd; ++i) {
        const float z = x[i] * sc;
        x[i] = mul != 1.0f ? z * mul : z;
    }
}

// ------------------------------------------------------------------ exact router primitives
float tree64(float * p) {
    for (int off = 32; off >= 1; off >>= 1) {
        float nxt[64];
        for (int l = 0; l < 64; ++l) nxt[l] = p[l] + p[l ^ off];
        std::memcpy(p, nxt, sizeof(nxt));
    }
    return p[0];
}
double tree64d(double * p) {
    for (int off = 32; off >= 1; off >>= 1) {
        double nxt[64];
        for (int l = 0; l < 64; ++l) nxt[l] = p[l] + p[l ^ off];
        std::memcpy(p, nxt, sizeof(nxt));
    }
    return p[0];
}
float lane_dot(const float * w, const float * x, int64_t n) {
    float p[64];
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int64_t i = l; i < n; i += 64) acc = std::fma(w[i], x[i], acc);
        p[l] = acc;
    }
    return tree64(p);
}
// router_dim-long dot: 8 partial fmaf chains over contiguous eighths (partial p: i = p*n/8 ...
// (p+1)*n/8 - 1 ascending), then a xor butterfly over the partials (offsets 4, 2, 1):
// ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7))
float chain8_dot(const float * w, const float * x, int64_t n) {
    const int64_t b = n / 8;
    float p[8];
    for (int l = 0; l < 8; ++l) {
        float acc = 0.0f;
        for (int64_t i = l * b; i < (l + 1) * b; ++i) acc = std::fma(w[i], x[i], acc);
        p[l] = acc;
    }
    for (int off = 4; off >= 1; off >>= 1) {
        float nxt[8];
        for (int l = 0; l < 8; ++l) nxt[l] = p[l] + p[l ^ off];
        std::memcpy(p, nxt, sizeof(nxt));
    }
    return p[0];
}
void router_rms(const float * x, const float * w, int64_t n, float eps, float * y) {
    double p[64];
    for (int l = 0; l < 64; ++l) {
        double acc = 0.0;
        for (int64_t i = l; i < n; i += 64) acc += (double) (x[i] * x[i]);
        p[l] = acc;
    }
    const double s = tree64d(p);
    const float mean = (float) (s / (double) n);
    const float scale = 1.0f / std::sqrt(mean + eps);
    for (int64_t i = 0; i < n; ++i) y[i] = (x[i] * scale) * w[i];
}

// ------------------------------------------------------------------ RoPE (ggml NORMAL mode)
// theta_i = pos * base^(-2i/hd), generated by repeated multiplication by base^(-2/hd) in fp32; sin
// and cos by z_sincos (the library's sin / cos are not part of the contract)
void rope_inplace(float * x, int n_heads, int hd, int pos, float base) {
    const float theta_scale = std::pow(base, -2.0f / (float) hd);
    std::vector<float> c(hd / 2), s(hd / 2);
    float theta = (float) pos;
    for (int i = 0; i < hd / 2; ++i) { z_sincos(theta, s[i], c[i]); theta *= theta_scale; }
    for (int h = 0; h < n_heads; ++h) {
        float * v = x + (int64_t) h * hd;
        for (int i = 0; i < hd / 2; ++i) {
            const float x0 = v[2 * i], x1 = v[2 * i + 1];
            v[2 * i]     = x0 * c[i] - x1 * s[i];
            v[2 * i + 1] = x0 * s[i] + x1 * c[i];
        }
    }
}

} // namespace

// ====================================================================== model
struct orc_layer {
    tensor attn_norm, ffn_norm, wq, wk, wv, wo, attn_temp, gater;
    tensor ffn_up, ffn_gate, ffn_down;
    tensor gate_exps, up_exps, down_exps, router_down, router_down_b, router_mlp0, router_mlp0_b,
           router_mlp2, router_mlp2_b, router_mlp4, router_norm, router_bias, router_eda_scale;
    bool is_moe = false;
    int top_k = 0, n_exp = 0;
    std::vector<float> logit_bias;                // harness-only
    std::vector<float> mask;                      // runtime expert mask, 0 / -inf (src/zonos2.cpp:203-239)
    // router weights as fp32 (dequantized once)
    std::vector<float> r_down, r_down_b, r_m0, r_m0_b, r_m2, r_m2_b, r_m4, r_norm, r_bias, r_eda;
};

struct orc_model {
    orc_hparams hp{};
    std::vector<int32_t> expert_used;
    std::map<std::string, tensor> t;
    std::vector<tensor> audio_embd;
    tensor text_embd, spk_lda_w, spk_lda_b, spk_proj_w, spk_proj_b, output_norm, output;
    std::vector<orc_layer> layers;
    std::vector<uint8_t> layer_skip;              // depth prune: nonzero = block bypassed (zonos2.h:116-121)
    int rd = 0, kmax = 0;
    bool finalized = false;
};

struct orc_kv {                                   // shapes copied: any model of the same shape may use it
    int n_layer = 0, nkv = 0, hd = 0;
    int n_slots = 0, S = 0;
    std::vector<std::vector<uint16_t>> k, v;      // per layer [slot][row][nkv][hd]
};

namespace {

bool kv_fits(const orc_model & m, const orc_kv & kv) {
    return kv.n_layer == (int) m.hp.n_layer && kv.nkv == (int) m.hp.n_head_kv && kv.hd == (int) m.hp.head_dim;
}

std::vector<float> to_f32(const tensor & t) {
    const int64_t n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    std::vector<float> out((size_t) n);
    const int64_t rows = n / t.ne[0];
    for (int64_t r = 0; r < rows; ++r)
        dequant_row(t.type, t.data + r * row_nbytes(t.type, t.ne[0]), out.data() + r * t.ne[0], t.ne[0]);
    return out;
}

const float * f32p(const tensor & t) { return (const float *) t.data; }

// get_rows on an embedding table [d, rows]
void table_row(const tensor & t, int64_t id, float * y) {
    dequant_row(t.type, t.data + id * row_nbytes(t.type, t.ne[0]), y, t.ne[0]);
}

// EDA router for one token (src/zonos2-graph.cpp:199-220). Exact contract, see header comment.
void router_token(const orc_model & m, const orc_layer & ly, const float * x, const float * state_in,
                  float * rh, float * logits, float * probs, int32_t * sel, float * w) {
    const int d = m.hp.n_embd, rd = m.rd, E = ly.n_exp, k = ly.top_k;
    for (int o = 0; o < rd; ++o) {
        float v = lane_dot(ly.r_down.data() + (int64_t) o * d, x, d) + ly.r_down_b[o];
        if (!ly.r_eda.empty() && state_in) v = v + state_in[o] * ly.r_eda[o];
        rh[o] = v;
    }
    std::vector<float> rn(rd), h1(rd), h2(rd), lg(E), pr(E);
    router_rms(rh, ly.r_norm.data(), rd, m.hp.rms_eps, rn.data());
    for (int o = 0; o < rd; ++o) h1[o] = z_gelu(chain8_dot(ly.r_m0.data() + (int64_t) o * rd, rn.data(), rd) + ly.r_m0_b[o]);
    for (int o = 0; o < rd; ++o) h2[o] = z_gelu(chain8_dot(ly.r_m2.data() + (int64_t) o * rd, h1.data(), rd) + ly.r_m2_b[o]);
    for (int e = 0; e < E; ++e) {
        lg[e] = chain8_dot(ly.r_m4.data() + (int64_t) e * rd, h2.data(), rd);
        if (!ly.logit_bias.empty()) lg[e] = lg[e] + ly.logit_bias[e];
        if (!ly.mask.empty()) lg[e] = lg[e] + ly.mask[e];          // graph.cpp:212
    }
    float mx = -INFINITY;
    for (int e = 0; e < E; ++e) mx = std::max(mx, lg[e]);
    std::vector<float> ex(E);
    double part[64];
    for (int l = 0; l < 64; ++l) part[l] = 0.0;
    for (int e = 0; e < E; ++e) { ex[e] = z_expf(lg[e] - mx); part[e % 64] += (double) ex[e]; }
    const float inv = (float) (1.0 / tree64d(part));
    for (int e = 0; e < E; ++e) pr[e] = ex[e] * inv;
    std::vector<float> sc(E);
    for (int e = 0; e < E; ++e) sc[e] = pr[e] + ly.r_bias[e];
    if (!ly.mask.empty()) for (int e = 0; e < E; ++e) sc[e] = sc[e] + ly.mask[e];   // graph.cpp:218
    std::vector<int> idx(E);
    std::iota(idx.begin(), idx.end(), 0);
    std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) { return sc[a] > sc[b]; });
    for (int j = 0; j < k; ++j) { sel[j] = idx[j]; w[j] = pr[idx[j]]; }
    if (logits) std::memcpy(logits, lg.data(), sizeof(float) * E);
    if (probs) std::memcpy(probs, pr.data(), sizeof(float) * E);
}

// mul_mat_id gate/up + SwiGLU + down + route weight, k-sum in route order (graph.cpp:222-238)
void experts_fwd(const orc_model & m, const orc_layer & ly, int T, const float * x, const int32_t * sel,
                 const float * w, float * eo, float * out) {
    const int d = m.hp.n_embd, ff = (int) ly.up_exps.ne[1], k = ly.top_k;
    const int64_t R = (int64_t) T * k;
    std::vector<qact> ax(T), axg(T);
    for (int t = 0; t < T; ++t) {
        quantize_act(act_kind_for(ly.up_exps.type), x + (int64_t) t * d, d, ax[t]);
        quantize_act(act_kind_for(ly.gate_exps.type), x + (int64_t) t * d, d, axg[t]);
    }
    std::vector<float> y((size_t) R * ff);
    const int64_t rbu = row_nbytes(ly.up_exps.type, d), rbg = row_nbytes(ly.gate_exps.type, d);
    const int64_t ch = 64;
    parallel_for(R * ((ff + ch - 1) / ch), [&](int64_t it) {
        const int64_t r = it / ((ff + ch - 1) / ch), c = it % ((ff + ch - 1) / ch);
        const int t = (int) (r / k), e = sel[r];
        const uint8_t * up = ly.up_exps.data + (int64_t) e * ff * rbu;
        const uint8_t * gt = ly.gate_exps.data + (int64_t) e * ff * rbg;
        for (int64_t o = c * ch; o < std::min<int64_t>(ff, (c + 1) * ch); ++o) {
            const float u = dot_row(ly.up_exps.type, up + o * rbu, ax[t]);
            const float g = dot_row(ly.gate_exps.type, gt + o * rbg, axg[t]);
            y[r * ff + o] = u * z_silu(g);
        }
    });
    std::vector<qact> ay(R);
    for (int64_t r = 0; r < R; ++r) quantize_act(act_kind_for(ly.down_exps.type), y.data() + r * ff, ff, ay[r]);
    const int64_t rbd = row_nbytes(ly.down_exps.type, ff);
    std::vector<float> e_out((size_t) R * d);
    parallel_for(R * ((d + ch - 1) / ch), [&](int64_t it) {
        const int64_t r = it / ((d + ch - 1) / ch), c = it % ((d + ch - 1) / ch);
        const int e = sel[r];
        const uint8_t * dn = ly.down_exps.data + (int64_t) e * d * rbd;
        for (int64_t o = c * ch; o < std::min<int64_t>(d, (c + 1) * ch); ++o)
            e_out[r * d + o] = dot_row(ly.down_exps.type, dn + o * rbd, ay[r]) * w[r];
    });
    if (eo) std::memcpy(eo, e_out.data(), sizeof(float) * R * d);
    for (int t = 0; t < T; ++t)
        for (int i = 0; i < d; ++i) {
            float s = e_out[((int64_t) t * k) * d + i];
            for (int j = 1; j < k; ++j) s = s + e_out[((int64_t) t * k + j) * d + i];
            out[(int64_t) t * d + i] = s;
        }
}

void dense_fwd(const orc_layer & ly, int T, const float * x, float * out) {
    const int64_t ff = ly.ffn_up.ne[1], d = ly.ffn_up.ne[0];
    std::vector<float> up((size_t) T * ff), gt((size_t) T * ff);
    matmul(ly.ffn_up, 0, T, x, up.data());
    matmul(ly.ffn_gate, 0, T, x, gt.data());
    for (int64_t i = 0; i < (int64_t) T * ff; ++i) up[i] = up[i] * z_silu(gt[i]);
    (void) d;
    matmul(ly.ffn_down, 0, T, up.data(), out);
}

// Decode attention for T columns: QKV + gate projections, QK-norm, |temp|, RoPE, KV append (f16),
// flash_attn_ext over the slot's band [0, n_past] (graph.cpp:107-175). The query is rounded to f16 as
// ggml's CPU flash attention does for an F16 cache. ggml's accumulation order inside flash_attn_ext
// is not known here; the order is fixed to the device decode kernels' split softmax: chunks of
// ATT_ROWS cache rows, each with its own max / exp sum / unnormalised P.V in fp32, merged with
// weights exp(m_c - M) as written below.
constexpr int ATT_ROWS = 64;
void attention_fwd(const orc_model & m, orc_kv & kv, int L, int T, const int32_t * slot_idx, const int32_t * n_past,
                   const float * cur, float * q_cap, float * k_cap, float * v_cap, float * g_cap,
                   float * attn_o, float * attn_out) {
    const orc_layer & ly = m.layers[L];
    const int d = m.hp.n_embd, hd = m.hp.head_dim, nh = m.hp.n_head, nkv = m.hp.n_head_kv;
    const int S = kv.S;
    std::vector<float> q((size_t) T * nh * hd), k((size_t) T * nkv * hd), v((size_t) T * nkv * hd), g((size_t) T * nh);
    matmul(ly.gater, 0, T, cur, g.data());
    matmul(ly.wq, 0, T, cur, q.data());
    matmul(ly.wk, 0, T, cur, k.data());
    matmul(ly.wv, 0, T, cur, v.data());
    for (auto & x : g) x = z_sigmoid(x);
    const float * temp = f32p(ly.attn_temp);
    for (int t = 0; t < T; ++t) {
        for (int h = 0; h < nh; ++h) {
            float * qh = &q[((int64_t) t * nh + h) * hd];
            qk_norm(qh, hd, m.hp.qk_norm_eps, temp[h]);
        }
        for (int h = 0; h < nkv; ++h) {
            float * kh = &k[((int64_t) t * nkv + h) * hd];
            qk_norm(kh, hd, m.hp.qk_norm_eps, 1.0f);
        }
        rope_inplace(&q[(int64_t) t * nh * hd], nh, hd, n_past[t], m.hp.rope_freq_base);
        rope_inplace(&k[(int64_t) t * nkv * hd], nkv, hd, n_past[t], m.hp.rope_freq_base);
        uint16_t * kc = kv.k[L].data() + ((int64_t) slot_idx[t] * S + n_past[t]) * nkv * hd;
        uint16_t * vc = kv.v[L].data() + ((int64_t) slot_idx[t] * S + n_past[t]) * nkv * hd;
        for (int i = 0; i < nkv * hd; ++i) { kc[i] = to_f16(k[(int64_t) t * nkv * hd + i]); vc[i] = to_f16(v[(int64_t) t * nkv * hd + i]); }
    }
    if (q_cap) std::memcpy(q_cap, q.data(), q.size() * 4);
    if (k_cap) std::memcpy(k_cap, k.data(), k.size() * 4);
    if (v_cap) std::memcpy(v_cap, v.data(), v.size() * 4);
    if (g_cap) std::memcpy(g_cap, g.data(), g.size() * 4);
    const float scale = 1.0f / std::sqrt((float) hd);
    const int grp = nh / nkv;
    // parts of the chunk merge's weighted sum: 8 / hpb, hpb = the smallest power of two <= 8 that
    // divides the group and whose heads span whole 256-element blocks (else 1)
    int hpb = 0;
    for (int hb = 1; hb <= 8 && !hpb; hb *= 2)
        if (grp % hb == 0 && (hb * hd) % 256 == 0) hpb = hb;
    const int parts = 8 / (hpb ? hpb : 1);
    std::vector<float> o((size_t) T * nh * hd);
    parallel_for((int64_t) T * nh, [&](int64_t it) {
        const int t = (int) (it / nh), h = (int) (it % nh), gk = h / grp;
        const int n = n_past[t] + 1, nc = (n_past[t] + ATT_ROWS) / ATT_ROWS;
        const uint16_t * kb = kv.k[L].data() + (int64_t) slot_idx[t] * S * nkv * hd;
        const uint16_t * vb = kv.v[L].data() + (int64_t) slot_idx[t] * S * nkv * hd;
        std::vector<float> qh(hd), mc(nc), lc(nc), oc((size_t) nc * hd, 0.0f);
        for (int i = 0; i < hd; ++i) qh[i] = from_f16(to_f16(q[((int64_t) t * nh + h) * hd + i]));
        // per chunk of ATT_ROWS rows: scores (fma chain over the head dims), chunk max, exp, sum
        // (xor butterfly, lane = row), unnormalised P.V (fma chain over the rows)
        for (int c = 0; c < nc; ++c) {
            const int r0 = c * ATT_ROWS, nr = std::min(ATT_ROWS, n - r0);
            float sc[ATT_ROWS], pe[64];
            float mx = -INFINITY;
            for (int r = 0; r < nr; ++r) {
                const uint16_t * kr = kb + ((int64_t) (r0 + r) * nkv + gk) * hd;
                float acc = 0.0f;
                for (int i = 0; i < hd; ++i) acc = std::fma(qh[i], from_f16(kr[i]), acc);
                sc[r] = acc * scale;
                mx = std::max(mx, sc[r]);
            }
            for (int l = 0; l < 64; ++l) pe[l] = l < nr ? z_expf(sc[l] - mx) : 0.0f;
            float * ov = &oc[(size_t) c * hd];
            for (int r = 0; r < nr; ++r) {
                const uint16_t * vr = vb + ((int64_t) (r0 + r) * nkv + gk) * hd;
                for (int i = 0; i < hd; ++i) ov[i] = std::fma(pe[r], from_f16(vr[i]), ov[i]);
            }
            mc[c] = mx;
            lc[c] = tree64(pe);
        }
        // merge: weights e_c = exp(m_c - M); denominator: lane l folds chunks l, l + 64, ... with fma,
        // then the xor butterfly; numerator: part p folds chunks p, p + parts, ... with fma, and the
        // parts add in order; out = num * (gate / den)
        float M = -INFINITY;
        for (int c = 0; c < nc; ++c) M = std::max(M, mc[c]);
        std::vector<float> e(nc);
        float dl[64];
        for (int l = 0; l < 64; ++l) dl[l] = 0.0f;
        for (int c = 0; c < nc; ++c) { e[c] = z_expf(mc[c] - M); dl[c % 64] = std::fma(e[c], lc[c], dl[c % 64]); }
        const float den = tree64(dl);
        const float gd = g[(int64_t) t * nh + h] / den;
        for (int i = 0; i < hd; ++i) {
            float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            for (int c = 0; c < nc; ++c) acc[c % parts] = std::fma(e[c], oc[(size_t) c * hd + i], acc[c % parts]);
            float num = 0.0f;
            for (int p = 0; p < parts; ++p) num += acc[p];
            o[((int64_t) t * nh + h) * hd + i] = num * gd;
        }
    });
    if (attn_o) std::memcpy(attn_o, o.data(), o.size() * 4);
    matmul(ly.wo, 0, T, o.data(), attn_out);
    (void) d;
}

float * cap_at(float * base, int L, int64_t per_layer) { return base ? base + (int64_t) L * per_layer : nullptr; }

int check_layer(const orc_model * m, int L) {
    if (!m || !m->finalized) return fail("model not finalized");
    if (L < 0 || L >= m->hp.n_layer) return fail("layer out of range");
    return 0;
}

} // namespace

// ====================================================================== C API
extern "C" {

const char * orc_last_error(void) { return g_err.c_str(); }
int orc_set_threads(int n) { g_threads = n; return 0; }

orc_model * orc_model_create(const orc_hparams * hp) {
    if (!hp || hp->n_layer <= 0 || !hp->expert_used) { g_err = "bad hparams"; return nullptr; }
    auto * m = new orc_model();
    m->hp = *hp;
    m->expert_used.assign(hp->expert_used, hp->expert_used + hp->n_layer);
    m->hp.expert_used = m->expert_used.data();
    return m;
}

int orc_model_set(orc_model * m, const char * name, int type, const int64_t ne[4], const void * data) {
    if (!m || !name || !data || blk_bytes(type) < 0) return fail("bad tensor");
    if (ne[0] % blk_elems(type)) return fail(std::string("row not block aligned: ") + name);
    tensor t; t.type = type; t.data = (const uint8_t *) data;
    for (int i = 0; i < 4; ++i) t.ne[i] = ne[i] > 0 ? ne[i] : 1;
    m->t[name] = t;
    return 0;
}

int orc_model_finalize(orc_model * m) {
    if (!m) return fail("null model");
    auto & hp = m->hp;
    std::string missing;
    auto T = [&](const std::string & n) { auto it = m->t.find(n); return it == m->t.end() ? tensor() : it->second; };
    auto R = [&](const std::string & n) { tensor x = T(n); if (!x.ok()) missing += n + " "; return x; };
    m->audio_embd.resize(hp.n_codebooks);
    for (int i = 0; i < hp.n_codebooks; ++i) m->audio_embd[i] = R("audio_embd." + std::to_string(i) + ".weight");
    m->text_embd = R("text_embd.weight");
    m->output_norm = R("output_norm.weight");
    m->output = R("output.weight");
    m->spk_lda_w = T("spk_lda.weight"); m->spk_lda_b = T("spk_lda.bias");
    m->spk_proj_w = T("spk_proj.weight"); m->spk_proj_b = T("spk_proj.bias");
    m->layers.assign(hp.n_layer, orc_layer());
    m->kmax = 0; m->rd = 0;
    for (int L = 0; L < hp.n_layer; ++L) {
        orc_layer & ly = m->layers[L];
        const std::string b = "blk." + std::to_string(L) + ".";
        ly.attn_norm = R(b + "attn_norm.weight"); ly.ffn_norm = R(b + "ffn_norm.weight");
        ly.wq = R(b + "attn_q.weight"); ly.wk = R(b + "attn_k.weight"); ly.wv = R(b + "attn_v.weight");
        ly.wo = R(b + "attn_output.weight"); ly.attn_temp = R(b + "attn_temp"); ly.gater = R(b + "attn_gate.weight");
        ly.top_k = hp.expert_used[L];
        ly.is_moe = ly.top_k > 0;
        if (!ly.is_moe) {
            ly.ffn_up = R(b + "ffn_up.weight"); ly.ffn_gate = R(b + "ffn_gate.weight"); ly.ffn_down = R(b + "ffn_down.weight");
            continue;
        }
        ly.gate_exps = R(b + "ffn_gate_exps.weight"); ly.up_exps = R(b + "ffn_up_exps.weight");
        ly.down_exps = R(b + "ffn_down_exps.weight");
        ly.router_down = R(b + "router_down.weight"); ly.router_down_b = R(b + "router_down.bias");
        ly.router_mlp0 = R(b + "router_mlp0.weight"); ly.router_mlp0_b = R(b + "router_mlp0.bias");
        ly.router_mlp2 = R(b + "router_mlp2.weight"); ly.router_mlp2_b = R(b + "router_mlp2.bias");
        ly.router_mlp4 = R(b + "router_mlp4.weight"); ly.router_norm = R(b + "router_norm.weight");
        ly.router_bias = R(b + "router_bias"); ly.router_eda_scale = T(b + "router_eda_scale");
        if (!missing.empty()) continue;
        ly.n_exp = (int) ly.up_exps.ne[2];
        if (ly.top_k > ly.n_exp) return fail("top_k > n_expert at layer " + std::to_string(L));
        m->kmax = std::max(m->kmax, ly.top_k);
        m->rd = (int) ly.router_down.ne[1];
        ly.r_down = to_f32(ly.router_down); ly.r_down_b = to_f32(ly.router_down_b);
        ly.r_m0 = to_f32(ly.router_mlp0); ly.r_m0_b = to_f32(ly.router_mlp0_b);
        ly.r_m2 = to_f32(ly.router_mlp2); ly.r_m2_b = to_f32(ly.router_mlp2_b);
        ly.r_m4 = to_f32(ly.router_mlp4); ly.r_norm = to_f32(ly.router_norm);
        ly.r_bias = to_f32(ly.router_bias);
        if (ly.router_eda_scale.ok()) ly.r_eda = to_f32(ly.router_eda_scale);
    }
    if (!missing.empty()) return fail("missing tensors: " + missing);
    // 1-D tensors are read as fp32 vectors (the reference keeps them F32, quantize.cpp:117)
    std::vector<const tensor *> vecs = {&m->output_norm};
    if (m->spk_lda_b.ok()) vecs.push_back(&m->spk_lda_b);
    if (m->spk_proj_b.ok()) vecs.push_back(&m->spk_proj_b);
    for (auto & ly : m->layers) { vecs.push_back(&ly.attn_norm); vecs.push_back(&ly.ffn_norm); vecs.push_back(&ly.attn_temp); }
    for (const tensor * t : vecs) if (t->type != 0) return fail("1-D norm/bias/temp tensors must be F32");
    m->finalized = true;
    return 0;
}

int orc_model_set_logit_bias(orc_model * m, int layer, const float * bias) {
    if (int rc = check_layer(m, layer)) return rc;
    orc_layer & ly = m->layers[layer];
    if (!ly.is_moe) return fail("layer is not MoE");
    if (bias) ly.logit_bias.assign(bias, bias + ly.n_exp); else ly.logit_bias.clear();
    return 0;
}

// zonos2_set_expert_mask for one layer (src/zonos2.cpp:228-234): keep[e] != 0 -> 0, else -inf
int orc_model_set_expert_mask(orc_model * m, int layer, const uint8_t * keep) {
    if (int rc = check_layer(m, layer)) return rc;
    orc_layer & ly = m->layers[layer];
    if (!ly.is_moe) return fail("layer is not MoE");
    ly.mask.clear();
    if (keep) for (int e = 0; e < ly.n_exp; ++e) ly.mask.push_back(keep[e] ? 0.0f : -INFINITY);
    return 0;
}

int orc_model_set_layer_skip(orc_model * m, const uint8_t * skip) {
    if (!m) return fail("null model");
    if (skip) m->layer_skip.assign(skip, skip + m->hp.n_layer); else m->layer_skip.clear();
    return 0;
}

void orc_model_free(orc_model * m) { delete m; }

orc_kv * orc_kv_create(const orc_model * m, int n_slots, int slot_cap_frames) {
    if (!m || n_slots <= 0 || slot_cap_frames <= 0) { g_err = "bad kv args"; return nullptr; }
    auto * kv = new orc_kv();
    kv->n_layer = m->hp.n_layer; kv->nkv = m->hp.n_head_kv; kv->hd = m->hp.head_dim; kv->n_slots = n_slots;
    kv->S = ((slot_cap_frames + 255) / 256) * 256;            // graph.cpp:610, 644
    const int64_t per = (int64_t) n_slots * kv->S * m->hp.n_head_kv * m->hp.head_dim;
    kv->k.assign(m->hp.n_layer, std::vector<uint16_t>((size_t) per, 0));
    kv->v.assign(m->hp.n_layer, std::vector<uint16_t>((size_t) per, 0));
    return kv;
}

int orc_kv_slot_cap(const orc_kv * kv) { return kv ? kv->S : 0; }

int orc_kv_write(orc_kv * kv, int L, int slot, int row0, int n, const uint16_t * k, const uint16_t * v) {
    if (!kv || L < 0 || L >= kv->n_layer || slot < 0 || slot >= kv->n_slots || row0 < 0 || n < 0 || row0 + n > kv->S)
        return fail("kv_write out of range");
    const int64_t w = (int64_t) kv->nkv * kv->hd;
    const int64_t off = ((int64_t) slot * kv->S + row0) * w;
    if (k) std::memcpy(kv->k[L].data() + off, k, (size_t) n * w * 2);
    if (v) std::memcpy(kv->v[L].data() + off, v, (size_t) n * w * 2);
    return 0;
}

int orc_kv_read(const orc_kv * kv, int L, int slot, int row0, int n, uint16_t * k, uint16_t * v) {
    if (!kv || L < 0 || L >= kv->n_layer || slot < 0 || slot >= kv->n_slots || row0 < 0 || n < 0 || row0 + n > kv->S)
        return fail("kv_read out of range");
    const int64_t w = (int64_t) kv->nkv * kv->hd;
    const int64_t off = ((int64_t) slot * kv->S + row0) * w;
    if (k) std::memcpy(k, kv->k[L].data() + off, (size_t) n * w * 2);
    if (v) std::memcpy(v, kv->v[L].data() + off, (size_t) n * w * 2);
    return 0;
}

void orc_kv_free(orc_kv * kv) { delete kv; }

// rows_of_a_slot: several rows may belong to one slot (distinct n_past; all rows' K/V are appended
// before the attention, so a slot's rows attend to each other causally); emb_map: per row -1 (ids)
// or the row of emb it takes (NULL: every row takes emb[t] when emb is given).
static int step_impl(orc_model * m, orc_kv * kv, int T, const int32_t * slot_idx, const int32_t * n_past,
                     const int32_t * ids, const float * emb, const int32_t * emb_map, float * logits, orc_capture * cap,
                     bool rows_of_a_slot) {
    if (!m || !m->finalized || !kv) return fail("model/kv not ready");
    if (!kv_fits(*m, *kv)) return fail("kv cache shape differs from the model");
    if (T <= 0 || !slot_idx || !n_past || (!ids && !emb) || !logits) return fail("bad step args");
    const auto & hp = m->hp;
    const int d = hp.n_embd, W = hp.n_codebooks + 1, nh = hp.n_head, nkv = hp.n_head_kv, hd = hp.head_dim;
    for (int t = 0; t < T; ++t) {
        if (slot_idx[t] < 0 || slot_idx[t] >= kv->n_slots) return fail("slot out of range");
        if (n_past[t] < 0 || n_past[t] >= kv->S) return fail("n_past out of range");
        for (int u = 0; u < t; ++u)
            if (slot_idx[u] == slot_idx[t] && (!rows_of_a_slot || n_past[u] == n_past[t])) return fail("duplicate slot row");
    }
    // embedding sum in column order (graph.cpp:248-260), then emb_norm (graph.cpp:300)
    std::vector<float> x((size_t) T * d), res((size_t) T * d), cur((size_t) T * d), tmp(d);
    for (int t = 0; t < T; ++t) {
        float * e = &x[(int64_t) t * d];
        const int er = emb ? (emb_map ? emb_map[t] : t) : -1;
        if (er >= 0) std::memcpy(e, emb + (int64_t) er * d, sizeof(float) * d);
        else {
            for (int kk = 0; kk < W; ++kk) {
                const tensor & tb = kk < hp.n_codebooks ? m->audio_embd[kk] : m->text_embd;
                const int id = ids[(int64_t) t * W + kk];
                if (id < 0 || id >= tb.ne[1]) return fail("token id out of range");
                table_row(tb, id, tmp.data());
                if (kk == 0) std::memcpy(e, tmp.data(), sizeof(float) * d);
                else for (int i = 0; i < d; ++i) e[i] = e[i] + tmp[i];
            }
        }
        rms_norm(e, nullptr, d, hp.rms_eps, e);
    }
    const int K = std::max(1, m->kmax), E = std::max(1, hp.n_expert), rd = std::max(1, m->rd);
    std::vector<float> state;                                  // EDA state threaded across MoE layers
    bool have_state = false;
    std::vector<float> ffn((size_t) T * d), attn_out((size_t) T * d);
    for (int L = 0; L < hp.n_layer; ++L) {
        const orc_layer & ly = m->layers[L];
        if (L == 0) res = x;
        else for (size_t i = 0; i < res.size(); ++i) res[i] = x[i] + res[i];
        if (L < (int) m->layer_skip.size() && m->layer_skip[L]) {   // graph.cpp:334-341: identity block
            for (size_t i = 0; i < res.size(); ++i) x[i] = 0.0f * res[i];
            continue;
        }
        if (cap && cap->res_in) std::memcpy(cap_at(cap->res_in, L, (int64_t) T * d), res.data(), res.size() * 4);
        for (int t = 0; t < T; ++t) rms_norm(&res[(int64_t) t * d], f32p(ly.attn_norm), d, hp.rms_eps, &cur[(int64_t) t * d]);
        if (cap && cap->attn_in) std::memcpy(cap_at(cap->attn_in, L, (int64_t) T * d), cur.data(), cur.size() * 4);
        attention_fwd(*m, *kv, L, T, slot_idx, n_past, cur.data(),
                      cap ? cap_at(cap->q, L, (int64_t) T * nh * hd) : nullptr,
                      cap ? cap_at(cap->k, L, (int64_t) T * nkv * hd) : nullptr,
                      cap ? cap_at(cap->v, L, (int64_t) T * nkv * hd) : nullptr,
                      cap ? cap_at(cap->gate, L, (int64_t) T * nh) : nullptr,
                      cap ? cap_at(cap->attn_o, L, (int64_t) T * nh * hd) : nullptr, attn_out.data());
        if (cap && cap->attn_out) std::memcpy(cap_at(cap->attn_out, L, (int64_t) T * d), attn_out.data(), attn_out.size() * 4);
        for (size_t i = 0; i < res.size(); ++i) res[i] = attn_out[i] + res[i];
        for (int t = 0; t < T; ++t) rms_norm(&res[(int64_t) t * d], f32p(ly.ffn_norm), d, hp.rms_eps, &cur[(int64_t) t * d]);
        if (cap && cap->ffn_in) std::memcpy(cap_at(cap->ffn_in, L, (int64_t) T * d), cur.data(), cur.size() * 4);
        if (ly.is_moe) {
            std::vector<float> rh((size_t) T * m->rd), lg((size_t) T * ly.n_exp), pr((size_t) T * ly.n_exp), w((size_t) T * ly.top_k);
            std::vector<int32_t> sel((size_t) T * ly.top_k);
            for (int t = 0; t < T; ++t)
                router_token(*m, ly, &cur[(int64_t) t * d], have_state ? &state[(int64_t) t * m->rd] : nullptr,
                             &rh[(int64_t) t * m->rd], &lg[(int64_t) t * ly.n_exp], &pr[(int64_t) t * ly.n_exp],
                             &sel[(int64_t) t * ly.top_k], &w[(int64_t) t * ly.top_k]);
            state = rh; have_state = true;
            if (cap) {
                for (int t = 0; t < T; ++t) {
                    if (cap->router_state) std::memcpy(cap->router_state + ((int64_t) L * T + t) * rd, &rh[(int64_t) t * m->rd], m->rd * 4);
                    if (cap->router_logits) std::memcpy(cap->router_logits + ((int64_t) L * T + t) * E, &lg[(int64_t) t * ly.n_exp], ly.n_exp * 4);
                    if (cap->probs) std::memcpy(cap->probs + ((int64_t) L * T + t) * E, &pr[(int64_t) t * ly.n_exp], ly.n_exp * 4);
                    if (cap->sel) std::memcpy(cap->sel + ((int64_t) L * T + t) * K, &sel[(int64_t) t * ly.top_k], ly.top_k * 4);
                    if (cap->weights) std::memcpy(cap->weights + ((int64_t) L * T + t) * K, &w[(int64_t) t * ly.top_k], ly.top_k * 4);
                }
            }
            experts_fwd(*m, ly, T, cur.data(), sel.data(), w.data(), nullptr, ffn.data());
        } else {
            dense_fwd(ly, T, cur.data(), ffn.data());
        }
        if (cap && cap->ffn_out) std::memcpy(cap_at(cap->ffn_out, L, (int64_t) T * d), ffn.data(), ffn.size() * 4);
        x = ffn;
    }
    for (size_t i = 0; i < res.size(); ++i) res[i] = x[i] + res[i];
    for (int t = 0; t < T; ++t) rms_norm(&res[(int64_t) t * d], f32p(m->output_norm), d, hp.rms_eps, &cur[(int64_t) t * d]);
    if (cap && cap->out_norm) std::memcpy(cap->out_norm, cur.data(), cur.size() * 4);
    const int64_t nout = (int64_t) hp.n_codebooks * hp.audio_vocab;
    matmul(m->output, 0, T, cur.data(), logits);
    const float c = hp.logit_softcap;
    if (c > 0.0f)                                               // graph.cpp:359-362
        for (int64_t i = 0; i < (int64_t) T * nout; ++i) logits[i] = z_softcap(logits[i], c);
    return 0;
}

int orc_step(orc_model * m, orc_kv * kv, int T, const int32_t * slot_idx, const int32_t * n_past,
             const int32_t * ids, const float * emb, float * logits, orc_capture * cap) {
    return step_impl(m, kv, T, slot_idx, n_past, ids, emb, nullptr, logits, cap, false);
}

int orc_step_mixed(orc_model * m, orc_kv * kv, int T, const int32_t * slot_idx, const int32_t * n_past,
                   const int32_t * ids, const int32_t * emb_map, const float * emb, float * logits) {
    return step_impl(m, kv, T, slot_idx, n_past, ids, emb, emb_map, logits, nullptr, true);
}

int orc_prefill(orc_model * m, orc_kv * kv, int slot, const int32_t * ids, int n0,
                const float * spk, int spk_pos, const float * delta, float * last_logits) {
    if (!m || !m->finalized || !kv) return fail("model/kv not ready");
    if (!kv_fits(*m, *kv)) return fail("kv cache shape differs from the model");
    if (slot < 0 || slot >= kv->n_slots) return fail("slot out of range");
    if (n0 <= 0 || n0 > kv->S) return fail("n0 exceeds slot_cap");
    const auto & hp = m->hp;
    const int d = hp.n_embd, W = hp.n_codebooks + 1, nh = hp.n_head, nkv = hp.n_head_kv, hd = hp.head_dim;
    const int S = kv->S, n = n0;
    std::vector<float> x((size_t) n * d), res((size_t) n * d), cur((size_t) n * d), tmp(d);
    for (int t = 0; t < n; ++t) {
        float * e = &x[(int64_t) t * d];
        for (int kk = 0; kk < W; ++kk) {
            const tensor & tb = kk < hp.n_codebooks ? m->audio_embd[kk] : m->text_embd;
            const int id = ids[(int64_t) t * W + kk];
            if (id < 0 || id >= tb.ne[1]) return fail("token id out of range");
            table_row(tb, id, tmp.data());
            if (kk == 0) std::memcpy(e, tmp.data(), sizeof(float) * d);
            else for (int i = 0; i < d; ++i) e[i] = e[i] + tmp[i];
        }
    }
    if (spk && spk_pos >= 0 && spk_pos < n) {                  // graph.cpp:262-297
        if (!m->spk_lda_w.ok() || !m->spk_proj_w.ok()) return fail("speaker tensors missing");
        const int64_t lda = m->spk_lda_w.ne[1];
        std::vector<float> sl(lda), sp(d);
        matmul(m->spk_lda_w, 0, 1, spk, sl.data());
        const float * lb = f32p(m->spk_lda_b);
        for (int64_t i = 0; i < lda; ++i) sl[i] = sl[i] + lb[i];
        matmul(m->spk_proj_w, 0, 1, sl.data(), sp.data());
        const float * pb = f32p(m->spk_proj_b);
        for (int i = 0; i < d; ++i) { sp[i] = sp[i] + pb[i]; if (delta) sp[i] = sp[i] + delta[i]; }
        std::memcpy(&x[(int64_t) spk_pos * d], sp.data(), sizeof(float) * d);
    }
    for (int t = 0; t < n; ++t) rms_norm(&x[(int64_t) t * d], nullptr, d, hp.rms_eps, &x[(int64_t) t * d]);
    std::vector<float> state; bool have_state = false;
    std::vector<float> ffn((size_t) n * d), ao((size_t) n * d);
    const float scale = 1.0f / std::sqrt((float) hd);
    const int grp = nh / nkv;
    for (int L = 0; L < hp.n_layer; ++L) {
        const orc_layer & ly = m->layers[L];
        if (L == 0) res = x; else for (size_t i = 0; i < res.size(); ++i) res[i] = x[i] + res[i];
        if (L < (int) m->layer_skip.size() && m->layer_skip[L]) {
            for (size_t i = 0; i < res.size(); ++i) x[i] = 0.0f * res[i];
            continue;
        }
        for (int t = 0; t < n; ++t) rms_norm(&res[(int64_t) t * d], f32p(ly.attn_norm), d, hp.rms_eps, &cur[(int64_t) t * d]);
        // manual causal attention over the n new rows with fp32 K/V (graph.cpp:155-169)
        std::vector<float> q((size_t) n * nh * hd), k((size_t) n * nkv * hd), v((size_t) n * nkv * hd), g((size_t) n * nh);
        matmul(ly.gater, 0, n, cur.data(), g.data());
        matmul(ly.wq, 0, n, cur.data(), q.data());
        matmul(ly.wk, 0, n, cur.data(), k.data());
        matmul(ly.wv, 0, n, cur.data(), v.data());
        for (auto & z : g) z = z_sigmoid(z);
        const float * temp = f32p(ly.attn_temp);
        for (int t = 0; t < n; ++t) {
            for (int h = 0; h < nh; ++h) {
                float * qh = &q[((int64_t) t * nh + h) * hd];
                qk_norm(qh, hd, hp.qk_norm_eps, temp[h]);
            }
            for (int h = 0; h < nkv; ++h) { float * kh = &k[((int64_t) t * nkv + h) * hd]; qk_norm(kh, hd, hp.qk_norm_eps, 1.0f); }
            rope_inplace(&q[(int64_t) t * nh * hd], nh, hd, t, hp.rope_freq_base);
            rope_inplace(&k[(int64_t) t * nkv * hd], nkv, hd, t, hp.rope_freq_base);
            uint16_t * kc = kv->k[L].data() + ((int64_t) slot * S + t) * nkv * hd;
            uint16_t * vc = kv->v[L].data() + ((int64_t) slot * S + t) * nkv * hd;
            for (int i = 0; i < nkv * hd; ++i) { kc[i] = to_f16(k[(int64_t) t * nkv * hd + i]); vc[i] = to_f16(v[(int64_t) t * nkv * hd + i]); }
        }
        std::vector<float> o((size_t) n * nh * hd);
        parallel_for((int64_t) n * nh, [&](int64_t it) {
            const int t = (int) (it / nh), h = (int) (it % nh), gk = h / grp;
            std::vector<float> s(t + 1);
            float mx = -INFINITY;
            for (int p = 0; p <= t; ++p) {
                double acc = 0.0;
                for (int i = 0; i < hd; ++i) acc += (double) q[((int64_t) t * nh + h) * hd + i] * k[((int64_t) p * nkv + gk) * hd + i];
                s[p] = (float) acc * scale;
                mx = std::max(mx, s[p]);
            }
            double sum = 0.0;
            std::vector<double> acc(hd, 0.0);
            for (int p = 0; p <= t; ++p) {
                const double e = z_expf(s[p] - mx);
                sum += e;
                for (int i = 0; i < hd; ++i) acc[i] += e * v[((int64_t) p * nkv + gk) * hd + i];
            }
            for (int i = 0; i < hd; ++i) o[((int64_t) t * nh + h) * hd + i] = (float) (acc[i] / sum) * g[(int64_t) t * nh + h];
        });
        matmul(ly.wo, 0, n, o.data(), ao.data());
        for (size_t i = 0; i < res.size(); ++i) res[i] = ao[i] + res[i];
        for (int t = 0; t < n; ++t) rms_norm(&res[(int64_t) t * d], f32p(ly.ffn_norm), d, hp.rms_eps, &cur[(int64_t) t * d]);
        if (ly.is_moe) {
            std::vector<float> rh((size_t) n * m->rd), w((size_t) n * ly.top_k);
            std::vector<int32_t> sel((size_t) n * ly.top_k);
            for (int t = 0; t < n; ++t)
                router_token(*m, ly, &cur[(int64_t) t * d], have_state ? &state[(int64_t) t * m->rd] : nullptr,
                             &rh[(int64_t) t * m->rd], nullptr, nullptr, &sel[(int64_t) t * ly.top_k], &w[(int64_t) t * ly.top_k]);
            state = rh; have_state = true;
            experts_fwd(*m, ly, n, cur.data(), sel.data(), w.data(), nullptr, ffn.data());
        } else dense_fwd(ly, n, cur.data(), ffn.data());
        x = ffn;
    }
    for (size_t i = 0; i < res.size(); ++i) res[i] = x[i] + res[i];
    const int64_t nout = (int64_t) hp.n_codebooks * hp.audio_vocab;
    std::vector<float> hl(d);
    rms_norm(&res[(int64_t) (n - 1) * d], f32p(m->output_norm), d, hp.rms_eps, hl.data());
    matmul(m->output, 0, 1, hl.data(), last_logits);
    const float c = hp.logit_softcap;
    if (c > 0.0f) for (int64_t i = 0; i < nout; ++i) last_logits[i] = z_softcap(last_logits[i], c);
    return 0;
}

int orc_router(orc_model * m, int L, int T, const float * ffn_in, const float * state_in,
               float * rh, float * logits, float * probs, int32_t * sel, float * w) {
    if (int rc = check_layer(m, L)) return rc;
    const orc_layer & ly = m->layers[L];
    if (!ly.is_moe) return fail("layer is not MoE");
    const int d = m->hp.n_embd, rd = m->rd, E = ly.n_exp, k = ly.top_k;
    for (int t = 0; t < T; ++t)
        router_token(*m, ly, ffn_in + (int64_t) t * d, state_in ? state_in + (int64_t) t * rd : nullptr,
                     rh + (int64_t) t * rd, logits ? logits + (int64_t) t * E : nullptr,
                     probs ? probs + (int64_t) t * E : nullptr, sel + (int64_t) t * k, w + (int64_t) t * k);
    return 0;
}

// Token->expert grouping inside ggml_mul_mat_id: a stable counting sort of the flat route index
// r = t*k + j by expert (rows of an expert in ascending token, then j).
int orc_group(int T, int k, int E, const int32_t * sel, int32_t * counts, int32_t * offsets, int32_t * perm) {
    std::vector<int32_t> c(E, 0);
    for (int r = 0; r < T * k; ++r) { if (sel[r] < 0 || sel[r] >= E) return fail("expert id out of range"); ++c[sel[r]]; }
    std::vector<int32_t> off(E + 1, 0);
    for (int e = 0; e < E; ++e) off[e + 1] = off[e] + c[e];
    std::vector<int32_t> pos(off.begin(), off.end() - 1);
    for (int r = 0; r < T * k; ++r) perm[pos[sel[r]]++] = r;
    if (counts) std::memcpy(counts, c.data(), sizeof(int32_t) * E);
    if (offsets) std::memcpy(offsets, off.data(), sizeof(int32_t) * (E + 1));
    return 0;
}

int orc_experts(orc_model * m, int L, int T, const float * ffn_in, const int32_t * sel, const float * w,
                float * expert_out, float * out) {
    if (int rc = check_layer(m, L)) return rc;
    const orc_layer & ly = m->layers[L];
    if (!ly.is_moe) return fail("layer is not MoE");
    for (int r = 0; r < T * ly.top_k; ++r) if (sel[r] < 0 || sel[r] >= ly.n_exp) return fail("expert id out of range");
    experts_fwd(*m, ly, T, ffn_in, sel, w, expert_out, out);
    return 0;
}

int orc_dense_ffn(orc_model * m, int L, int T, const float * ffn_in, float * out) {
    if (int rc = check_layer(m, L)) return rc;
    if (m->layers[L].is_moe) return fail("layer is MoE");
    dense_fwd(m->layers[L], T, ffn_in, out);
    return 0;
}

int orc_attention(orc_model * m, orc_kv * kv, int L, int T, const int32_t * slot_idx, const int32_t * n_past,
                  const float * attn_in, float * attn_o, float * attn_out) {
    if (int rc = check_layer(m, L)) return rc;
    if (!kv || !kv_fits(*m, *kv)) return fail("kv cache shape differs from the model");
    attention_fwd(*m, *kv, L, T, slot_idx, n_past, attn_in, nullptr, nullptr, nullptr, nullptr, attn_o, attn_out);
    return 0;
}

int orc_dequant(int type, const void * src, float * dst, int64_t n) {
    if (blk_bytes(type) < 0 || n % blk_elems(type)) return fail("bad dequant args");
    dequant_row(type, (const uint8_t *) src, dst, n);
    return 0;
}

int orc_matmul(int type, const void * w, int64_t n_in, int64_t n_out, int T, const float * x, float * y) {
    if (blk_bytes(type) < 0 || n_in % blk_elems(type)) return fail("bad matmul args");
    tensor t; t.type = type; t.ne[0] = n_in; t.ne[1] = n_out; t.data = (const uint8_t *) w;
    matmul(t, 0, T, x, y);
    return 0;
}

int orc_quant_act(int act, const float * x, int64_t n, int8_t * q, float * d, int16_t * bsum, uint16_t * h) {
    qact a;
    quantize_act(act, x, n, a);
    if (q && !a.q.empty()) std::memcpy(q, a.q.data(), a.q.size());
    if (d && !a.d.empty()) std::memcpy(d, a.d.data(), a.d.size() * 4);
    if (bsum && !a.bsum.empty()) std::memcpy(bsum, a.bsum.data(), a.bsum.size() * 2);
    if (h && !a.h.empty()) std::memcpy(h, a.h.data(), a.h.size() * 2);
    return 0;
}

float orc_expf(float x) { return z_expf(x); }
void orc_sincos(float x, float * s, float * c) { z_sincos(x, *s, *c); }
float orc_softcap(float x, float cap) { return z_softcap(x, cap); }
float orc_erff(float x) { return z_erff(x); }
float orc_gelu_erf(float x) { return z_gelu(x); }
float orc_silu(float x) { return z_silu(x); }
int orc_rope(float * x, int n_heads, int hd, int pos, float base) { rope_inplace(x, n_heads, hd, pos, base); return 0; }
uint16_t orc_f32_to_f16(float x) { return to_f16(x); }
float orc_f16_to_f32(uint16_t h) { return from_f16(h); }

} // extern "C"

// ------------------------------------------------------------------ frame sampler
// exp(x) in double: x = n ln2 + r (ln2 in two parts, Cody-Waite), exp(r) by the degree-13 Taylor
// polynomial in Horner form with fma, times 2^n.
double orc_exp_d(double x) {
    if (x < -745.0) return 0.0;
    const double n = std::rint(x * 0x1.71547652b82fep+0);
    double r = std::fma(-n, 0x1.62e42fee00000p-1, x);
    r = std::fma(-n, 0x1.a39ef35793c76p-33, r);
    static const double c[14] = {0x1.6124613a86d09p-33, 0x1.1eed8eff8d898p-29, 0x1.ae64567f544e4p-26, 0x1.27e4fb7789f5cp-22,
                                 0x1.71de3a556c734p-19, 0x1.a01a01a01a01ap-16, 0x1.a01a01a01a01ap-13, 0x1.6c16c16c16c17p-10,
                                 0x1.1111111111111p-7, 0x1.5555555555555p-5, 0x1.5555555555555p-3, 0.5, 1.0, 1.0};
    double p = c[0];
    for (int i = 1; i < 14; ++i) p = std::fma(p, r, c[i]);
    return std::ldexp(p, (int) n);
}

int orc_sample(const float * in, int vocab, float temperature, int top_k, float top_p, float min_p,
               float rep_penalty, int rep_codebooks, int greedy, int cb, const int32_t * hist, int hist_len,
               double u, int exp_mode) {
    if (greedy) {
        int best = 0;
        for (int i = 1; i < vocab; ++i) if (in[i] > in[best]) best = i;
        return best;
    }
    std::vector<float> lg(in, in + vocab);
    if (rep_penalty != 1.0f && cb < rep_codebooks)
        for (int i = 0; i < hist_len; ++i) {
            const int t = hist[i];
            if (t >= 0 && t < vocab) lg[t] = lg[t] > 0.0f ? lg[t] / rep_penalty : lg[t] * rep_penalty;
        }
    if (temperature > 0.0f)
        for (float & v : lg) v /= temperature;
    std::vector<int> cand(vocab);
    for (int i = 0; i < vocab; ++i) cand[i] = i;
    const int k = top_k > 0 && top_k < vocab ? top_k : vocab;
    const auto by_logit = [&lg](int a, int b) { return lg[a] > lg[b]; };
    if (k < vocab) {
        std::partial_sort(cand.begin(), cand.begin() + k, cand.end(), by_logit);
        cand.resize(k);
    }
    const size_t n = cand.size();
    float mx = -1e30f;
    for (const int i : cand) mx = std::max(mx, lg[i]);
    std::vector<float> p(n);
    double z = 0.0;
    for (size_t j = 0; j < n; ++j) {
        const float x = lg[cand[j]] - mx;
        p[j] = exp_mode ? (float) orc_exp_d((double) x) : std::exp(x);
        z += p[j];
    }
    for (float & v : p) v = (float) (v / z);
    std::vector<int> rank(n);
    for (size_t j = 0; j < n; ++j) rank[j] = (int) j;
    std::sort(rank.begin(), rank.end(), [&p](int a, int b) { return p[a] > p[b]; });
    std::vector<char> keep(n, 1);
    if (top_p > 0.0f && top_p < 1.0f) {
        double c = 0.0;
        bool reached = false;
        for (const int r : rank) {
            if (reached) keep[r] = 0;
            c += p[r];
            if (c >= top_p) reached = true;
        }
    }
    if (min_p > 0.0f) {
        const float floor_p = min_p * p[rank[0]];
        for (size_t j = 0; j < n; ++j) if (p[j] < floor_p) keep[j] = 0;
    }
    double mass = 0.0;
    for (size_t j = 0; j < n; ++j) { if (!keep[j]) p[j] = 0.0f; mass += p[j]; }
    if (mass <= 0.0) return cand[rank[0]];
    const double r = u * (mass - 0.0) + 0.0;
    double acc = 0.0;
    for (size_t j = 0; j < n; ++j) {
        acc += p[j];
        if (acc >= r) return cand[j];
    }
    return cand[rank[0]];
}
