// z2h_common.h — device-side helpers shared by the decode-step kernels (gfx950, wave64).
//
// The exp / erf / GELU / SiLU implementations and the xor-butterfly reductions are part of the
// router's bit-exact contract (the CPU oracle restates them operation for operation): every source
// file is compiled with -ffp-contract=off, and fused multiply-adds are only the explicit fmaf calls.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace z2d {

constexpr int WAVE = 64;

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// exp: Cody-Waite reduction by ln2 (high part exact in the fma) + degree-7 Taylor polynomial.
__device__ __forceinline__ float z_expf(float x) {
    if (x > 88.72283f) return __builtin_inff();
    if (x < -103.97208f) return 0.0f;
    const float n = rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(n, -0.693145751953125f, x);
    r = __builtin_fmaf(n, -1.428606765330187e-06f, r);
    float p = 1.98412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return ldexpf(p, (int) n);
}

// fp32 pair -> f16 hi / lo pairs: hi = f16(x), lo = f16(x - hi) (x - hi is exact in fp32), so
// hi + lo carries x to about 2^-22 relative; low half = the first value.
__device__ __forceinline__ uint32_t f16_split2(float x0, float x1, uint32_t & lo) {
    const _Float16 h0 = (_Float16) x0, h1 = (_Float16) x1;
    const _Float16 l0 = (_Float16) (x0 - (float) h0), l1 = (_Float16) (x1 - (float) h1);
    lo = (uint32_t) __builtin_bit_cast(uint16_t, l0) | ((uint32_t) __builtin_bit_cast(uint16_t, l1) << 16);
    return (uint32_t) __builtin_bit_cast(uint16_t, h0) | ((uint32_t) __builtin_bit_cast(uint16_t, h1) << 16);
}

// exp in double for the sampler's softmax: x = n ln2 + r with ln2 split in two (Cody-Waite; n ln2_hi
// is exact for |n| < 2^21), |r| <= ln2 / 2, exp(r) by its degree-13 Taylor polynomial (truncation
// < 2^-58 relative) in Horner form with fma, scaled by 2^n. z_expf_cr rounds it to float: the
// correctly rounded expf except where exp(x) lies within ~2 double ulps of a float rounding boundary.
__device__ __forceinline__ double z_exp_d(double x) {
    if (x < -745.0) return 0.0;
    const double n = rint(x * 0x1.71547652b82fep+0);
    double r = __builtin_fma(-n, 0x1.62e42fee00000p-1, x);
    r = __builtin_fma(-n, 0x1.a39ef35793c76p-33, r);
    double p = 0x1.6124613a86d09p-33;                                    // 1/13!
    p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);
    p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);
    p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);
    p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);
    p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);
    p = __builtin_fma(p, r, 0x1.1111111111111p-7);
    p = __builtin_fma(p, r, 0x1.5555555555555p-5);
    p = __builtin_fma(p, r, 0x1.5555555555555p-3);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return ldexp(p, (int) n);
}
__device__ __forceinline__ float z_expf_cr(float x) { return (float) z_exp_d((double) x); }

// Logit softcap cap * tanh(x / cap): y = x * (1/cap) in fp32; tanh(|y|) in double, below 2^-10 by
// its Taylor series to y^5 (next term < 2^-60 relative), above it as 1 - 2 / (exp(2|y|) + 1); rounded
// to fp32, the sign restored, times cap. Every operation is IEEE double / fp32 as written, so the
// CPU oracle reproduces it bit for bit.
__device__ __forceinline__ float z_softcap(float x, float cap) {
    const float y = x * (1.0f / cap);
    const double a = fabs((double) y);
    double t;
    if (a < 0x1p-10) {
        const double a2 = a * a;
        t = a + (a * a2) * (-1.0 / 3.0 + a2 * (2.0 / 15.0));
    } else {
        t = 1.0 - 2.0 / (z_exp_d(2.0 * a) + 1.0);
    }
    return copysignf((float) t, y) * cap;
}

// erf: Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7).
__device__ __forceinline__ float z_erff(float x) {
    const float ax = fabsf(x);
    const float t = 1.0f / (1.0f + 0.3275911f * ax);
    float p = __builtin_fmaf(1.061405429f, t, -1.453152027f);
    p = __builtin_fmaf(p, t, 1.421413741f);
    p = __builtin_fmaf(p, t, -0.284496736f);
    p = __builtin_fmaf(p, t, 0.254829592f);
    p = p * t;
    const float y = 1.0f - p * z_expf(-(ax * ax));
    return copysignf(y, x);
}

// sin and cos of a RoPE angle (0 <= x < 2^24): the angle is reduced modulo 2 pi in double
// precision (the fp32 angle is exact in double; 2 pi in double is off by < 2.5e-16, so the reduced
// angle is good to ~1e-13 for angles below 2^24), then by quadrant to [-pi/4, pi/4], where degree-9 /
// degree-8 Taylor polynomials are accurate to < 4e-9. No library call, so no large-argument path.
__device__ __forceinline__ void z_sincos(float x, float & s, float & c) {
    const double xd = (double) x;
    const double k2 = rint(xd * 0.15915494309189533577);                 // turns
    const double rd = __builtin_fma(-k2, 6.28318530717958647692, xd);    // in [-pi, pi]
    const double q = rint(rd * 0.63661977236758134308);                  // quadrant, |q| <= 2
    const float r = (float) __builtin_fma(-q, 1.57079632679489661923, rd);
    const float r2 = r * r;
    float sp = 2.75573192e-6f;                                           // 1/9!
    sp = __builtin_fmaf(sp, r2, -1.98412698e-4f);
    sp = __builtin_fmaf(sp, r2, 8.33333333e-3f);
    sp = __builtin_fmaf(sp, r2, -1.66666667e-1f);
    const float sr = __builtin_fmaf(sp * r2, r, r);
    float cp = 2.48015873e-5f;                                           // 1/8!
    cp = __builtin_fmaf(cp, r2, -1.38888889e-3f);
    cp = __builtin_fmaf(cp, r2, 4.16666667e-2f);
    cp = __builtin_fmaf(cp, r2, -0.5f);
    const float cr = __builtin_fmaf(cp, r2, 1.0f);
    const int qi = ((int) q) & 3;
    s = qi == 0 ? sr : qi == 1 ? cr : qi == 2 ? -sr : -cr;
    c = qi == 0 ? cr : qi == 1 ? -sr : qi == 2 ? -cr : sr;
}

__device__ __forceinline__ float z_gelu(float x) { return (0.5f * x) * (1.0f + z_erff(x * 0.70710678118654752f)); }
__device__ __forceinline__ float z_silu(float x) { return x / (1.0f + z_expf(-x)); }
__device__ __forceinline__ float z_sigmoid(float x) { return 1.0f / (1.0f + z_expf(-x)); }

// Reductions over the 64 lanes with the tree of an xor butterfly (offsets 32, 16, 8, 4, 2, 1): at each
// level a node adds the two nodes of the level below that differ in one lane bit. Only lane 0's
// chain of the tree is formed (lane i < off adds lane i + off), the two cross-row levels by gfx950's
// lane-swap instructions and the four in-row levels by DPP row shifts, none of which goes through
// LDS; lane 0's value is then broadcast. Every addition is the one the butterfly makes (a + b and
// b + a are the same IEEE value), so the result equals the butterfly's bit for bit.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v))); }
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t) dpp_i<CTRL>((int) (uint32_t) u), hi = (uint32_t) dpp_i<CTRL>((int) (uint32_t) (u >> 32));
    return __builtin_bit_cast(double, ((uint64_t) hi << 32) | lo);
}
constexpr int DPP_ROW_SHL = 0x100;     // lane i reads lane i + n of its 16-lane row
// Lane i < 32 receives lane i + 32 (v_permlane32_swap trades rows 2-3 of its first operand for rows
// 0-1 of its second; with both operands v the second's rows 0-1 become v's rows 2-3).
__device__ __forceinline__ int up32_i(int v) {
    return (int) __builtin_amdgcn_permlane32_swap((unsigned) v, (unsigned) v, false, false)[1];
}
// Lane i of rows 0 and 2 receives lane i + 16 (v_permlane16_swap: rows 1 and 3 of the first operand
// for rows 0 and 2 of the second).
__device__ __forceinline__ int up16_i(int v) {
    return (int) __builtin_amdgcn_permlane16_swap((unsigned) v, (unsigned) v, false, false)[1];
}
__device__ __forceinline__ float up32_f(float v) { return __builtin_bit_cast(float, up32_i(__builtin_bit_cast(int, v))); }
__device__ __forceinline__ float up16_f(float v) { return __builtin_bit_cast(float, up16_i(__builtin_bit_cast(int, v))); }
__device__ __forceinline__ double up32_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t) up32_i((int) (uint32_t) u), hi = (uint32_t) up32_i((int) (uint32_t) (u >> 32));
    return __builtin_bit_cast(double, ((uint64_t) hi << 32) | lo);
}
__device__ __forceinline__ double up16_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t) up16_i((int) (uint32_t) u), hi = (uint32_t) up16_i((int) (uint32_t) (u >> 32));
    return __builtin_bit_cast(double, ((uint64_t) hi << 32) | lo);
}
constexpr int DPP_QUAD_XOR1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;   // lane i of each 8-lane half-row reads lane 7 - i
constexpr int DPP_ROW_MIRROR = 0x140;        // lane i of each 16-lane row reads lane 15 - i
// Largest value over each aligned group of 8 lanes (xor 1 and xor 2 within quads, then the mirrored
// quad), or of 32 lanes (then the mirrored half-row, and the row 16 lanes away by a lane swap):
// every lane of the group ends with it. A maximum does not depend on the order it is taken in.
__device__ __forceinline__ float max8_f(float m) {
    m = fmaxf(m, dpp_f<DPP_QUAD_XOR1>(m));
    m = fmaxf(m, dpp_f<DPP_QUAD_XOR2>(m));
    return fmaxf(m, dpp_f<DPP_ROW_HALF_MIRROR>(m));
}
__device__ __forceinline__ float max32_f(float m) {
    m = max8_f(m);
    m = fmaxf(m, dpp_f<DPP_ROW_MIRROR>(m));
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, m), __builtin_bit_cast(unsigned, m), false, false);
    const unsigned r0 = r[0], r1 = r[1];
    return fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
__device__ __forceinline__ float lane0_f(float v) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)); }
__device__ __forceinline__ double lane0_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) u, 0);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) (u >> 32), 0);
    return __builtin_bit_cast(double, ((uint64_t) hi << 32) | lo);
}

__device__ __forceinline__ float wave_tree_f(float v) {
    v = v + up32_f(v);
    v = v + up16_f(v);
    v = v + dpp_f<DPP_ROW_SHL + 8>(v);
    v = v + dpp_f<DPP_ROW_SHL + 4>(v);
    v = v + dpp_f<DPP_ROW_SHL + 2>(v);
    v = v + dpp_f<DPP_ROW_SHL + 1>(v);
    return lane0_f(v);
}
__device__ __forceinline__ double wave_tree_d(double v) {
    v = v + up32_d(v);
    v = v + up16_d(v);
    v = v + dpp_d<DPP_ROW_SHL + 8>(v);
    v = v + dpp_d<DPP_ROW_SHL + 4>(v);
    v = v + dpp_d<DPP_ROW_SHL + 2>(v);
    v = v + dpp_d<DPP_ROW_SHL + 1>(v);
    return lane0_d(v);
}
__device__ __forceinline__ float wave_max_f(float v) {
    v = fmaxf(v, up32_f(v));
    v = fmaxf(v, up16_f(v));
    v = fmaxf(v, dpp_f<DPP_ROW_SHL + 8>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_SHL + 4>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_SHL + 2>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_SHL + 1>(v));
    return lane0_f(v);
}

// Block barrier that orders LDS only. __syncthreads() also waits for every global access the wave
// has in flight, which would turn a weight prefetch issued before a staging barrier into a stall;
// blocks that exchange data only through LDS use this one, and their loads stay in flight across it.
__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float c) {
    half2_t ha, hb;
    __builtin_memcpy(&ha, &a, 4);
    __builtin_memcpy(&hb, &b, 4);
    return __builtin_amdgcn_fdot2(ha, hb, c, false);
}

// acc + a.lo * b.lo, then + a.hi * b.hi, for two f16 pairs: fp32 fmas in that order (the f16 x f16
// products are exact in fp32, so each adds with one rounding; each compiles to one v_fma_mix_f32)
__device__ __forceinline__ float fma_f16x2(uint32_t a, uint32_t b, float acc) {
    acc = __builtin_fmaf(h2f(b & 0xffffu), h2f(a & 0xffffu), acc);
    return __builtin_fmaf(h2f(b >> 16), h2f(a >> 16), acc);
}

// Q4_K 6-bit scale / min of sub-block j from the 12 packed bytes (GGUF K-quant layout).
__device__ __forceinline__ void q4k_sm(const uint8_t * sc, int j, int & s, int & m) {
    if (j < 4) { s = sc[j] & 63; m = sc[j + 4] & 63; }
    else {
        s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

} // namespace z2d
