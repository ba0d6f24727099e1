// z2_formats.h — GGUF tensor types and block formats used by the decode-step weights.
//
// Block layouts follow the public GGUF/ggml storage format (the reference only consumes them
// through ggml: src/zonos2.cpp:100-119 streams the bytes unchanged into the backend):
//   Q8_0  32 weights / 34 B : fp16 d; int8 q[32]                          w = d*q
//   Q4_K 256 weights / 144 B: fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128] w = d*sc*q - dmin*m
//   Q6_K 256 weights / 210 B: u8 ql[128]; u8 qh[64]; i8 sc[16]; fp16 d    w = d*sc*(q-32)
// Host-side only (generator, GGUF I/O, device repack); the device kernels have their own decode.
#pragma once
#include <cstdint>
#include <cstring>
#include <cmath>

namespace z2 {

enum gguf_type : int32_t { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };

constexpr int QK8_0 = 32;
constexpr int QK_K  = 256;

struct blk_q8_0 { uint16_t d; int8_t qs[QK8_0]; };
struct blk_q4_k { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; };
struct blk_q6_k { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; uint16_t d; };
static_assert(sizeof(blk_q8_0) == 34, "q8_0 size");
static_assert(sizeof(blk_q4_k) == 144, "q4_k size");
static_assert(sizeof(blk_q6_k) == 210, "q6_k size");

inline int64_t type_block(int t) {
    switch (t) { case T_F32: case T_F16: return 1; case T_Q8_0: return QK8_0; default: return QK_K; }
}
inline int64_t type_block_bytes(int t) {
    switch (t) {
        case T_F32: return 4; case T_F16: return 2; case T_Q8_0: return 34;
        case T_Q4_K: return 144; case T_Q6_K: return 210; default: return -1;
    }
}
inline bool type_known(int t) { return type_block_bytes(t) > 0; }
inline int64_t row_bytes(int t, int64_t n) { return n / type_block(t) * type_block_bytes(t); }

// IEEE binary16 <-> binary32, round-to-nearest-even, with subnormals, inf and NaN.
inline uint16_t f32_to_f16(float f) {
    uint32_t x; std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);            // rounds to >= 65520 -> inf
    if (ax < 0x38800000u) {                                                // result is subnormal or 0
        if (ax < 0x33000000u) return (uint16_t) sign;                      // below 2^-25 rounds to 0
        // value = m * 2^(e-150); in units of the f16 subnormal step 2^-24 that is m * 2^(e-126)
        const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t sh = 126 - e;                                       // 14..24 bits dropped
        uint32_t r = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (r & 1u))) r += 1u;              // may carry into 0x400
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax - 0x38000000u) >> 13);                               // rebias exponent 127->15
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1u;
    return (uint16_t)(sign | r);
}

inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = sign;
        else {                                                             // subnormal: normalise
            int sh = 0; uint32_t mm = m;
            while (!(mm & 0x400u)) { mm <<= 1; ++sh; }
            x = sign | ((uint32_t)(113 - sh) << 23) | ((mm & 0x3ffu) << 13);
        }
    } else if (e == 31) x = sign | 0x7f800000u | (m << 13);
    else x = sign | ((e + 112u) << 23) | (m << 13);
    float f; std::memcpy(&f, &x, 4); return f;
}

} // namespace z2
