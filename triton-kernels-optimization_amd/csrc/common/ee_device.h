// ee_device.h -- device helpers for the gfx950 kernels (wave64, CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ee_kernel_args.h"

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define EE_DEV static __device__ __forceinline__

EE_DEV int lane_id() { return (int)(threadIdx.x & 63); }
EE_DEV int wave_id() { return (int)(threadIdx.x >> 6); }

// Butterfly reductions across the 64 lanes of a wave (every lane gets the result).
EE_DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
EE_DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

EE_DEV f16x2 f16x2_from_bits(uint32_t u) {
    union { uint32_t u; f16x2 h; } c;
    c.u = u;
    return c.h;
}
EE_DEV uint32_t bits_of(f16x2 h) {
    union { uint32_t u; f16x2 h; } c;
    c.h = h;
    return c.u;
}
EE_DEV float f16_lo(uint32_t u) { return (float)f16x2_from_bits(u).x; }
EE_DEV float f16_hi(uint32_t u) { return (float)f16x2_from_bits(u).y; }
EE_DEV uint32_t pack_f16x2(float lo, float hi) {
    f16x2 h;
    h.x = (f16)lo;   // v_cvt_f16_f32: round to nearest even
    h.y = (f16)hi;
    return bits_of(h);
}
EE_DEV float f16_round(float x) { return (float)(f16)x; }

// Routing partition bookkeeping: rows of tier t start at counts[0] + ... + counts[t-1].
EE_DEV int64_t tier_offset(const int32_t* counts, int tier) {
    int64_t off = 0;
    for (int t = 0; t < tier; ++t) off += counts[t];
    return off;
}

// binary32 -> OCP e4m3fn code, round-to-nearest-even, saturating to +-448,
// NaN -> 0x7f|sign.  Exact integer arithmetic (no dependence on hardware
// conversion modes).
EE_DEV uint32_t e4m3_rne_sat(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 24) & 0x80u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7fu;
    if (ax >= 0x43e00000u) return sign | 0x7eu;                  // |f| >= 448 (incl. inf)
    const int E = (int)(ax >> 23) - 127;
    if ((ax >> 23) == 0) return sign;
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t q;
    int shift;
    uint32_t base;
    if (E >= -6) {
        shift = 20;
        base = (uint32_t)(E + 7) << 3;
        q = mant;
    } else {
        shift = 14 - E;
        base = 0;
        q = mant | 0x800000u;
    }
    if (shift > 31) return sign;
    uint32_t r = q >> shift;
    const uint32_t rem = q & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    r += (rem > half || (rem == half && (r & 1u))) ? 1u : 0u;
    return sign | (base + r);                                    // carry into the exponent is the next binade
}
