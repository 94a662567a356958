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

// Reductions across the 64 lanes of a wave, all lanes active; every lane gets
// the (wave-uniform) result.  Within each 16-lane row, four DPP steps
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror)
// leave the row's result in all its lanes; the four rows are then combined
// from v_readlane.  No LDS traffic, unlike __shfl_xor (ds_bpermute).
template <int CTRL>
EE_DEV uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
EE_DEV float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
EE_DEV float lane_f32(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

EE_DEV float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}
// IEEE 754-2019 maximum (v_maximum_f32 / v_pk_maximum3_f16): a NaN operand gives NaN.
EE_DEV float fmaximum(float a, float b) { return __builtin_elementwise_maximum(a, b); }
EE_DEV float wave_maximum(float v) {
    v = fmaximum(v, dpp_f32<0xB1>(v));
    v = fmaximum(v, dpp_f32<0x4E>(v));
    v = fmaximum(v, dpp_f32<0x141>(v));
    v = fmaximum(v, dpp_f32<0x140>(v));
    return fmaximum(fmaximum(lane_f32(v, 0), lane_f32(v, 16)), fmaximum(lane_f32(v, 32), lane_f32(v, 48)));
}
EE_DEV float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}
EE_DEV int32_t wave_sum_i32(int32_t v) {
    v += (int32_t)dpp_u32<0xB1>((uint32_t)v);
    v += (int32_t)dpp_u32<0x4E>((uint32_t)v);
    v += (int32_t)dpp_u32<0x141>((uint32_t)v);
    v += (int32_t)dpp_u32<0x140>((uint32_t)v);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
EE_DEV uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));
    v = max(v, dpp_u32<0x4E>(v));
    v = max(v, dpp_u32<0x141>(v));
    v = max(v, dpp_u32<0x140>(v));
    const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
    const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
    return max(a, b);
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
// x as an f32 register value.  hipcc folds an f32 multiply whose only use is an
// f32 -> fp16 conversion into v_fma_mix{lo,hi}_f16(a, b, 0): one rounding,
// straight to fp16, even under -ffp-contract=off.  Every fp16 result here is
// the reference's f32 value rounded to fp16 (f32 op, then .to(float16)), so
// conversions take their operand through this barrier, which costs no
// instruction.
EE_DEV float f32_rn(float x) {
    asm("" : "+v"(x));
    return x;
}
EE_DEV uint32_t pack_f16x2(float lo, float hi) {
    f16x2 h;
    h.x = (f16)f32_rn(lo);   // v_cvt_f16_f32: round to nearest even
    h.y = (f16)f32_rn(hi);
    return bits_of(h);
}
EE_DEV float f16_round(float x) { return (float)(f16)f32_rn(x); }

// SiLU * up of two fp16 pairs: fp16( f32(fp16(silu(g))) * f32(u) ) per half,
// silu(g) = g / (1 + e^-g) in f32 -- torch's fp16 F.silu(gate) * up, op by op.
// No contraction: 1 + e^-g is one rounded add, as in torch.
EE_DEV float silu_f32(float g) {
#pragma clang fp contract(off)
    return g / (1.0f + expf(-g));
}
// fp16 bits (low half) of fp16(silu_f32(g)), mostly without its expf and IEEE
// division.  Fast form: e = 2^(-g log2 e) by v_exp_f32, s = g * v_rcp_f32(1 + e).
// It lies within (6 + |g| min(e, 1)) f32 ulps of silu_f32(g): the product
// -g log2 e rounds to 2^-24 relative, which moves e by |g| 2^-24 relative and
// 1 + e by e / (1 + e) of that; plus a few ulps of the hardware's exp and rcp,
// the add, the multiply and silu_f32's own roundings.  Where s (1 - eps) and
// s (1 + eps) round to the same fp16 value, silu_f32(g) rounds to it too
// (rounding is monotonic); elsewhere (about 0.1% of N(0, 2) gates, and
// non-finite ones) silu_f32 itself.  The bracket is a product, not a sum, so
// a zero s keeps its sign.  Checked on the GPU against silu_f32 for every fp16
// gate: the same bits for all of them.
EE_DEV uint32_t silu_f16(float g) {
#pragma clang fp contract(off)
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    const float s = g * __builtin_amdgcn_rcpf(1.0f + e);
    const float eps = (6.0f + fabsf(g) * fminf(e, 1.0f)) * 1.1920928955078125e-07f;
    const uint32_t b = pack_f16x2(s * (1.0f - eps), s * (1.0f + eps));
    if ((b & 0xffffu) == (b >> 16) && fabsf(g) < 65536.0f) return b & 0xffffu;
    return pack_f16x2(silu_f32(g), 0.0f) & 0xffffu;
}
// The GEMM epilogues' form: branch-free, so that the compiler overlaps the
// evaluations of a whole block (with one wave per SIMD, a per-element fallback
// branch as in silu_f16 exposes each evaluation's latency; measured slower).
EE_DEV uint32_t silu_mul2(uint32_t g2, uint32_t u2) {
#pragma clang fp contract(off)
    const float a0 = f16_round(silu_f32(f16_lo(g2)));
    const float a1 = f16_round(silu_f32(f16_hi(g2)));
    return pack_f16x2(a0 * f16_lo(u2), a1 * f16_hi(u2));
}
// The same bits through silu_f16, for eek_silu_mul (many waves per SIMD hide the
// branches).  fp16(f32(a) * f32(u)) for fp16 a and u is the packed fp16 multiply:
// the f32 product of two fp16 values is exact, so both round it once.
EE_DEV uint32_t silu_mul2_fast(uint32_t g2, uint32_t u2) {
    const uint32_t a2 = silu_f16(f16_lo(g2)) | (silu_f16(f16_hi(g2)) << 16);
    return bits_of(f16x2_from_bits(a2) * f16x2_from_bits(u2));
}

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
