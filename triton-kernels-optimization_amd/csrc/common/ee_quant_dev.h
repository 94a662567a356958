// ee_quant_dev.h -- the arithmetic of the per-row activation quantisers, shared
// by quant.hip's quantiser kernels and llama.hip's norm kernel that quantises
// the rows it produces, so that both write the same codes bit for bit.
// Include after `#pragma clang fp contract(off)`: every multiply and add here
// is its own rounded f32 operation.
#pragma once
#include "ee_device.h"

#define INV127 (1.0f / 127.0f)
#define INV448 (1.0f / 448.0f)

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

// amax of |fp16| on raw bits: for non-negative halves the integer order is the
// numeric order, and NaN patterns sort above inf, so NaN propagates like amax.
EE_DEV uint32_t absmax_bits(uint32_t acc, uint32_t u) {
    union { uint32_t u; u16x2 v; } a, b;
    a.u = acc;
    b.u = u & 0x7fff7fffu;
    a.v = __builtin_elementwise_max(a.v, b.v);
    return a.u;
}

struct RowScale {
    float s;     // scale stored per row
    float mul;   // F8: fp16(1/s); I8 dispatcher: RN(RN(1/s) * (1 + 2^-21))
};

EE_DEV RowScale row_scale(int mode, float amax) {
    RowScale r;
    if (mode == EE_QUANT_I8_DISPATCH) {
        r.s = f16_round(amax * INV127);
        r.mul = (1.0f / r.s) * (1.0f + 0x1p-21f);
    } else if (mode == EE_QUANT_I8_ENGINE) {
        float s = amax * INV127;
        if (s < 1e-8f) s = 1e-8f;            // clamp(min=1e-8); NaN stays NaN
        r.s = s;
        r.mul = 0.f;
    } else if (mode == EE_QUANT_F8_ROW) {
        r.s = f16_round(amax * INV448);
        r.mul = f16_round(1.0f / r.s);
    } else {                                  // EE_QUANT_F8_TENSOR: amax is the tensor's
        r.s = (amax > 0.0f && amax < INFINITY) ? amax / 448.0f : 1.0f;
        r.mul = 1.0f / r.s;
    }
    return r;
}

EE_DEV uint32_t quant_one(int mode, float x, const RowScale& rs) {
    if (mode == EE_QUANT_I8_DISPATCH) {
        // trunc(x / s) as trunc(x * mul): for fp16 x and s with |x| <= amax a
        // non-integer quotient lies >= 2^-19 (relative) from the nearest integer,
        // and mul errs upward by 2^-22 .. 2^-20.7, so no integer is crossed and
        // exact-integer quotients are not rounded below -- the same code for every
        // reachable (amax, x) pair (checked exhaustively by tests/rcp_trunc_check.c).
        // s = 0 gives mul = inf, as x / 0 does.
        const float q = x * rs.mul;
        int32_t iv;
        if (fabsf(q) < 2147483648.0f) iv = (int32_t)q;                 // truncation
        else iv = (q > 0.0f) ? 0x7fffffff : (int32_t)0x80000000;       // saturate; NaN -> 0 byte
        return (uint32_t)iv & 0xffu;
    } else if (mode == EE_QUANT_I8_ENGINE) {
        float r = rintf(x / rs.s);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        return (r != r) ? 0u : ((uint32_t)(int32_t)r & 0xffu);
    } else if (mode == EE_QUANT_F8_TENSOR) {
        return e4m3_rne_sat(x * rs.mul);
    } else {
        // fp16 x fp16 -> fp16 (RNE), as the reference multiplies its fp16 tile by the
        // fp16 inverse scale.  Written as a half-precision product on purpose: the
        // widened form fp16(x * inv) is lowered to v_fma_mix(x, inv, +0.0), which
        // turns a -0 product into +0 and would change the code of -0 (0x80 -> 0x00).
        const f16 p = (f16)x * (f16)rs.mul;
        return e4m3_rne_sat((float)p);
    }
}

// Per-row switches of the fast conversions.
struct QuantFast {
    bool f8, i8;
    f16x2 mul2;
};
EE_DEV QuantFast quant_fast(int mode, float amax, const RowScale& rs) {
    QuantFast f;
    // FP8 rows whose amax and fp16 inverse scale are finite: every product
    // fp16(x * inv) is finite with |p| < 464, where the hardware e4m3 conversion
    // (round to nearest even; checked against e4m3_rne_sat on every fp16 value)
    // gives the same code -- two codes per instruction.  Zero, tiny and
    // non-finite rows take quant_one.
    f.f8 = mode == EE_QUANT_F8_ROW && fabsf(amax) < INFINITY && fabsf(rs.mul) < INFINITY;
    // INT8 dispatcher rows with 0 < s < inf and a finite amax: every |x * mul| is
    // below 2^31 (s >= the smallest fp16 subnormal bounds it by ~1.3e5), so the
    // truncating conversion needs no saturation; the low byte is the int8 code.
    f.i8 = mode == EE_QUANT_I8_DISPATCH && fabsf(amax) < INFINITY && rs.s > 0.0f && fabsf(rs.mul) < INFINITY;
    f.mul2 = f16x2{(f16)rs.mul, (f16)rs.mul};
    return f;
}

// The 8 codes of one 16-byte chunk v (8 fp16 values) of a row: packed in the
// return value and one per entry of q.
EE_DEV u32x2 quant_chunk(int mode, const QuantFast& fast, const RowScale& rs, const u32x4& v, uint32_t (&q)[8]) {
    u32x2 o;
    if (fast.f8) {
        s16x2 r0 = {0, 0}, r1 = {0, 0};
        r0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r0, f16x2_from_bits(v[0]) * fast.mul2, 1.0f, false);
        r0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r0, f16x2_from_bits(v[1]) * fast.mul2, 1.0f, true);
        r1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r1, f16x2_from_bits(v[2]) * fast.mul2, 1.0f, false);
        r1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(r1, f16x2_from_bits(v[3]) * fast.mul2, 1.0f, true);
        o = u32x2{__builtin_bit_cast(uint32_t, r0), __builtin_bit_cast(uint32_t, r1)};
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = (o[i >> 2] >> ((i & 3) * 8)) & 0xffu;
        return o;
    }
    if (fast.i8) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = v[i >> 1];
            q[i] = (uint32_t)(int32_t)(((i & 1) ? f16_hi(u) : f16_lo(u)) * rs.mul) & 0xffu;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = v[i >> 1];
            q[i] = quant_one(mode, (i & 1) ? f16_hi(u) : f16_lo(u), rs);
        }
    }
    return u32x2{q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24), q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24)};
}
