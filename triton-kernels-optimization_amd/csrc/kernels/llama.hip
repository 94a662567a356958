// llama.hip -- the Llama block's elementwise work around the entropy-gated
// linears for gfx950: RMSNorm fused with the residual add, and rotary
// embedding fused with the q/k/v head-major layout.  Each follows the torch
// op sequence it replaces, op by op and in the same precision.
#include "../common/ee_device.h"

// Every multiply and add below stands for one torch op, rounded on its own:
// no contraction into FMAs (which would skip the fp16 rounding of a product
// before the add that follows it).
#pragma clang fp contract(off)
#include "../common/ee_quant_dev.h"

// eek_add_rmsnorm: s = x + y (fp16, as torch adds fp16 tensors: f32 sum
// rounded once to fp16), then RMSNorm as LlamaRMSNorm computes it in f32:
//   xf = f32(s); r = rsqrt(mean(xf * xf) + eps); n = fp16(xf * r);
//   out = fp16(f32(w) * f32(n)).
// One wave per row; lane l holds 16-byte chunks l, l + 64, ... (NC of them:
// the launcher picks the smallest of 1, 2, 4, 8 that covers the row, which
// keeps the register count, and so the occupancy, to what the row needs).
// The mean's f32 sum runs in a different order than torch's reduction, so a
// row can differ from torch in the last bit of its mean.
template <int NC>
EE_DEV void rmsnorm_row(const EeRmsNormArgs& a, int64_t row, int lane, u32x4 (&o)[NC], bool store_n = true) {
    const int nc = (int)(a.D >> 3);                   // 16-byte chunks per row
    const uint16_t* xr = a.x + row * a.ld_x;
    u32x4 s[NC];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + 64 * i;
        if (c < nc) {
            u32x4 v = *(const u32x4*)(xr + 8 * c);
            if (a.y) {
                const u32x4 yv = *(const u32x4*)(a.y + row * a.ld_y + 8 * c);
                // torch's fp16 add (f32 sum rounded to fp16) is the RNE fp16 sum: one
                // packed add per two elements
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = bits_of(f16x2_from_bits(v[j]) + f16x2_from_bits(yv[j]));
                *(u32x4*)(a.x_out + row * a.ld_xo + 8 * c) = v;
            }
            s[i] = v;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = f16_lo(v[j]), hi = f16_hi(v[j]);
                ss += lo * lo;
                ss += hi * hi;
            }
        }
    }
    const float r = rsqrtf(wave_sum(ss) * a.inv_d + a.eps);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + 64 * i;
        if (c < nc) {
            const u32x4 w = *(const u32x4*)(a.w + 8 * c);
            // n = fp16(xf * r) from the f32 product; w * n, a product of two fp16
            // values, is exact in f32, so its fp16 rounding is one packed fp16 multiply
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t n = pack_f16x2(f16_lo(s[i][j]) * r, f16_hi(s[i][j]) * r);
                o[i][j] = bits_of(f16x2_from_bits(w[j]) * f16x2_from_bits(n));
            }
            if (store_n) *(u32x4*)(a.n_out + row * a.ld_n + 8 * c) = o[i];
        }
    }
}

template <int NC>
EE_DEV void add_rmsnorm(const EeRmsNormArgs& a) {
    const int64_t row = (int64_t)blockIdx.x * (EE_BLOCK / 64) + wave_id();
    if (row >= a.T) return;
    u32x4 o[NC];
    rmsnorm_row<NC>(a, row, lane_id(), o);
}

// eek_add_rmsnorm_route: the same norm over the rows of a routing partition in
// slot order (slot i is source row idx[i]; slots [0, c0) are INT8, [c0, c0 + c1)
// FP8, the rest FP16), which also quantises the normalised rows of the INT8 and
// FP8 slots into slot i of the routed linear's workspace: the codes and scales
// the routed quantiser (quant.hip, EE_QUANT_ROUTED_I8_F8) would write from
// n_out, with the same arithmetic (ee_quant_dev.h), without reading n_out back.
// n_out receives the FP16 slots' rows only, the ones the routed GEMM reads.
template <int NC>
EE_DEV void add_rmsnorm_route(const EeRmsNormRouteArgs& ra) {
    const EeRmsNormArgs& a = ra.n;
    const int lane = lane_id();
    const int64_t slot = (int64_t)blockIdx.x * (EE_BLOCK / 64) + wave_id();
    if (slot >= a.T) return;
    const int64_t row = ra.idx[slot];
    const int64_t c0 = ra.counts[0], c01 = c0 + ra.counts[1];
    u32x4 o[NC];
    rmsnorm_row<NC>(a, row, lane, o, slot >= c01);
    if (slot >= c01) return;                          // FP16 slot: the GEMM reads n_out
    const int mode = slot < c0 ? EE_QUANT_I8_DISPATCH : EE_QUANT_F8_ROW;
    const int nc = (int)(a.D >> 3);
    uint32_t am = 0;
#pragma unroll
    for (int i = 0; i < NC; ++i)
        if (lane + 64 * i < nc)
#pragma unroll
            for (int j = 0; j < 4; ++j) am = absmax_bits(am, o[i][j]);
    am = max(am & 0xffffu, am >> 16);
    const float amax = f16_lo(wave_max_u32(am));
    const RowScale rs = row_scale(mode, amax);
    const QuantFast fast = quant_fast(mode, amax, rs);
    uint8_t* cr = ra.codes + slot * ra.ld_c;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + 64 * i;
        if (c < nc) {
            uint32_t q[8];
            *(u32x2*)(cr + 8 * c) = quant_chunk(mode, fast, rs, o[i], q);
        }
    }
    if (lane == 0) ra.scale[slot] = rs.s;
}

#define EE_RMSNORM(NC)                                                                                       \
    extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_add_rmsnorm_c##NC(EeRmsNormArgs a) {          \
        add_rmsnorm<NC>(a);                                                                                  \
    }                                                                                                        \
    extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_add_rmsnorm_route_c##NC(EeRmsNormRouteArgs a) { \
        add_rmsnorm_route<NC>(a);                                                                            \
    }
EE_RMSNORM(1)
EE_RMSNORM(2)
EE_RMSNORM(4)
EE_RMSNORM(8)

// Rotary embedding of 8 + 8 elements: x1 = elements j .. j+7 of the first
// half, x2 = the same positions of the second half (h = d/2):
//   out[j]   = fp16( fp16(x[j] * cos[j])     + fp16(-x[j+h] * sin[j]) )
//   out[j+h] = fp16( fp16(x[j+h] * cos[j+h]) + fp16( x[j]   * sin[j+h]) )
// which is torch's x * cos + rotate_half(x) * sin, each op rounded to fp16.
// Packed fp16 multiplies and adds give exactly those roundings: a product of
// two fp16 values is exact in f32, so rounding it once to fp16 is the RNE fp16
// product; the f32 sum of two fp16 values is exact whenever it can matter (an
// addend more than 2^13 below the other is under an eighth of the result's
// fp16 ulp), so its fp16 rounding is the RNE fp16 sum.
EE_DEV void rope8(const u32x4& x1, const u32x4& x2, const u32x4& c1, const u32x4& s1, const u32x4& c2,
                  const u32x4& s2, u32x4& o1, u32x4& o2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f16x2 a = f16x2_from_bits(x1[j]), b = f16x2_from_bits(x2[j]);
        o1[j] = bits_of(a * f16x2_from_bits(c1[j]) - b * f16x2_from_bits(s1[j]));
        o2[j] = bits_of(b * f16x2_from_bits(c2[j]) + a * f16x2_from_bits(s2[j]));
    }
}
// fp16(v * scale) for packed fp16 v: torch's f32 product rounded to fp16.  A power
// of two (1/sqrt(d) for d = 4^k) is one exact packed fp16 multiply.
EE_DEV void scale8(u32x4& o, float scale, bool pow2) {
    if (pow2) {
        const f16x2 s2 = {(f16)scale, (f16)scale};
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = bits_of(f16x2_from_bits(o[j]) * s2);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = pack_f16x2(f16_lo(o[j]) * scale, f16_hi(o[j]) * scale);
    }
}

// Work items (32-bit indices: the launcher checks that they fit): the v_t units
// first (each moves 16 rows, the longest items, so they start with the first
// workgroups), then the q/k chunk pairs, then the plain v chunks.
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_qkv_rope(EeQkvRopeArgs a) {
    const uint32_t d = (uint32_t)a.d, h = d >> 1;
    const uint32_t cpr = d >> 4;                      // 8-element chunk pairs per head row
    const uint32_t HH = (uint32_t)(a.Hq + a.Hkv), S = (uint32_t)a.S;
    const uint32_t T = (uint32_t)a.B * S;
    const uint32_t n_qk = T * HH * cpr;
    // v: 16-byte chunks of each token's heads, or with v_t one unit per 16 tokens x
    // 8 d of a kv head, transposed in registers
    const uint32_t n_v = a.v_t ? (uint32_t)a.B * a.Hkv * (S >> 4) * (d >> 3) : T * a.Hkv * (d >> 3);
    const uint32_t stride = gridDim.x * EE_BLOCK;
    const uint32_t n_vt = a.v_t ? n_v : 0;
    const float q_scale = a.q_scale;
    const bool pow2 = q_scale > 0.0f && (__float_as_uint(q_scale) & 0x007fffffu) == 0 && q_scale >= 0x1p-14f &&
                      q_scale <= 0x1p15f;        // an exact fp16 power of two
    for (uint32_t i0 = blockIdx.x * EE_BLOCK + threadIdx.x; i0 < n_qk + n_v; i0 += stride) {
        const uint32_t i = i0 < n_vt ? i0 + n_qk : i0 - n_vt;   // index in the order q/k, v
        if (i < n_qk) {
            const uint32_t c = i % cpr, th = i / cpr;
            const uint32_t head = th % HH, t = th / HH;
            const uint32_t b = t / S, sp = t - b * S;
            const uint16_t* src = a.qkv + (int64_t)t * a.ld + head * d + 8 * c;
            const u32x4 x1 = *(const u32x4*)src, x2 = *(const u32x4*)(src + h);
            const uint16_t* cr = a.cos_t + sp * d + 8 * c;
            const uint16_t* sr = a.sin_t + sp * d + 8 * c;
            const u32x4 c1 = *(const u32x4*)cr, c2 = *(const u32x4*)(cr + h);
            const u32x4 s1 = *(const u32x4*)sr, s2 = *(const u32x4*)(sr + h);
            const bool isq = head < (uint32_t)a.Hq;
            u32x4 o1, o2;
            rope8(x1, x2, c1, s1, c2, s2, o1, o2);
            if (isq && q_scale != 1.0f) {
                scale8(o1, q_scale, pow2);
                scale8(o2, q_scale, pow2);
            }
            uint16_t* dst = isq ? a.q + ((int64_t)(b * a.Hq + head) * S + sp) * d
                                : a.k + ((int64_t)(b * a.Hkv + (head - a.Hq)) * S + sp) * d;
            *(u32x4*)(dst + 8 * c) = o1;
            *(u32x4*)(dst + h + 8 * c) = o2;
        } else if (a.v_t) {
            // V^T [B, Hkv, d, S]: row dd holds v[.., dd] of every token; within each
            // group of 16 tokens the stored order is 0-3, 8-11, 4-7, 12-15 (the
            // K-slot order of the attention kernel's probability fragments).
            const uint32_t iv = i - n_qk;
            const uint32_t c = iv % (d >> 3), r1 = iv / (d >> 3);
            const uint32_t g = r1 % (S >> 4), bh = r1 / (S >> 4);
            const uint32_t head = bh % (uint32_t)a.Hkv, b = bh / (uint32_t)a.Hkv;
            const uint16_t* src = a.qkv + (int64_t)(b * S + 16 * g) * a.ld + (HH + head) * d + 8 * c;
            u32x4 x[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) x[j] = *(const u32x4*)(src + (int64_t)j * a.ld);
            // stored position p holds token perm(p): chunks of 4 in the order 0, 2, 1, 3
            constexpr int perm[16] = {0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;   // high or low halves
                uint32_t w[8];
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    w[k] = __builtin_amdgcn_perm(x[perm[2 * k + 1]][e >> 1], x[perm[2 * k]][e >> 1], sel);
                uint16_t* dst = a.v + ((int64_t)(b * a.Hkv + head) * d + 8 * c + e) * S + 16 * g;
                *(u32x4*)dst = u32x4{w[0], w[1], w[2], w[3]};
                *(u32x4*)(dst + 8) = u32x4{w[4], w[5], w[6], w[7]};
            }
        } else {
            const uint32_t iv = i - n_qk;
            const uint32_t c = iv % (d >> 3), th = iv / (d >> 3);
            const uint32_t head = th % (uint32_t)a.Hkv, t = th / (uint32_t)a.Hkv;
            const uint32_t b = t / S, sp = t - b * S;
            const u32x4 v = *(const u32x4*)(a.qkv + (int64_t)t * a.ld + (HH + head) * d + 8 * c);
            *(u32x4*)(a.v + ((int64_t)(b * a.Hkv + head) * S + sp) * d + 8 * c) = v;
        }
    }
}
