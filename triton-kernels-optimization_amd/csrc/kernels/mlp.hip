// mlp.hip -- the MLP activation of the fused entropy-gated MLP for gfx950.
//
// eek_silu_mul: act[m, j] = fp16( f32(fp16(silu(g))) * f32(u) ),  g = gu[m, j],
// u = gu[m, F + j], silu(g) = g / (1 + e^-g) in f32.  That is the value of
// F.silu(F.linear(x, gate_w)) * F.linear(x, up_w) on fp16 tensors in the
// reference's baseline (EE/test_engine.py:36-41): silu evaluated in f32 and
// rounded to fp16, then the fp16 product evaluated in f32 and rounded.  gu is
// the output of one GEMM over the concatenated [gate; up] weights.
// Each thread handles 8 consecutive j (16-byte loads and store) when F, the
// strides and the pointers allow it, else single elements.
#include "../common/ee_device.h"

EE_DEV float silu_f32(float g) { return g / (1.0f + expf(-g)); }

EE_DEV uint32_t silu_mul2(uint32_t g2, uint32_t u2) {
    const float a0 = f16_round(silu_f32(f16_lo(g2)));
    const float a1 = f16_round(silu_f32(f16_hi(g2)));
    return pack_f16x2(a0 * f16_lo(u2), a1 * f16_hi(u2));
}

extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_silu_mul(EeSiluMulArgs a) {
    const int64_t stride = (int64_t)gridDim.x * EE_BLOCK;
    if (a.vec) {
        const int64_t per_row = a.F / 8;
        const int64_t total = a.M * per_row;
        for (int64_t i = (int64_t)blockIdx.x * EE_BLOCK + threadIdx.x; i < total; i += stride) {
            const int64_t m = i / per_row, j = (i - m * per_row) * 8;
            const uint16_t* row = a.gu + m * a.ld_gu;
            const u32x4 g = *(const u32x4*)(row + j);
            const u32x4 u = *(const u32x4*)(row + a.F + j);
            *(u32x4*)(a.act + m * a.ld_act + j) =
                u32x4{silu_mul2(g[0], u[0]), silu_mul2(g[1], u[1]), silu_mul2(g[2], u[2]), silu_mul2(g[3], u[3])};
        }
    } else {
        const int64_t total = a.M * a.F;
        for (int64_t i = (int64_t)blockIdx.x * EE_BLOCK + threadIdx.x; i < total; i += stride) {
            const int64_t m = i / a.F, j = i - m * a.F;
            const uint16_t* row = a.gu + m * a.ld_gu;
            a.act[m * a.ld_act + j] = (uint16_t)silu_mul2(row[j], row[a.F + j]);
        }
    }
}
