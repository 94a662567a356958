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
// interleave = 1: gu holds gate and up in alternating blocks of 32 columns
// (the layout the fused GEMM epilogue pairs): gate of j at 64 * (j / 32) +
// j % 32, up 32 columns after it.
#include "../common/ee_device.h"

// No contraction: each multiply and add is one rounded operation, as in torch.
#pragma clang fp contract(off)

// column of gate value j in gu, and the distance to its up value
EE_DEV int64_t gate_col(int64_t j, int64_t F, int interleave) { return interleave ? ((j >> 5) << 6) + (j & 31) : j; }

extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_silu_mul(EeSiluMulArgs a) {
    const int64_t stride = (int64_t)gridDim.x * EE_BLOCK;
    if (a.vec) {
        const int64_t per_row = a.F / 8;
        const int64_t total = a.M * per_row;
        for (int64_t i = (int64_t)blockIdx.x * EE_BLOCK + threadIdx.x; i < total; i += stride) {
            const int64_t m = i / per_row, j = (i - m * per_row) * 8;
            const uint16_t* row = a.gu + m * a.ld_gu + gate_col(j, a.F, a.interleave);
            const u32x4 g = *(const u32x4*)row;
            const u32x4 u = *(const u32x4*)(row + (a.interleave ? 32 : a.F));
            *(u32x4*)(a.act + m * a.ld_act + j) =
                u32x4{silu_mul2_fast(g[0], u[0]), silu_mul2_fast(g[1], u[1]), silu_mul2_fast(g[2], u[2]), silu_mul2_fast(g[3], u[3])};
        }
    } else {
        const int64_t total = a.M * a.F;
        for (int64_t i = (int64_t)blockIdx.x * EE_BLOCK + threadIdx.x; i < total; i += stride) {
            const int64_t m = i / a.F, j = i - m * a.F;
            const uint16_t* row = a.gu + m * a.ld_gu + gate_col(j, a.F, a.interleave);
            a.act[m * a.ld_act + j] = (uint16_t)silu_mul2_fast(row[0], row[a.interleave ? 32 : a.F]);
        }
    }
}

// Gate rows then up rows -> blocks of 32 alternating (one row per work item,
// 4-byte words).  Used once per weight, at preparation.
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_interleave_rows(EeInterleaveArgs a) {
    const int64_t words = a.row_bytes >> 2;
    const int64_t total = 2 * a.F * words;
    const int64_t stride = (int64_t)gridDim.x * EE_BLOCK;
    for (int64_t i = (int64_t)blockIdx.x * EE_BLOCK + threadIdx.x; i < total; i += stride) {
        const int64_t dr = i / words, w = i - dr * words;
        const int64_t k = dr >> 6, r = dr & 63;
        const int64_t sr = r < 32 ? 32 * k + r : a.F + 32 * k + (r - 32);
        ((uint32_t*)(a.dst + dr * a.ld_dst_bytes))[w] = ((const uint32_t*)(a.src + sr * a.ld_src_bytes))[w];
    }
}
