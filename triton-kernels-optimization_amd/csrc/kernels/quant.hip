// quant.hip -- per-row activation quantisers and offline weight preparation
// for gfx950.
//
// Activation quantisers (one read of the row, one write of the codes):
//   EE_QUANT_I8_DISPATCH  EE/python/kernels.py:336-338
//       s = fp16(amax * f32(1/127));  code = int8(trunc(f32(x) / s))
//   EE_QUANT_I8_ENGINE    EE/test_cubin.py:93-103  (also EE/python/dispatch.py:43-48
//                         per weight channel)
//       s = max(amax * f32(1/127), 1e-8);  code = clamp(rne(f32(x) / s), -127, 127)
//   EE_QUANT_F8_ROW       EE/python/kernels.py:361,144,159-160
//       s = fp16(amax * f32(1/448));  inv = fp16(1/s);  code = e4m3(fp16(x * inv))
// `amax * f32(1/d)` is how PyTorch evaluates `tensor / python_float` on the
// GPU, which is where the reference ran these lines.  Divisions x / s are
// IEEE binary32 divisions (correctly rounded), as in the reference.
// With a routing partition (idx, counts, tier; off = rows of lower tiers) the
// kernel reads source rows idx[off + r] and writes codes/scales to partition
// slot off + r of a full-height workspace, so the three tiers share one
// buffer without host-side offsets.
#include "../common/ee_device.h"

// Every epilogue / quantiser multiply and add is its own rounded f32
// operation, as in the reference: no contraction into FMAs.  (Conversions to
// fp16 take their operand through f32_rn, which keeps a product from being
// folded into the conversion.)
#pragma clang fp contract(off)
#include "../common/ee_quant_dev.h"

// EE_QUANT_F8_TENSOR: max |x| of the whole tensor from the per-block maxima of
// eek_absmax_partial (fp16 bits; NaN sorts above inf).  Wave-uniform.
EE_DEV float tensor_amax(const EeQuantArgs& a) {
    uint32_t m = 0;
    for (int i = lane_id(); i < a.n_tmax; i += 64) m = max(m, a.tmax[i]);
    return f16_lo(wave_max_u32(m));
}

template <int VPT, int WPR>
EE_DEV void quant_vec(const EeQuantArgs& a) {
    constexpr int RPB = 4 / WPR;
    __shared__ uint32_t slot[4];
    const int lane = lane_id();
    const int w = wave_id();
    const int wr = w % WPR;
    const int64_t lr = (int64_t)blockIdx.x * RPB + w / WPR;
    // EE_QUANT_ROUTED_I8_F8: slots [0, counts[0]) take INT8 codes, the next counts[1] FP8
    const bool dual = a.mode == EE_QUANT_ROUTED_I8_F8;
    const int64_t rows = dual ? (int64_t)a.counts[0] + a.counts[1] : (a.counts ? (int64_t)a.counts[a.tier] : a.M);
    const bool valid = lr < rows;
    const int64_t off = (a.counts && !dual) ? tier_offset(a.counts, a.tier) : 0;
    const int mode = dual ? (lr < a.counts[0] ? EE_QUANT_I8_DISPATCH : EE_QUANT_F8_ROW) : a.mode;
    int64_t src = 0;
    if (valid) src = a.idx ? (int64_t)a.idx[off + lr] : lr;
    const int64_t dst = off + lr;                 // routed: partition slot; else the row itself
    const uint16_t* xr = a.x + src * a.ld_x;
    const int K = (int)a.K;

    u32x4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c0 = ((j * WPR + wr) * 64 + lane) * 8;
        if (c0 + 8 <= K) {
            v[j] = *(const u32x4*)(xr + c0);
        } else {
            uint16_t e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = (c0 + i < K) ? xr[c0 + i] : (uint16_t)0;
            v[j] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                         e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
        }
    }
    uint32_t am = 0;
#pragma unroll
    for (int j = 0; j < VPT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) am = absmax_bits(am, v[j][i]);
    am = max(am & 0xffffu, am >> 16);
    am = wave_max_u32(am);
    if (WPR > 1) {
        if (lane == 0) slot[w] = am;
        __syncthreads();
        const int base = (w / WPR) * WPR;
        am = slot[base];
#pragma unroll
        for (int i = 1; i < WPR; ++i) am = max(am, slot[base + i]);
    }
    if (!valid) return;
    const float amax = mode == EE_QUANT_F8_TENSOR ? tensor_amax(a) : f16_lo(am);
    const RowScale rs = row_scale(mode, amax);
    const QuantFast fast = quant_fast(mode, amax, rs);
    uint8_t* cr = (uint8_t*)a.codes + dst * a.ld_c;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c0 = ((j * WPR + wr) * 64 + lane) * 8;
        if (c0 >= K) continue;
        uint32_t q[8];
        const u32x2 o = quant_chunk(mode, fast, rs, v[j], q);
        if (c0 + 8 <= K) {
            *(u32x2*)(cr + c0) = o;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (c0 + i < K) cr[c0 + i] = (uint8_t)q[i];
        }
    }
    if (wr == 0 && lane == 0) a.scale[dst] = rs.s;
}

// Any K, any alignment: one wave per row, two passes over the row.
EE_DEV void quant_generic(const EeQuantArgs& a) {
    const int lane = lane_id();
    const int64_t lr = (int64_t)blockIdx.x * 4 + wave_id();
    const bool dual = a.mode == EE_QUANT_ROUTED_I8_F8;
    const int64_t rows = dual ? (int64_t)a.counts[0] + a.counts[1] : (a.counts ? (int64_t)a.counts[a.tier] : a.M);
    if (lr >= rows) return;
    const int64_t off = (a.counts && !dual) ? tier_offset(a.counts, a.tier) : 0;
    const int mode = dual ? (lr < a.counts[0] ? EE_QUANT_I8_DISPATCH : EE_QUANT_F8_ROW) : a.mode;
    const int64_t src = a.idx ? (int64_t)a.idx[off + lr] : lr;
    const int64_t dst = off + lr;
    const uint16_t* xr = a.x + src * a.ld_x;
    uint32_t am = 0;
    for (int64_t c = lane; c < a.K; c += 64) am = max(am, (uint32_t)(xr[c] & 0x7fffu));
    am = wave_max_u32(am);
    const RowScale rs = row_scale(mode, mode == EE_QUANT_F8_TENSOR ? tensor_amax(a) : f16_lo(am));
    uint8_t* cr = (uint8_t*)a.codes + dst * a.ld_c;
    for (int64_t c = lane; c < a.K; c += 64) cr[c] = (uint8_t)quant_one(mode, f16_lo(xr[c]), rs);
    if (lane == 0) a.scale[dst] = rs.s;
}

#define EE_Q_VEC(V, W)                                                                             \
    extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_quant_v##V##_w##W(EeQuantArgs a) { \
        quant_vec<V, W>(a);                                                                        \
    }
#define EE_Q_VEC_W(V) EE_Q_VEC(V, 1) EE_Q_VEC(V, 2) EE_Q_VEC(V, 4)
EE_Q_VEC_W(1)
EE_Q_VEC_W(2)
EE_Q_VEC_W(3)
EE_Q_VEC_W(4)
EE_Q_VEC_W(5)
EE_Q_VEC_W(6)
EE_Q_VEC_W(7)
EE_Q_VEC_W(8)

extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_quant_generic(EeQuantArgs a) { quant_generic(a); }

// First pass of the per-tensor FP8 scale: out[b] = max |x| over the rows
// b*4 + w, b*4 + w + 4*gridDim.x, ... (w = wave), as fp16 bits.
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_absmax_partial(EeAbsmaxArgs a) {
    __shared__ uint32_t red[4];
    const int lane = lane_id(), w = wave_id();
    uint32_t m = 0;
    for (int64_t r = (int64_t)blockIdx.x * 4 + w; r < a.M; r += (int64_t)gridDim.x * 4) {
        const uint16_t* xr = a.x + r * a.ld_x;
        const bool vec = ((uintptr_t)xr & 15) == 0;
        for (int64_t c = (int64_t)lane * 8; c < a.K; c += 512) {
            if (vec && c + 8 <= a.K) {
                const u32x4 v = *(const u32x4*)(xr + c);
#pragma unroll
                for (int i = 0; i < 4; ++i) m = absmax_bits(m, v[i]);
            } else {
                for (int i = 0; i < 8; ++i)
                    if (c + i < a.K) m = absmax_bits(m, (uint32_t)xr[c + i]);
            }
        }
    }
    m = max(m & 0xffffu, m >> 16);
    m = wave_max_u32(m);
    if (lane == 0) red[w] = m;
    __syncthreads();
    if (threadIdx.x == 0) a.out[blockIdx.x] = max(max(red[0], red[1]), max(red[2], red[3]));
}

// ---------------------------------------------------------------------------
// Weight preparation.  The GEMMs read B as [N, K] (K contiguous, the MFMA
// operand order); the reference's buffer is B int8 [K, N] (N contiguous,
// EE/python/dispatch.py:44-48).  These kernels move between the two and
// derive the FP8 / W8A16 tier operands from the int8 codes once per layer.
// ---------------------------------------------------------------------------

// dst[c, r] = src[r, c] for int8 [R, C]; 64x64 tiles through LDS.
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_transpose_i8(EeWeightArgs a) {
    __shared__ uint8_t tile[64][65];
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    const uint8_t* src = (const uint8_t*)a.src;
    uint8_t* dst = (uint8_t*)a.dst;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < a.R && c < a.C) tile[i][tx] = src[r * a.ld_src + c];
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (r < a.R && c < a.C) dst[c * a.ld_dst + r] = tile[tx][i];
    }
}

// e4m3 weight codes of the FP8 tier: dst = e4m3(fp16(b)) for int8 b
// (EE/python/kernels.py:166), elementwise over [R, C].
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_pack_b_f8(EeWeightArgs a) {
    const int64_t n = a.R * a.C;
    for (int64_t i = (int64_t)blockIdx.x * EE_BLOCK + threadIdx.x; i < n; i += (int64_t)gridDim.x * EE_BLOCK) {
        const int64_t r = i / a.C, c = i - r * a.C;
        const int8_t b = ((const int8_t*)a.src)[r * a.ld_src + c];
        ((uint8_t*)a.dst)[r * a.ld_dst + c] = (uint8_t)e4m3_rne_sat((float)b);
    }
}

// W8A16 tier weights: dst[n, k] = fp16(fp16(b[n, k]) * fp16(scale[n]))
// (EE/python/kernels.py:215,232-233), src int8 [N, K] codes.
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_pack_b_f16(EeWeightArgs a) {
    const int64_t n = a.R * a.C;
    for (int64_t i = (int64_t)blockIdx.x * EE_BLOCK + threadIdx.x; i < n; i += (int64_t)gridDim.x * EE_BLOCK) {
        const int64_t r = i / a.C, c = i - r * a.C;
        const float s16 = f16_round(a.scale[r]);
        const int8_t b = ((const int8_t*)a.src)[r * a.ld_src + c];
        ((uint16_t*)a.dst)[r * a.ld_dst + c] = (uint16_t)pack_f16x2((float)b * s16, 0.0f);
    }
}
