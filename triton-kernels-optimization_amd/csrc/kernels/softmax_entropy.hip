// softmax_entropy.hip -- fused row softmax + Shannon entropy for gfx950.
//
// Computes, for every row r of fp16 logits x (S columns, causal optional):
//   m = max x,  s = x - m,  Z = sum e^s,  p = e^s / Z  (stored fp16, RNE)
//   H = ln Z - sum p*s   (masked columns contribute 0)
// which is the function of the reference's fused_softmax_entropy_kernel
// (EE/python/kernels.py:264-312).  H is evaluated in the cancellation-free
// form  H = ln(c0) + log1p(Z'/c0) - T/(c0 + Z')  with c0 = number of entries
// equal to the max, Z' = sum of e^s over the other entries and T = sum e^s*s;
// every term is non-negative, so nearly one-hot rows keep full relative
// precision (the plain ln Z form loses ~1e-4 relative at H ~ 5e-4 in f32).
//
// Layout: row-major rows, unit column stride.  One to eight wave64s per row;
// each lane holds VPT 16-byte vectors (8 fp16) of the row in registers, so
// the row is read from HBM exactly once and the probabilities are written
// once: 2 bytes in + 2 bytes out per element + 4 bytes of H per row.
#include "../common/ee_device.h"

#define LOG2E 1.4426950408889634f
#define LN2 0.69314718055994531f

// Rows per block for WPR waves per row (the block holds RPB * WPR waves).
template <int WPR>
struct SeGeom {
    static constexpr int RPB = WPR == 1 ? 4 : (WPR == 2 ? 2 : 1);
    static constexpr int BLOCK = RPB * WPR * 64;
};

EE_DEV int tier_of(float h, double tl, double th) {
    const double d = (double)h;
    return d < tl ? 0 : (d < th ? 1 : 2);
}

// ln x for x >= 1: v_log_f32 (log2, within 1 ulp of the result) times ln 2.
EE_DEV float ln_ge1(float x) { return __builtin_amdgcn_logf(x) * LN2; }
// log1p(x) for x >= 0 (Goldberg): u = 1 + x; x ln(u) / (u - 1) with u - 1 exact,
// which cancels u's rounding, or x where u rounds to 1.  A few ulps relative.
EE_DEV float log1p_ge0(float x) {
    const float u = 1.0f + x;
    return u == 1.0f ? x : ln_ge1(u) * (x * __builtin_amdgcn_rcpf(u - 1.0f));
}
// Entropy from the reduced partial sums (see header comment): c0 >= 1 counts the
// entries at the max, z >= 0, t <= 0, so every term is >= 0; the quotients take
// v_rcp_f32 (1 ulp).  Within ~1e-6 relative of the libm form (logf, log1pf and
// IEEE divisions: ~120 dependent instructions, evaluated once per row).
EE_DEV float entropy_from(float c0, float z, float t) {
    return ln_ge1(c0) + log1p_ge0(z * __builtin_amdgcn_rcpf(c0)) - t * __builtin_amdgcn_rcpf(c0 + z);
}

// s = x - m for the low / high fp16 half of a packed word: one v_fma_mix_f32
// (x * 1 + (-m), a single rounding, the same value as converting x and then
// subtracting).
EE_DEV float sub_lo(uint32_t u, float negm) {
    float r;
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(u), "v"(negm));
    return r;
}
EE_DEV float sub_hi(uint32_t u, float negm) {
    float r;
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(u), "v"(negm));
    return r;
}
// (x - m) log2 e in one v_fma_mix_f32: x * log2e + (-m log2e), one rounding.
// The waves of a row that hold no entry equal to the max take this form (one
// instruction per element instead of two); it is within 2^-24 |m log2 e| of
// the two-step value, so e changes by at most a few f32 ulps.
EE_DEV float sub2_lo(uint32_t u, float l2e, float negml) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(u), "s"(l2e), "v"(negml));
    return r;
}
EE_DEV float sub2_hi(uint32_t u, float l2e, float negml) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(u), "s"(l2e), "v"(negml));
    return r;
}
// fp16(e0 * s) | fp16(e1 * s) << 16, each product rounded once to fp16
// (v_fma_mixlo_f16 / v_fma_mixhi_f16 with a zero addend).
EE_DEV uint32_t scale_pack_f16x2(float e0, float e1, float s) {
    uint32_t r;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "=v"(r) : "v"(e0), "v"(s));
    asm("v_fma_mixhi_f16 %0, %1, %2, 0" : "+v"(r) : "v"(e1), "v"(s));
    return r;
}

// Row kernel: WPR wave64s per row (one to eight), VPT 16-byte vectors per lane
// (S <= VPT * WPR * 512).  Passes over the registers:
//  1. max with packed fp16 IEEE maximum (NaN anywhere, or no finite entry,
//     makes the row NaN, as the reference's e^(x - m) / Z does);
//  2. -inf (masked or padded) entries clamped to -65504 with a packed max, so
//     they give e = 0 and e * s = 0 without a per-element guard;
//  3. e = 2^((x - m) log2 e), Z' and T = sum e * s.  Only a wave whose lanes
//     hold an entry equal to the row max (one wave of the row, typically) needs
//     the per-element test that keeps those entries out of Z' and counts them
//     (c0); the others take the test-free loop;
//  4. probabilities p = fp16(e / Z) from the kept e (VPT <= 4) or recomputed e,
//     stored before
//  5. H, which only the row's first wave evaluates (its stores drain meanwhile).
// The row's registers: lane l of wave wr of the row holds 16-byte vectors
// j = 0 .. VPT-1 at column ((j * WPR + wr) * 64 + l) * 8; entries past the row
// (or past the causal limit) read as -inf and are not loaded.
// NT: non-temporal loads (the _nt kernels: logits read once from HBM).
template <int VPT, int WPR, bool NT = false>
EE_DEV void se_load(const EeSoftmaxArgs& a, int64_t r, int wr, int lane, u32x4 (&v)[VPT]) {
    const int S = a.S;
    const int nvalid = a.causal ? min(S, (int)(r % S) + 1) : S;
    const uint16_t* xr = a.x + r * a.ld_x;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c0 = ((j * WPR + wr) * 64 + lane) * 8;
        if (c0 + 8 <= nvalid) {
            if constexpr (NT) v[j] = __builtin_nontemporal_load((const u32x4*)(xr + c0));
            else v[j] = *(const u32x4*)(xr + c0);
        } else {
            uint16_t e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = (c0 + i < nvalid) ? xr[c0 + i] : (uint16_t)0xFC00u;  // -inf
            v[j] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                         e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
        }
    }
}

// H of a row from its reduced sums, and its tier, written by lane 0.
EE_DEV void se_entropy_out(const EeSoftmaxArgs& a, int64_t row, bool dead, float cz, float z, float t, int lane) {
    const float H = dead ? NAN : entropy_from(cz, z, t);
    if (lane == 0) {
        a.h[row] = H;
        if (a.tier) a.tier[row] = tier_of(H, a.tau_low, a.tau_high);
    }
}

// Steps 1-5 for one row held in v (red: the block's cross-wave partials when WPR > 1).
template <int VPT, int WPR>
EE_DEV void se_process(const EeSoftmaxArgs& a, u32x4 (&v)[VPT], int64_t row, bool valid, int w, int wr, int lane,
                       float (*red)[4]) {
    constexpr bool KEEP_E = VPT <= 4;
    const int S = a.S;

    // ---- 1. max
    f16x2 mx2 = f16x2_from_bits(0xFC00FC00u);
#pragma unroll
    for (int j = 0; j < VPT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx2 = __builtin_elementwise_maximum(mx2, f16x2_from_bits(v[j][i]));
    const float m_lane = fmaximum((float)mx2.x, (float)mx2.y);
    float m = wave_maximum(m_lane);
    if constexpr (WPR > 1) {
        if (lane == 0) red[w][0] = m;
        __syncthreads();
        const int base = (w / WPR) * WPR;
        m = red[base][0];
#pragma unroll
        for (int i = 1; i < WPR; ++i) m = fmaximum(m, red[base + i][0]);
    }
    const bool dead = !(m > -INFINITY);
    const bool has_max = __builtin_amdgcn_ballot_w64(m_lane == m) != 0;   // wave-uniform
    if (dead) m = 0.0f;
    const float negm = -m;

    // ---- 2. -inf -> -65504 (after the max, so NaN rows stay dead).  IEEE maximum
    // (NaN-propagating) needs no canonicalising max of its input first, as maxnum
    // does: one v_pk_maximum3_f16 per two elements.
    const f16x2 lowest = f16x2_from_bits(0xFBFFFBFFu);
#pragma unroll
    for (int j = 0; j < VPT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) v[j][i] = bits_of(__builtin_elementwise_maximum(f16x2_from_bits(v[j][i]), lowest));

    // ---- 3. sums
    float ek[KEEP_E ? VPT * 8 : 1];
    float z0 = 0.f, z1 = 0.f, t0 = 0.f, t1 = 0.f;
    int cnt = 0;
    const float negml = negm * LOG2E;
    if (!has_max) {
        // s2 = (x - m) log2 e; T accumulates e * s2 and is scaled by ln 2 below
#pragma unroll
        for (int j = 0; j < VPT; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t u = v[j][i >> 1];
                const float s2 = (i & 1) ? sub2_hi(u, LOG2E, negml) : sub2_lo(u, LOG2E, negml);
                const float e = __builtin_amdgcn_exp2f(s2);
                if (i & 1) { z1 += e; t1 = fmaf(e, s2, t1); }
                else       { z0 += e; t0 = fmaf(e, s2, t0); }
                if (KEEP_E) ek[j * 8 + i] = e;
            }
    } else {
#pragma unroll
        for (int j = 0; j < VPT; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t u = v[j][i >> 1];
                const float s = (i & 1) ? sub_hi(u, negm) : sub_lo(u, negm);
                const float e = __builtin_amdgcn_exp2f(s * LOG2E);
                const bool at_max = (s == 0.0f);
                cnt += at_max ? 1 : 0;
                if (i & 1) { z1 += at_max ? 0.0f : e; t1 = fmaf(e, s, t1); }
                else       { z0 += at_max ? 0.0f : e; t0 = fmaf(e, s, t0); }
                if (KEEP_E) ek[j * 8 + i] = e;
            }
    }
    float z = wave_sum(z0 + z1);
    float t = wave_sum(t0 + t1);
    if (!has_max) t *= LN2;
    float cz = has_max ? (float)wave_sum_i32(cnt) : 0.0f;   // cnt is 0 in every lane elsewhere
    if constexpr (WPR > 1) {
        if (lane == 0) { red[w][1] = z; red[w][2] = t; red[w][3] = cz; }
        __syncthreads();
        const int base = (w / WPR) * WPR;
        z = red[base][1]; t = red[base][2]; cz = red[base][3];
#pragma unroll
        for (int i = 1; i < WPR; ++i) { z += red[base + i][1]; t += red[base + i][2]; cz += red[base + i][3]; }
    }
    if (!valid) return;
    // One wave x 4 vectors (eight waves per SIMD, 64 VGPRs) has no registers to keep
    // the row sums through the stores: it evaluates H first.
    constexpr bool H_FIRST = WPR == 1 && VPT == 4;
    if constexpr (H_FIRST) se_entropy_out(a, row, dead, cz, z, t, lane);

    // ---- 4. one write of the probabilities, issued before H is evaluated so that
    // the stores drain while the row's first wave computes it (1/Z from v_rcp_f32,
    // within 1 ulp; Z >= 1)
    if (a.p != nullptr) {
        const float invZ = dead ? NAN : __builtin_amdgcn_rcpf(cz + z);
        uint16_t* pr = a.p + row * a.ld_p;
    #pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int c0 = ((j * WPR + wr) * 64 + lane) * 8;
            if (c0 >= S) continue;
            float ev[8];
    #pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (KEEP_E) {
                    ev[i] = ek[j * 8 + i];
                } else {                                  // the e of step 3, recomputed
                    const uint32_t u = v[j][i >> 1];
                    ev[i] = __builtin_amdgcn_exp2f(has_max ? ((i & 1) ? sub_hi(u, negm) : sub_lo(u, negm)) * LOG2E
                                                           : ((i & 1) ? sub2_hi(u, LOG2E, negml) : sub2_lo(u, LOG2E, negml)));
                }
            }
            const u32x4 o{scale_pack_f16x2(ev[0], ev[1], invZ), scale_pack_f16x2(ev[2], ev[3], invZ),
                          scale_pack_f16x2(ev[4], ev[5], invZ), scale_pack_f16x2(ev[6], ev[7], invZ)};
            if (c0 + 8 <= S) {
                // written once, read by a later kernel: non-temporal (measured 5% faster
                // at [4096, 14336], where the kernel runs at ~93% of a plain copy)
                __builtin_nontemporal_store(o, (u32x4*)(pr + c0));
            } else {
    #pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (c0 + i < S) pr[c0 + i] = (uint16_t)(o[i >> 1] >> ((i & 1) * 16));
            }
        }
    }
    // ---- 5. H and the tier, by the row's first wave
    if (!H_FIRST && wr == 0) se_entropy_out(a, row, dead, cz, z, t, lane);
}

template <int VPT, int WPR, bool NT = false>
EE_DEV void softmax_entropy_vec(const EeSoftmaxArgs& a) {
    typedef SeGeom<WPR> G;
    __shared__ float red[G::RPB * WPR][4];
    const int lane = lane_id();
    const int w = wave_id();
    const int wr = w % WPR;
    const int64_t row = (int64_t)blockIdx.x * G::RPB + w / WPR;
    const bool valid = row < a.rows;
    const int64_t r = valid ? row : a.rows - 1;    // keep every wave in the barriers
    u32x4 v[VPT];
    se_load<VPT, WPR, NT>(a, r, wr, lane, v);
    se_process<VPT, WPR>(a, v, row, valid, w, wr, lane, red);
}

// Short rows (one wave per row): each wave takes RPW consecutive rows and
// issues all their loads before working on the first, so a wave keeps
// RPW x VPT x 1 KB of the input in flight instead of VPT x 1 KB.
template <int VPT, int RPW>
EE_DEV void softmax_entropy_rows(const EeSoftmaxArgs& a) {
    const int lane = lane_id();
    const int w = wave_id();
    const int64_t row0 = ((int64_t)blockIdx.x * (EE_BLOCK / 64) + w) * RPW;
    u32x4 v[RPW][VPT];
#pragma unroll
    for (int q = 0; q < RPW; ++q) se_load<VPT, 1>(a, min(row0 + q, a.rows - 1), 0, lane, v[q]);
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        if (row0 + q >= a.rows) break;                // wave-uniform; no barriers in se_process<., 1>
        se_process<VPT, 1>(a, v[q], row0 + q, true, w, 0, lane, nullptr);
    }
}

// Any row length, any alignment: one wave per row, three passes over the row
// (max, sums, store) with 2-byte loads.  Used when the vector kernel's
// preconditions (16-byte aligned rows, S <= 8 * 512 * 4) do not hold.
EE_DEV void softmax_entropy_generic(const EeSoftmaxArgs& a) {
    const int lane = lane_id();
    const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
    if (row >= a.rows) return;                     // no barriers below
    const int S = a.S;
    const int nvalid = a.causal ? min(S, (int)(row % S) + 1) : S;
    const uint16_t* xr = a.x + row * a.ld_x;
    float m = -INFINITY;
    for (int c = lane; c < nvalid; c += 64) m = fmaximum(m, f16_lo(xr[c]));
    m = wave_maximum(m);
    const bool dead = !(m > -INFINITY);                // NaN or no finite entry: NaN row
    if (dead) m = 0.0f;
    float cz = 0.f, z = 0.f, t = 0.f;
    for (int c = lane; c < nvalid; c += 64) {
        const float s = fmaxf(f16_lo(xr[c]) - m, -256.0f);
        const float e = __builtin_amdgcn_exp2f(s * LOG2E);
        const bool at_max = (s == 0.0f);
        cz += at_max ? 1.0f : 0.0f;
        z += at_max ? 0.0f : e;
        t = fmaf(e, s, t);
    }
    z = wave_sum(z);
    t = wave_sum(t);
    cz = wave_sum(cz);
    const float H = dead ? NAN : entropy_from(cz, z, t);
    if (lane == 0) {
        a.h[row] = H;
        if (a.tier) a.tier[row] = tier_of(H, a.tau_low, a.tau_high);
    }
    if (a.p == nullptr) return;
    const float invZ = dead ? NAN : 1.0f / (cz + z);
    uint16_t* pr = a.p + row * a.ld_p;
    for (int c = lane; c < S; c += 64) {
        float e = 0.0f;
        if (c < nvalid) e = __builtin_amdgcn_exp2f(fmaxf(f16_lo(xr[c]) - m, -256.0f) * LOG2E);
        pr[c] = (uint16_t)pack_f16x2(e * invZ, 0.0f);
    }
}

#define EE_SE_VEC(V, W)                                                                        \
    extern "C" __global__ void __launch_bounds__(SeGeom<W>::BLOCK) eek_softmax_entropy_v##V##_w##W( \
        EeSoftmaxArgs a) {                                                                     \
        softmax_entropy_vec<V, W>(a);                                                          \
    }
// The same within 64 VGPRs, for eight waves per SIMD: with 4 vectors per lane the
// kept e values take the kernel to 65-72 VGPRs (seven waves per SIMD), and at
// [4096, 4096] (8192 waves for 7168 slots) the last 1024 waves ran as a second
// round: 15.1 -> 14.2 us cold at 63 VGPRs.  (Three, five, six and seven waves per
// row do not fit 64 without spilling and keep the plain form.)
#define EE_SE_VEC_8W(V, W)                                                                     \
    extern "C" __global__ void __launch_bounds__(SeGeom<W>::BLOCK)                             \
        __attribute__((amdgpu_waves_per_eu(8))) eek_softmax_entropy_v##V##_w##W(EeSoftmaxArgs a) { \
        softmax_entropy_vec<V, W>(a);                                                          \
    }
// Non-temporal twins of the multi-wave layouts, for logits too large to have
// stayed in cache (the launcher's choice): from HBM 3-5% faster, from the caches
// ~13% slower (configs 0-2, measured both ways).
#define EE_SE_VEC_NT(V, W, EPU)                                                                \
    extern "C" __global__ void __launch_bounds__(SeGeom<W>::BLOCK)                             \
        __attribute__((amdgpu_waves_per_eu(EPU))) eek_softmax_entropy_v##V##_w##W##_nt(EeSoftmaxArgs a) { \
        softmax_entropy_vec<V, W, true>(a);                                                    \
    }
#define EE_SE_VEC_W(V) EE_SE_VEC(V, 1) EE_SE_VEC(V, 2) EE_SE_VEC(V, 3) EE_SE_VEC(V, 4) \
                       EE_SE_VEC(V, 5) EE_SE_VEC(V, 6) EE_SE_VEC(V, 7) EE_SE_VEC(V, 8)
EE_SE_VEC_W(1)
EE_SE_VEC_W(2)
EE_SE_VEC_W(3)
EE_SE_VEC_8W(4, 1)
EE_SE_VEC_8W(4, 2)
EE_SE_VEC(4, 3)
EE_SE_VEC_8W(4, 4)
EE_SE_VEC(4, 5)
EE_SE_VEC(4, 6)
EE_SE_VEC(4, 7)
EE_SE_VEC_8W(4, 8)
// short rows, several per wave
#define EE_SE_ROWS(V, R) \
    extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_softmax_entropy_v##V##_r##R(EeSoftmaxArgs a) { \
        softmax_entropy_rows<V, R>(a);                                                                  \
    }
EE_SE_ROWS(1, 2)
EE_SE_ROWS(1, 4)
EE_SE_ROWS(2, 2)
// rows longer than 4 * 8 * 512: eight waves, probabilities from recomputed e
EE_SE_VEC(5, 8)
EE_SE_VEC(6, 8)
EE_SE_VEC(7, 8)
EE_SE_VEC(8, 8)
EE_SE_VEC_NT(4, 2, 8)
EE_SE_VEC_NT(4, 4, 8)
EE_SE_VEC_NT(4, 8, 8)
EE_SE_VEC_NT(5, 8, 1)
EE_SE_VEC_NT(6, 8, 1)
EE_SE_VEC_NT(7, 8, 1)
EE_SE_VEC_NT(8, 8, 1)

extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_softmax_entropy_generic(EeSoftmaxArgs a) {
    softmax_entropy_generic(a);
}
