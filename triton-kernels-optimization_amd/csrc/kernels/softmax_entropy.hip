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
// Layout: row-major rows, unit column stride.  One to four wave64s per row;
// each lane holds VPT 16-byte vectors (8 fp16) of the row in registers, so
// the row is read from HBM exactly once and the probabilities are written
// once: 2 bytes in + 2 bytes out per element + 4 bytes of H per row.
#include "../common/ee_device.h"

#define LOG2E 1.4426950408889634f

// Combine per-wave partials of the WPR waves that share a row.
template <int WPR>
EE_DEV float row_reduce_max(float v, float (*slot)[4], int q) {
    if (WPR == 1) return v;
    const int w = wave_id();
    if (lane_id() == 0) slot[w][q] = v;
    __syncthreads();
    const int base = (w / WPR) * WPR;
    float r = slot[base][q];
#pragma unroll
    for (int i = 1; i < WPR; ++i) r = fmaximum(r, slot[base + i][q]);
    return r;
}
template <int WPR>
EE_DEV void row_reduce_sum3(float& x, float& y, float& z, float (*slot)[4]) {
    if (WPR == 1) return;
    const int w = wave_id();
    if (lane_id() == 0) { slot[w][1] = x; slot[w][2] = y; slot[w][3] = z; }
    __syncthreads();
    const int base = (w / WPR) * WPR;
    x = slot[base][1]; y = slot[base][2]; z = slot[base][3];
#pragma unroll
    for (int i = 1; i < WPR; ++i) { x += slot[base + i][1]; y += slot[base + i][2]; z += slot[base + i][3]; }
}

EE_DEV int tier_of(float h, double tl, double th) {
    const double d = (double)h;
    return d < tl ? 0 : (d < th ? 1 : 2);
}

// Entropy from the reduced partial sums (see header comment).
EE_DEV float entropy_from(float c0, float z, float t) {
    return logf(c0) + log1pf(z / c0) - t / (c0 + z);
}

template <int VPT, int WPR>
EE_DEV void softmax_entropy_vec(const EeSoftmaxArgs& a) {
    constexpr int RPB = 4 / WPR;                  // rows per 256-thread block
    constexpr bool KEEP_E = VPT <= 4;             // keep e^s in registers for the store pass
    __shared__ float slot[4][4];

    const int lane = lane_id();
    const int w = wave_id();
    const int wr = w % WPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + w / WPR;
    const bool valid = row < a.rows;
    const int64_t r = valid ? row : a.rows - 1;    // keep every wave in the barriers
    const int S = a.S;
    const int nvalid = a.causal ? min(S, (int)(r % S) + 1) : S;
    const uint16_t* xr = a.x + r * a.ld_x;

    // ---- one read of the row: VPT x 16 B per lane, lanes adjacent in memory
    u32x4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c0 = ((j * WPR + wr) * 64 + lane) * 8;
        if (c0 + 8 <= nvalid) {
            v[j] = *(const u32x4*)(xr + c0);
        } else {
            uint16_t e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = (c0 + i < nvalid) ? xr[c0 + i] : (uint16_t)0xFC00u;  // -inf
            v[j] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                         e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
        }
    }

    // ---- max: packed fp16 maximum is exact and propagates NaN, so a NaN
    // anywhere in the row (or no finite entry) makes the whole row NaN, as the
    // reference's e^(x - m) / Z does.
    f16x2 mx2 = f16x2_from_bits(0xFC00FC00u);
#pragma unroll
    for (int j = 0; j < VPT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx2 = __builtin_elementwise_maximum(mx2, f16x2_from_bits(v[j][i]));
    float m = fmaximum((float)mx2.x, (float)mx2.y);
    m = wave_maximum(m);
    m = row_reduce_max<WPR>(m, slot, 0);
    const bool dead = !(m > -INFINITY);
    if (dead) m = 0.0f;

    // ---- exact sums: c0 (entries at the max, counted by ballot on the scalar
    // unit), Z' (e over the others), T = sum e*s
    int nmax = 0;
    float z0 = 0.f, z1 = 0.f, t0 = 0.f, t1 = 0.f;
    float ek[KEEP_E ? VPT * 8 : 1];
#pragma unroll
    for (int j = 0; j < VPT; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = v[j][i >> 1];
            const float xv = (i & 1) ? f16_hi(u) : f16_lo(u);
            const float s = fmaxf(xv - m, -256.0f);          // -inf (masked) -> e = 0, e*s = 0
            const float e = __builtin_amdgcn_exp2f(s * LOG2E);
            const bool at_max = (s == 0.0f);
            nmax += __builtin_popcountll(__builtin_amdgcn_ballot_w64(at_max));
            if (i & 1) { z1 += at_max ? 0.0f : e; t1 = fmaf(e, s, t1); }
            else       { z0 += at_max ? 0.0f : e; t0 = fmaf(e, s, t0); }
            if (KEEP_E) ek[j * 8 + i] = e;
        }
    float z = wave_sum(z0 + z1);
    float t = wave_sum(t0 + t1);
    float cz = (float)nmax;                                  // already the wave's count
    row_reduce_sum3<WPR>(z, t, cz, slot);
    const float H = dead ? NAN : entropy_from(cz, z, t);
    if (valid && wr == 0 && lane == 0) {
        a.h[row] = H;
        if (a.tier) a.tier[row] = tier_of(H, a.tau_low, a.tau_high);
    }
    if (a.p == nullptr || !valid) return;

    // ---- one write of the probabilities
    const float invZ = dead ? NAN : 1.0f / (cz + z);
    uint16_t* pr = a.p + row * a.ld_p;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c0 = ((j * WPR + wr) * 64 + lane) * 8;
        if (c0 >= S) continue;
        float pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float e;
            if (KEEP_E) {
                e = ek[j * 8 + i];
            } else {
                const uint32_t u = v[j][i >> 1];
                const float xv = (i & 1) ? f16_hi(u) : f16_lo(u);
                e = __builtin_amdgcn_exp2f(fmaxf(xv - m, -256.0f) * LOG2E);
            }
            pv[i] = e * invZ;
        }
        const u32x4 o{pack_f16x2(pv[0], pv[1]), pack_f16x2(pv[2], pv[3]),
                      pack_f16x2(pv[4], pv[5]), pack_f16x2(pv[6], pv[7])};
        if (c0 + 8 <= S) {
            *(u32x4*)(pr + c0) = o;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (c0 + i < S) pr[c0 + i] = (uint16_t)(o[i >> 1] >> ((i & 1) * 16));
        }
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

#define EE_SE_VEC(V, W)                                                                  \
    extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_softmax_entropy_v##V##_w##W( \
        EeSoftmaxArgs a) {                                                               \
        softmax_entropy_vec<V, W>(a);                                                    \
    }
#define EE_SE_VEC_W(V) EE_SE_VEC(V, 1) EE_SE_VEC(V, 2) EE_SE_VEC(V, 4)
EE_SE_VEC_W(1)
EE_SE_VEC_W(2)
EE_SE_VEC_W(3)
EE_SE_VEC_W(4)
EE_SE_VEC_W(5)
EE_SE_VEC_W(6)
EE_SE_VEC_W(7)
EE_SE_VEC_W(8)

extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_softmax_entropy_generic(EeSoftmaxArgs a) {
    softmax_entropy_generic(a);
}
