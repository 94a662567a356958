// attention.hip -- causal grouped-query attention fused with the Shannon
// entropy of its probability rows, head_dim 64, fp16, for gfx950.
//
// For one (batch, query head) and query s the kernel computes, over keys c <= s:
//   x_c = fp16(q_s . k_c)       (q already carries 1/sqrt(64); the fp16 rounding
//                                is the one an fp16 product q k^T stores),
//   m = max x,  Z = sum_c e^(x_c - m),  p_c = e^(x_c - m) / Z,
//   out_s = fp16(sum_c p_c v_c),  H_s = ln Z - sum_c p_c (x_c - m),
// i.e. the attention of an HF Llama layer and the entropy that
// softmax_entropy.hip takes of its probability rows (the quantity of
// EE/python/kernels.py:264-312 and dispatch.py:243-245), without writing the
// S x S scores or probabilities anywhere.
//
// Keys stream through LDS in blocks of 64 (K rows and V^T rows, direct-to-LDS
// DMA, double-buffered) with an online maximum.  Per lane and query row the
// kernel keeps z = sum e^(x - m) and t = sum e^(x - m) (x - m) over its keys,
// rescaled by e^(m_old - m_new) when the running max m grows; H = ln Z - T / Z
// over the lane pair.  (softmax_entropy.hip uses a cancellation-free form that
// keeps full relative precision for nearly one-hot rows; here H has ~1e-7
// absolute error there, which routing at thresholds of order 1 does not see,
// and the per-element test that form needs (a compare, two selects and an add
// per score) would add roughly a third to the per-score VALU work, which at
// head_dim 64 bounds the kernel, not the MFMAs.)  The
// output accumulates fp16(e^(x - m)) v in f32, rescaled the same way, and is
// divided by Z at the end.
//
// Workgroup: one block of 64 queries of W query heads (W = 2 or 4 waves, one
// head each) that share one kv head, so every K/V block staged in LDS serves W
// heads and every wave has the same causal key range.  A wave holds its 64
// queries as two 32-row blocks.  MFMAs are v_mfma_f32_32x32x16_f16 with the
// key (or V^T) fragment as the first operand, so each lane ends up with one
// query row: row reductions stay in the lane and its partner lane l ^ 32.
// The probabilities feed the second product straight from the score
// registers: lane l < 32 holds keys 16c + {0..3, 8..11} of each 16-key chunk c,
// lane l + 32 keys 16c + {4..7, 12..15}; V^T stores each 16-key group in that
// order (0-3, 8-11, 4-7, 12-15), so one 16-byte read gives a lane the V^T
// fragment whose K slots match (written by eek_qkv_rope with v_t set).
#include "../common/ee_device.h"

#define LOG2E 1.4426950408889634f
#define ATT_STAGE 16384                 // K block 64 x 128 B, then V^T block 64 x 128 B

#define LPTR(p) ((void __attribute__((address_space(3)))*)(p))

// 16 bytes per lane from global memory (wave-uniform base + 32-bit per-lane byte
// offset) straight into LDS at lds_base + 16 * lane (lds_base wave-uniform);
// tracked by the explicit vmcnt wait of each step.
EE_DEV void att_dma16(const void* sbase, uint32_t voff, uint32_t lds_base) {
    const uint32_t lb = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_base);   // uniform by construction
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lb), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}
#define ATT_WAITCNT_VM0() __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8) | (0 << 14))
#define ATT_WAITCNT_LGKM0() __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14))

// 16-byte chunk c of the 128-byte LDS row r sits at chunk c ^ ((r >> 1) & 7):
// the 16 rows one ds_read_b128 pass serves hit 16 distinct bank groups.
EE_DEV uint32_t att_off(int row, int chunk) { return (uint32_t)(row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4)); }

// (x - m) log2(e) for the low / high fp16 half of a packed word in one
// v_fma_mix_f32: x * log2(e) + (-m log2(e)), a single rounding.
EE_DEV float att_l2_lo(uint32_t u, float negm2) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(u), "v"(LOG2E), "v"(negm2));
    return r;
}
EE_DEV float att_l2_hi(uint32_t u, float negm2) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(u), "v"(LOG2E), "v"(negm2));
    return r;
}

EE_DEV f32x16 mma16(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int W>
EE_DEV void attn_causal_d64(const EeAttnArgs& a) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * ATT_STAGE];
    const int lane = (int)(threadIdx.x & 63), wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int r32 = lane & 31, hi = lane >> 5;
    const int nqb = a.S >> 6, hgroups = a.Hq / W, G = a.Hq / a.Hkv;
    const int ngrp = a.B * hgroups;
    // Query block order: the first half of the grid runs the longest key ranges
    // (qb = nqb - 1, nqb - 2, ...), the second half the mirror images (qb = 0, 1,
    // ...), so workgroup i + N/2, which the dispatcher places beside workgroup i
    // (two fit per CU), brings qb' = nqb - 1 - qb: nqb + 1 key steps per CU.
    const int rank = (int)blockIdx.x / ngrp, hrank = (nqb + 1) >> 1;
    const int qb = rank < hrank ? nqb - 1 - rank : rank - hrank;
    const int grp = (int)blockIdx.x % ngrp;
    const int b = grp / hgroups, hg = grp % hgroups;
    const int hq = hg * W + wave, hkv = (hg * W) / G;
    const int q0 = qb << 6, nsteps = qb + 1;
    const int64_t S = a.S;

    // DMA of step st into buffer st & 1: 16 instructions of 8 LDS rows (1 KB),
    // 0-7 the K rows of keys 64 st .. 64 st + 63, 8-15 the V^T rows d of those
    // keys; wave w issues instructions w, w + W, ...  Lane l lands at row
    // 8 (i % 8) + l / 8, physical chunk l % 8, which holds logical chunk
    // (l % 8) ^ swz(row), swz(row) = (row >> 1) & 7.
    // Row r = 8 (i % 8) + l / 8 of instruction i has swz(r) = (4 (i & 1) + (l >> 4)) & 7,
    // so two per-lane byte offsets per operand (i even, odd) plus wave-uniform
    // offsets address every instruction.
    const int64_t kvh = (int64_t)b * a.Hkv + hkv;
    const uint16_t* kbase = a.k + kvh * S * 64;       // wave-uniform
    const uint16_t* vbase = a.vt + kvh * 64 * S;
    uint32_t ko[2], vo[2];
#pragma unroll
    for (int par = 0; par < 2; ++par) {
        const int lc = (lane & 7) ^ ((4 * par + (lane >> 4)) & 7);
        ko[par] = (uint32_t)(((lane >> 3) * 64 + lc * 8) * 2);
        vo[par] = (uint32_t)(((int64_t)(lane >> 3) * S + lc * 8) * 2);
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)LPTR(smem);
    auto issue = [&](int st) {
        const uint32_t sb = lds0 + (uint32_t)((st & 1) * ATT_STAGE);
#pragma unroll
        for (int j = 0; j < 16 / W; ++j) {
            const int i = wave + j * W, g = i & 7;
            if (i < 8) att_dma16(kbase, ko[g & 1] + (uint32_t)(((st << 6) + 8 * g) * 128), sb + (uint32_t)(g * 1024));
            else att_dma16(vbase, vo[g & 1] + (uint32_t)((8 * g * S + (st << 6)) * 2), sb + (uint32_t)(8192 + g * 1024));
        }
    };
    issue(0);

    // q fragments: row block rb (queries q0 + 32 rb + (l & 31)), d chunk dc
    // (d = 16 dc + 8 (l >> 5) .. + 7).
    const uint16_t* qrow = a.q + (((int64_t)b * a.Hq + hq) * S + q0) * 64;
    u32x4 qf[2][4];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int dc = 0; dc < 4; ++dc) qf[rb][dc] = *(const u32x4*)(qrow + (rb * 32 + r32) * 64 + dc * 16 + hi * 8);

    // Running row max (below every clamped score at the start), and per lane
    // z = sum e, t = sum e * (x - m) log2(e) over the lane's keys.
    f32x16 o[2][2];
    float m[2], z[2], t[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        m[rb] = -131008.0f;
        z[rb] = t[rb] = 0.0f;
#pragma unroll
        for (int db = 0; db < 2; ++db) o[rb][db] = f32x16{};
    }

    for (int st = 0; st < nsteps; ++st) {
        ATT_WAITCNT_VM0();                            // this wave's share of step st has landed
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();                 // all of it has; step st - 1's buffer is free
        asm volatile("" ::: "memory");
        if (st + 1 < nsteps) issue(st + 1);
        const uint8_t* sk = smem + (st & 1) * ATT_STAGE;
        const uint8_t* sv = sk + 8192;

        // scores, rounded to fp16 and packed: xh[rb][kb][w] holds keys r = 2w, 2w + 1 of
        // block (rb, kb); lane holds query 32 rb + (l & 31), key 64 st + 32 kb +
        // 8 (r / 4) + 4 (l >> 5) + r % 4.  On the diagonal step, keys > query become
        // -65504 (e = 0, e * (x - m) = 0).
        uint32_t xh[2][2][8];
        f16x2 mx2[2] = {f16x2{(f16)-65504.0f, (f16)-65504.0f}, f16x2{(f16)-65504.0f, (f16)-65504.0f}};
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            u32x4 kf[4];
#pragma unroll
            for (int dc = 0; dc < 4; ++dc) kf[dc] = *(const u32x4*)(sk + att_off(kb * 32 + r32, dc * 2 + hi));
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                f32x16 acc = f32x16{};
#pragma unroll
                for (int dc = 0; dc < 4; ++dc) acc = mma16(kf[dc], qf[rb][dc], acc);
                if (st == qb) {                       // wave-uniform: the diagonal step only
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int kk = kb * 32 + (r >> 2) * 8 + hi * 4 + (r & 3);
                        acc[r] = kk > rb * 32 + r32 ? -65504.0f : fmaxf(acc[r], -65504.0f);
                    }
                }
#pragma unroll
                for (int w = 0; w < 8; ++w) {
                    xh[rb][kb][w] = pack_f16x2(acc[2 * w], acc[2 * w + 1]);
                    mx2[rb] = __builtin_elementwise_max(mx2[rb], f16x2_from_bits(xh[rb][kb][w]));
                }
            }
        }

        __builtin_amdgcn_sched_barrier(0);           // phases stay apart: the scheduler would hoist LDS reads
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            float ml = fmaxf((float)mx2[rb].x, (float)mx2[rb].y);
            ml = fmaxf(ml, __shfl_xor(ml, 32));
            const float mn = fmaxf(m[rb], ml);
            // rescale to the new max (alpha = 1 if unchanged; 0 at the first step,
            // where m starts below every score): t is kept in log2 units
            const float d2 = (m[rb] - mn) * LOG2E;
            const float alpha = __builtin_amdgcn_exp2f(d2);
            t[rb] = alpha * (t[rb] + d2 * z[rb]);
            z[rb] = alpha * z[rb];
            if (__any(mn > m[rb])) {                  // wave vote: skip the rescale when no row max grew
#pragma unroll
                for (int db = 0; db < 2; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[rb][db][r] *= alpha;
            }
            m[rb] = mn;
            const float negm2 = -mn * LOG2E;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int w = 0; w < 8; ++w) {
                    float e2[2];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float s2 = h ? att_l2_hi(xh[rb][kb][w], negm2) : att_l2_lo(xh[rb][kb][w], negm2);
                        const float e = __builtin_amdgcn_exp2f(s2);
                        z[rb] += e;
                        t[rb] += e * s2;
                        e2[h] = e;
                    }
                    xh[rb][kb][w] = pack_f16x2(e2[0], e2[1]);   // now the fp16 probability (unnormalised)
                }
        }
        __builtin_amdgcn_sched_barrier(0);
        // out[rb][db] += P V: lane holds query 32 rb + (l & 31), d = 32 db + 8 (r / 4) + 4 (l >> 5) + r % 4
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const u32x4 vf = *(const u32x4*)(sv + att_off(db * 32 + r32, cc * 2 + hi));
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    const int kb = cc >> 1, w0 = (cc & 1) * 4;
                    const u32x4 pf = u32x4{xh[rb][kb][w0], xh[rb][kb][w0 + 1], xh[rb][kb][w0 + 2], xh[rb][kb][w0 + 3]};
                    o[rb][db] = mma16(vf, pf, o[rb][db]);
                }
            }
    }

    // Row totals over the lane pair, entropy, normalisation.
    ATT_WAITCNT_LGKM0();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();                     // every wave is done with the K/V buffers
    asm volatile("" ::: "memory");
    uint8_t* tile = smem + wave * 8192;               // 64 rows x 128 B of this wave's output
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const float L = z[rb] + __shfl_xor(z[rb], 32);
        const float ts = t[rb] + __shfl_xor(t[rb], 32);
        const float Hs = logf(L) - 0.69314718055994531f * ts / L;
        const int qrow_i = q0 + rb * 32 + r32;
        if (hi == 0) a.h[((int64_t)b * a.Hq + hq) * S + qrow_i] = Hs;
        const float inv = 1.0f / L;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = db * 32 + q * 8 + hi * 4;
                *(u32x2*)(tile + att_off(rb * 32 + r32, col >> 3) + ((col >> 2) & 1) * 8) =
                    u32x2{pack_f16x2(o[rb][db][4 * q] * inv, o[rb][db][4 * q + 1] * inv),
                          pack_f16x2(o[rb][db][4 * q + 2] * inv, o[rb][db][4 * q + 3] * inv)};
            }
    }
    // Each wave reads back only its own tile: rows of 128 contiguous bytes of out.
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int row = k * 8 + (lane >> 3), ch = lane & 7;
        const u32x4 v = *(const u32x4*)(tile + att_off(row, ch));
        uint16_t* dst = a.out + ((int64_t)b * S + q0 + row) * a.ld_out + (int64_t)hq * 64 + ch * 8;
        __builtin_nontemporal_store(v, (u32x4*)dst);
    }
}

// One entry per workgroup width W (query heads sharing a kv head per workgroup).
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
eek_attn_causal_d64_w4(EeAttnArgs a) { attn_causal_d64<4>(a); }
extern "C" __global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(2)))
eek_attn_causal_d64_w2(EeAttnArgs a) { attn_causal_d64<2>(a); }
