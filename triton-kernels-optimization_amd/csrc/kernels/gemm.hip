// gemm.hip -- MFMA GEMMs of the three precision tiers for gfx950: the 128 x 128
// tile kernels (config 0, small grids, routed tiers; the 256 x 256 ones are in
// gemm256.hip).
//
//   EE_GEMM_I8 : int8 x int8 -> int32; C = fp16((f32(acc) * a_scale[m]) * b_scale[n])
//                (EE/python/kernels.py:50-110)
//   EE_GEMM_F8 : e4m3 x e4m3 -> f32; C = fp16((acc * a_scale[m]) * b_scale[n])
//                (EE/python/kernels.py:118-180; codes from quant.hip)
//   EE_GEMM_F16: fp16 x fp16 -> f32; C = fp16(acc)
//                (EE/python/kernels.py:192-246; W8A16 weights pre-dequantised
//                bit-exactly by eek_pack_b_f16)
//
// Operands: A [M, K] and B [N, K], both K-contiguous, which is the order the
// MFMA register fragments want (16 consecutive K bytes per lane and operand).
//
// Pipelined kernels (K * elem_size a multiple of 128 bytes): a 512-thread
// workgroup computes a 128 x 128 tile of C as four 64 x 64 quadrants of 32 x 32
// blocks; K advances in 128-byte stages that direct-to-LDS loads
// (global_load_lds_dwordx4, no VGPR staging) stream into a ring of LDS stages;
// LDS rows are 128 bytes, 16-byte chunk c of row r at chunk c ^ ((r >> 1) & 7).
// Per block and K slice the MFMAs are the pipes of ee_gemm_dev.h: INT8 four
// 16x16x64 per 64-byte slice, FP8 one 32x32x64, FP16 four 16x16x32.
//   eek_gemm_{i8,f8,f16}: loader waves (4 compute waves + 4 DMA waves);
//   eek_gemm_{i8,f16}_w8: 8 waves that each compute and load (Gemm8);
//   eek_gemm_{i8,f8}_persist, eek_gemm_routed[_persist]: persistent and routed grids;
//   eek_gemm_w8a16: the FP16 tier on int8 weight codes dequantised in registers.
// eek_gemm_{i8,f8,f16}_generic (K a multiple of 16 bytes only): 256 threads,
// two register-staged LDS buffers and a zero-filled K tail; each wave owns a
// 64 x 64 quadrant as 4 x 4 blocks of 16x16 MFMAs (16x16x64 i8, 16x16x128
// e4m3, 16x16x32 f16).
//
// The MFMA is issued with B as its first operand, so each lane ends up with
// rows of C and four consecutive columns of each (one 8-byte store).
// Routing: with a device row count counts[tier] (off = rows of lower tiers),
// A row m is a[a_idx[off + m]] (gather from the activations) or, without
// a_idx, a[off + m] (the quantiser's partition slot), a_scale is read at
// off + m, and C row m is c[c_idx[off + m]] (scatter).  The grid covers the
// upper bound M and surplus workgroups exit at once.
#include "../common/ee_device.h"
#include "../common/ee_gemm_dev.h"

// Every epilogue / quantiser multiply and add is its own rounded f32
// operation, as in the reference: no contraction into FMAs.  (Conversions to
// fp16 take their operand through f32_rn, which keeps a product from being
// folded into the conversion.)
#pragma clang fp contract(off)

#define BM 128
#define BN 128
#define LDS_STAGE ((BM + BN) * BKB)     // 32 KB
#define NSTAGE 5                        // pipelined kernel: LDS stages (5 x 32 KB = all 160 KB)

template <int KIND> struct AccT { typedef f32x4 type; };
template <> struct AccT<EE_GEMM_I8> { typedef i32x4 type; };


// Workgroup -> tile.  Consecutive workgroup ids land on different XCDs
// (round robin over 8); renumber so each XCD owns a contiguous run of tiles,
// ordered M-fastest, so an XCD's L2 sees few distinct B column panels.
EE_DEV void tile_of(int bid, int nblk, int tiles_m, int& tm, int& tn) {
    int logical = bid;
    if ((nblk & 7) == 0) logical = (bid & 7) * (nblk >> 3) + (bid >> 3);
    tm = logical % tiles_m;
    tn = logical / tiles_m;
}

// One 128-byte K stage from LDS into the 4 x 4 accumulator blocks of a wave.
template <int KIND, typename acc_t>
EE_DEV void mfma_stage(const uint8_t* s, acc_t (&acc)[4][4], int wm, int wn, int lane) {
    const int fr = lane & 15, fg = lane >> 4;
    if constexpr (KIND == EE_GEMM_F8) {
        i32x8 af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ra = wm * 64 + i * 16 + fr, rb = BM + wn * 64 + i * 16 + fr;
            const u32x4 a0 = *(const u32x4*)(s + lds_off(ra, 2 * fg));
            const u32x4 a1 = *(const u32x4*)(s + lds_off(ra, 2 * fg + 1));
            const u32x4 b0 = *(const u32x4*)(s + lds_off(rb, 2 * fg));
            const u32x4 b1 = *(const u32x4*)(s + lds_off(rb, 2 * fg + 1));
            af[i] = i32x8{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
            bf[i] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[j], af[i], acc[i][j], 0, 0, 0, 0, 0, 0);
    } else {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            u32x4 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                af[i] = *(const u32x4*)(s + lds_off(wm * 64 + i * 16 + fr, kk * 4 + fg));
                bf[i] = *(const u32x4*)(s + lds_off(BM + wn * 64 + i * 16 + fr, kk * 4 + fg));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (KIND == EE_GEMM_I8)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i32x4(bf[j]), as_i32x4(af[i]), acc[i][j],
                                                                         0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(bf[j]), as_f16x8(af[i]),
                                                                          acc[i][j], 0, 0, 0);
                }
        }
    }
}

// Dequantising epilogue: lane holds C[m0 + wm*64 + i*16 + fr][n0 + wn*64 + j*16 + 4*fg + 0..3].
template <int KIND, typename acc_t>
EE_DEV void epilogue(const EeGemmArgs& g, const acc_t (&acc)[4][4], int m0, int n0, int M, int64_t off, int wm,
                     int wn, int lane) {
    const int fr = lane & 15, fg = lane >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + wm * 64 + i * 16 + fr;
        if (m >= M) continue;
        const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
        const float as = (KIND == EE_GEMM_F16) ? 0.0f : g.a_scale[off + m];
        uint16_t* cr = g.c + crow * g.ldc;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 64 + j * 16 + 4 * fg;
            if (n >= g.N) continue;                 // N is a multiple of 4
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (KIND == EE_GEMM_I8) {
                    float v = (float)acc[i][j][r];
                    v = v * as;
                    o[r] = v * g.b_scale[n + r];
                } else if constexpr (KIND == EE_GEMM_F8) {
                    const float v = acc[i][j][r] * as;
                    o[r] = v * g.b_scale[n + r];
                } else {
                    o[r] = acc[i][j][r];
                }
            }
            *(u32x2*)(cr + n) = u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
            if constexpr (KIND == EE_GEMM_I8) {
                if (g.acc) *(i32x4*)(g.acc + crow * g.ldc + n) = acc[i][j];
            }
        }
    }
}



template <class P>
struct FragsP {
    typename P::frag_t a[2], b[2];
};
template <int KIND>
using Frags = FragsP<Pipe<KIND>>;

// Fragments of one K slice: lane l reads row (l & 31) of each 32-row block, K
// chunk slice * SB/16 + (l >> 5) * LSTEP (and the chunk CSTEP after it when
// CPF == 2): lanes 0-31 and 32-63 cover the two K halves of each MFMA's operand.
// 16x16 pipes (SUB16): rows (l & 15) and 16 + (l & 15) of each block, chunk 4 slice + (l >> 4).
// JB: 32-column B blocks of the wave (2, or 1 in the 64-wide FP16 tiles).
template <int KIND, int JB = 2>
EE_DEV void read_frags(const uint8_t* s, int slice, int wm, int wn, int lane, Frags<KIND>& f) {
    typedef Pipe<KIND> P;
    static_assert(JB == 2 || P::SUB16, "one-block waves are the 16x16 pipes'");
    if constexpr (P::SUB16) {
        const int c = slice * 4 + (lane >> 4), r = lane & 15;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ra = wm * 64 + i * 32 + r, rb = BM + wn * 64 + i * 32 + r;   // swz(x + 16) == swz(x)
            f.a[i].h[0] = *(const i32x4*)(s + lds_off(ra, c));
            f.a[i].h[1] = *(const i32x4*)(s + lds_off(ra + 16, c));
            if constexpr (JB == 2) {
                f.b[i].h[0] = *(const i32x4*)(s + lds_off(rb, c));
                f.b[i].h[1] = *(const i32x4*)(s + lds_off(rb + 16, c));
            } else if (i == 0) {                      // the wave's one block: B rows 32 wn ..
                const int rb1 = BM + wn * 32 + r;
                f.b[0].h[0] = *(const i32x4*)(s + lds_off(rb1, c));
                f.b[0].h[1] = *(const i32x4*)(s + lds_off(rb1 + 16, c));
            }
        }
    } else {
        const int r = lane & 31;
        const int c0 = slice * (P::SB / 16) + (lane >> 5) * P::LSTEP;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ra = wm * 64 + i * 32 + r, rb = BM + wn * 64 + i * 32 + r;
            if constexpr (P::CPF == 1) {
                f.a[i] = *(const u32x4*)(s + lds_off(ra, c0));
                f.b[i] = *(const u32x4*)(s + lds_off(rb, c0));
            } else {
                const u32x4 a0 = *(const u32x4*)(s + lds_off(ra, c0)), a1 = *(const u32x4*)(s + lds_off(ra, c0 + P::CSTEP));
                const u32x4 b0 = *(const u32x4*)(s + lds_off(rb, c0)), b1 = *(const u32x4*)(s + lds_off(rb, c0 + P::CSTEP));
                f.a[i] = i32x8{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
                f.b[i] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
            }
        }
    }
}

template <int KIND, int JB = 2>
EE_DEV void mma_all(const Frags<KIND>& f, typename Pipe<KIND>::acc_t (&acc)[2][2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[i][j] = Pipe<KIND>::mma(f.b[j], f.a[i], acc[i][j]);
}

// Scheduling groups for one slice: the LDS reads of the next slice (8
// ds_read_b128) spread over the MFMAs of the current slice -- one read per two
// 16x16 MFMAs (INT8, FP16), two reads per 32x32x64 e4m3 MFMA (FP8).  Against
// issuing every read first (same box, three alternating runs): C0 INT8 18.64 ->
// 18.2 us, FP16 33.2 -> 32.1, FP8 18.5 -> 18.2; the reads no longer queue at the
// LDS in one burst while the matrix core waits for the first MFMA's operands.
template <int KIND, int JB = 2>
EE_DEV void interleave() {
    constexpr int NR = (2 + JB) * Pipe<KIND>::CPF, NM = (Pipe<KIND>::SUB16 ? 8 : 2) * JB;
    if constexpr (NM % NR == 0) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);         // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, NM / NR, 0);   // MFMA
        }
    } else if constexpr (NR % NM == 0) {
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, NR / NM, 0);   // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         // MFMA
        }
    } else {                                          // (the 64-wide FP16 tiles: 6 reads, 8 MFMAs)
        __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);   // DS read
        __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);   // MFMA
    }
}

// 32x32 epilogue: lane l, register r of block (i, j) holds
// C[m0 + wm*64 + 32i + (l & 31)][n0 + wn*64 + 32j + 8*(r/4) + 4*(l >> 5) + r%4].
template <int KIND, class P = Pipe<KIND>>
EE_DEV void epilogue32(const EeGemmArgs& g, const typename P::acc_t (&acc)[2][2], int m0, int n0, int M,
                       int64_t off, int wm, int wn, int lane) {
    if constexpr (P::SUB16) {                         // quarter q at row_of(q), col_of(q)
        static_assert(KIND != EE_GEMM_F8, "FP8 runs 32x32 MFMAs");
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int m = m0 + wm * 64 + i * 32 + P::row_of(q, lane);
                    const int n = n0 + wn * 64 + j * 32 + P::col_of(q, lane);
                    if (m >= M || n >= g.N) continue;
                    const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
                    const float as = (KIND == EE_GEMM_F16) ? 0.0f : g.a_scale[off + m];
                    float o[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        o[r] = deq<KIND>(acc[i][j][4 * q + r], as, KIND == EE_GEMM_F16 ? 0.0f : g.b_scale[n + r]);
                    *(u32x2*)(g.c + crow * g.ldc + n) = u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
                    if constexpr (KIND == EE_GEMM_I8) {
                        if (g.acc)
                            *(i32x4*)(g.acc + crow * g.ldc + n) = i32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1],
                                                                        acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                    }
                }
        return;
    } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = m0 + wm * 64 + i * 32 + (lane & 31);
        if (m >= M) continue;
        const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
        const float as = (KIND == EE_GEMM_F16) ? 0.0f : g.a_scale[off + m];
        uint16_t* cr = g.c + crow * g.ldc;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wn * 64 + j * 32 + 8 * q + 4 * (lane >> 5);
                if (n >= g.N) continue;             // N is a multiple of 4
                float o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (KIND == EE_GEMM_I8) {
                        float v = (float)acc[i][j][4 * q + r];
                        v = v * as;
                        o[r] = v * g.b_scale[n + r];
                    } else if constexpr (KIND == EE_GEMM_F8) {
                        const float v = acc[i][j][4 * q + r] * as;
                        o[r] = v * g.b_scale[n + r];
                    } else {
                        o[r] = acc[i][j][4 * q + r];
                    }
                }
                *(u32x2*)(cr + n) = u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
                if constexpr (KIND == EE_GEMM_I8) {
                    if (g.acc)
                        *(i32x4*)(g.acc + crow * g.ldc + n) =
                            i32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                }
            }
        }
    }
    }
}

// Epilogue through LDS: the wave's 64 x 64 fp16 tile is written to a free 8 KB
// LDS region in the 32x32 MFMA layout, read back as rows, and stored 16 bytes
// per lane -- each store instruction covers 8 rows x 128 contiguous bytes of C
// instead of 32 rows x 16 bytes.  (The optional int32 accumulators keep the
// direct path; they are a debug output.)
// Per-lane dequantisation scales of a wave's 64 x 64 quadrant: lane l needs the
// column scales of columns j*32 + 8q + 4(l >> 5) + 0..3 (8 vectors of 4) and the
// row scales of rows i*32 + (l & 31).  Loaded before the K loop so that their
// latency is hidden behind it.
struct TileScales {
    f32x4 bs[2][4];
    float as[2];
};
// The same for the 16x16 layout (Lay16): lane l needs, per 32-column block j, the
// scales of columns j*32 + col_of(0 | 2, l) + 0..3 and, per 32-row block i, of rows
// i*32 + row_of(0 | 1, l).
struct TileScalesL16 {
    f32x4 bs[2][2];
    float as[2][2];
};
template <class P>
using TileScalesOf = std::conditional_t<P::SUB16, TileScalesL16, TileScales>;

template <int KIND, class P = Pipe<KIND>>
EE_DEV void load_scales(const EeGemmArgs& g, int m0, int n0, int M, int64_t off, int wm, int wn, int lane,
                        TileScalesOf<P>& sc) {
    if constexpr (KIND != EE_GEMM_F16 && P::SUB16) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int n = n0 + wn * 64 + j * 32 + P::col_of(2 * c, lane);
                sc.bs[j][c] = (n < g.N) ? *(const f32x4*)(g.b_scale + n) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int m = m0 + wm * 64 + i * 32 + P::row_of(h, lane);
                sc.as[i][h] = (m < M) ? g.a_scale[off + m] : 0.0f;
            }
    } else if constexpr (KIND != EE_GEMM_F16) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wn * 64 + j * 32 + 8 * q + 4 * (lane >> 5);
                sc.bs[j][q] = (n < g.N) ? *(const f32x4*)(g.b_scale + n) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int m = m0 + wm * 64 + i * 32 + (lane & 31);
            sc.as[i] = (m < M) ? g.a_scale[off + m] : 0.0f;
        }
    }
}


// SwiGLU epilogue of a wave's 64 x 64 quadrant (swiglu weights: column block
// j = 0 holds gate values, j = 1 the up values of the same 32 outputs):
// act = fp16(fp16(silu(fp16(gate))) * fp16(up)), the fp16 gate and up being
// exactly what the plain epilogue would store.  The 64 x 32 act block goes
// through the wave's LDS region to act columns (n0 + 64 wn) / 2 ...
template <int KIND, class P = Pipe<KIND>>
EE_DEV void epilogue32_lds_swiglu(const EeGemmArgs& g, const typename P::acc_t (&acc)[2][2],
                                  const TileScalesOf<P>& sc, uint8_t* tile, int m0, int n0, int M, int64_t off,
                                  int wm, int wn, int lane) {
    if constexpr (P::SUB16) {                         // act column col_of(q) of row row_of(q)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float gv[4], uv[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (KIND == EE_GEMM_F16) {
                        gv[r] = acc[i][0][4 * q + r];
                        uv[r] = acc[i][1][4 * q + r];
                    } else {
                        gv[r] = deq<KIND>(acc[i][0][4 * q + r], sc.as[i][P::rq(q)], sc.bs[0][P::cq(q)][r]);
                        uv[r] = deq<KIND>(acc[i][1][4 * q + r], sc.as[i][P::rq(q)], sc.bs[1][P::cq(q)][r]);
                    }
                }
                const int rl = i * 32 + P::row_of(q, lane), ca = P::col_of(q, lane);
                *(u32x2*)(tile + lds_off(rl, ca >> 3) + ((ca >> 2) & 1) * 8) =
                    u32x2{silu_mul2(pack_f16x2(gv[0], gv[1]), pack_f16x2(uv[0], uv[1])),
                          silu_mul2(pack_f16x2(gv[2], gv[3]), pack_f16x2(uv[2], uv[3]))};
            }
    } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rl = i * 32 + (lane & 31);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float gv[4], uv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                gv[r] = deq<KIND>(acc[i][0][4 * q + r], sc.as[i], sc.bs[0][q][r]);
                uv[r] = deq<KIND>(acc[i][1][4 * q + r], sc.as[i], sc.bs[1][q][r]);
            }
            // act column 8q + 4(l >> 5) + 0..3 of the block: chunk q, half l >> 5
            *(u32x2*)(tile + lds_off(rl, q) + (lane >> 5) * 8) =
                u32x2{silu_mul2(pack_f16x2(gv[0], gv[1]), pack_f16x2(uv[0], uv[1])),
                      silu_mul2(pack_f16x2(gv[2], gv[3]), pack_f16x2(uv[2], uv[3]))};
        }
    }
    }
    const int na = g.N >> 1;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int rl = k * 16 + (lane >> 2), ch = lane & 3;
        const u32x4 v = *(const u32x4*)(tile + lds_off(rl, ch));
        const int m = m0 + wm * 64 + rl;
        const int n = ((n0 + wn * 64) >> 1) + ch * 8;
        if (m >= M || n >= na) continue;
        const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
        store_row16(g.c + crow * g.ldc + n, v, true);
    }
}

// JB = 1: the wave's 64 x 32 block of a 64-wide FP16 tile (columns n0 + 32 wn ..).
template <int KIND, int SW, class P = Pipe<KIND>, int JB = 2>
EE_DEV void epilogue32_lds(const EeGemmArgs& g, const typename P::acc_t (&acc)[2][2], const TileScalesOf<P>& sc,
                           uint8_t* tile, int m0, int n0, int M, int64_t off, int wm, int wn, int lane) {
    static_assert(JB == 2 || (P::SUB16 && SW == 0 && KIND == EE_GEMM_F16), "one-block waves: 16x16 FP16, no SwiGLU");
    if constexpr (SW) {
        epilogue32_lds_swiglu<KIND, P>(g, acc, sc, tile, m0, n0, M, off, wm, wn, lane);
        return;
    }
    if constexpr (P::SUB16) {                         // quarter q at row_of(q), col_of(q)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < JB; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int rl = i * 32 + P::row_of(q, lane), cl = j * 32 + P::col_of(q, lane);
                    float o[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if constexpr (KIND == EE_GEMM_F16) o[r] = acc[i][j][4 * q + r];
                        else o[r] = deq<KIND>(acc[i][j][4 * q + r], sc.as[i][P::rq(q)], sc.bs[j][P::cq(q)][r]);
                    }
                    *(u32x2*)(tile + lds_off(rl, cl >> 3) + ((cl >> 2) & 1) * 8) =
                        u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
                }
    } else {
    // 1. dequantise and write: lane l holds rows i*32 + (l & 31), columns j*32 + 8q + 4(l >> 5) + 0..3.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rl = i * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int cl = j * 32 + 8 * q + 4 * (lane >> 5);
                float o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (KIND == EE_GEMM_I8) {
                        float v = (float)acc[i][j][4 * q + r];
                        v = v * sc.as[i];
                        o[r] = v * sc.bs[j][q][r];
                    } else if constexpr (KIND == EE_GEMM_F8) {
                        const float v = acc[i][j][4 * q + r] * sc.as[i];
                        o[r] = v * sc.bs[j][q][r];
                    } else {
                        o[r] = acc[i][j][4 * q + r];
                    }
                }
                // row rl: 128 bytes = 8 chunks of 16; column cl is chunk cl/8, half (cl/4)&1
                *(u32x2*)(tile + lds_off(rl, cl >> 3) + ((cl >> 2) & 1) * 8) =
                    u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
            }
        }
    }
    }
    // 2. read back row-contiguous and store (each wave reads only its own region:
    //    64 rows of 4 JB chunks of 16 bytes)
#pragma unroll
    for (int k = 0; k < 4 * JB; ++k) {
        const int rl = k * (16 / JB) + (lane >> (JB + 1)), ch = lane & (4 * JB - 1);
        const u32x4 v = *(const u32x4*)(tile + lds_off(rl, ch));
        const int m = m0 + wm * 64 + rl;
        const int n = n0 + wn * (32 * JB) + ch * 8;
        if (m >= M || n >= g.N) continue;
        const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
        uint16_t* dst = g.c + crow * g.ldc + n;
        // C is written once and read by a later kernel: non-temporal stores keep
        // it from lingering dirty in L2 (measured ~0.5 us per launch at C0).
        if (n + 8 <= g.N && ((uintptr_t)dst & 15) == 0) {
            __builtin_nontemporal_store(v, (u32x4*)dst);
        } else {                                           // N % 8 == 4 tail, or C only 8-byte aligned
            __builtin_nontemporal_store(u32x2{v[0], v[1]}, (u32x2*)dst);
            if (n + 4 < g.N) __builtin_nontemporal_store(u32x2{v[2], v[3]}, (u32x2*)(dst + 4));
        }
    }
}

// Pipelined kernel, 512 threads: waves 0-3 compute (one 64 x 64 quadrant each:
// LDS fragment reads + MFMAs only), waves 4-7 load (direct-to-LDS DMA of the
// stages and their vmcnt waits).  Each SIMD runs one wave of each kind, so the
// loaders' issue and waits never stall the MFMA stream.  One s_barrier per K
// stage serves both roles: barrier kt means "stage kt has landed" for the
// compute waves and "stage kt-1 has been read" for the loaders, which then
// refill that stage's buffer with stage kt-1+NSTAGE.
#define GEMM_THREADS 512

// One 128 x 128 C tile (tile coordinates tm, tn) of the pipelined GEMM;
// smem is the workgroup's NSTAGE * LDS_STAGE bytes of LDS (1 KB aligned).
// TNW = 64: a 128 x 64 tile (tn counts 64-column tiles), FP16 without SwiGLU only:
// each compute wave owns 64 x 32, the loaders fetch 64 B rows.  The same MFMAs on
// the same K slices in the same order as the 128-wide tile, so the same bits.
template <int KIND, int SW = 0, int TNW = BN>
EE_DEV void gemm_tile(const EeGemmArgs& g, int tm, int tn, uint8_t* smem) {
    typedef Pipe<KIND> P;
    typedef typename P::acc_t acc_t;
    static_assert(TNW == BN || (TNW == 64 && KIND == EE_GEMM_F16 && SW == 0), "64-wide tiles: FP16, no SwiGLU");
    constexpr int ESZ = (KIND == EE_GEMM_F16) ? 2 : 1;
    constexpr int BG = TNW / 32;                      // B row groups of 8 per loader wave
    constexpr int JB = TNW / 64;                      // 32-column blocks per compute wave
    constexpr int LOADS = 4 + BG;                     // DMA instructions per loader wave per stage (4 A + BG B)
    constexpr int NSL = BKB / P::SB;                  // K slices per stage (4 or 2)

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = g.counts ? g.counts[g.tier] : g.M;
    const int64_t off = g.counts ? tier_offset(g.counts, g.tier) : 0;
    const int m0 = tm * BM, n0 = tn * TNW;
    if (m0 >= M) return;                              // whole workgroup, before any barrier
    if constexpr (TNW != BN) {
        if (n0 >= g.N) return;
    }
    const int nk = (int)((int64_t)g.K * ESZ / BKB);   // K * ESZ is a multiple of BKB here

    if (wave >= 4) {
        // ------------------------------------------------------------ loader waves
        // One global_load_lds_dwordx4 fills 8 LDS rows (1 KB): lane l lands at row
        // r = 8*grp + l/8, physical chunk l%8, which holds logical chunk
        // (l%8) ^ swz(r).  Loader w fills row groups 4w..4w+3 of A and of B.
        const int lw = wave - 4, lrow = lane >> 3;
        const uint8_t* pa[4];
        const uint8_t* pb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = (lw * 4 + i) * 8 + lrow;
            const int lchunk = (lane & 7) ^ swz(r);   // swz(BM + r) == swz(r): BM is a multiple of 16
            const int m = min(m0 + r, M - 1);
            const int64_t ar = g.a_idx ? (int64_t)g.a_idx[off + m] : off + m;
            pa[i] = (const uint8_t*)g.a + ar * g.lda * ESZ + lchunk * 16;
            if constexpr (BG == 4) {
                const int n = min(n0 + r, g.N - 1);
                pb[i] = (const uint8_t*)g.b + (int64_t)n * g.ldb * ESZ + lchunk * 16;
            } else if (i < BG) {                      // B row groups 2 lw, 2 lw + 1
                const int rb = (lw * BG + i) * 8 + lrow;
                const int n = min(n0 + rb, g.N - 1);
                pb[i] = (const uint8_t*)g.b + (int64_t)n * g.ldb * ESZ + ((lane & 7) ^ swz(rb)) * 16;
            }
        }
        auto issue = [&](int kt) {
            const uint32_t s = lds_addr(smem) + (uint32_t)((kt % NSTAGE) * LDS_STAGE);
            const int64_t kb = (int64_t)kt * BKB;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int grp = lw * 4 + i;
                dma16(pa[i] + kb, s + grp * 8 * BKB);
                if constexpr (BG == 4) dma16(pb[i] + kb, s + (BM + grp * 8) * BKB);
                else if (i < BG) dma16(pb[i] + kb, s + (BM + (lw * BG + i) * 8) * BKB);
            }
        };
#pragma unroll
        for (int st = 0; st < NSTAGE; ++st)
            if (st < nk) issue(st);
        for (int kt = 0; kt < nk; ++kt) {
            // This wave's loads of stage kt must be done; the stages issued after it
            // may stay in flight.  Before barrier kt those are stages kt+1 .. kt+NSTAGE-1
            // when kt == 0 (prologue) and kt+1 .. kt+NSTAGE-2 after (the refill of stage
            // kt+NSTAGE-1 was issued after barrier kt-1), capped at the last stage.
            const int last = kt == 0 ? NSTAGE - 1 : kt + NSTAGE - 2;
            const int after = min(last, nk - 1) - kt;
            if (after >= 4) WAITCNT_VM(4 * LOADS);
            else if (after == 3) WAITCNT_VM(3 * LOADS);
            else if (after == 2) WAITCNT_VM(2 * LOADS);
            else if (after == 1) WAITCNT_VM(LOADS);
            else WAITCNT_VM(0);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();             // barrier kt
            asm volatile("" ::: "memory");
            if (kt >= 1 && kt - 1 + NSTAGE < nk) issue(kt - 1 + NSTAGE);   // stage kt-1's buffer is free
        }
        return;
    }

    // ---------------------------------------------------------------- compute waves
    const int wm = wave >> 1, wn = wave & 1;
    acc_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = acc_t{};

    // Fragments alternate between f0 and f1 slice by slice (NSL is even): the
    // reads of slice s+1 are issued before the MFMAs of slice s, and the reads of
    // the next stage's slice 0 before the MFMAs of this stage's last slice.  The
    // barrier for stage kt+1 therefore sits before those last MFMAs; by then every
    // read of stage kt has completed (lgkmcnt 0), which is what the loaders need to
    // refill its buffer after that barrier.  (Reading two slices ahead measured
    // slower: LDS latency is not what bounds this loop.)
    // The last stage is peeled off the loop: were its final slice (whose reads are
    // still in flight) and the steady-state final slice one block, the waitcnt
    // pass would make the steady state wait for the next stage's reads as well.
    TileScalesOf<P> sc;
    if (!g.acc) load_scales<KIND>(g, m0, n0, M, off, wm, wn, lane, sc);
    Frags<KIND> f0, f1;
    auto stage = [&](int kt, bool more) {
        const uint8_t* s = smem + (kt % NSTAGE) * LDS_STAGE;
#pragma unroll
        for (int sl = 0; sl < NSL; ++sl) {
            Frags<KIND>& cur = (sl & 1) ? f1 : f0;
            Frags<KIND>& nxt = (sl & 1) ? f0 : f1;
            if (sl + 1 < NSL) {
                read_frags<KIND, JB>(s, sl + 1, wm, wn, lane, nxt);
            } else if (more) {
                // keep the previous slice's MFMAs ahead of this wait: they cover its latency
                __builtin_amdgcn_sched_barrier(0);
                WAITCNT_LGKM0();
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();         // barrier kt+1: stage kt+1 has landed
                asm volatile("" ::: "memory");
                read_frags<KIND, JB>(smem + ((kt + 1) % NSTAGE) * LDS_STAGE, 0, wm, wn, lane, nxt);
            }
            mma_all<KIND, JB>(cur, acc);
            interleave<KIND, JB>();
        }
    };
    __builtin_amdgcn_s_barrier();                     // barrier 0: stage 0 has landed
    asm volatile("" ::: "memory");
    read_frags<KIND, JB>(smem, 0, wm, wn, lane, f0);
    for (int kt = 0; kt + 1 < nk; ++kt) stage(kt, true);
    stage(nk - 1, false);
    // Buffer nk % NSTAGE is free: no DMA is in flight after the last barrier
    // (the loaders waited for all of theirs before it), and its last stage,
    // nk - NSTAGE, was read before barrier nk - NSTAGE + 1.
    if constexpr (TNW != BN) {                        // FP16: no int32 accumulator output
        uint8_t* tile = smem + (nk % NSTAGE) * LDS_STAGE + wave * (64 * BKB);
        epilogue32_lds<KIND, SW, P, JB>(g, acc, sc, tile, m0, n0, M, off, wm, wn, lane);
    } else if (g.acc) {
        epilogue32<KIND>(g, acc, m0, n0, M, off, wm, wn, lane);
    } else {
        uint8_t* tile = smem + (nk % NSTAGE) * LDS_STAGE + wave * (64 * BKB);
        epilogue32_lds<KIND, SW>(g, acc, sc, tile, m0, n0, M, off, wm, wn, lane);
    }
}

// ---------------------------------------------------------------- W8A16 on int8 weights
// The reference's FP16 tier (EE/python/kernels.py:192-246) keeps int8 weights
// and dequantises them in SRAM: w = fp16(fp16(b) * fp16(b_scale[n])) (:215,
// :233), then an fp16 dot with f32 accumulation.  This kernel does the same
// from int8 codes in HBM, so B costs 1 byte per element instead of the 2 of
// pre-dequantised fp16 weights.  Loader-wave pipeline as gemm_tile, with:
//  * stages of 64 K elements: A fp16 128 rows x 128 B (the usual swizzle) and
//    B int8 128 rows x 64 B, 16-byte chunk c of row r stored at chunk
//    c ^ ((r >> 2) & 3) -- conflict-free ds_read_b128 over 16 rows;
//  * K order: in each 32-element block, lanes 0-31 take elements 0-7 (first
//    MFMA) and 8-15 (second), lanes 32-63 take 16-23 and 24-31, so one 16-byte
//    B read per lane feeds two MFMAs; A uses the same mapping (each MFMA sums a
//    consistent set of products);
//  * dequantisation in registers: byte b -> fp16 bits 0x6400 | (b ^ 0x80) is
//    1024 + (b + 128) exactly, minus 1152 gives fp16(b); times fp16(scale) in
//    one RNE fp16 multiply, the reference's w exactly.
#define W8_KE 64                                  // K elements per stage
#define W8_STAGE (BM * 128 + BN * 64)             // 24 KB
#define W8_NSTAGE 5
#define W8_EPI (W8_NSTAGE * W8_STAGE)             // 120 KB: the epilogue tiles, 4 x 8 KB
#define W8_LDS (W8_EPI + 4 * 64 * BKB)            // 152 KB

EE_DEV uint32_t w8_boff(int r, int c) { return (uint32_t)(BM * 128 + r * 64 + ((c ^ swz64(r)) << 4)); }

template <int SW>
EE_DEV void gemm_tile_w8a16(const EeGemmArgs& g, int tm, int tn, uint8_t* smem) {
    typedef f32x16 acc_t;
    constexpr int LOADS = 6;                          // per loader wave per stage: 4 A + 2 B
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = g.counts ? g.counts[g.tier] : g.M;
    const int64_t off = g.counts ? tier_offset(g.counts, g.tier) : 0;
    const int m0 = tm * BM, n0 = tn * BN;
    if (m0 >= M) return;                              // whole workgroup, before any barrier
    const int nk = g.K / W8_KE;                       // K is a multiple of 64 here

    if (wave >= 4) {
        const int lw = wave - 4;
        const uint8_t* pa[4];
        const uint8_t* pb[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {                 // A: row groups of 8 rows x 128 B
            const int r = (lw * 4 + i) * 8 + (lane >> 3);
            const int lchunk = (lane & 7) ^ swz(r);
            const int m = min(m0 + r, M - 1);
            const int64_t ar = g.a_idx ? (int64_t)g.a_idx[off + m] : off + m;
            pa[i] = (const uint8_t*)g.a + ar * g.lda * 2 + lchunk * 16;
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {                 // B: row groups of 16 rows x 64 B
            const int r = (lw * 2 + q) * 16 + (lane >> 2);
            const int lchunk = (lane & 3) ^ ((r >> 2) & 3);
            const int n = min(n0 + r, g.N - 1);
            pb[q] = (const uint8_t*)g.b + (int64_t)n * g.ldb + lchunk * 16;
        }
        auto issue = [&](int kt) {
            const uint32_t s = lds_addr(smem) + (uint32_t)((kt % W8_NSTAGE) * W8_STAGE);
#pragma unroll
            for (int i = 0; i < 4; ++i) dma16(pa[i] + (int64_t)kt * 128, s + (lw * 4 + i) * 8 * 128);
#pragma unroll
            for (int q = 0; q < 2; ++q) dma16(pb[q] + (int64_t)kt * 64, s + BM * 128 + (lw * 2 + q) * 16 * 64);
        };
#pragma unroll
        for (int st = 0; st < W8_NSTAGE; ++st)
            if (st < nk) issue(st);
        for (int kt = 0; kt < nk; ++kt) {
            const int last = kt == 0 ? W8_NSTAGE - 1 : kt + W8_NSTAGE - 2;
            const int after = min(last, nk - 1) - kt;
            if (after >= 4) WAITCNT_VM(4 * LOADS);
            else if (after == 3) WAITCNT_VM(3 * LOADS);
            else if (after == 2) WAITCNT_VM(2 * LOADS);
            else if (after == 1) WAITCNT_VM(LOADS);
            else WAITCNT_VM(0);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();             // barrier kt
            asm volatile("" ::: "memory");
            if (kt >= 1 && kt - 1 + W8_NSTAGE < nk) issue(kt - 1 + W8_NSTAGE);
        }
        return;
    }

    // ---------------------------------------------------------------- compute waves
    const int wm = wave >> 1, wn = wave & 1, h = lane >> 5;
    acc_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = acc_t{};
    f16x2 s2[2];                                      // fp16(b_scale[n]) of this lane's B row in block j
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        const f16 sv = (f16)f32_rn(n < g.N ? g.b_scale[n] : 0.0f);
        s2[j] = f16x2{sv, sv};
    }
    // fragments of one 32-element K block t of a stage: A rows (i), B rows (j)
    struct Fr { u32x4 a[2][2]; u32x4 b[2]; };        // a[i][u]: u = first / second MFMA
    auto read = [&](const uint8_t* s, int t, Fr& f) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ra = wm * 64 + i * 32 + (lane & 31);
#pragma unroll
            for (int u = 0; u < 2; ++u) f.a[i][u] = *(const u32x4*)(s + lds_off(ra, 4 * t + 2 * h + u));
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) f.b[j] = *(const u32x4*)(s + w8_boff(wn * 64 + j * 32 + (lane & 31), 2 * t + h));
    };
    auto mma = [&](const Fr& f) {
        u32x4 w[2][2];                                // w[j][u]: 8 fp16 weights for MFMA u
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint32_t d[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) dq4(f.b[j][q], s2[j], d[2 * q], d[2 * q + 1]);
            w[j][0] = u32x4{d[0], d[1], d[2], d[3]};
            w[j][1] = u32x4{d[4], d[5], d[6], d[7]};
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, w[j][u]),
                                                                       __builtin_bit_cast(f16x8, f.a[i][u]),
                                                                       acc[i][j], 0, 0, 0);
    };
    TileScales sc;                                    // unused by the fp16 epilogue
    Fr f0, f1;
    auto stage = [&](int kt, bool more) {
        const uint8_t* s = smem + (kt % W8_NSTAGE) * W8_STAGE;
        read(s, 1, f1);                               // block 1 of this stage
        mma(f0);
        if (more) {
            __builtin_amdgcn_sched_barrier(0);
            WAITCNT_LGKM0();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();             // barrier kt+1: stage kt+1 has landed
            asm volatile("" ::: "memory");
            read(smem + ((kt + 1) % W8_NSTAGE) * W8_STAGE, 0, f0);
        }
        mma(f1);
    };
    __builtin_amdgcn_s_barrier();                     // barrier 0: stage 0 has landed
    asm volatile("" ::: "memory");
    read(smem, 0, f0);
    for (int kt = 0; kt + 1 < nk; ++kt) stage(kt, true);
    stage(nk - 1, false);
    uint8_t* tile = smem + W8_EPI + wave * (64 * BKB);
    epilogue32_lds<EE_GEMM_F16, SW, PipeF16x32>(g, acc, sc, tile, m0, n0, M, off, wm, wn, lane);   // 32x32 layout
}

template <int SW>
EE_DEV void gemm_w8a16(const EeGemmArgs& g) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[W8_LDS];
    int tm, tn;
    tile_of((int)blockIdx.x, (int)gridDim.x, (g.M + BM - 1) / BM, tm, tn);
    gemm_tile_w8a16<SW>(g, tm, tn, smem);
}

// A 32 x 32 accumulator block through LDS: register group q (4 values) of lane l
// at byte (q * 64 + l) * 16 of a 4 KB slot, so a ds_write_b128 / ds_read_b128
// covers 1 KB of consecutive banks.  (Elements are converted one scalar at a
// time: hipcc turns __builtin_bit_cast of a vector element into element 0.)
EE_DEV uint32_t word_of(int32_t v) { return (uint32_t)v; }
EE_DEV uint32_t word_of(float v) { return __float_as_uint(v); }
template <typename acc_t>
EE_DEV void xchg_put(uint8_t* slot, const acc_t& v, int lane) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t w[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = word_of(v[4 * q + r]);
        *(u32x4*)(slot + (q * 64 + lane) * 16) = u32x4{w[0], w[1], w[2], w[3]};
    }
}
EE_DEV void xchg_put(uint8_t* slot, const I32x4x4& v, int lane) {
#pragma unroll
    for (int q = 0; q < 4; ++q) *(u32x4*)(slot + (q * 64 + lane) * 16) = __builtin_bit_cast(u32x4, v.q[q]);
}
template <int KIND>
EE_DEV void xchg_add(const uint8_t* slot, I32x4x4& v, int lane) {
#pragma unroll
    for (int q = 0; q < 4; ++q) v.q[q] += __builtin_bit_cast(i32x4, *(const u32x4*)(slot + (q * 64 + lane) * 16));
}
EE_DEV void xchg_put(uint8_t* slot, const F32x4x4& v, int lane) {
#pragma unroll
    for (int q = 0; q < 4; ++q) *(u32x4*)(slot + (q * 64 + lane) * 16) = __builtin_bit_cast(u32x4, v.q[q]);
}
template <int KIND>
EE_DEV void xchg_add(const uint8_t* slot, F32x4x4& v, int lane) {
#pragma unroll
    for (int q = 0; q < 4; ++q) v.q[q] += __builtin_bit_cast(f32x4, *(const u32x4*)(slot + (q * 64 + lane) * 16));
}
template <int KIND, typename acc_t>
EE_DEV void xchg_add(const uint8_t* slot, acc_t& v, int lane) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const u32x4 x = *(const u32x4*)(slot + (q * 64 + lane) * 16);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t w = x[r];
            if constexpr (KIND == EE_GEMM_I8) v[4 * q + r] += (int32_t)w;
            else v[4 * q + r] += __uint_as_float(w);
        }
    }
}

// ---------------------------------------------------------------------------
// Fused 8-wave pipeline (512 threads).  Wave w = (kq, wm, wn) = (w >> 2,
// (w >> 1) & 1, w & 1) accumulates the 64 x 64 quadrant (wm, wn) over its half
// of every stage's K slices, HPS = NSL / 2 slices starting at kq * HPS, and
// issues one eighth of every stage's DMA (row groups 2w, 2w+1 of A and B: 4
// instructions) in the shadow of its own MFMAs.  On gfx950 that is what lets
// the operand stream overlap the MFMAs: a wave that issues only MFMAs holds
// back the memory traffic of the other wave on its SIMD (separate loader waves
// measured DMA time + MFMA time), and eight waves rather than four keep the
// LDS fragment reads at full rate.  At the end the two K halves of each
// quadrant are summed through LDS (exact for int32; one fixed order for f32):
// wave kq keeps row block kq of the quadrant and gets its partner's partial
// of it, then dequantises and stores that 32 x 64 block.
//
// Schedule: barrier kt+1 sits before the MFMAs of the wave's last slice of
// stage kt; the refill of stage kt+4 (into stage kt-1's buffer, free after
// barrier kt) is spread over the HPS slices that follow barrier kt.
#define GEMM8_THREADS 512

// Per-lane scales of one 32-row block (row block rb) of quadrant (wm, wn).
template <int KIND>
EE_DEV void load_scales_blk(const EeGemmArgs& g, int m0, int n0, int M, int64_t off, int wm, int wn, int rb, int lane,
                            TileScales& sc) {
    if constexpr (KIND != EE_GEMM_F16) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wn * 64 + j * 32 + 8 * q + 4 * (lane >> 5);
                sc.bs[j][q] = (n < g.N) ? *(const f32x4*)(g.b_scale + n) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        const int m = m0 + wm * 64 + rb * 32 + (lane & 31);
        sc.as[0] = (m < M) ? g.a_scale[off + m] : 0.0f;
        sc.as[1] = 0.0f;
    }
}

// SwiGLU form of epilogue_blk_lds: the 32 x 64 block's gate (j = 0) and up
// (j = 1) halves become a 32 x 32 act block at act columns (n0 + 64 wn) / 2 ...
template <int KIND>
EE_DEV void epilogue_blk_lds_swiglu(const EeGemmArgs& g, const typename Pipe<KIND>::acc_t (&acc)[2],
                                    const TileScales& sc, uint8_t* tile, int m0, int n0, int M, int64_t off, int wm,
                                    int wn, int rb, int lane) {
    const int rl0 = lane & 31;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float gv[4], uv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            gv[r] = deq<KIND>(acc[0][4 * q + r], sc.as[0], sc.bs[0][q][r]);
            uv[r] = deq<KIND>(acc[1][4 * q + r], sc.as[0], sc.bs[1][q][r]);
        }
        *(u32x2*)(tile + lds_off(rl0, q) + (lane >> 5) * 8) =
            u32x2{silu_mul2(pack_f16x2(gv[0], gv[1]), pack_f16x2(uv[0], uv[1])),
                  silu_mul2(pack_f16x2(gv[2], gv[3]), pack_f16x2(uv[2], uv[3]))};
    }
    const int na = g.N >> 1;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int rl = k * 16 + (lane >> 2), ch = lane & 3;
        const u32x4 v = *(const u32x4*)(tile + lds_off(rl, ch));
        const int m = m0 + wm * 64 + rb * 32 + rl;
        const int n = ((n0 + wn * 64) >> 1) + ch * 8;
        if (m >= M || n >= na) continue;
        const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
        store_row16(g.c + crow * g.ldc + n, v, true);
    }
}

// Epilogue of one 32 x 64 block (row block rb of quadrant (wm, wn)) held as
// acc[0..1] (column blocks), through a 4 KB LDS tile: dequantise, write in the
// MFMA layout, read back as rows and store 16 bytes per lane, non-temporal.
template <int KIND, int SW>
EE_DEV void epilogue_blk_lds(const EeGemmArgs& g, const typename Pipe<KIND>::acc_t (&acc)[2], const TileScales& sc,
                             uint8_t* tile, int m0, int n0, int M, int64_t off, int wm, int wn, int rb, int lane) {
    if constexpr (SW) {
        epilogue_blk_lds_swiglu<KIND>(g, acc, sc, tile, m0, n0, M, off, wm, wn, rb, lane);
        return;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int cl = j * 32 + 8 * q + 4 * (lane >> 5);
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (KIND == EE_GEMM_I8) {
                    float v = (float)acc[j][4 * q + r];
                    v = v * sc.as[0];
                    o[r] = v * sc.bs[j][q][r];
                } else if constexpr (KIND == EE_GEMM_F8) {
                    const float v = acc[j][4 * q + r] * sc.as[0];
                    o[r] = v * sc.bs[j][q][r];
                } else {
                    o[r] = acc[j][4 * q + r];
                }
            }
            *(u32x2*)(tile + lds_off(lane & 31, cl >> 3) + ((cl >> 2) & 1) * 8) =
                u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int rl = k * 8 + (lane >> 3), ch = lane & 7;
        const u32x4 v = *(const u32x4*)(tile + lds_off(rl, ch));
        const int m = m0 + wm * 64 + rb * 32 + rl;
        const int n = n0 + wn * 64 + ch * 8;
        if (m >= M || n >= g.N) continue;
        const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
        uint16_t* dst = g.c + crow * g.ldc + n;
        // C is written once and read by a later kernel: non-temporal stores keep
        // it from lingering dirty in L2.
        if (n + 8 <= g.N && ((uintptr_t)dst & 15) == 0) {
            __builtin_nontemporal_store(v, (u32x4*)dst);
        } else {                                           // N % 8 == 4 tail, or C only 8-byte aligned
            __builtin_nontemporal_store(u32x2{v[0], v[1]}, (u32x2*)dst);
            if (n + 4 < g.N) __builtin_nontemporal_store(u32x2{v[2], v[3]}, (u32x2*)(dst + 4));
        }
    }
}

// Debug epilogue (int32 accumulators requested): direct stores of the block.
template <int KIND>
EE_DEV void epilogue_blk_direct(const EeGemmArgs& g, const typename Pipe<KIND>::acc_t (&acc)[2], int m0, int n0, int M,
                                int64_t off, int wm, int wn, int rb, int lane) {
    const int m = m0 + wm * 64 + rb * 32 + (lane & 31);
    if (m >= M) return;
    const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
    const float as = (KIND == EE_GEMM_F16) ? 0.0f : g.a_scale[off + m];
    uint16_t* cr = g.c + crow * g.ldc;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = n0 + wn * 64 + j * 32 + 8 * q + 4 * (lane >> 5);
            if (n >= g.N) continue;                 // N is a multiple of 4
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (KIND == EE_GEMM_I8) {
                    float v = (float)acc[j][4 * q + r];
                    v = v * as;
                    o[r] = v * g.b_scale[n + r];
                } else if constexpr (KIND == EE_GEMM_F8) {
                    const float v = acc[j][4 * q + r] * as;
                    o[r] = v * g.b_scale[n + r];
                } else {
                    o[r] = acc[j][4 * q + r];
                }
            }
            *(u32x2*)(cr + n) = u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
            if constexpr (KIND == EE_GEMM_I8) {
                if (g.acc)
                    *(i32x4*)(g.acc + crow * g.ldc + n) =
                        i32x4{acc[j][4 * q], acc[j][4 * q + 1], acc[j][4 * q + 2], acc[j][4 * q + 3]};
            }
        }
}

// The 16x16x64 accumulator layout (PipeI8x16): register 4q + r of column block
// j of row block rb holds row rb*32 + row_of(q, l), column j*32 + col_of(q, l) + r
// of the quadrant; a lane needs two row scales and two column-scale vectors per j.
struct TileScales16 {
    f32x4 bs[2][2];
    float as[2];
};
template <int KIND, class P>
EE_DEV void load_scales_blk16(const EeGemmArgs& g, int m0, int n0, int M, int64_t off, int wm, int wn, int rb,
                              int lane, TileScales16& sc) {
    if constexpr (KIND != EE_GEMM_F16) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int n = n0 + wn * 64 + j * 32 + P::col_of(2 * c, lane);
                sc.bs[j][c] = (n < g.N) ? *(const f32x4*)(g.b_scale + n) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int m = m0 + wm * 64 + rb * 32 + P::row_of(h, lane);
            sc.as[h] = (m < M) ? g.a_scale[off + m] : 0.0f;
        }
    }
}
// epilogue_blk_lds (and its SwiGLU form) for that layout.
template <int KIND, int SW, class P>
EE_DEV void epilogue_blk_lds16(const EeGemmArgs& g, const typename P::acc_t (&acc)[2], const TileScales16& sc,
                               uint8_t* tile, int m0, int n0, int M, int64_t off, int wm, int wn, int rb, int lane) {
    // (the lane through an empty asm: addresses derived from it are computed here,
    // not merged with the K loop's and held across it)
    asm volatile("" : "+v"(lane));
    if constexpr (SW) {                               // gate (j = 0) and up (j = 1) -> act columns (n0 + 64 wn) / 2 ..
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float gv[4], uv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                gv[r] = deq<KIND>(acc[0][4 * q + r], sc.as[P::rq(q)], sc.bs[0][P::cq(q)][r]);
                uv[r] = deq<KIND>(acc[1][4 * q + r], sc.as[P::rq(q)], sc.bs[1][P::cq(q)][r]);
            }
            const int ca = P::col_of(q, lane);
            *(u32x2*)(tile + lds_off(P::row_of(q, lane), ca >> 3) + ((ca >> 2) & 1) * 8) =
                u32x2{silu_mul2(pack_f16x2(gv[0], gv[1]), pack_f16x2(uv[0], uv[1])),
                      silu_mul2(pack_f16x2(gv[2], gv[3]), pack_f16x2(uv[2], uv[3]))};
        }
        const int na = g.N >> 1;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int rl = k * 16 + (lane >> 2), ch = lane & 3;
            const u32x4 v = *(const u32x4*)(tile + lds_off(rl, ch));
            const int m = m0 + wm * 64 + rb * 32 + rl;
            const int n = ((n0 + wn * 64) >> 1) + ch * 8;
            if (m >= M || n >= na) continue;
            const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
            store_row16(g.c + crow * g.ldc + n, v, true);
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int cl = j * 32 + P::col_of(q, lane);
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = deq<KIND>(acc[j][4 * q + r], sc.as[P::rq(q)], sc.bs[j][P::cq(q)][r]);
            *(u32x2*)(tile + lds_off(P::row_of(q, lane), cl >> 3) + ((cl >> 2) & 1) * 8) =
                u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int rl = k * 8 + (lane >> 3), ch = lane & 7;
        const u32x4 v = *(const u32x4*)(tile + lds_off(rl, ch));
        const int m = m0 + wm * 64 + rb * 32 + rl;
        const int n = n0 + wn * 64 + ch * 8;
        if (m >= M || n >= g.N) continue;
        const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
        store_row16(g.c + crow * g.ldc + n, v, n + 8 <= g.N);
    }
}
// epilogue_blk_direct (int32 accumulators requested, INT8) for that layout.
template <int KIND, class P>
EE_DEV void epilogue_blk_direct16(const EeGemmArgs& g, const typename P::acc_t (&acc)[2], int m0, int n0, int M,
                                  int64_t off, int wm, int wn, int rb, int lane) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = m0 + wm * 64 + rb * 32 + P::row_of(q, lane);
            const int n = n0 + wn * 64 + j * 32 + P::col_of(q, lane);
            if (m >= M || n >= g.N) continue;
            const int64_t crow = g.c_idx ? (int64_t)g.c_idx[off + m] : (int64_t)m;
            const float as = (KIND == EE_GEMM_F16) ? 0.0f : g.a_scale[off + m];
            float o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = deq<KIND>(acc[j][4 * q + r], as, KIND == EE_GEMM_F16 ? 0.0f : g.b_scale[n + r]);
            *(u32x2*)(g.c + crow * g.ldc + n) = u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
            if constexpr (KIND == EE_GEMM_I8) {
                if (g.acc) *(i32x4*)(g.acc + crow * g.ldc + n) = acc[j].q[q];
            }
        }
}

template <int KIND, int SW = 0>
struct Gemm8 {
    // INT8: 16x16x64 MFMAs on 64-byte slices (PipeI8x16)
    typedef std::conditional_t<KIND == EE_GEMM_I8, PipeI8x16, Pipe<KIND>> P;
    typedef typename P::acc_t acc_t;
    static constexpr int ESZ = (KIND == EE_GEMM_F16) ? 2 : 1;
    static constexpr int LOADS = 4;                    // DMA instructions per wave per stage
    static constexpr int NSL = BKB / P::SB;            // K slices per stage (4 or 2)
    static constexpr int HPS = NSL / 2;                // slices per wave per stage
    static constexpr int PPS = 2 / HPS;                // DMA parts (2 instructions) per slice

    const EeGemmArgs& g;
    uint8_t* smem;
    uint32_t lds0;
    int lane, wave, kq, wm, wn, nk;
    const uint8_t* pa[2];
    const uint8_t* pb[2];
    acc_t acc[2][2];
    FragsP<P> fr[2];
    uint32_t fo16;                                     // SUB16: byte of row l & 15, chunk (l >> 4) of slice 0

    __device__ __forceinline__ Gemm8(const EeGemmArgs& g_, uint8_t* smem_) : g(g_), smem(smem_) {}

    __device__ __forceinline__ void issue_part(int kt, int part) {
        const uint32_t s = lds0 + (uint32_t)((kt % NSTAGE) * LDS_STAGE);
        const int64_t kb = (int64_t)kt * BKB;
        const int grp = wave * 2 + part;
        dma16(pa[part] + kb, s + grp * 8 * BKB);
        dma16(pb[part] + kb, s + (BM + grp * 8) * BKB);
    }
    // This wave's loads of stage kt done; the stages issued after it may stay in
    // flight: before barrier kt those are kt+1 .. kt+NSTAGE-1 (kt == 0) or
    // kt+1 .. kt+NSTAGE-2, capped at the last stage.
    __device__ __forceinline__ void wait_stage(int kt) const {
        const int last = kt == 0 ? NSTAGE - 1 : kt + NSTAGE - 2;
        const int after = min(last, nk - 1) - kt;
        if (after >= 4) WAITCNT_VM(4 * LOADS);
        else if (after == 3) WAITCNT_VM(3 * LOADS);
        else if (after == 2) WAITCNT_VM(2 * LOADS);
        else if (after == 1) WAITCNT_VM(LOADS);
        else WAITCNT_VM(0);
    }

    // One stage kt.  PAR: parity of the fragment buffer of the wave's first slice.
    // RPRE: the slices before barrier kt+1 refill stage kt+4 (buffer of stage
    // kt-1, free since barrier kt); RPOST: the slice after barrier kt+1 refills
    // stage kt+5; WAITN: stages issued after stage kt+1 that may stay in flight at
    // barrier kt+1 (vmcnt = WAITN * LOADS); MORE: a stage kt+1 exists.  The
    // runtime form (GENERIC) decides all of these from kt and nk.
    template <int PAR, bool GENERIC, bool RPRE, bool RPOST, int WAITN, bool MORE>
    __device__ __forceinline__ void stage(int kt) {
        const uint8_t* s = smem + (kt % NSTAGE) * LDS_STAGE;
        const bool more = GENERIC ? (kt + 1 < nk) : MORE;
#pragma unroll
        for (int h = 0; h < HPS; ++h) {
            FragsP<P>& cur = fr[(PAR + h) & 1];
            FragsP<P>& nxt = fr[(PAR + h + 1) & 1];
            int dkt = -1, dp0 = 0;
            bool rd = false;
            const uint8_t* rs = s;
            int rsl = kq * HPS + h + 1;
            if (h + 1 < HPS) {
                rd = true;
                if (GENERIC ? (kt >= 1 && kt + NSTAGE - 1 < nk) : RPRE) { dkt = kt + NSTAGE - 1; dp0 = (h + 1) * PPS; }
            } else if (more) {
                __builtin_amdgcn_sched_barrier(0);
                if (GENERIC) wait_stage(kt + 1);
                else WAITCNT_VM(WAITN * LOADS);
                WAITCNT_LGKM0();
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();         // barrier kt+1: stage kt+1 landed, stage kt read
                asm volatile("" ::: "memory");
                rd = true;
                rs = smem + ((kt + 1) % NSTAGE) * LDS_STAGE;
                rsl = kq * HPS;
                if (GENERIC ? (kt + NSTAGE < nk) : RPOST) { dkt = kt + NSTAGE; dp0 = 0; }
            }
            // MFMA (0,0) | reads A0 B0 B1 | MFMA (0,1) | DMA | MFMA (1,0) | read A1 | MFMA (1,1):
            // every fragment of the next slice lands two or more MFMAs before its use.
            acc[0][0] = P::mma(cur.b[0], cur.a[0], acc[0][0]);
            __builtin_amdgcn_sched_barrier(0);
            if (rd) { read_frag(rs, rsl, nxt.a[0], 0); read_frag(rs, rsl, nxt.b[0], 2); read_frag(rs, rsl, nxt.b[1], 3); }
            __builtin_amdgcn_sched_barrier(0);
            acc[0][1] = P::mma(cur.b[1], cur.a[0], acc[0][1]);
            __builtin_amdgcn_sched_barrier(0);
            if (dkt >= 0)
#pragma unroll
                for (int p = 0; p < PPS; ++p) issue_part(dkt, dp0 + p);
            __builtin_amdgcn_sched_barrier(0);
            acc[1][0] = P::mma(cur.b[0], cur.a[1], acc[1][0]);
            __builtin_amdgcn_sched_barrier(0);
            if (rd) read_frag(rs, rsl, nxt.a[1], 1);
            __builtin_amdgcn_sched_barrier(0);
            acc[1][1] = P::mma(cur.b[1], cur.a[1], acc[1][1]);
        }
    }
    // One fragment of one K slice: which = 0, 1 (A row block), 2, 3 (B row block).
    __device__ __forceinline__ void read_frag(const uint8_t* s, int slice, typename P::frag_t& f, int which) const {
        if constexpr (P::SUB16) {                     // rows base + (l & 15), +16; chunk 4 slice + (l >> 4)
            // (base % 16 == 0: swz(base + x) == swz(x); the lane's offset for the slice goes
            // through an empty asm, so that each read adds it to the block's base rather
            // than the compiler holding a hoisted address per block and buffer)
            const int base = which < 2 ? wm * 64 + which * 32 : BM + wn * 64 + (which - 2) * 32;
            uint32_t o = fo16 ^ (uint32_t)((slice & 1) << 6);  // chunk 4 + c ^ s == (c ^ s) ^ 4 for c < 4
            asm volatile("" : "+v"(o));
            const uint8_t* p = s + base * BKB + o;
            f.h[0] = *(const i32x4*)p;
            f.h[1] = *(const i32x4*)(p + 16 * BKB);
        } else {
            const int r = lane & 31;
            const int c0 = slice * (P::SB / 16) + (lane >> 5) * P::LSTEP;
            const int row = which < 2 ? wm * 64 + which * 32 + r : BM + wn * 64 + (which - 2) * 32 + r;
            if constexpr (P::CPF == 1) {
                f = *(const u32x4*)(s + lds_off(row, c0));
            } else {
                const u32x4 x0 = *(const u32x4*)(s + lds_off(row, c0)),
                            x1 = *(const u32x4*)(s + lds_off(row, c0 + P::CSTEP));
                f = i32x8{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
            }
        }
    }
    // The last five stages (kt0 = nk - 5 .. nk - 1, nk >= 6), first one of parity P0.
    template <int P0>
    __device__ __forceinline__ void tail(int kt0) {
        constexpr int D = HPS & 1;                     // parity step per stage
        stage<P0, false, true, false, 3, true>(kt0);
        stage<(P0 + D) & 1, false, false, false, 2, true>(kt0 + 1);
        stage<(P0 + 2 * D) & 1, false, false, false, 1, true>(kt0 + 2);
        stage<(P0 + 3 * D) & 1, false, false, false, 0, true>(kt0 + 3);
        stage<(P0 + 4 * D) & 1, false, false, false, 0, false>(kt0 + 4);
    }
    __device__ __forceinline__ void run(int tm, int tn) {
        const int tid = threadIdx.x;
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        kq = wave >> 2;
        wm = (wave >> 1) & 1;
        wn = wave & 1;
        if constexpr (P::SUB16) fo16 = lds_off(lane & 15, lane >> 4);
        const int M = g.counts ? g.counts[g.tier] : g.M;
        const int64_t off = g.counts ? tier_offset(g.counts, g.tier) : 0;
        const int m0 = tm * BM, n0 = tn * BN;
        if (m0 >= M) return;                          // whole workgroup, before any barrier
        nk = (int)((int64_t)g.K * ESZ / BKB);         // K * ESZ is a multiple of BKB here

        // Scales of the wave's final block first: they are the oldest loads the
        // first stage wait covers.
        std::conditional_t<P::SUB16, TileScales16, TileScales> sc;
        if (!g.acc) {
            if constexpr (P::SUB16) load_scales_blk16<KIND, P>(g, m0, n0, M, off, wm, wn, kq, lane, sc);
            else load_scales_blk<KIND>(g, m0, n0, M, off, wm, wn, kq, lane, sc);
        }
        // DMA: one global_load_lds_dwordx4 fills 8 LDS rows (1 KB): lane l lands at
        // row r = 8*grp + l/8, physical chunk l%8, which holds logical chunk
        // (l%8) ^ swz(r).  Wave w fills row groups 2w, 2w+1 of A and of B.
        const int lrow = lane >> 3;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = (wave * 2 + i) * 8 + lrow;
            const int lchunk = (lane & 7) ^ swz(r);   // swz(BM + r) == swz(r): BM is a multiple of 16
            const int m = min(m0 + r, M - 1);
            const int64_t ar = g.a_idx ? (int64_t)g.a_idx[off + m] : off + m;
            pa[i] = (const uint8_t*)g.a + ar * g.lda * ESZ + lchunk * 16;
            const int n = min(n0 + r, g.N - 1);
            pb[i] = (const uint8_t*)g.b + (int64_t)n * g.ldb * ESZ + lchunk * 16;
        }
        lds0 = lds_addr(smem);
#pragma unroll
        for (int st = 0; st < NSTAGE; ++st)
            if (st < nk) { issue_part(st, 0); issue_part(st, 1); }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = acc_t{};

        wait_stage(0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();                 // barrier 0: stage 0 has landed
        asm volatile("" ::: "memory");
        read_frag(smem, kq * HPS, fr[0].a[0], 0);
        read_frag(smem, kq * HPS, fr[0].b[0], 2);
        read_frag(smem, kq * HPS, fr[0].b[1], 3);
        read_frag(smem, kq * HPS, fr[0].a[1], 1);
        constexpr int D = HPS & 1;
        if (nk >= 6) {
            // stage 0 (stage 4 came with the prologue), steady state, tail
            stage<0, false, false, true, 3, true>(0);
            int kt = 1;
            if constexpr (D == 0) {
                for (; kt <= nk - 6; ++kt) stage<0, false, true, true, 3, true>(kt);
                tail<0>(kt);
            } else {
                for (; kt + 1 <= nk - 6; kt += 2) {
                    stage<1, false, true, true, 3, true>(kt);
                    stage<0, false, true, true, 3, true>(kt + 1);
                }
                if (kt <= nk - 6) { stage<1, false, true, true, 3, true>(kt); ++kt; }
                if (kt & 1) tail<1>(kt);
                else tail<0>(kt);
            }
        } else if constexpr (D == 0) {
            for (int kt = 0; kt < nk; ++kt) stage<0, true, false, false, 0, false>(kt);
        } else {
            int kt = 0;
            for (; kt + 1 < nk; kt += 2) {
                stage<0, true, false, false, 0, false>(kt);
                stage<1, true, false, false, 0, false>(kt + 1);
            }
            if (kt < nk) stage<0, true, false, false, 0, false>(kt);
        }

        // Pair exchange.  After the last barrier every buffer but stage nk-1's is
        // free (all DMA landed before it; stage nk-1-i was read before barrier
        // nk-i), i.e. buffers (nk + i) % NSTAGE, i = 0..3.  Wave w's 8 KB receive
        // slot is quarter (w & 3) of buffer (nk + 1 + (w >> 2)) % NSTAGE; its
        // 4 KB epilogue tile is in buffer nk % NSTAGE.
        acc_t blk[2];
        {
            const int partner = wave ^ 4;
            uint8_t* dst = smem + ((nk + 1 + (partner >> 2)) % NSTAGE) * LDS_STAGE + (partner & 3) * 8192;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                xchg_put(dst + j * 4096, kq ? acc[0][j] : acc[1][j], lane);
                blk[j] = kq ? acc[1][j] : acc[0][j];
            }
            WAITCNT_LGKM0();                          // this wave's LDS writes are done
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();             // every partner's half has landed
            asm volatile("" ::: "memory");
            const uint8_t* src = smem + ((nk + 1 + (wave >> 2)) % NSTAGE) * LDS_STAGE + (wave & 3) * 8192;
#pragma unroll
            for (int j = 0; j < 2; ++j) xchg_add<KIND>(src + j * 4096, blk[j], lane);
        }
        if (g.acc) {
            if constexpr (P::SUB16) epilogue_blk_direct16<KIND, P>(g, blk, m0, n0, M, off, wm, wn, kq, lane);
            else epilogue_blk_direct<KIND>(g, blk, m0, n0, M, off, wm, wn, kq, lane);
        } else {
            uint8_t* tile = smem + (nk % NSTAGE) * LDS_STAGE + wave * 4096;
            if constexpr (P::SUB16) epilogue_blk_lds16<KIND, SW, P>(g, blk, sc, tile, m0, n0, M, off, wm, wn, kq, lane);
            else epilogue_blk_lds<KIND, SW>(g, blk, sc, tile, m0, n0, M, off, wm, wn, kq, lane);
        }
    }
};

template <int KIND, int SW = 0>
EE_DEV void gemm_pipelined_8w(const EeGemmArgs& g) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTAGE * LDS_STAGE];
    int tm, tn;
    tile_of((int)blockIdx.x, (int)gridDim.x, (g.M + BM - 1) / BM, tm, tn);
    Gemm8<KIND, SW> k(g, smem);
    k.run(tm, tn);
}

template <int KIND, int SW = 0>
EE_DEV void gemm_pipelined(const EeGemmArgs& g) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTAGE * LDS_STAGE];
    int tm, tn;
    tile_of((int)blockIdx.x, (int)gridDim.x, (g.M + BM - 1) / BM, tm, tn);
    gemm_tile<KIND, SW>(g, tm, tn, smem);
}

template <int KIND>
EE_DEV void gemm_generic(const EeGemmArgs& g) {
    typedef typename AccT<KIND>::type acc_t;
    constexpr int ESZ = (KIND == EE_GEMM_F16) ? 2 : 1;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * LDS_STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int M = g.counts ? g.counts[g.tier] : g.M;
    const int64_t off = g.counts ? tier_offset(g.counts, g.tier) : 0;
    const int tiles_m = (g.M + BM - 1) / BM;
    int tm, tn;
    tile_of((int)blockIdx.x, (int)gridDim.x, tiles_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    if (m0 >= M) return;                              // whole workgroup, before any barrier

    const int64_t Kb = (int64_t)g.K * ESZ;
    const int nk = (int)((Kb + BKB - 1) / BKB);
    const int ch = tid & 7, rr = tid >> 3;            // loader: chunk, first row

    const uint8_t* pa[4];
    const uint8_t* pb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = min(m0 + rr + 32 * i, M - 1);
        const int64_t ar = g.a_idx ? (int64_t)g.a_idx[off + m] : off + m;
        pa[i] = (const uint8_t*)g.a + ar * g.lda * ESZ + ch * 16;
        const int n = min(n0 + rr + 32 * i, g.N - 1);
        pb[i] = (const uint8_t*)g.b + (int64_t)n * g.ldb * ESZ + ch * 16;
    }

    u32x4 ra[4], rb[4];
    auto gload = [&](int kt) {
        const bool kin = (int64_t)kt * BKB + ch * 16 < Kb;   // K is a multiple of 16 bytes
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ra[i] = kin ? *(const u32x4*)(pa[i] + (int64_t)kt * BKB) : u32x4{0, 0, 0, 0};
            rb[i] = kin ? *(const u32x4*)(pb[i] + (int64_t)kt * BKB) : u32x4{0, 0, 0, 0};
        }
    };
    auto lstore = [&](int buf) {
        uint8_t* s = smem + buf * LDS_STAGE;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = rr + 32 * i;
            *(u32x4*)(s + lds_off(r, ch)) = ra[i];
            *(u32x4*)(s + lds_off(BM + r, ch)) = rb[i];
        }
    };

    acc_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = acc_t{0, 0, 0, 0};

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
        mfma_stage<KIND>(smem + buf * LDS_STAGE, acc, wm, wn, lane);
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }
    epilogue<KIND>(g, acc, m0, n0, M, off, wm, wn, lane);
}

// ---------------------------------------------------------------- persistent loader-wave GEMM
// One workgroup per CU walks a list of tiles.  The stage ring runs on across
// tile boundaries: the loader waves keep streaming the next tile's first
// stages while the compute waves finish the current tile's MFMAs and
// epilogue, so the pipeline fills once per workgroup instead of once per
// tile.  Four DMA stages (128 KB) plus a 32 KB epilogue buffer the DMA never
// touches.  Global stage s lives in buffer s % NSTAGE_P; barrier s means
// "stage s has landed" for the compute waves and "stage s-1 has been read"
// for the loaders, exactly as in gemm_tile.  The compute code and the K order
// are gemm_tile's, so outputs are bit-identical to it.  1-byte operands only
// (INT8 and FP8): every tile of one launch then has the same stage count.
#define NSTAGE_P 4
#define EPI_BUF (NSTAGE_P * LDS_STAGE)

// The work of one tile: its GEMM, tile coordinates, row count and slot offset.
struct PTile {
    const EeGemmArgs* g;
    int tier, tm, tn, M;
    int64_t off;
};


// Tiles of a plain GEMM for workgroup b of G.
struct SeqPlain {
    const EeGemmArgs* g;
    TileDeal d;
    __device__ __forceinline__ SeqPlain(const EeGemmArgs& ga, int b, int G)
        : g(&ga), d((ga.M + BM - 1) / BM, (ga.N + BN - 1) / BN, 0, b, G) {}
    __device__ __forceinline__ int count() const { return d.count(); }
    __device__ __forceinline__ PTile tile(int i) const {
        int tm, tn;
        d.coords(d.tile_index(d.first_round + i), tm, tn);
        return PTile{g, g->tier, tm, tn, g->M, 0};
    }
};

// The INT8 and FP8 tiles of a routed launch: M-tiles 0 .. T0-1 are INT8
// (slots 0 .. c0-1), T0 .. T0+T1-1 FP8 (slots c0 ..).
struct SeqRouted {
    const EeRoutedGemmArgs* r;
    int T0, c0, c1;
    TileDeal d;
    __device__ __forceinline__ SeqRouted(const EeRoutedGemmArgs& ra, int t0, int t01, int k0, int k1, int nN, int nF,
                                         int b, int G)
        : r(&ra), T0(t0), c0(k0), c1(k1), d(t01, nN, nF, b, G) {}
    __device__ __forceinline__ int count() const { return d.count(); }
    __device__ __forceinline__ PTile tile(int i) const {
        int tmg, tn;
        d.coords(d.tile_index(d.first_round + i), tmg, tn);
        return tmg < T0 ? PTile{&r->t[0], 0, tmg, tn, c0, 0} : PTile{&r->t[1], 1, tmg - T0, tn, c1, c0};
    }
};

template <class Seq>
EE_DEV void persist_loader(const Seq& seq, int ntiles, int nk, uint8_t* smem, int lw, int lane) {
    constexpr int LOADS = 8;                          // DMA instructions per loader wave per stage
    const int lrow = lane >> 3;
    const uint8_t* pa[4];
    const uint8_t* pb[4];
    const int total = ntiles * nk;
    int issued = 0, cur = -1;
    auto issue = [&]() {
        const int i = issued / nk, kt = issued - i * nk;
        if (i != cur) {                               // the issue cursor enters tile i
            cur = i;
            const PTile t = seq.tile(i);
            const int m0 = t.tm * BM, n0 = t.tn * BN;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = (lw * 4 + q) * 8 + lrow;
                const int lchunk = (lane & 7) ^ swz(r);
                const int m = min(m0 + r, t.M - 1);
                const int64_t ar = t.g->a_idx ? (int64_t)t.g->a_idx[t.off + m] : t.off + m;
                pa[q] = (const uint8_t*)t.g->a + ar * t.g->lda + lchunk * 16;
                const int n = min(n0 + r, t.g->N - 1);
                pb[q] = (const uint8_t*)t.g->b + (int64_t)n * t.g->ldb + lchunk * 16;
            }
        }
        const uint32_t s = lds_addr(smem) + (uint32_t)((issued % NSTAGE_P) * LDS_STAGE);
        const int64_t kb = (int64_t)kt * BKB;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int grp = lw * 4 + q;
            dma16(pa[q] + kb, s + grp * 8 * BKB);
            dma16(pb[q] + kb, s + (BM + grp * 8) * BKB);
        }
        ++issued;
    };
    while (issued < NSTAGE_P && issued < total) issue();
    for (int s = 0; s < total; ++s) {
        // this wave's loads of stage s are done; the (issued - 1 - s) stages issued after it may still fly
        const int after = issued - 1 - s;
        if (after >= 3) WAITCNT_VM(3 * LOADS);
        else if (after == 2) WAITCNT_VM(2 * LOADS);
        else if (after == 1) WAITCNT_VM(LOADS);
        else WAITCNT_VM(0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();                 // barrier s
        asm volatile("" ::: "memory");
        if (s >= 1 && issued < total) issue();        // stage s-1's buffer is free: it gets stage s-1+NSTAGE_P
    }
}

// Compute waves (0-3) on one tile whose first stage is global stage s0.
template <int KIND, int SW = 0>
EE_DEV void persist_compute(const PTile& t, int nk, int s0, uint8_t* smem, int wave, int lane) {
    typedef Pipe<KIND> P;
    typedef typename P::acc_t acc_t;
    constexpr int NSL = BKB / P::SB;
    const EeGemmArgs& g = *t.g;
    const int m0 = t.tm * BM, n0 = t.tn * BN;
    const int wm = wave >> 1, wn = wave & 1;
    acc_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = acc_t{};
    TileScalesOf<P> sc;
    if (!g.acc) load_scales<KIND>(g, m0, n0, t.M, t.off, wm, wn, lane, sc);
    Frags<KIND> f0, f1;
    auto stage = [&](int kt, bool more) {
        const uint8_t* s = smem + ((s0 + kt) % NSTAGE_P) * LDS_STAGE;
#pragma unroll
        for (int sl = 0; sl < NSL; ++sl) {
            Frags<KIND>& cur = (sl & 1) ? f1 : f0;
            Frags<KIND>& nxt = (sl & 1) ? f0 : f1;
            if (sl + 1 < NSL) {
                read_frags<KIND>(s, sl + 1, wm, wn, lane, nxt);
            } else if (more) {
                __builtin_amdgcn_sched_barrier(0);
                WAITCNT_LGKM0();
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();         // barrier s0+kt+1
                asm volatile("" ::: "memory");
                read_frags<KIND>(smem + ((s0 + kt + 1) % NSTAGE_P) * LDS_STAGE, 0, wm, wn, lane, nxt);
            }
            mma_all<KIND>(cur, acc);
            interleave<KIND>();
        }
    };
    WAITCNT_LGKM0();                                  // the previous tile's LDS reads are complete
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();                     // barrier s0: the tile's first stage has landed
    asm volatile("" ::: "memory");
    read_frags<KIND>(smem + (s0 % NSTAGE_P) * LDS_STAGE, 0, wm, wn, lane, f0);
    for (int kt = 0; kt + 1 < nk; ++kt) stage(kt, true);
    stage(nk - 1, false);
    if (g.acc) epilogue32<KIND>(g, acc, m0, n0, t.M, t.off, wm, wn, lane);
    else epilogue32_lds<KIND, SW>(g, acc, sc, smem + EPI_BUF + wave * (64 * BKB), m0, n0, t.M, t.off, wm, wn, lane);
}

template <int KIND, int SW = 0>
EE_DEV void gemm_persistent(const EeGemmArgs& g) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[(NSTAGE_P + 1) * LDS_STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const SeqPlain seq(g, (int)blockIdx.x, (int)gridDim.x);
    const int nt = seq.count();
    const int nk = g.K / BKB;
    if (wave >= 4) {
        persist_loader(seq, nt, nk, smem, wave - 4, lane);
        return;
    }
    for (int i = 0; i < nt; ++i) persist_compute<KIND, SW>(seq.tile(i), nk, i * nk, smem, wave, lane);
}

// Kernel entries; each GEMM also has a _swiglu twin whose epilogue writes
// fp16(fp16(silu(gate)) * up) of gate|up-interleaved weights instead of C (one
// epilogue per kernel keeps the register budget of each).
#define EE_GEMM_ENTRY(NAME, BODY)                                                                         \
    extern "C" __global__ void __launch_bounds__(GEMM_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) \
    NAME(EeGemmArgs g) { BODY<0>(g); }                                                                  \
    extern "C" __global__ void __launch_bounds__(GEMM_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) \
    NAME##_swiglu(EeGemmArgs g) { BODY<1>(g); }
template <int SW> EE_DEV void body_i8(const EeGemmArgs& g) { gemm_pipelined<EE_GEMM_I8, SW>(g); }
template <int SW> EE_DEV void body_f8(const EeGemmArgs& g) { gemm_pipelined<EE_GEMM_F8, SW>(g); }
template <int SW> EE_DEV void body_f16(const EeGemmArgs& g) { gemm_pipelined<EE_GEMM_F16, SW>(g); }
template <int SW> EE_DEV void body_i8_w8(const EeGemmArgs& g) { gemm_pipelined_8w<EE_GEMM_I8, SW>(g); }
template <int SW> EE_DEV void body_f16_w8(const EeGemmArgs& g) { gemm_pipelined_8w<EE_GEMM_F16, SW>(g); }
EE_GEMM_ENTRY(eek_gemm_i8, body_i8)
EE_GEMM_ENTRY(eek_gemm_f8, body_f8)
EE_GEMM_ENTRY(eek_gemm_f16, body_f16)
EE_GEMM_ENTRY(eek_gemm_i8_w8, body_i8_w8)
EE_GEMM_ENTRY(eek_gemm_f16_w8, body_f16_w8)
template <int SW> EE_DEV void body_w8a16(const EeGemmArgs& g) { gemm_w8a16<SW>(g); }
EE_GEMM_ENTRY(eek_gemm_w8a16, body_w8a16)

// The routed linear's three tier GEMMs in one launch.  Tier t owns partition
// slots [off_t, off_t + counts[t]) (off_t = counts[0] + ... + counts[t-1]) and
// the ceil(counts[t] / 128) M-tile indices after those of the lower tiers, so
// an M-tile never mixes tiers; workgroups past the last tile exit at once.
// The grid holds r.mt_max = ceil(M / 128) + 2 M-tile slots (the sum of the
// three ceilings is at most that) times ceil(N / 128) N-tiles.
// FP16 halves (r.f16_half_cus > 0, no SwiGLU): an FP16 tile costs two 1-byte
// tiles, so the FP16 tier takes two M-tile indices per M-tile, one per 128 x 64
// column half (mt_max then counts them: at most 2 ceil(M / 128) + 2), where the
// grid with the halves fits one round of the r.f16_half_cus CUs, or where the
// whole-tile grid takes between one and two rounds (its FP16 tiles then set a
// ragged second round).  Measured on MI355X, 20/40/40 % tiers: 1024 x 4096 x
// 4096 52.5 -> 47.0 us, 2048 x 5632 x 2048 67.4 -> 62.8; but halves that push a
// one-round grid into a second round lose (1024 x 2048 x 2560: 23.4 -> 27.8),
// and past two rounds the halves' extra operand stream outweighs the balance.
// Same bits: the halves sum K exactly as the whole tile.
template <int SW>
EE_DEV void gemm_routed(const EeRoutedGemmArgs& r) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTAGE * LDS_STAGE];
    const int32_t* counts = r.t[0].counts;
    const int T0 = (counts[0] + BM - 1) / BM;
    const int T1 = (counts[1] + BM - 1) / BM;
    const int T2 = (counts[2] + BM - 1) / BM;
    int tm, tn;
    tile_of((int)blockIdx.x, (int)gridDim.x, r.mt_max, tm, tn);
    if constexpr (SW == 0) {
        const int nN = (r.t[2].N + BN - 1) / BN;
        const int wf = (T0 + T1 + T2) * nN, wh = (T0 + T1 + 2 * T2) * nN, cus = r.f16_half_cus;
        if (cus > 0 && T2 > 0 && (wh <= cus || (wf > cus && wf <= 2 * cus)) && tm >= T0 + T1) {
            const int v = tm - T0 - T1;
            if (v < 2 * T2) gemm_tile<EE_GEMM_F16, 0, 64>(r.t[2], v >> 1, 2 * tn + (v & 1), smem);
            return;
        }
    }
    if (tm < T0) gemm_tile<EE_GEMM_I8, SW>(r.t[0], tm, tn, smem);
    else if (tm < T0 + T1) gemm_tile<EE_GEMM_F8, SW>(r.t[1], tm - T0, tn, smem);
    else if (tm < T0 + T1 + T2) {
        if (r.f16_w8) {
            Gemm8<EE_GEMM_F16, SW> k(r.t[2], smem);
            k.run(tm - T0 - T1, tn);
        } else {
            gemm_tile<EE_GEMM_F16, SW>(r.t[2], tm - T0 - T1, tn, smem);
        }
    }
}
extern "C" __global__ void __launch_bounds__(GEMM_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
eek_gemm_routed(EeRoutedGemmArgs r) {
    gemm_routed<0>(r);
}
extern "C" __global__ void __launch_bounds__(GEMM_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
eek_gemm_routed_swiglu(EeRoutedGemmArgs r) {
    gemm_routed<1>(r);
}

template <int SW> EE_DEV void body_i8_persist(const EeGemmArgs& g) { gemm_persistent<EE_GEMM_I8, SW>(g); }
template <int SW> EE_DEV void body_f8_persist(const EeGemmArgs& g) { gemm_persistent<EE_GEMM_F8, SW>(g); }
EE_GEMM_ENTRY(eek_gemm_i8_persist, body_i8_persist)
EE_GEMM_ENTRY(eek_gemm_f8_persist, body_f8_persist)

// eek_gemm_routed as a persistent grid (at most one workgroup per CU): each
// workgroup runs its INT8 and FP8 tiles through the cross-tile pipeline, then
// its W8A16 tiles, one Gemm8 run each (the pipeline ee_gemm uses for that
// tier, so routed and per-tier outputs stay bit-identical).  TileDeal levels
// the work: W8A16 tiles first, round robin, then the 1-byte tiles.
template <int SW>
EE_DEV void gemm_routed_persist(const EeRoutedGemmArgs& r) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[(NSTAGE_P + 1) * LDS_STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int32_t* counts = r.t[0].counts;
    const int c0 = counts[0], c1 = counts[1], c2 = counts[2];
    const int T0 = (c0 + BM - 1) / BM, T1 = (c1 + BM - 1) / BM, T2 = (c2 + BM - 1) / BM;
    const int nN = (r.t[0].N + BN - 1) / BN;
    const int b = (int)blockIdx.x, G = (int)gridDim.x;
    const int nF = T2 * nN;
    const SeqRouted seq(r, T0, T0 + T1, c0, c1, nN, nF, b, G);
    const int nt = seq.count();
    const int nk = r.t[0].K / BKB;
    if (nt > 0) {
        if (wave >= 4) {
            persist_loader(seq, nt, nk, smem, wave - 4, lane);
        } else {
            for (int i = 0; i < nt; ++i) {
                const PTile t = seq.tile(i);
                if (t.tier == 0) persist_compute<EE_GEMM_I8, SW>(t, nk, i * nk, smem, wave, lane);
                else persist_compute<EE_GEMM_F8, SW>(t, nk, i * nk, smem, wave, lane);
            }
        }
    }
    // W8A16 tiles f = b, b + G, ...: M-tile f % T2, N-tile f / T2
    for (int f = b; f < nF; f += G) {
        __syncthreads();                              // the LDS is free: earlier tiles' reads and DMA are done
        Gemm8<EE_GEMM_F16, SW> k(r.t[2], smem);
        k.run(f % T2, f / T2);
    }
}
extern "C" __global__ void __launch_bounds__(GEMM_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
eek_gemm_routed_persist(EeRoutedGemmArgs r) {
    gemm_routed_persist<0>(r);
}
extern "C" __global__ void __launch_bounds__(GEMM_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
eek_gemm_routed_persist_swiglu(EeRoutedGemmArgs r) {
    gemm_routed_persist<1>(r);
}

// Fallback for any K that is a multiple of 16 bytes (zero-filled K tail).
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_gemm_i8_generic(EeGemmArgs g) { gemm_generic<EE_GEMM_I8>(g); }
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_gemm_f8_generic(EeGemmArgs g) { gemm_generic<EE_GEMM_F8>(g); }
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_gemm_f16_generic(EeGemmArgs g) { gemm_generic<EE_GEMM_F16>(g); }
