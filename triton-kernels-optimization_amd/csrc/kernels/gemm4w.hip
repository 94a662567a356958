// gemm4w.hip -- persistent 256 x 256-tile MFMA GEMMs of the three precision
// tiers on four waves per workgroup (gfx950): one wave per SIMD, each wave
// owning a 128 x 128 quarter of the tile with its accumulators in AGPRs.
//
//   EE_GEMM_I8 : int8 x int8 -> int32 (v_mfma_i32_16x16x64_i8, four per 32x32 block
//                and 64-byte K slice);
//                C = fp16((f32(acc) * a_scale[m]) * b_scale[n])     (EE/python/kernels.py:50-110)
//   EE_GEMM_F8 : e4m3 x e4m3 -> f32 (v_mfma_scale_f32_32x32x64_f8f6f4);
//                C = fp16((acc * a_scale[m]) * b_scale[n])           (EE/python/kernels.py:118-180)
//   EE_GEMM_F16: fp16 x fp16 -> f32 (v_mfma_f32_16x16x32_f16, four per 32x32 block
//                and 64-byte K slice); C = fp16(acc)
//                (EE/python/kernels.py:192-246, W8A16 weights pre-dequantised)
//   EE_GEMM_W8A16: the same GEMM from the int8 weight codes and f32 column
//                scales, dequantised in registers to exactly the pre-dequantised
//                weights (dq4): the same MFMAs on the same fragment values in the
//                same order, so the same bits as EE_GEMM_F16 on those weights,
//                with B streamed at 1 byte per element.
//
// Why four waves.  The eight-wave 256-tile pipeline (gemm256.hip) gives each
// wave a 128 x 64 block, so every A row of a stage is read from LDS by four
// waves and every B row by two: 192 KB of fragment reads per 64 KB stage.  A
// 128 x 128 block per wave has each stage row read by two waves: 128 KB per
// stage, and each fragment read feeds twice the MFMAs.  The 16 blocks of
// 32 x 32 take all 256 AGPRs as accumulators; the fragments of two K slices
// (double buffered) and the DMA offsets fit in the 256 architectural VGPRs.
// With one wave per SIMD the wave's own instruction stream keeps the matrix
// core busy: each 64-byte K slice is 1024 clocks of MFMA (64 16x16x64 i8, 64
// 16x16x32 f16 or 16 32x32x64 e4m3) into which the reads of the next slice's
// 8 fragments and the direct-to-LDS loads of a stage are interleaved.
//
// Every 32 x 32 block sums its K slices in order with the MFMA and fragment
// layout of the other pipelines (ee_gemm_dev.h), so FP8 and FP16 outputs are
// bit-identical to the 8-wave 256-tile and the 128-tile kernels, and INT8 to
// every kernel.
//
// LDS: a ring of two 64 KB stages (128 K bytes of 256 A rows and 256 B rows,
// the 128-byte swizzled rows of ee_gemm_dev.h), a 4 KB epilogue slot per wave,
// and two 3 KB scale areas.  Stage s: slice 0's MFMAs read slice 1's
// fragments; barrier s+1 (every wave has read stage s and waited for its part
// of stage s+1); slice 1's MFMAs issue stage s+2 into stage s's buffer and
// read slice 0 of stage s+1.  Every stage runs this one schedule, across tile
// boundaries too: the epilogue of a tile runs between two stages, with the
// next tile's first stage landed and its slice-0 fragments in registers.
//
// The epilogue issues no loads: a tile's row scales, column scales and
// (routed) C row numbers are DMA'd into the scale area of its parity with the
// tile's first stage, and read back from LDS.  Outputs are dequantised in
// registers, staged through the wave's slot 32 x 64 at a time and stored as
// row-contiguous 16-byte vectors.
//
// Persistent grid: one workgroup per CU walks its tiles (TileDeal: 8 x 4
// blocks of tiles per XCD per round).
#include "../common/ee_device.h"
#include "../common/ee_gemm_dev.h"
#include "../common/ee_gemm_seq.h"

#pragma clang fp contract(off)

#define G4_THREADS 256

// Tile 256 x TN (TN = 256 or 128).  The waves form a WM x WN grid over the tile:
// wave w owns rows WR (w / WN) .. + WR - 1 and columns WC (w % WN) .. + WC - 1
// as NI x NJ blocks of 32 x 32.  A stage holds 128 K bytes of each A row and BRB
// K bytes of each B row: 128, or 64 for int8 W8A16 codes (64 K elements, as the
// fp16 A rows' 128 bytes).  2 x 2 waves of 128 x (TN / 2), except W8A16 256 x 256
// tiles: 1 x 4 waves of 256 x 64, so that each B column's codes are dequantised
// by one wave of the workgroup instead of two.
template <int TN, int BRB = BKB, int WN_ = 2>
struct G4Geom {
    static constexpr int STAGE = T2M * BKB + TN * BRB;   // 64, 48, 48 or 40 KB
    static constexpr int SLOTS = 2 * STAGE;           // after the ring of two stages
    static constexpr int SLOT = 32 * 64 * 2;          // 32 rows x 64 fp16 columns per wave
    static constexpr int SCALES = SLOTS + 4 * SLOT;   // two scale areas (tile parity)
    static constexpr int SA = 0, SB = T2M * 4, SC = SB + TN * 4;   // a_scale, b_scale, C rows
    static constexpr int SCALE_SZ = SC + T2M * 4;
    static constexpr int LDS = SCALES + 2 * SCALE_SZ; // 150, 117, 118 or 101 KB
    static constexpr int WN = WN_, WM = 4 / WN_;     // the wave grid
    static constexpr int WR = T2M / WM, WC = TN / WN; // rows and columns of a wave's block
    static constexpr int NI = WR / 32, NJ = WC / 32;  // its 32-row and 32-column blocks
    static constexpr int AG = 8;                      // A row groups (of 8 rows) per wave and stage
    static constexpr int BROWS = 1024 / BRB;          // B rows per DMA instruction (8 or 16)
    static constexpr int BG = TN / BROWS / 4;         // B row groups per wave and stage
    static constexpr int BRB_ = BRB;
    static constexpr int PARTS = AG + BG;             // DMA instructions per wave and stage
};

template <int KIND, int SW, class Seq, int TN = 256>
struct G4 {
    static constexpr bool W8 = KIND == EE_GEMM_W8A16;       // int8 B codes, dequantised in registers
    static constexpr bool F16T = KIND == EE_GEMM_F16 || W8;  // the FP16 tier: fp16 A, no scales in the epilogue
    typedef G4Geom<TN, W8 ? 64 : BKB, W8 && TN == 256 ? 4 : 2> GE;
    static constexpr int NI = GE::NI, NJ = GE::NJ, WR = GE::WR, WC = GE::WC;
    typedef std::conditional_t<KIND == EE_GEMM_I8, PipeI8x16, std::conditional_t<W8, PipeF16x16, Pipe<KIND>>> P;
    typedef typename P::acc_t acc_t;
    typedef typename P::frag_t frag_t;
    static constexpr int ESZ = F16T ? 2 : 1;                 // bytes per A element
    static constexpr int ESZB = KIND == EE_GEMM_F16 ? 2 : 1; // bytes per B element
    static_assert(BKB / P::SB == 2, "two K slices per stage");
    static_assert(NJ % 2 == 0, "the epilogue stores pairs of 32-column blocks");
    static constexpr int NBLK = NI * NJ;              // 32 x 32 blocks per wave
    static constexpr int NFR = NI + NJ;               // fragments per slice

    const EeGemmArgs& g;
    uint8_t* smem;
    const Seq& seq;
    int M;                                            // rows (counts[tier] when routed)
    int64_t off;                                      // partition slot of row 0 (routed), else 0
    uint32_t lds0;
    int lane, wave, wm, wn;
    int nk, ntiles;                                   // stages per tile (>= 2), tiles of this workgroup
    // DMA cursor: the next stage to issue is (itile, ikt), global number iss.
    int iss, itile, ikt;
    const uint8_t* abase;
    const uint8_t* bbase;
    uint32_t aoff[GE::AG], boff[GE::BG];
    acc_t acc[NI][NJ];
    struct RawB {                                     // W8: 8 codes of each of the lane's two B rows
        u32x2 h[2];
    };
    typedef std::conditional_t<W8, RawB, frag_t> bfrag_t;
    struct Frags {
        frag_t a[NI];
        bfrag_t b[NJ];
    } fr[2];
    frag_t wb[W8 ? NJ : 1];                           // W8: the slice's dequantised B fragments
    f16x2 bs2[W8 ? NJ : 1][2];                        // W8: {s, s}, s = fp16(b_scale) of the lane's B rows

    __device__ __forceinline__ G4(const EeGemmArgs& g_, uint8_t* smem_, const Seq& seq_, int M_, int64_t off_)
        : g(g_), smem(smem_), seq(seq_), M(M_), off(off_) {}

    __device__ __forceinline__ void coords(int i, int& m0, int& n0) const {
        int tm, tn;
        seq.coords(i, tm, tn);
        m0 = tm * T2M;
        n0 = tn * TN;
    }

    // DMA rows of tile i: one global_load_lds_dwordx4 fills 8 LDS rows (1 KB);
    // lane l lands at row 8 * grp + l / 8, physical chunk l % 8, which holds
    // logical chunk (l % 8) ^ swz(row) (W8 B: 16 rows of 64 bytes, row 16 * grp
    // + l / 4, physical chunk l % 4 holding (l % 4) ^ swz64(row)).  Wave w fills
    // A row groups 8w .. 8w+7 and B row groups BG w .. BG w + BG-1 (rows clamped
    // to the operand: rows
    // beyond it load a valid row whose results are never stored).  Un-routed:
    // offsets from the tile's first row; routed: A row m is a[a_idx[off + m]] or
    // a[off + m], offsets from the operand's start (the launcher checks that
    // they fit 32 bits).  Then the tile's scales and C rows into the scale area
    // of its parity: wave w takes rows 64w .. 64w+63 and, for w < TN / 64,
    // columns 64w .. 64w+63 (clamped likewise).
    __device__ __forceinline__ void dma_tile(int i) {
        int m0, n0;
        coords(i, m0, n0);
        int lane = this->lane;
        asm volatile("" : "+v"(lane));                // lane-dependent offsets computed here, not hoisted
        constexpr bool routed = Seq::ROUTED;
        abase = (const uint8_t*)g.a + (routed ? 0 : (int64_t)m0 * g.lda * ESZ);
        bbase = (const uint8_t*)g.b + (int64_t)n0 * g.ldb * ESZB;
#pragma unroll
        for (int q = 0; q < GE::AG; ++q) {
            const int r = (wave * GE::AG + q) * 8 + (lane >> 3);
            const int lchunk = (lane & 7) ^ swz(r);
            const int m = min(m0 + r, M - 1);
            const int64_t ar = !routed ? (int64_t)(m - m0) : Seq::GATHER ? (int64_t)g.a_idx[off + m] : off + m;
            uint32_t pr = (uint32_t)ar * (uint32_t)(g.lda * ESZ);
            asm volatile("" : "+v"(pr));
            aoff[q] = pr + (uint32_t)(lchunk * 16);
        }
#pragma unroll
        for (int q = 0; q < GE::BG; ++q) {
            const int r = W8 ? (wave * GE::BG + q) * 16 + (lane >> 2) : (wave * GE::BG + q) * 8 + (lane >> 3);
            const int lchunk = W8 ? (lane & 3) ^ swz64(r) : (lane & 7) ^ swz(r);   // swz(T2M + r) == swz(r)
            const int n = min(n0 + r, g.N - 1) - n0;
            uint32_t pr = (uint32_t)n * (uint32_t)(g.ldb * ESZB);
            asm volatile("" : "+v"(pr));
            boff[q] = pr + (uint32_t)(lchunk * 16);
        }
        const uint32_t sa = lds0 + (uint32_t)(GE::SCALES + (i & 1) * GE::SCALE_SZ);
        const int mr = min(m0 + wave * 64 + lane, M - 1);
        if constexpr (!F16T) dma4(g.a_scale + off + mr, sa + GE::SA + wave * 256);
        if constexpr (KIND != EE_GEMM_F16)
            if (wave < TN / 64) dma4(g.b_scale + min(n0 + wave * 64 + lane, g.N - 1), sa + GE::SB + wave * 256);
        if constexpr (routed)
            if (g.c_idx) dma4(g.c_idx + off + mr, sa + GE::SC + wave * 256);
    }
    // Part P (0 .. PARTS-1) of the next stage: A row group 8w + P, then B row
    // group BG w + P - 8: one s_add writing m0 (the part's LDS rows) and the
    // load, from the stage's SGPR base (operand start + K offset of the stage)
    // and the lane's row offset.  Past the workgroup's last stage the cursor
    // re-issues its last tile's stages (valid rows, into ring buffers nobody
    // reads again), so that every stage runs one schedule; run() waits for
    // them before the workgroup ends.
    template <int PT>
    __device__ __forceinline__ void issue_part() {
        if constexpr (PT == 0) {
            if (ikt == nk) {
                ikt = 0;
                if (itile + 1 < ntiles) {
                    ++itile;
                    dma_tile(itile);
                }
            }
        }
        const uint32_t s = lds0 + (uint32_t)((iss & 1) * GE::STAGE);
        if constexpr (PT < GE::AG)
            dma16_at<PT * 8 * BKB>(abase + (uint32_t)ikt * BKB, aoff[PT], s + wave * (GE::AG * 8 * BKB));
        else
            dma16_at<(PT - GE::AG) * 1024>(bbase + (uint32_t)ikt * GE::BRB_, boff[PT - GE::AG],
                                           s + T2M * BKB + wave * GE::BG * 1024);
        if constexpr (PT == GE::PARTS - 1) {
            ++ikt;
            ++iss;
        }
    }
    template <int OFF>
    static __device__ __forceinline__ void dma16_at(const uint8_t* sbase, uint32_t voff, uint32_t lds_sgpr) {
        asm volatile("s_add_u32 m0, %0, %3\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_sgpr), "v"(voff), "s"(sbase),
                     "i"(OFF)
                     : "memory", "m0", "scc");
    }
    template <int PT = 0>
    __device__ __forceinline__ void issue_stage() {
        if constexpr (PT < GE::PARTS) {
            issue_part<PT>();
            issue_stage<PT + 1>();
        }
    }

    // Fragments of K slice SL from the stage at st.  Byte offsets from a stage's
    // start, per slice (offA / offB, set up in run()):
    // SUB16: rows row0 + (l & 15) and row0 + 16 + (l & 15), chunk 4 SL + (l >> 4)
    // (swz(row0 + x) == swz(x) for row0 % 32 == 0);
    // 32x32 forms: row row0 + (l & 31), chunk SL * SB/16 + (l >> 5) * LSTEP and
    // the chunk CSTEP after it (offsets x = 0, 1).
    // Fragment K: 0..NI-1 A row block K (rows WR wm + 32 K), NI.. B row block K - NI
    // (rows 256 + WC wn + 32 (K - NI)); each read takes the block's offset as its
    // immediate.  W8 B: the 8 codes of K elements 32 SL + 8 (l >> 4) .. +7 of rows
    // (l & 15) and 16 + (l & 15), two ds_read_b64 (byte 32 SL + 8 (l >> 4) of the
    // 64-byte row: chunk 2 SL + (l >> 5), half (l >> 4) & 1).
    static constexpr int XR = P::SUB16 ? 1 : 2;
    uint32_t offA[2][XR], offB[2][XR];
    template <int SL, int K>
    __device__ __forceinline__ void rd_frag(const uint8_t* st, Frags& f) {
        constexpr int rel = K < NI ? K * 32 * BKB : (K - NI) * 32 * GE::BRB_;
        uint32_t o0, o1 = 0;
        if constexpr (K < NI) {
            o0 = offA[SL][0];
            if constexpr (XR == 2) o1 = offA[SL][XR - 1];
        } else {
            o0 = offB[SL][0];
            if constexpr (XR == 2) o1 = offB[SL][XR - 1];
        }
        if constexpr (W8 && K >= NI) {
            const uint8_t* q = st + o0 + rel;
            RawB v;
            v.h[0] = *(const u32x2*)q;
            v.h[1] = *(const u32x2*)(q + 16 * 64);
            f.b[K - NI] = v;
            return;
        }
        frag_t v;
        if constexpr (P::SUB16) {
            const uint8_t* q = st + o0 + rel;
            v.h[0] = *(const i32x4*)q;
            v.h[1] = *(const i32x4*)(q + 16 * BKB);
        } else {
            const u32x4 x0 = *(const u32x4*)(st + o0 + rel), x1 = *(const u32x4*)(st + o1 + rel);
            v = i32x8{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
        }
        if constexpr (K < NI) f.a[K] = v;
        else if constexpr (!W8) f.b[K - NI] = v;
    }
    template <int SL, int K = 0>
    __device__ __forceinline__ void rd_all(const uint8_t* st, Frags& f) {
        if constexpr (K < NFR) {
            rd_frag<SL, K>(st, f);
            rd_all<SL, K + 1>(st, f);
        }
    }

#define G4_SB() __builtin_amdgcn_sched_barrier(0)
    // MFMA Q of block (I, J) on fragments f: SUB16 blocks are four 16x16 MFMAs
    // (quarter Q: B half Q >> 1, A half Q & 1), exactly PipeI8x16 / PipeF16x16's
    // mma; the 32x32 forms are one.  W8 takes B from the dequantised wb[J].
    static constexpr int NQ = P::SUB16 ? 4 : 1;       // MFMAs per block
    static constexpr int NM = NBLK * NQ;              // MFMAs per slice
    template <int I, int J, int Q>
    __device__ __forceinline__ void mma_q(const Frags& f) {
        if constexpr (!P::SUB16) {
            acc[I][J] = P::mma(f.b[J], f.a[I], acc[I][J]);
        } else if constexpr (KIND == EE_GEMM_I8) {
            acc[I][J].q[Q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.b[J].h[Q >> 1], f.a[I].h[Q & 1], acc[I][J].q[Q], 0, 0, 0);
        } else if constexpr (W8) {
            acc[I][J].q[Q] = P::m16(wb[J].h[Q >> 1], f.a[I].h[Q & 1], acc[I][J].q[Q]);
        } else {
            acc[I][J].q[Q] = P::m16(f.b[J].h[Q >> 1], f.a[I].h[Q & 1], acc[I][J].q[Q]);
        }
    }
    // Block order within a slice: by block rows (I outer), or for W8 by block
    // columns (J outer), so that each dequantised B fragment is dead after its
    // column's 16 MFMAs and one set of wb registers serves every slice.  Either
    // order gives every accumulator the same MFMAs in the same K order.
    static constexpr bool JMAJ = W8;
    static constexpr int blk_i(int b) { return JMAJ ? b % NI : b / NJ; }
    static constexpr int blk_j(int b) { return JMAJ ? b / NI : b % NJ; }
    // Fragment read order: by first use in the next slice (a0 b0 .. b3, then
    // a1 .. a3; W8: b0, whose dequantisation comes first, then a0 .. a3, b1 ..).
    static constexpr int rd_order(int r) {
        return W8 ? (r == 0 ? NI : r <= NI ? r - 1 : r) : (r == 0 ? 0 : r <= NJ ? NI - 1 + r : r - NJ);
    }
    // The ops of a slice: RD: the NFR fragment reads of the next slice; DMA: the
    // PARTS parts of the stage being issued.  Op o of n goes after MFMA
    // (o * span) / n, span = 3/4 of the slice's MFMAs for reads (the last reads
    // land before the next slice) and all of them for the loads.  Spread that far,
    // the 64 loads per CU and stage queue less at the address unit: measured at
    // C1 (timestamps, same box, interleaved), loop clocks 155.6k -> 151.9k (FP16)
    // and 77.4k -> 76.3k (INT8) against loads over 3/4 of the slice, and a burst
    // over half of it costs 11%.
    static constexpr int n_ops(bool rd, bool dma) { return (rd ? NFR : 0) + (dma ? GE::PARTS : 0); }
    static constexpr int op_at(int m, bool rd, bool dma) {   // first op after MFMA m (m may be NM: the end)
        const int n = n_ops(rd, dma), span = rd ? (NM * 3) / 4 : NM;
        // ops o with (o * span) / n < m ... count them: smallest o with o * span >= m * n
        return m >= span ? n : (m * n + span - 1) / span;
    }
    template <int SL, bool RD, bool DMA, int O>
    __device__ __forceinline__ void op(const uint8_t* rs, Frags& nf) {
        if constexpr (RD && DMA) {
            constexpr int n = NFR + GE::PARTS;
            constexpr int r0 = (O * NFR) / n, r1 = ((O + 1) * NFR) / n;   // reads before op O, through it
            if constexpr (r1 > r0) rd_frag<SL, rd_order(r1 - 1)>(rs, nf);
            else issue_part<O - r0>();
        } else if constexpr (RD) {
            rd_frag<SL, rd_order(O)>(rs, nf);
        } else if constexpr (DMA) {
            issue_part<O>();
        }
    }
    template <int SL, bool RD, bool DMA, int O, int OE>
    __device__ __forceinline__ void ops(const uint8_t* rs, Frags& nf) {
        if constexpr (O < OE) {
            op<SL, RD, DMA, O>(rs, nf);
            ops<SL, RD, DMA, O + 1, OE>(rs, nf);
        }
    }
    // W8 dequantisation: unit U (0..3) of B fragment J from raw codes f.b[J]:
    // half U >> 1, codes 4 (U & 1) .. +3 -> fp16 words 2 (U & 1), +1 of wb[J].
    template <int J, int U>
    __device__ __forceinline__ void dq_unit(const Frags& f) {
        constexpr int h = U >> 1, d = U & 1;
        uint32_t lo, hi;
        dq4(f.b[J].h[h][d], bs2[J][h], lo, hi);
        asm volatile("" : "+v"(lo), "+v"(hi));        // computed here, not sunk past the stage barrier
        wb[J].h[h][2 * d] = (int)lo;
        wb[J].h[h][2 * d + 1] = (int)hi;
    }
    template <int J, int U = 0>
    __device__ __forceinline__ void dq_frag(const Frags& f) {
        if constexpr (U < 4) {
            dq_unit<J, U>(f);
            dq_frag<J, U + 1>(f);
        }
    }
    // The units in flight, one step per MFMA: dq4's four dependent steps (xor;
    // the two perms; the two bias subtracts; the two scale multiplies), each a
    // full MFMA after the one before, so that no VALU op waits on its operand
    // and at most two issue between two MFMAs (the matrix core is never left
    // without a queued MFMA).
    uint32_t dq_x[1], dq_p[2];                        // W8: the unit in flight
    template <int J, int U, int S>
    __device__ __forceinline__ void dq_part(const Frags& f) {
        constexpr int h = U >> 1, d = U & 1;
        if constexpr (S == 0) {
            dq_x[0] = f.b[J].h[h][d] ^ 0x80808080u;
        } else if constexpr (S == 1) {
            dq_p[0] = __builtin_amdgcn_perm(0x64646464u, dq_x[0], 0x04010400u);
            dq_p[1] = __builtin_amdgcn_perm(0x64646464u, dq_x[0], 0x04030402u);
        } else if constexpr (S == 2) {
            const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
            dq_p[0] = bits_of(f16x2_from_bits(dq_p[0]) - bias);
            dq_p[1] = bits_of(f16x2_from_bits(dq_p[1]) - bias);
        } else {
            uint32_t lo = bits_of(f16x2_from_bits(dq_p[0]) * bs2[J][h]);
            uint32_t hi = bits_of(f16x2_from_bits(dq_p[1]) * bs2[J][h]);
            asm volatile("" : "+v"(lo), "+v"(hi));    // computed here, not sunk past the stage barrier
            wb[J].h[h][2 * d] = (int)lo;
            wb[J].h[h][2 * d + 1] = (int)hi;
        }
    }
    // Block column c's CM MFMAs carry the 16 steps of fragment c + 1 of this
    // slice, or after the last column, of fragment 0 of the next slice (NEXT: its
    // codes were read during this slice): step 4 u + s (unit u, step s) after
    // MFMA c CM + (4 u + s) CM / 16.  Unit u writes half u >> 1; the next column's
    // first MFMAs read half 0, so the last unit (half 1) is read at least two
    // MFMAs after its last step.
    static constexpr int CM = NI * NQ;                // MFMAs per block column (16 or 32)
    template <int C, bool NEXT, int MI>
    __device__ __forceinline__ void dq_step() {
        constexpr int c = MI / CM, p = MI % CM, SP = CM / 16;
        if constexpr (p % SP == 0) {
            constexpr int k = p / SP, u = k / 4, st = k % 4;
            if constexpr (c + 1 < NJ) dq_part<c + 1, u, st>(fr[C]);
            else if constexpr (NEXT) dq_part<0, u, st>(fr[1 - C]);
        }
    }
    // The lane's b_scale pairs of tile t, from its scale area.
    __device__ __forceinline__ void load_bscales(int t) {
        const uint8_t* sb = smem + GE::SCALES + (t & 1) * GE::SCALE_SZ + GE::SB;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const f16 v = (f16)f32_rn(*(const float*)(sb + (wn * WC + j * 32 + h * 16 + (lane & 15)) * 4));
                bs2[j][h] = f16x2{v, v};
            }
    }

    // The MFMAs of one K slice on fragments fr[C], block by block (blk_i, blk_j),
    // one MFMA at a time with the slice's ops between them (RD: slice SL of the
    // stage at rs into fr[1 - C]).
    template <int C, int SL, bool RD, bool DMA, int MI = 0>
    __device__ __forceinline__ void slice(const uint8_t* rs) {
        if constexpr (MI < NM) {
            constexpr int b = MI / NQ, q = MI % NQ;
            mma_q<blk_i(b), blk_j(b), q>(fr[C]);
            G4_SB();
            if constexpr (W8) dq_step<C, RD, MI>();
            if constexpr (RD && DMA) {                // reads over 3/4 of the slice, the stage's loads over all of it
                ops<SL, true, false, op_at(MI, true, false), op_at(MI + 1, true, false)>(rs, fr[1 - C]);
                ops<SL, false, true, op_at(MI, false, true), op_at(MI + 1, false, true)>(rs, fr[1 - C]);
            } else {
                ops<SL, RD, DMA, op_at(MI, RD, DMA), op_at(MI + 1, RD, DMA)>(rs, fr[1 - C]);
            }
            G4_SB();
            slice<C, SL, RD, DMA, MI + 1>(rs);
        }
    }

    // Stage cs from buffer cs & 1; its slice-0 fragments are in fr[0].  Slice 0's
    // MFMAs read slice 1 into fr[1]; barrier cs+1 (stage cs+1 landed, stage cs
    // read); slice 1's MFMAs issue stage cs+2 and, RD, read slice 0 of stage
    // cs+1 into fr[0].  A tile's last stage reads nothing: the fragments of the
    // next tile's first stage are read after the epilogue, so that they do not
    // hold registers through it.
    template <bool RD>
    __device__ __forceinline__ void stage(int cs) {
        slice<0, 1, true, false>(smem + (cs & 1) * GE::STAGE);
        G4_SB();
        WAITCNT_VM(0);
        WAITCNT_LGKM0();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();                 // barrier cs+1: stage cs+1 landed, stage cs read
        asm volatile("" ::: "memory");
        slice<1, 0, RD, true>(smem + ((cs + 1) & 1) * GE::STAGE);
        G4_SB();
    }

    // Dequantise and store tile t (m0, n0): for each 32-row block and pair of
    // 32-column blocks, quarter q of block (i, j) holds rows row_of(q) and
    // columns j * 32 + col_of(q) .. +3 of the block; they are dequantised with
    // the row's a_scale and the four columns' b_scale (from the tile's scale
    // area), written to the wave's slot as fp16 and stored as 16-byte row
    // vectors.  SwiGLU: blocks 2p (gate) and 2p + 1 (up) hold the same 32
    // outputs; their act values fp16(fp16(silu(gate)) * up) are staged instead.
    static constexpr int q_of_cq(int c) { return P::SUB16 ? 2 * c : c; }
    __device__ __forceinline__ void epilogue(int t) {
        int m0, n0;
        coords(t, m0, n0);
        const int N = g.N;
        int lane = this->lane;
        asm volatile("" : "+v"(lane));                // epilogue addresses computed here, not hoisted
        const int nb = n0 + wn * WC;                  // first column of the wave's block
        const uint8_t* sc = smem + GE::SCALES + (t & 1) * GE::SCALE_SZ;
        uint8_t* slot = smem + GE::SLOTS + wave * GE::SLOT;
        auto crow_of = [&](int r) -> int32_t {        // C row of wave row r (0..127), -1 beyond M
            const int m = m0 + wm * WR + r;
            if (m >= M) return -1;
            if constexpr (Seq::ROUTED)
                if (g.c_idx) return *(const int32_t*)(sc + GE::SC + (wm * WR + r) * 4);
            return m;
        };
        // An un-routed tile wholly inside C with 16-byte aligned rows stores without
        // per-row tests: a wave-uniform base (the wave's first output) plus a 32-bit
        // byte offset per lane.
        const bool fast = !Seq::ROUTED && m0 + T2M <= M && n0 + TN <= N && ((uintptr_t)g.c & 15) == 0 &&
                          (g.ldc & 7) == 0;
        const int64_t ldc = g.ldc;
        const uint8_t* cwave = (const uint8_t*)(g.c + (int64_t)(m0 + wm * WR) * ldc + (SW ? (nb >> 1) : nb));
        constexpr int SCPR = SW ? NJ * 2 : 8;         // 16-byte chunks per stored row of a pass
        const uint32_t lofs = (uint32_t)(((lane / SCPR) * ldc + (lane % SCPR) * 8) * 2);
        auto fast_store = [&](int row, int col, const u32x4& v) {   // row, col: uniform, from the wave's origin
            const uint8_t* b = cwave + ((int64_t)row * ldc + col) * 2;
            __builtin_nontemporal_store(v, (u32x4*)(b + lofs));
        };
        auto bsc = [&](int j, int c) -> f32x4 {       // b_scale of column group c of block j
            if constexpr (F16T) return f32x4{1.f, 1.f, 1.f, 1.f};
            else return *(const f32x4*)(sc + GE::SB + (wn * WC + j * 32 + P::col_of(q_of_cq(c), lane)) * 4);
        };
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            G4_SB();                                  // one block row's accumulators at a time
            const int mb = m0 + wm * WR + i * 32;     // first row of this 32-row block
            float as[P::NRQ] = {};
            if constexpr (!F16T)
#pragma unroll
                for (int h = 0; h < P::NRQ; ++h)
                    as[h] = *(const float*)(sc + GE::SA + (wm * WR + i * 32 + P::row_of(h, lane)) * 4);
            if constexpr (KIND == EE_GEMM_I8) {
                if (!Seq::ROUTED && g.acc) {          // debug output: int32 accumulators, direct stores
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int m = mb + P::row_of(q, lane), n = nb + j * 32 + P::col_of(q, lane);
                            if (m < M && n < N)
                                *(i32x4*)(g.acc + (int64_t)m * g.ldc + n) =
                                    i32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                          acc[i][j][4 * q + 3]};
                        }
                }
            }
            if constexpr (SW) {
#pragma unroll
                for (int pr = 0; pr < NJ / 2; ++pr) {
                    f32x4 bg[P::NCQ], bu[P::NCQ];
#pragma unroll
                    for (int c = 0; c < P::NCQ; ++c) {
                        bg[c] = bsc(2 * pr, c);
                        bu[c] = bsc(2 * pr + 1, c);
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        float gv[4], uv[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            gv[r] = deq<KIND>(acc[i][2 * pr][4 * q + r], as[P::rq(q)], bg[P::cq(q)][r]);
                            uv[r] = deq<KIND>(acc[i][2 * pr + 1][4 * q + r], as[P::rq(q)], bu[P::cq(q)][r]);
                        }
                        const int ca = pr * 32 + P::col_of(q, lane);
                        *(u32x2*)(slot + lds_off(P::row_of(q, lane), ca >> 3) + ((ca >> 2) & 1) * 8) =
                            u32x2{silu_mul2(pack_f16x2(gv[0], gv[1]), pack_f16x2(uv[0], uv[1])),
                                  silu_mul2(pack_f16x2(gv[2], gv[3]), pack_f16x2(uv[2], uv[3]))};
                    }
                }
                constexpr int CPR = NJ * 2;           // 16-byte chunks per act row (NJ * 16 columns)
                constexpr int RPR = 64 / CPR;         // rows per store round
                const int na = N >> 1;
#pragma unroll
                for (int k = 0; k < 32 / RPR; ++k) {
                    const int rl = k * RPR + lane / CPR, ch = lane % CPR;
                    const u32x4 v = *(const u32x4*)(slot + lds_off(rl, ch));
                    if (fast) {
                        fast_store(i * 32 + k * RPR, 0, v);
                    } else {
                        const int n = (nb >> 1) + ch * 8;
                        const int32_t crow = crow_of(i * 32 + rl);
                        if (crow >= 0 && n < na) store_row16(g.c + (int64_t)crow * g.ldc + n, v, true);
                    }
                }
            } else {
#pragma unroll
                for (int jp = 0; jp < NJ / 2; ++jp) {
                    G4_SB();
#pragma unroll
                    for (int jj = 0; jj < 2; ++jj) {
                        const int j = 2 * jp + jj;
                        f32x4 bs[P::NCQ];
#pragma unroll
                        for (int c = 0; c < P::NCQ; ++c) bs[c] = bsc(j, c);
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int cl = jj * 32 + P::col_of(q, lane);
                            float o[4];
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                if constexpr (F16T) o[r] = acc[i][j][4 * q + r];
                                else o[r] = deq<KIND>(acc[i][j][4 * q + r], as[P::rq(q)], bs[P::cq(q)][r]);
                            }
                            *(u32x2*)(slot + lds_off(P::row_of(q, lane), cl >> 3) + ((cl >> 2) & 1) * 8) =
                                u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
                        }
                    }
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int rl = k * 8 + (lane >> 3), ch = lane & 7;
                        const u32x4 v = *(const u32x4*)(slot + lds_off(rl, ch));
                        if (fast) {
                            fast_store(i * 32 + k * 8, jp * 64, v);
                        } else {
                            const int n = nb + jp * 64 + ch * 8;
                            const int32_t crow = crow_of(i * 32 + rl);
                            if (crow >= 0 && n < N) store_row16(g.c + (int64_t)crow * g.ldc + n, v, n + 8 <= N);
                        }
                    }
                }
            }
        }
    }

    // Zero accumulators, each 4-register group through an empty asm that keeps it
    // in AGPRs: without it hipcc shares one zero group among the first MFMAs of
    // a tile and then copies accumulators between AGPRs and VGPRs at the top of
    // every stage.
    template <typename V>
    static __device__ __forceinline__ V zero4() {
        V z = {};
        asm volatile("" : "+a"(z));
        return z;
    }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                if constexpr (P::SUB16) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[i][j].q[q] = zero4<std::remove_reference_t<decltype(acc[i][j].q[q])>>();
                } else {
                    acc[i][j] = zero4<acc_t>();
                }
            }
    }

    __device__ __forceinline__ void run() {
        const int tid = threadIdx.x;
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        wm = wave / GE::WN;
        wn = wave % GE::WN;
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
            for (int x = 0; x < XR; ++x) {
                uint32_t o;
                if constexpr (P::SUB16) o = lds_off(lane & 15, lane >> 4) ^ (uint32_t)(sl << 6);
                else o = lds_off(lane & 31, sl * (P::SB / 16) + (lane >> 5) * P::LSTEP + x * P::CSTEP);
                uint32_t oa = (uint32_t)(wm * WR * BKB) + o, ob = (uint32_t)((T2M + wn * WC) * BKB) + o;
                if constexpr (W8) {
                    const int r = lane & 15, g4 = lane >> 4;
                    ob = (uint32_t)(T2M * BKB + (wn * WC + r) * 64 + (((2 * sl + (g4 >> 1)) ^ swz64(r)) << 4) +
                                    (g4 & 1) * 8);
                }
                asm volatile("" : "+v"(oa), "+v"(ob));
                offA[sl][x] = oa;
                offB[sl][x] = ob;
            }
        ntiles = seq.count();
        if (ntiles <= 0) return;                      // whole workgroup, before any barrier
        nk = (int)((int64_t)g.K * ESZ / BKB);         // a multiple of BKB, at least 2 stages (launcher)
        lds0 = lds_addr(smem);
        iss = 0;
        itile = -1;
        ikt = nk;
        issue_stage();                                // stage 0 (and tile 0's scales) -> buffer 0
        issue_stage();                                // stage 1 -> buffer 1
        WAITCNT_VM(GE::PARTS);                        // stage 0 landed; stage 1 may stay in flight
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();                 // barrier 0
        asm volatile("" ::: "memory");
        rd_all<0>(smem, fr[0]);
        if constexpr (W8) {
            load_bscales(0);
            dq_frag<0>(fr[0]);
        }
        int cs = 0;
        for (int t = 0; t < ntiles; ++t) {
            zero();
            for (int kt = 0; kt + 1 < nk; ++kt, ++cs) stage<true>(cs);
            stage<false>(cs);
            ++cs;
            epilogue(t);
            if (t + 1 < ntiles) {                     // slice 0 of the next tile's first stage (landed)
                G4_SB();
                rd_all<0>(smem + (cs & 1) * GE::STAGE, fr[0]);
                if constexpr (W8) {
                    load_bscales(t + 1);
                    dq_frag<0>(fr[0]);
                }
            }
        }
        WAITCNT_VM(0);                                // the re-issued stages have landed
    }
};

// A grid of 256 x 256 tiles whose last round is at most half full (config 2:
// 896 tiles on 256 CUs, 3.5 rounds) runs that round as 256 x 128 halves, one
// per workgroup: the full rounds first, then the halves, in the same tile
// order (both halves of a tile on one XCD).  The halves sum K in the same
// order, so the output bits do not change.
template <int KIND, int SW, int TN>
EE_DEV void gemm4w(const EeGemmArgs& g) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[G4<KIND, SW, Seq256<TN>, TN>::GE::LDS];
    const int b = (int)blockIdx.x, G = (int)gridDim.x;
    const Seq256<TN> seq(g, b, G);
    if constexpr (TN == 256) {
        const int nT = seq.d.nA, full = nT / G, rem = nT - full * G;
        if (rem > 0 && 2 * rem <= G) {
            if (full > 0) {
                const Seq256<TN> s1(g, b, G, full);
                G4<KIND, SW, Seq256<TN>, TN> k(g, smem, s1, g.M, 0);
                k.run();
                __syncthreads();                      // every wave's reads of the ring, slots and scales are done
            }
            const int h = seq.d.half_pos(2 * rem, full == 0);   // one position per workgroup
            Seq256Half sh{0, 0, 0};
            if (h < 2 * rem) {
                int tm, tn;
                seq.d.coords(full * G + (h >> 1), tm, tn);
                const int tn2 = 2 * tn + (h & 1);
                if (tn2 * 128 < g.N) sh = Seq256Half{1, tm, tn2};
            }
            if (sh.n > 0) {
                G4<KIND, SW, Seq256Half, 128> k(g, smem, sh, g.M, 0);
                k.run();
            }
            return;
        }
    }
    G4<KIND, SW, Seq256<TN>, TN> k(g, smem, seq, g.M, 0);
    k.run();
}

// ---------------------------------------------------------------- routed
// The routed linear's three tier GEMMs as one persistent grid of 256 x 256
// tiles on the four-wave pipeline: the deal of gemm256.hip's routed grid
// (tier t owns ceil(counts[t] / 256) M-tiles of its partition slots; FP16
// tiles, twice a 1-byte tile's work, dealt first round robin, as 256 x 128
// halves where that shortens the estimated makespan; then the INT8 and FP8
// tiles in TileDeal rounds), each phase one G4 pipeline.  Every tile sums K in
// the order of the un-routed kernels, so routed rows equal ee_gemm's rows of
// their tier bit for bit.
// The last round R of a deal's 1-byte tiles and its first logical tile, when that
// round is at most half full (it then runs as 256 x 128 halves).
EE_DEV bool half_last_round(const TileDeal& d, int G, int& R, int& base) {
    R = -1;
    base = 0;
    if (d.rF == 0) {
        R = (d.nA + G - 1) / G - 1;
        base = R * G;
    } else if (d.nA > d.skip * d.P) {
        const int q = (d.nA - d.skip * d.P + G - 1) / G - 1;
        R = d.skip + q;
        base = d.skip * d.P + q * G;
    }
    return R >= 0 && d.nA > base && 2 * (d.nA - base) <= G;
}

template <int SW>
EE_DEV void gemm4w_routed(const EeRoutedGemmArgs& r) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[G4Geom<256>::LDS];
    const int32_t* counts = r.t[0].counts;
    const int c0 = counts[0], c1 = counts[1], c2 = counts[2];
    const int T0 = (c0 + T2M - 1) / T2M, T1 = (c1 + T2M - 1) / T2M, T2 = (c2 + T2M - 1) / T2M;
    const int N = r.t[0].N;
    const int nN = (N + 255) / 256;
    const int b = (int)blockIdx.x, G = (int)gridDim.x;
    // W8A16 tiles: 256 x 256, or 256 x 128 halves where that shortens the estimated
    // makespan (in 1-byte-tile units: a full W8A16 tile costs 2, a half ~1.15).
    // Every workgroup reads the same counts, so every workgroup makes the same choice.
    int nF = T2 * nN, skip = 2;
    bool half = false;
    {
        const int nFh = T2 * ((N + 127) / 128), nA = (T0 + T1) * nN;
        const int full20 = 20 * max(2 * ((nF + G - 1) / G), (2 * nF + nA + G - 1) / G);
        const int half20 = max(23 * ((nFh + G - 1) / G), 20 * (((23 * nFh + 19) / 20 + nA + G - 1) / G));
        if (nF > 0 && half20 < full20) {
            half = true;
            nF = nFh;
            skip = 1;
        }
    }
    // One round of 1-byte tiles, no W8A16 tiles, and an INT8 tier of one tile row
    // (config 4's ~95 INT8 rows per 4096): each INT8 tile streams all of its B
    // columns for a few rows, with no other tile sharing them in L2, so it sets the
    // makespan where B comes from HBM.  The INT8 tiles then run as 256 x 128
    // halves on the last 2 nN workgroups and the FP8 tiles on the others, spread
    // over the XCDs (same tiles, same K order, so the same bits).
    if (nF == 0 && T0 == 1 && T1 > 0 && 2 * (T0 + T1) * nN > G && (T1 + 2) * nN <= G) {
        const int G8 = G - 2 * nN;
        if (b >= G8) {
            const int h = b - G8, tn2 = h;           // half h: columns 128 h ..
            if (tn2 * 128 < N) {
                const SeqR1Half sh{1, 0, tn2};
                G4<EE_GEMM_I8, SW, SeqR1Half, 128> k(r.t[0], smem, sh, c0, 0);
                k.run();
            }
        } else {
            const TileDeal d8(T1, nN, 0, b, G8);
            const SeqR1 s8{d8, 0, d8.count(), 0, T1, nN};
            G4<EE_GEMM_F8, SW, SeqR1, 256> k(r.t[1], smem, s8, c1, c0);
            k.run();
        }
        return;
    }
    const TileDeal d(T0 + T1, nN, nF, b, G, skip);
    // phase FP16
    const SeqRF sf{b, G, b < nF ? (nF - b + G - 1) / G : 0, T2};
    if (sf.n > 0) {
        if (half) {
            G4<EE_GEMM_F16, SW, SeqRF, 128> k(r.t[2], smem, sf, c2, (int64_t)c0 + c1);
            k.run();
        } else {
            G4<EE_GEMM_F16, SW, SeqRF, 256> k(r.t[2], smem, sf, c2, (int64_t)c0 + c1);
            k.run();
        }
    }
    // The 1-byte tiles: the INT8 ones come first (logical index < T0 * nN).  A last
    // round at most half full runs as 256 x 128 halves, one per workgroup (both
    // halves of a tile on one XCD), as gemm4w does: halves sum K in the same order,
    // so their rows do not change.  (Config 4's per-token gate|up grid: 836 units of
    // work on 256 workgroups, a fourth round of 68 tiles.)  The halves run first.
    bool had_half = false;
    int R, last_base;
    if (half_last_round(d, G, R, last_base)) {
        const int rem = d.nA - last_base;
        const int h = d.half_pos(2 * rem, d.rF == 0 && last_base == 0);   // one position per workgroup
        if (h < 2 * rem) {
            const int a = last_base + (h >> 1);
            const bool i8 = a < T0 * nN;
            int tm, tn;
            if (i8) band_coords(a, T0, nN, tm, tn);
            else band_coords(a - T0 * nN, T1, nN, tm, tn);
            const int tn2 = 2 * tn + (h & 1);
            if (tn2 * 128 < N) {
                if (sf.n > 0) __syncthreads();        // the previous phase's LDS reads and DMA are done
                const SeqR1Half sh{1, tm, tn2};
                if (i8) {
                    G4<EE_GEMM_I8, SW, SeqR1Half, 128> k(r.t[0], smem, sh, c0, 0);
                    k.run();
                } else {
                    G4<EE_GEMM_F8, SW, SeqR1Half, 128> k(r.t[1], smem, sh, c1, c0);
                    k.run();
                }
                had_half = true;
            }
        }
    }
    int n1 = d.count();
    if (half_last_round(d, G, R, last_base)) n1 = max(0, min(n1, R - d.first_round));   // tiles before it
    int ni8 = 0;
    while (ni8 < n1 && d.tile_index(d.first_round + ni8) < T0 * nN) ++ni8;
    if (ni8 > 0) {
        if (sf.n > 0 || had_half) __syncthreads();
        const SeqR1 s8{d, 0, ni8, T0, T1, nN};
        G4<EE_GEMM_I8, SW, SeqR1, 256> k(r.t[0], smem, s8, c0, 0);
        k.run();
    }
    if (n1 > ni8) {
        if (sf.n > 0 || had_half || ni8 > 0) __syncthreads();
        const SeqR1 s8{d, ni8, n1 - ni8, T0, T1, nN};
        G4<EE_GEMM_F8, SW, SeqR1, 256> k(r.t[1], smem, s8, c1, c0);
        k.run();
    }
}

#define EE_G4_ENTRY(NAME, KIND, TN)                                                                        \
    extern "C" __global__ void __launch_bounds__(G4_THREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))   \
    NAME(EeGemmArgs g) { gemm4w<KIND, 0, TN>(g); }                                                        \
    extern "C" __global__ void __launch_bounds__(G4_THREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))   \
    NAME##_swiglu(EeGemmArgs g) { gemm4w<KIND, 1, TN>(g); }
EE_G4_ENTRY(eek_gemm4w_i8, EE_GEMM_I8, 256)
EE_G4_ENTRY(eek_gemm4w_f8, EE_GEMM_F8, 256)
EE_G4_ENTRY(eek_gemm4w_f16, EE_GEMM_F16, 256)
EE_G4_ENTRY(eek_gemm4w_w8a16, EE_GEMM_W8A16, 256)
// 256 x 128 tiles
EE_G4_ENTRY(eek_gemm4wn128_i8, EE_GEMM_I8, 128)
EE_G4_ENTRY(eek_gemm4wn128_f8, EE_GEMM_F8, 128)
EE_G4_ENTRY(eek_gemm4wn128_f16, EE_GEMM_F16, 128)
EE_G4_ENTRY(eek_gemm4wn128_w8a16, EE_GEMM_W8A16, 128)
// the routed grid
extern "C" __global__ void __launch_bounds__(G4_THREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
eek_gemm4w_routed(EeRoutedGemmArgs r) { gemm4w_routed<0>(r); }
extern "C" __global__ void __launch_bounds__(G4_THREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
eek_gemm4w_routed_swiglu(EeRoutedGemmArgs r) { gemm4w_routed<1>(r); }
