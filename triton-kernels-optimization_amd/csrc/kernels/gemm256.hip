// gemm256.hip -- persistent 256 x 256-tile MFMA GEMMs of the three precision
// tiers for gfx950 (the large-M shapes: configs 1-4).
//
//   EE_GEMM_I8 : int8 x int8 -> int32 (v_mfma_i32_16x16x64_i8, four per 32x32 block
//                and 64-byte K slice: the same MFMA time as the 32x32x32 form at a
//                lower power draw);
//                C = fp16((f32(acc) * a_scale[m]) * b_scale[n])     (EE/python/kernels.py:50-110)
//   EE_GEMM_F8 : e4m3 x e4m3 -> f32 (v_mfma_scale_f32_32x32x64_f8f6f4);
//                C = fp16((acc * a_scale[m]) * b_scale[n])           (EE/python/kernels.py:118-180)
//   EE_GEMM_F16: fp16 x fp16 -> f32 (v_mfma_f32_16x16x32_f16, four per 32x32 block
//                and 64-byte K slice); C = fp16(acc)
//                (EE/python/kernels.py:192-246, W8A16 weights pre-dequantised)
//
// Why a 256 x 256 tile.  A CU computing a T x T tile streams 2T bytes of
// operands per K byte for 2T^2 ops: at the MFMA rate of 8192 int8/fp8 ops per
// clock a 128 x 128 tile needs 64 B/clk per CU from L2, a 256 x 256 tile 32.
// A gfx950 CU streams at most ~58 B/clk from L2 with every CU streaming (a
// timing-only direct-to-LDS stream kernel measured on MI355X),
// and the GEMM loops reach ~38 of it beside their fragment reads, so 128-wide
// tiles are operand-stream bound and 256-wide tiles can be MFMA bound.
//
// Workgroup: 512 threads, 8 wave64s, two per SIMD.  Wave w owns rows
// 128 (w >> 2) .. +127 and columns 64 (w & 3) .. +63 of the tile as 4 x 2
// blocks of 32 x 32 (128 accumulator registers), summing K in order, slice
// after slice -- the same K order as the 128-tile loader-wave kernels, so FP8
// and FP16 outputs are bit-identical to theirs and INT8 to every kernel.
//
// LDS: a ring of two 64 KB stages (128 K bytes of 256 A rows and 256 B rows,
// the usual 128-byte swizzled rows) plus a 4 KB epilogue slot per wave.  All
// eight waves issue the direct-to-LDS DMA of the stages in the shadow of their
// own MFMAs (4 A and 4 B row groups of 8 rows each per wave and stage).
// Barrier s+1 sits before the MFMAs of stage s's last K slice: by then every
// wave has read stage s (lgkmcnt 0) and waited for its part of stage s+1
// (vmcnt 0), so stage s+2 is issued into stage s's buffer right after it,
// while the last slice's MFMAs run and slice 0 of stage s+1 is read (FP16:
// half of it there, half during the next slice).
//
// Persistent grid: one workgroup per CU walks its tiles (TileDeal: 8 x 4
// blocks of tiles per XCD per round); the stage sequence and the ring run on
// across tile boundaries.  At a tile's end the epilogue loads the scales,
// issues the next DMA stage, then dequantises 32 x 64 blocks through the
// wave's LDS slot and stores 16-byte row vectors.
#include "../common/ee_device.h"
#include "../common/ee_gemm_dev.h"
#include "../common/ee_gemm_seq.h"

#pragma clang fp contract(off)


#define T2_SLOT 4096                      // per-wave epilogue slot (32 x 64 fp16)
#define T2_THREADS 512

// Tile TN columns wide (256 or 128).  Waves: TN = 256: wm = w >> 2, wn = w & 3, 128 x 64
// each (4 x 2 blocks); TN = 128: wm = w >> 1, wn = w & 1, 64 x 64 each (2 x 2 blocks).
template <int TN>
struct G2Geom {
    static constexpr int STAGE = (T2M + TN) * BKB;    // 64 KB or 48 KB
    static constexpr int EPI = 2 * STAGE;             // the ring: two stages
    static constexpr int LDS = EPI + 8 * T2_SLOT;     // 160 KB or 128 KB
    static constexpr int WR = TN == 256 ? 128 : 64;   // rows of a wave's block
    static constexpr int NI = WR / 32;                // its 32-row blocks
    static constexpr int WMS = TN == 256 ? 2 : 1;     // wm = w >> WMS, wn = w & (2^WMS - 1)
    static constexpr int BG = TN / 64;                // B row groups of 8 each wave loads per stage
};

template <int KIND, int SW, class Seq, int TN = 256>
struct G256 {
    typedef G2Geom<TN> GE;
    static constexpr int NI = GE::NI, WR = GE::WR;
    // INT8: 16x16x64 MFMAs on 64-byte slices (PipeI8x16)
    typedef std::conditional_t<KIND == EE_GEMM_I8, PipeI8x16, Pipe<KIND>> P;
    typedef typename P::acc_t acc_t;
    typedef typename P::frag_t frag_t;
    static constexpr int ESZ = (KIND == EE_GEMM_F16) ? 2 : 1;
    static constexpr int NSL = BKB / P::SB;           // K slices per stage: 4 (32-byte slices) or 2 (64-byte)
    // DMA parts of stage s+2 issued in each slice of the window from barrier s+1
    // (slice w = 0: the last slice of stage s; w >= 1: slice w-1 of stage s+1).
    // All four are issued before barrier s+2 waits for them.  With four slices
    // per stage (32-byte slices) they spread over two: 2.5% faster for FP16 at
    // configs 1-2 than all four in the first; with two slices per stage they go
    // in the first (spread, the last loads land late: 3-8% slower).
    static constexpr int dma_count(int w) {
        if constexpr (NSL == 4) {
            constexpr int c[4] = {2, 2, 0, 0};
            return c[w];
        } else {
            return w == 0 ? 4 : 0;
        }
    }
    static constexpr int dma_first(int w) {
        int f = 0;
        for (int i = 0; i < w; ++i) f += dma_count(i);
        return f;
    }
    static_assert(dma_first(NSL) == 4, "every DMA part is issued within its window");

    const EeGemmArgs& g;
    uint8_t* smem;
    const Seq& seq;                                   // tiles of this workgroup: count(), coords(i, m0, n0)
    int M;                                            // rows (counts[tier] when routed)
    int64_t off;                                      // partition slot of row 0 (routed), else 0
    uint32_t lds0;
    int lane, wave, wm, wn;
    int nk, total;                                    // stages per tile, stages of this workgroup
    // DMA cursor: the next stage to issue is (itile, ikt), global number iss;
    // row group q of A (B) of that tile starts at abase + aoff[q] (bbase + boff[q]).
    int iss, itile, ikt;
    bool dmaon;                                       // the stage being issued is still issuing
    const uint8_t* abase;
    const uint8_t* bbase;
    uint32_t aoff[4], boff[GE::BG];
    acc_t acc[NI][2];
    // fragments: A single-buffered (row block i of the next slice is read right
    // after the last MFMA that uses row block i of this one); B double-buffered,
    // except for FP8, whose 32-byte fragments leave room for one B buffer only
    // (its slices run j-major, so each B block is also dead before its reload)
    static constexpr int NB = (P::CPF == 2) ? 1 : 2;
    frag_t fa[NI], fb[NB][2];
    uint32_t fo;                                      // SUB16: byte of row l & 15, chunk (l >> 4) of slice 0

    __device__ __forceinline__ G256(const EeGemmArgs& g_, uint8_t* smem_, const Seq& seq_, int M_, int64_t off_)
        : g(g_), smem(smem_), seq(seq_), M(M_), off(off_) {}

    __device__ __forceinline__ void coords(int i, int& m0, int& n0) const {
        int tm, tn;
        seq.coords(i, tm, tn);
        m0 = tm * T2M;
        n0 = tn * TN;
    }

    // DMA rows of tile i: one global_load_lds_dwordx4 fills 8 LDS rows (1 KB);
    // lane l lands at row 8 * grp + l / 8, physical chunk l % 8, which holds
    // logical chunk (l % 8) ^ swz(row).  Wave w fills row groups 4w .. 4w+3 of
    // A and of B (rows are clamped: out-of-range rows load a valid row whose
    // results are never stored).
    // Un-routed: offsets from the tile's first row.  Routed (g.counts): A row m
    // is a[a_idx[off + m]] or a[off + m], offsets from the operand's start (the
    // launcher checks that they fit 32 bits).
    __device__ __forceinline__ void dma_tile(int i) {
        int m0, n0;
        coords(i, m0, n0);
        // SUB16: the lane index through an empty asm, so that the lane-dependent
        // parts of the offsets are computed here rather than held across the K
        // loop (the 16x16 form's registers have no room for them)
        int lane = this->lane;
        if constexpr (P::SUB16) asm volatile("" : "+v"(lane));
        constexpr bool routed = Seq::ROUTED;
        abase = (const uint8_t*)g.a + (routed ? 0 : (int64_t)m0 * g.lda * ESZ);
        bbase = (const uint8_t*)g.b + (int64_t)n0 * g.ldb * ESZ;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = (wave * 4 + q) * 8 + (lane >> 3);
            const int lchunk = (lane & 7) ^ swz(r);
            const int m = min(m0 + r, M - 1);
            const int64_t ar = !routed ? (int64_t)(m - m0) : Seq::GATHER ? (int64_t)g.a_idx[off + m] : off + m;
            if constexpr (P::SUB16) {
                // the low 32 bits in 32-bit registers (the launcher checks that the
                // offsets fit): a 64-bit multiply-add would hold register pairs
                uint32_t pr = (uint32_t)ar * (uint32_t)(g.lda * ESZ);
                asm volatile("" : "+v"(pr));
                aoff[q] = pr + (uint32_t)(lchunk * 16);
            } else {
                aoff[q] = (uint32_t)(ar * g.lda * ESZ + lchunk * 16);
            }
        }
#pragma unroll
        for (int q = 0; q < GE::BG; ++q) {
            const int r = (wave * GE::BG + q) * 8 + (lane >> 3);
            const int lchunk = (lane & 7) ^ swz(r);   // swz(T2M + r) == swz(r)
            const int n = min(n0 + r, g.N - 1) - n0;
            if constexpr (P::SUB16) {
                uint32_t pr = (uint32_t)n * (uint32_t)(g.ldb * ESZ);
                asm volatile("" : "+v"(pr));
                boff[q] = pr + (uint32_t)(lchunk * 16);
            } else {
                boff[q] = (uint32_t)(n * g.ldb * ESZ + lchunk * 16);
            }
        }
    }
    // Part p (0..3) of the next stage: A row group 4w+p and, for p < BG, B row group BG w + p.
    __device__ __forceinline__ void issue_part(int p) {
        if (p == 0 && ikt == nk) {
            ++itile;
            ikt = 0;
            dma_tile(itile);
        }
        const uint32_t s = lds0 + (uint32_t)((iss & 1) * GE::STAGE);
        const uint32_t kb = (uint32_t)ikt * BKB;
        const int grp = wave * 4 + p;
        dma16s(abase, aoff[p] + kb, s + grp * 8 * BKB);
        if (p < GE::BG) dma16s(bbase, boff[p] + kb, s + (T2M + (wave * GE::BG + p) * 8) * BKB);
        if (p == 3) {
            ++ikt;
            ++iss;
        }
    }
    __device__ __forceinline__ void issue_stage() {
#pragma unroll
        for (int p = 0; p < 4; ++p) issue_part(p);
    }

    // Fragments of K slice sl of the stage at st: lane l reads row (l & 31) of
    // each 32-row block, chunk sl * SB/16 + (l >> 5) * LSTEP (and the chunk CSTEP
    // after it when CPF == 2).
    __device__ __forceinline__ void rd(const uint8_t* st, int sl, frag_t& f, int row) const {
        const int c0 = sl * (P::SB / 16) + (lane >> 5) * P::LSTEP;
        if constexpr (P::CPF == 1) {
            f = *(const u32x4*)(st + lds_off(row, c0));
        } else {
            const u32x4 x0 = *(const u32x4*)(st + lds_off(row, c0)), x1 = *(const u32x4*)(st + lds_off(row, c0 + P::CSTEP));
            f = i32x8{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
        }
    }
    // 16x16x64 fragments (SUB16) of the 32-row block at row0 (a multiple of 16, so
    // swz(row0 + x) == swz(x)): rows row0 + (l & 15) and row0 + 16 + (l & 15),
    // chunk 4 sl + (l >> 4), at byte fo ^ 64 sl of the block's first row and 2 KB on
    // (chunk 4 + c ^ s == (c ^ s) ^ 4 for c < 4: slice 1's offset flips bit 6).
    __device__ __forceinline__ void rd16(const uint8_t* st, int sl, frag_t& f, int row0) const {
        // (the offset through an empty asm: each read adds it to the block's base
        // instead of the compiler holding a hoisted address per block and buffer)
        uint32_t o = fo ^ (uint32_t)(sl << 6);
        asm volatile("" : "+v"(o));
        const uint8_t* p = st + row0 * BKB + o;
        f.h[0] = *(const i32x4*)p;
        f.h[1] = *(const i32x4*)(p + 16 * BKB);
    }
    __device__ __forceinline__ void rd_a(const uint8_t* st, int sl, int i) {
        if constexpr (P::SUB16) rd16(st, sl, fa[i], wm * WR + i * 32);
        else rd(st, sl, fa[i], wm * WR + i * 32 + (lane & 31));
    }
    __device__ __forceinline__ void rd_b(const uint8_t* st, int sl, int buf, int j) {
        if constexpr (P::SUB16) rd16(st, sl, fb[buf % NB][j], T2M + wn * 64 + j * 32);
        else rd(st, sl, fb[buf % NB][j], T2M + wn * 64 + j * 32 + (lane & 31));
    }
    // all fragments of slice sl into fa and fb[buf]
    __device__ __forceinline__ void rd_all(const uint8_t* st, int sl, int buf) {
        rd_a(st, sl, 0);
        rd_b(st, sl, buf, 0);
        rd_b(st, sl, buf, 1);
#pragma unroll
        for (int i = 1; i < NI; ++i) rd_a(st, sl, i);
    }

#define G2_SB() __builtin_amdgcn_sched_barrier(0)
    // Part p0 + k of the stage being issued, at the k-th DMA position of a slice
    // (k < np), while dmaon.
    __device__ __forceinline__ void dma_at(int k, int p0, int np) {
        if (k < np && dmaon) issue_part(p0 + k);
    }
    // The 8 MFMAs of the current slice (B fragments in buffer C), interleaved
    // with the reads of the next slice (from stage rs, slice rsl, when RD: B into
    // buffer 1 - C, A row block i right after its last MFMA here) and DMA parts
    // p0 .. p0+np-1 of the stage being issued.
    template <int C, bool RD>
    __device__ __forceinline__ void slice(const uint8_t* rs, int rsl, int p0, int np) {
        if constexpr (NB == 1) {
            if constexpr (NI == 2) slice_j2(RD, rs, rsl, p0, np);
            else slice_j(RD, rs, rsl, p0, np);
            return;
        } else if constexpr (NI == 2) {
            slice2<C>(RD, rs, rsl, p0, np);
            return;
        }
        constexpr int N = (1 - C) % NB;
        acc[0][0] = P::mma(fb[C][0], fa[0], acc[0][0]);
        G2_SB();
        if (RD) { rd_b(rs, rsl, N, 0); rd_b(rs, rsl, N, 1); }
        G2_SB();
        acc[0][1] = P::mma(fb[C][1], fa[0], acc[0][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 0);
        G2_SB();
        acc[1][0] = P::mma(fb[C][0], fa[1], acc[1][0]);
        G2_SB();
        dma_at(0, p0, np);
        G2_SB();
        acc[1][1] = P::mma(fb[C][1], fa[1], acc[1][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 1);
        dma_at(1, p0, np);
        G2_SB();
        acc[2][0] = P::mma(fb[C][0], fa[2], acc[2][0]);
        G2_SB();
        dma_at(2, p0, np);
        G2_SB();
        acc[2][1] = P::mma(fb[C][1], fa[2], acc[2][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 2);
        dma_at(3, p0, np);
        G2_SB();
        acc[3][0] = P::mma(fb[C][0], fa[3], acc[3][0]);
        G2_SB();
        acc[3][1] = P::mma(fb[C][1], fa[3], acc[3][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 3);
        G2_SB();
    }

    // Two row blocks (64 x 64 per wave): the same interleave over 4 MFMAs, the four
    // load parts of the next stage after the first two.
    template <int C>
    __device__ __forceinline__ void slice2(bool RD, const uint8_t* rs, int rsl, int p0, int np) {
        constexpr int N = (1 - C) % NB;
        acc[0][0] = P::mma(fb[C][0], fa[0], acc[0][0]);
        G2_SB();
        if (RD) { rd_b(rs, rsl, N, 0); rd_b(rs, rsl, N, 1); }
        G2_SB();
        acc[0][1] = P::mma(fb[C][1], fa[0], acc[0][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 0);
        dma_at(0, p0, np);
        dma_at(1, p0, np);
        G2_SB();
        acc[1][0] = P::mma(fb[C][0], fa[1], acc[1][0]);
        G2_SB();
        dma_at(2, p0, np);
        dma_at(3, p0, np);
        G2_SB();
        acc[1][1] = P::mma(fb[C][1], fa[1], acc[1][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 1);
        G2_SB();
    }
    __device__ __forceinline__ void slice_j2(bool RD, const uint8_t* rs, int rsl, int p0, int np) {
        acc[0][0] = P::mma(fb[0][0], fa[0], acc[0][0]);
        G2_SB();
        acc[1][0] = P::mma(fb[0][0], fa[1], acc[1][0]);
        G2_SB();
        if (RD) rd_b(rs, rsl, 0, 0);
        G2_SB();
        acc[0][1] = P::mma(fb[0][1], fa[0], acc[0][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 0);
        dma_at(0, p0, np);
        dma_at(1, p0, np);
        G2_SB();
        acc[1][1] = P::mma(fb[0][1], fa[1], acc[1][1]);
        G2_SB();
        if (RD) { rd_a(rs, rsl, 1); rd_b(rs, rsl, 0, 1); }
        dma_at(2, p0, np);
        dma_at(3, p0, np);
        G2_SB();
    }

    // The single-buffer form (FP8): MFMAs j-major; B block 0 is reread after
    // the fourth MFMA, A block i and B block 1 after their last use.
    __device__ __forceinline__ void slice_j(bool RD, const uint8_t* rs, int rsl, int p0, int np) {
        acc[0][0] = P::mma(fb[0][0], fa[0], acc[0][0]);
        G2_SB();
        acc[1][0] = P::mma(fb[0][0], fa[1], acc[1][0]);
        G2_SB();
        acc[2][0] = P::mma(fb[0][0], fa[2], acc[2][0]);
        G2_SB();
        acc[3][0] = P::mma(fb[0][0], fa[3], acc[3][0]);
        G2_SB();
        if (RD) rd_b(rs, rsl, 0, 0);
        G2_SB();
        acc[0][1] = P::mma(fb[0][1], fa[0], acc[0][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 0);
        dma_at(0, p0, np);
        G2_SB();
        acc[1][1] = P::mma(fb[0][1], fa[1], acc[1][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 1);
        dma_at(1, p0, np);
        G2_SB();
        acc[2][1] = P::mma(fb[0][1], fa[2], acc[2][1]);
        G2_SB();
        if (RD) rd_a(rs, rsl, 2);
        dma_at(2, p0, np);
        G2_SB();
        acc[3][1] = P::mma(fb[0][1], fa[3], acc[3][1]);
        G2_SB();
        if (RD) { rd_a(rs, rsl, 3); rd_b(rs, rsl, 0, 1); }
        dma_at(3, p0, np);
        G2_SB();
    }

    // Stage cs: slices 0 .. NSL-1 from buffer cs & 1; the stage starts with its
    // slice-0 fragments in fa / fb[0] (NSL is even).  Not the tile's last stage
    // (LAST = false): before the last slice's MFMAs, barrier cs+1, slice 0 of
    // stage cs+1 is read and stage cs+2 starts into this stage's buffer (when
    // dma2; its parts go out over the slices dma_count gives).  The tile's last
    // stage reads nothing for the next one: the epilogue and the tile change do
    // that (run()).
    template <bool LAST>
    __device__ __forceinline__ void stage(int cs, bool dma2) {
        const uint8_t* st = smem + (cs & 1) * GE::STAGE;
#pragma unroll
        for (int h = 0; h + 1 < NSL; h += 2) {
            slice<0, true>(st, h + 1, dma_first(h + 1), dma_count(h + 1));
            if (h + 2 < NSL) slice<1, true>(st, h + 2, dma_first(h + 2), dma_count(h + 2));
        }
        if (!LAST) {
            G2_SB();
            WAITCNT_VM(0);
            WAITCNT_LGKM0();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();             // barrier cs+1: stage cs+1 landed, stage cs read
            asm volatile("" ::: "memory");
            dmaon = dma2;
            slice<1, true>(smem + ((cs + 1) & 1) * GE::STAGE, 0, dma_first(0), dma_count(0));
        } else {
            slice<1, false>(st, 0, 0, 0);
            dmaon = false;
        }
    }

    // Dequantise and store the tile (m0, n0) from acc through the wave's LDS
    // slot.  Scales are loaded first; the wait for them also covers this wave's
    // part of the next DMA stage (the one barrier cs+1 will publish).
    __device__ __forceinline__ void epilogue32(int m0, int n0) {
        const int N = g.N;
        // The lane index through an empty asm: the epilogue's addresses are then
        // computed here instead of being hoisted out of the tile loop, where they
        // would hold ~20 VGPRs across the K loop.
        int lane = this->lane;
        asm volatile("" : "+v"(lane));
        f32x4 bs[2][4] = {};
        float as[NI] = {};
        if constexpr (KIND != EE_GEMM_F16) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int n = n0 + wn * 64 + j * 32 + 8 * q + 4 * (lane >> 5);
                    bs[j][q] = (n < N) ? *(const f32x4*)(g.b_scale + n) : f32x4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int m = m0 + wm * WR + i * 32 + (lane & 31);
                as[i] = (m < M) ? g.a_scale[off + m] : 0.0f;
            }
        }
        // C row of wave row r (0..127) of the tile, -1 beyond M.  Routed rows are
        // scattered through c_idx: lane l loads the C rows of wave rows l and
        // 64 + l here, with the scales, and each store round fetches its row
        // from the lane that holds it (ds_bpermute: a cross-lane move, no LDS
        // memory), two registers instead of a 16-entry table.
        int32_t cr[WR / 64];
        if constexpr (Seq::ROUTED) {
#pragma unroll
            for (int h = 0; h < WR / 64; ++h) {
                const int m = m0 + wm * WR + h * 64 + lane;
                cr[h] = (m < M) ? (g.c_idx ? g.c_idx[off + m] : m) : -1;
            }
        }
        auto crow_of = [&](int r) -> int32_t {
            if constexpr (Seq::ROUTED) {
                return __builtin_amdgcn_ds_bpermute((r & 63) << 2, cr[r >> 6]);
            } else {
                const int m = m0 + wm * WR + r;
                return m < M ? m : -1;
            }
        };
        WAITCNT_VM(0);
        asm volatile("" ::: "memory");
        uint8_t* slot = smem + GE::EPI + wave * T2_SLOT;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int mb = m0 + wm * WR + i * 32;     // first row of this 32 x 64 block
            const int nb = n0 + wn * 64;
            if constexpr (KIND == EE_GEMM_I8) {
                if (!Seq::ROUTED && g.acc) {          // debug output: int32 accumulators, direct stores
                    const int m = mb + (lane & 31);
                    if (m < M) {
#pragma unroll
                        for (int j = 0; j < 2; ++j)
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const int n = nb + j * 32 + 8 * q + 4 * (lane >> 5);
                                if (n < N)
                                    *(i32x4*)(g.acc + (int64_t)m * g.ldc + n) =
                                        i32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                              acc[i][j][4 * q + 3]};
                            }
                    }
                }
            }
            if constexpr (SW) {
                // columns j = 0 (gate) and j = 1 (up) of the same 32 outputs -> act
                // columns nb / 2 .. +31: fp16(fp16(silu(gate)) * up)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float gv[4], uv[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        gv[r] = deq<KIND>(acc[i][0][4 * q + r], as[i], bs[0][q][r]);
                        uv[r] = deq<KIND>(acc[i][1][4 * q + r], as[i], bs[1][q][r]);
                    }
                    *(u32x2*)(slot + lds_off(lane & 31, q) + (lane >> 5) * 8) =
                        u32x2{silu_mul2(pack_f16x2(gv[0], gv[1]), pack_f16x2(uv[0], uv[1])),
                              silu_mul2(pack_f16x2(gv[2], gv[3]), pack_f16x2(uv[2], uv[3]))};
                }
                const int na = N >> 1;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int rl = k * 16 + (lane >> 2), ch = lane & 3;
                    const u32x4 v = *(const u32x4*)(slot + lds_off(rl, ch));
                    const int n = (nb >> 1) + ch * 8;
                    const int32_t crow = crow_of(i * 32 + rl);
                    if (crow >= 0 && n < na) store_row16(g.c + (int64_t)crow * g.ldc + n, v, true);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int cl = j * 32 + 8 * q + 4 * (lane >> 5);
                        float o[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if constexpr (KIND == EE_GEMM_F16) o[r] = acc[i][j][4 * q + r];
                            else o[r] = deq<KIND>(acc[i][j][4 * q + r], as[i], bs[j][q][r]);
                        }
                        // row (lane & 31): 128 bytes = 8 chunks of 16; column cl is chunk cl / 8, half (cl / 4) & 1
                        *(u32x2*)(slot + lds_off(lane & 31, cl >> 3) + ((cl >> 2) & 1) * 8) =
                            u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
                    }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int rl = k * 8 + (lane >> 3), ch = lane & 7;
                    const u32x4 v = *(const u32x4*)(slot + lds_off(rl, ch));
                    const int n = nb + ch * 8;
                    const int32_t crow = crow_of(i * 32 + rl);
                    if (crow >= 0 && n < N) store_row16(g.c + (int64_t)crow * g.ldc + n, v, n + 8 <= N);
                }
            }
        }
    }

    // epilogue32 for the 16x16 accumulator layout (SUB16): quarter q of block (i, j)
    // holds rows row_of(q) and columns j * 32 + col_of(q) .. +3 of the block, whose
    // scales are bs[j][cq(q)] and as[rq(q)].  Lane l loads the row scales of wave
    // rows l and 64 + l (with the next stage's wait) and each block's lanes fetch
    // theirs from the lanes holding them (ds_bpermute).
    __device__ __forceinline__ void epilogue16(int m0, int n0) {
        G2_SB();                                      // nothing of it moves up among the last MFMAs
        const int N = g.N;
        int lane = this->lane;                        // (not hoisted out of the tile loop)
        asm volatile("" : "+v"(lane));
        f32x4 bs[2][P::NCQ] = {};
        float asv[WR / 64] = {};
        if constexpr (KIND != EE_GEMM_F16) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int c = 0; c < P::NCQ; ++c) {      // column group c: quarters 2c, 2c + 1
                    const int n = n0 + wn * 64 + j * 32 + P::col_of(2 * c, lane);
                    bs[j][c] = (n < N) ? *(const f32x4*)(g.b_scale + n) : f32x4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
            for (int h = 0; h < WR / 64; ++h) {
                const int m = m0 + wm * WR + h * 64 + lane;
                asv[h] = (m < M) ? g.a_scale[off + m] : 0.0f;
            }
        }
        int32_t cr[WR / 64];                          // C rows, as in epilogue32
        if constexpr (Seq::ROUTED) {
#pragma unroll
            for (int h = 0; h < WR / 64; ++h) {
                const int m = m0 + wm * WR + h * 64 + lane;
                cr[h] = (m < M) ? (g.c_idx ? g.c_idx[off + m] : m) : -1;
            }
        }
        auto crow_of = [&](int r) -> int32_t {
            if constexpr (Seq::ROUTED) {
                return __builtin_amdgcn_ds_bpermute((r & 63) << 2, cr[r >> 6]);
            } else {
                const int m = m0 + wm * WR + r;
                return m < M ? m : -1;
            }
        };
        WAITCNT_VM(0);
        asm volatile("" ::: "memory");
        uint8_t* slot = smem + GE::EPI + wave * T2_SLOT;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int mb = m0 + wm * WR + i * 32;     // first row of this 32 x 64 block
            const int nb = n0 + wn * 64;
            float as[P::NRQ] = {};
            if constexpr (KIND != EE_GEMM_F16)
#pragma unroll
                for (int h = 0; h < P::NRQ; ++h) {
                    const int r = i * 32 + P::row_of(h, lane);
                    as[h] = __int_as_float(__builtin_amdgcn_ds_bpermute((r & 63) << 2, __float_as_int(asv[r >> 6])));
                }
            if constexpr (KIND == EE_GEMM_I8) {
                if (!Seq::ROUTED && g.acc) {          // debug output: int32 accumulators, direct stores
#pragma unroll
                    for (int j = 0; j < 2; ++j)
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
                // gate (j = 0) and up (j = 1) of the same 32 outputs -> act columns nb / 2 .. +31
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float gv[4], uv[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        gv[r] = deq<KIND>(acc[i][0][4 * q + r], as[P::rq(q)], bs[0][P::cq(q)][r]);
                        uv[r] = deq<KIND>(acc[i][1][4 * q + r], as[P::rq(q)], bs[1][P::cq(q)][r]);
                    }
                    const int ca = P::col_of(q, lane);
                    *(u32x2*)(slot + lds_off(P::row_of(q, lane), ca >> 3) + ((ca >> 2) & 1) * 8) =
                        u32x2{silu_mul2(pack_f16x2(gv[0], gv[1]), pack_f16x2(uv[0], uv[1])),
                              silu_mul2(pack_f16x2(gv[2], gv[3]), pack_f16x2(uv[2], uv[3]))};
                }
                const int na = N >> 1;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int rl = k * 16 + (lane >> 2), ch = lane & 3;
                    const u32x4 v = *(const u32x4*)(slot + lds_off(rl, ch));
                    const int n = (nb >> 1) + ch * 8;
                    const int32_t crow = crow_of(i * 32 + rl);
                    if (crow >= 0 && n < na) store_row16(g.c + (int64_t)crow * g.ldc + n, v, true);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int cl = j * 32 + P::col_of(q, lane);
                        float o[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if constexpr (KIND == EE_GEMM_F16) o[r] = acc[i][j][4 * q + r];
                            else o[r] = deq<KIND>(acc[i][j][4 * q + r], as[P::rq(q)], bs[j][P::cq(q)][r]);
                        }
                        *(u32x2*)(slot + lds_off(P::row_of(q, lane), cl >> 3) + ((cl >> 2) & 1) * 8) =
                            u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
                    }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int rl = k * 8 + (lane >> 3), ch = lane & 7;
                    const u32x4 v = *(const u32x4*)(slot + lds_off(rl, ch));
                    const int n = nb + ch * 8;
                    const int32_t crow = crow_of(i * 32 + rl);
                    if (crow >= 0 && n < N) store_row16(g.c + (int64_t)crow * g.ldc + n, v, n + 8 <= N);
                }
            }
        }
    }

    __device__ __forceinline__ void epilogue(int m0, int n0) {
        if constexpr (P::SUB16) epilogue16(m0, n0);
        else epilogue32(m0, n0);
    }

    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = acc_t{};
    }

    // Barrier cs (each wave has waited for its part of stage cs and finished its
    // reads of stage cs-1), then stage cs+1 into the buffer stage cs-1 used, then
    // slice 0 of stage cs.
    __device__ __forceinline__ void enter(int cs) {
        dmaon = false;
        WAITCNT_LGKM0();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (cs + 1 < total && iss == cs + 1) issue_stage();
        rd_all(smem + (cs & 1) * GE::STAGE, 0, 0);
    }

    __device__ __forceinline__ void run() {
        const int tid = threadIdx.x;
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        wm = wave >> GE::WMS;
        wn = wave & ((1 << GE::WMS) - 1);
        if constexpr (P::SUB16) fo = lds_off(lane & 15, lane >> 4);
        const int ntiles = seq.count();
        if (ntiles <= 0) return;                      // whole workgroup, before any barrier
        nk = (int)((int64_t)g.K * ESZ / BKB);         // K * ESZ is a multiple of BKB here
        total = ntiles * nk;
        lds0 = lds_addr(smem);
        iss = 0;
        itile = -1;
        ikt = nk;
        dmaon = false;
        issue_stage();                                // stage 0 -> buffer 0
        if (total > 1) {
            issue_stage();                            // stage 1 -> buffer 1
            // stage 0 landed; stage 1's loads (4 A + BG B per wave) may stay in flight
            if constexpr (GE::BG == 4) WAITCNT_VM(8);
            else WAITCNT_VM(6);
        } else {
            WAITCNT_VM(0);
        }
        enter(0);
        int cs = 0;
        for (int t = 0; t < ntiles; ++t) {
            zero();
            for (int kt = 0; kt + 1 < nk; ++kt, ++cs) stage<false>(cs, cs + 2 < total);
            stage<true>(cs, false);
            int m0, n0;
            coords(t, m0, n0);
            epilogue(m0, n0);
            ++cs;
            if (cs < total) enter(cs);
        }
    }
};

// A grid of 256 x 256 tiles whose last round is at most half full (config 2:
// 896 tiles on 256 CUs, 3.5 rounds) runs that round as 256 x 128 halves, one
// per workgroup: the full rounds first, then the halves, in the same tile
// order (both halves of a tile on one XCD).  The halves sum K in the same
// order, so the output bits do not change.
template <int KIND, int SW, int TN>
EE_DEV void gemm256(const EeGemmArgs& g) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[G2Geom<TN>::LDS];
    const int b = (int)blockIdx.x, G = (int)gridDim.x;
    const Seq256<TN> seq(g, b, G);
    // (not for FP16 SwiGLU: a second pipeline instance in the kernel takes its
    // registers past 256; its grids run the last round as 256 x 256 tiles)
    if constexpr (TN == 256 && !(SW && KIND == EE_GEMM_F16)) {
        const int nT = seq.d.nA, full = nT / G, rem = nT - full * G;
        if (rem > 0 && 2 * rem <= G) {
            if (full > 0) {
                const Seq256<TN> s1(g, b, G, full);
                G256<KIND, SW, Seq256<TN>, TN> k(g, smem, s1, g.M, 0);
                k.run();
                __syncthreads();                      // every wave's reads of the ring and its slot are done
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
                G256<KIND, SW, Seq256Half, 128> k(g, smem, sh, g.M, 0);
                k.run();
            }
            return;
        }
    }
    G256<KIND, SW, Seq256<TN>, TN> k(g, smem, seq, g.M, 0);
    k.run();
}

// ---------------------------------------------------------------- routed
// The routed linear's three tier GEMMs as one persistent grid on 256 x 256
// tiles.  Tier t owns ceil(counts[t] / 256) M-tiles of its partition slots.
// FP16 (W8A16) tiles, twice the work of a 1-byte tile at the same K, are
// dealt first, round robin; the 1-byte tiles -- all INT8 tiles, then all FP8
// tiles, each tier in bands of 8 M-tiles along N -- follow in TileDeal rounds
// (workgroups holding an extra FP16 tile skip the first two).  A workgroup
// then runs its tiles in three phases (FP16, INT8, FP8), one G256 pipeline
// each; the tier order of the 1-byte list makes each phase a contiguous run.
// Every tile sums K in the order of the un-routed kernels, so routed rows equal
// ee_gemm's rows of the same tier bit for bit.

template <int SW, int TN>
EE_DEV void gemm256_routed(const EeRoutedGemmArgs& r) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[G2Geom<TN>::LDS];
    const int32_t* counts = r.t[0].counts;
    const int c0 = counts[0], c1 = counts[1], c2 = counts[2];
    const int T0 = (c0 + T2M - 1) / T2M, T1 = (c1 + T2M - 1) / T2M, T2 = (c2 + T2M - 1) / T2M;
    const int N = r.t[0].N;
    const int nN = (N + TN - 1) / TN;
    const int b = (int)blockIdx.x, G = (int)gridDim.x;
    // W8A16 tiles: 256 x TN, or 256 x 128 halves where that shortens the estimated
    // makespan (in 1-byte-tile units: a full W8A16 tile costs 2, a half ~1.15, as
    // measured).  A few FP16 rows -- one M-tile per column, as at config 4 -- then
    // no longer set the grid's length at twice a 1-byte tile's time.  Every
    // workgroup reads the same counts, so every workgroup makes the same choice.
    int nF = T2 * nN, skip = 2;
    bool half = false;
    if constexpr (TN == 256) {
        const int nFh = T2 * ((N + 127) / 128), nA = (T0 + T1) * nN;
        const int full20 = 20 * max(2 * ((nF + G - 1) / G), (2 * nF + nA + G - 1) / G);
        const int half20 = max(23 * ((nFh + G - 1) / G), 20 * (((23 * nFh + 19) / 20 + nA + G - 1) / G));
        if (nF > 0 && half20 < full20) {
            half = true;
            nF = nFh;
            skip = 1;
        }
    }
    const TileDeal d(T0 + T1, nN, nF, b, G, skip);
    // phase FP16
    const SeqRF sf{b, G, b < nF ? (nF - b + G - 1) / G : 0, T2};
    if (sf.n > 0) {
        if (half) {
            G256<EE_GEMM_F16, SW, SeqRF, 128> k(r.t[2], smem, sf, c2, (int64_t)c0 + c1);
            k.run();
        } else {
            G256<EE_GEMM_F16, SW, SeqRF, TN> k(r.t[2], smem, sf, c2, (int64_t)c0 + c1);
            k.run();
        }
    }
    // the 1-byte tiles: the INT8 ones come first (logical index < T0 * nN)
    const int n1 = d.count();
    int ni8 = 0;
    while (ni8 < n1 && d.tile_index(d.first_round + ni8) < T0 * nN) ++ni8;
    if (ni8 > 0) {
        if (sf.n > 0) __syncthreads();                // the previous phase's LDS reads and DMA are done
        const SeqR1 s8{d, 0, ni8, T0, T1, nN};
        G256<EE_GEMM_I8, SW, SeqR1, TN> k(r.t[0], smem, s8, c0, 0);
        k.run();
    }
    if (n1 > ni8) {
        if (sf.n > 0 || ni8 > 0) __syncthreads();
        const SeqR1 s8{d, ni8, n1 - ni8, T0, T1, nN};
        G256<EE_GEMM_F8, SW, SeqR1, TN> k(r.t[1], smem, s8, c1, c0);
        k.run();
    }
}

#define EE_G256_ENTRY(NAME, KIND, TN)                                                                       \
    extern "C" __global__ void __launch_bounds__(T2_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))   \
    NAME(EeGemmArgs g) { gemm256<KIND, 0, TN>(g); }                                                       \
    extern "C" __global__ void __launch_bounds__(T2_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))   \
    NAME##_swiglu(EeGemmArgs g) { gemm256<KIND, 1, TN>(g); }
EE_G256_ENTRY(eek_gemm256_i8, EE_GEMM_I8, 256)
EE_G256_ENTRY(eek_gemm256_f8, EE_GEMM_F8, 256)
EE_G256_ENTRY(eek_gemm256_f16, EE_GEMM_F16, 256)
// 256 x 128 tiles
EE_G256_ENTRY(eek_gemm256n128_i8, EE_GEMM_I8, 128)
EE_G256_ENTRY(eek_gemm256n128_f8, EE_GEMM_F8, 128)
EE_G256_ENTRY(eek_gemm256n128_f16, EE_GEMM_F16, 128)
#define EE_G256_ROUTED_ENTRY(NAME, TN)                                                                      \
    extern "C" __global__ void __launch_bounds__(T2_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))   \
    NAME(EeRoutedGemmArgs r) { gemm256_routed<0, TN>(r); }                                                \
    extern "C" __global__ void __launch_bounds__(T2_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))   \
    NAME##_swiglu(EeRoutedGemmArgs r) { gemm256_routed<1, TN>(r); }
EE_G256_ROUTED_ENTRY(eek_gemm256_routed, 256)
EE_G256_ROUTED_ENTRY(eek_gemm256n128_routed, 128)
