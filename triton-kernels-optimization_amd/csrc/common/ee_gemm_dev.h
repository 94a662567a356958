// ee_gemm_dev.h -- building blocks shared by the MFMA GEMM kernels (gfx950):
// the swizzled 128-byte LDS rows, the direct-to-LDS DMA and its waits, the
// MFMA shapes of the three tiers, the dequantising arithmetic of the
// epilogues and the XCD-aware deal of tiles to persistent workgroups.
#pragma once
#include <type_traits>

#include "ee_device.h"

// Every epilogue multiply is its own rounded f32 operation, as in the reference.
#pragma clang fp contract(off)

#define BKB 128                         // K bytes per LDS stage row

// 16-byte chunk c of LDS row r sits at chunk c ^ ((r >> 1) & 7).  gfx950's LDS
// serves a ds_read_b128 in passes of 16 lanes over 64 banks: the 16 rows of a
// pass then land on 16 distinct (row parity, chunk) bank groups.
EE_DEV int swz(int row) { return (row >> 1) & 7; }
EE_DEV uint32_t lds_off(int row, int chunk) { return (uint32_t)(row * BKB + ((chunk ^ swz(row)) << 4)); }

// 64-byte LDS rows (int8 W8A16 weight codes, 64 K elements per stage): chunk c
// of row r at chunk c ^ ((r >> 2) & 3), so that 16 rows x two 8-byte halves of
// a chunk pair (a ds_read_b64 pass of 32 lanes) fall on 32 distinct bank pairs,
// as do 16 rows of one chunk for a ds_read_b128 pass.
EE_DEV int swz64(int row) { return (row >> 2) & 3; }

EE_DEV i32x4 as_i32x4(u32x4 v) { return __builtin_bit_cast(i32x4, v); }
EE_DEV f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }

#define GPTR(p) ((const void __attribute__((address_space(1)))*)(p))
#define LPTR(p) ((void __attribute__((address_space(3)))*)(p))

// 16 bytes per lane from global memory straight into LDS at lds_base + 16 * lane
// (lds_base wave-uniform).  Issued as inline asm so that the compiler's wait
// model contains only the kernel's ds_reads (an LDS DMA it can see makes it
// fall back to waiting for every outstanding LDS read); the kernel tracks these
// loads itself with explicit vmcnt waits before each stage barrier.
EE_DEV void dma16(const uint8_t* gptr, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_base), "v"(gptr) : "memory", "m0");
}
EE_DEV uint32_t lds_addr(const uint8_t* p) { return (uint32_t)(uintptr_t)LPTR(p); }
// 4 bytes per lane from global memory into LDS at lds_base + 4 * lane (per-row
// scales and row indices of a tile, staged beside its operands).
EE_DEV void dma4(const void* gptr, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds_base), "v"(gptr) : "memory", "m0");
}
// The same load with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane
// byte offset (one VGPR per row group instead of a 64-bit address pair).
EE_DEV void dma16s(const uint8_t* sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_base), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt 7 << 4 |
// lgkmcnt 15 << 8 | vmcnt[5:4] << 14).
#define WAITCNT_VM(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14)))
// s_waitcnt lgkmcnt(0) with vmcnt and expcnt left unconstrained.
#define WAITCNT_LGKM0() __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14))

// ---------------------------------------------------------------------------
// Pipelined kernels: 32x32 blocks of C, K stages split into slices of one
// MFMA depth, fragments of slice s+1 read from LDS while the MFMAs of slice s
// run.  A block is one 32x32 MFMA per slice, or four 16x16 ones (PipeI8x16).
template <int KIND> struct Pipe;
// Where a lane's accumulators sit in its 32x32 block: registers 4q .. 4q+3 hold
// rows (A side, m) row_of(q, l) and columns (B side, n) col_of(q, l) .. +3.
// A lane's quarters span NRQ distinct rows (quarter q: the rq(q)-th) and NCQ
// distinct column groups (the cq(q)-th), which size the epilogue's scales.
// 32x32 MFMAs: every register of lane l is row l & 31; columns 8q + 4 (l >> 5).
struct Lay32 {
    static constexpr bool SUB16 = false;
    static constexpr int NRQ = 1, NCQ = 4;
    static EE_DEV int rq(int) { return 0; }
    static EE_DEV int cq(int q) { return q; }
    static EE_DEV int row_of(int, int lane) { return lane & 31; }
    static EE_DEV int col_of(int q, int lane) { return 8 * q + 4 * (lane >> 5); }
};
// 16x16 MFMAs on 64-byte K slices (INT8 16x16x64 i8, FP16 16x16x32 f16): a
// 32x32 block of a slice is four of them, the same MFMA time as the 32x32
// forms.  Fragment half h holds rows 16h + (l & 15) of the block, K bytes
// 16 (l >> 4) .. +15 of the slice, for A and B alike; accumulator quarter q is
// the 16 x 16 sub-block of A half q & 1 and B half q >> 1, lane l holding its
// row l & 15 and columns 4 (l >> 4) .. +3.  Measured on MI355X (timing-only
// fragment-read + MFMA loops: the same clocks per iteration either way), the 16x16 forms
// run at a 9-13% higher shader clock under the power limit than the 32x32
// forms of the same work.
struct Lay16 {
    static constexpr bool SUB16 = true;
    static constexpr int NRQ = 2, NCQ = 2;
    static EE_DEV int rq(int q) { return q & 1; }
    static EE_DEV int cq(int q) { return q >> 1; }
    static EE_DEV int row_of(int q, int lane) { return (q & 1) * 16 + (lane & 15); }
    static EE_DEV int col_of(int q, int lane) { return (q >> 1) * 16 + 4 * (lane >> 4); }
};
// The four quarters of one block's accumulators; element e is register e & 3 of quarter e >> 2.
struct I32x4x4 {
    i32x4 q[4];
    __device__ __forceinline__ int32_t operator[](int e) const { return q[e >> 2][e & 3]; }
};
struct F32x4x4 {
    f32x4 q[4];
    __device__ __forceinline__ float operator[](int e) const { return q[e >> 2][e & 3]; }
};
// The two 16-row halves of one fragment.
struct I32x4x2 {
    i32x4 h[2];
};
struct PipeI8x16 : Lay16 {
    static constexpr int SB = 64, CPF = 2, LSTEP = 0, CSTEP = 0;
    typedef I32x4x2 frag_t;
    typedef I32x4x4 acc_t;
    static EE_DEV acc_t mma(const frag_t& b, const frag_t& a, const acc_t& c) {
        acc_t r;
        r.q[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b.h[0], a.h[0], c.q[0], 0, 0, 0);
        r.q[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b.h[0], a.h[1], c.q[1], 0, 0, 0);
        r.q[2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b.h[1], a.h[0], c.q[2], 0, 0, 0);
        r.q[3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b.h[1], a.h[1], c.q[3], 0, 0, 0);
        return r;
    }
};
// INT8 slices are 64 K bytes deep, as FP8's, on four 16x16x64 MFMAs per block
// (int32 sums are exact in any order, so every INT8 kernel has the same bits).
template <> struct Pipe<EE_GEMM_I8> : PipeI8x16 {};
struct PipeF16x16 : Lay16 {                       // 16x16x32 f16: 64 K bytes (32 elements) per slice
    static constexpr int SB = 64, CPF = 2, LSTEP = 0, CSTEP = 0;
    typedef I32x4x2 frag_t;
    typedef F32x4x4 acc_t;
    static EE_DEV f32x4 m16(const i32x4& b, const i32x4& a, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, b), __builtin_bit_cast(f16x8, a), c, 0, 0, 0);
    }
    static EE_DEV acc_t mma(const frag_t& b, const frag_t& a, const acc_t& c) {
        acc_t r;
        r.q[0] = m16(b.h[0], a.h[0], c.q[0]);
        r.q[1] = m16(b.h[0], a.h[1], c.q[1]);
        r.q[2] = m16(b.h[1], a.h[0], c.q[2]);
        r.q[3] = m16(b.h[1], a.h[1], c.q[3]);
        return r;
    }
};
struct PipeF16x32 : Lay32 {                      // 32x32x16 f16: 32 K bytes per slice, 16 B per lane
    static constexpr int SB = 32, CPF = 1, LSTEP = 1, CSTEP = 0;
    typedef u32x4 frag_t;
    typedef f32x16 acc_t;
    static EE_DEV acc_t mma(const frag_t& b, const frag_t& a, const acc_t& c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, b), __builtin_bit_cast(f16x8, a), c, 0, 0, 0);
    }
};
template <> struct Pipe<EE_GEMM_F16> : PipeF16x16 {};
// 32x32 pipes' fragment chunks: lane l reads 16-byte chunk sl * SB/16 + (l >> 5) *
// LSTEP of its row and, when CPF == 2, the chunk CSTEP after it.
template <> struct Pipe<EE_GEMM_F8> : Lay32 {    // 32x32x64 e4m3: 64 K bytes per slice, 32 B per lane
    static constexpr int SB = 64, CPF = 2, LSTEP = 2, CSTEP = 1;
    typedef i32x8 frag_t;
    typedef f32x16 acc_t;
    static EE_DEV acc_t mma(const frag_t& b, const frag_t& a, const acc_t& c) {
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c, 0, 0, 0, 0, 0, 0);
    }
};

// 4 int8 weight codes (one dword) -> 4 fp16 w = fp16(fp16(b) * s) as two f16x2
// words (EE/python/kernels.py:215,233): byte b -> fp16 bits 0x6400 | (b ^ 0x80)
// is 1024 + (b + 128) exactly, minus 1152 is fp16(b); times fp16(scale) in one
// RNE fp16 multiply, which rounds the exact product as eek_pack_b_f16's f32
// product (exact: 8 x 11 significant bits) rounded to fp16 does.
EE_DEV void dq4(uint32_t w, f16x2 s2, uint32_t& lo, uint32_t& hi) {
    const uint32_t x = w ^ 0x80808080u;
    const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
    const f16x2 a = f16x2_from_bits(__builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) - bias;
    const f16x2 b = f16x2_from_bits(__builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) - bias;
    lo = bits_of(a * s2);
    hi = bits_of(b * s2);
}

// Dequantised value of one accumulator, as the fp16 epilogues compute it
// (left-to-right f32 multiplies; W8A16 accumulators are the value).
template <int KIND, typename E>
EE_DEV float deq(E acc, float as, float bs) {
    if constexpr (KIND == EE_GEMM_I8) {
        float v = (float)acc;
        v = v * as;
        return v * bs;
    } else if constexpr (KIND == EE_GEMM_F8) {
        const float v = acc * as;
        return v * bs;
    } else {
        return acc;
    }
}

// One 16-byte store of C or of the SwiGLU output: non-temporal (written once,
// read by a later kernel), 8-byte halves when the row is only 8-byte aligned.
EE_DEV void store_row16(uint16_t* dst, const u32x4& v, bool full) {
    if (full && ((uintptr_t)dst & 15) == 0) {
        __builtin_nontemporal_store(v, (u32x4*)dst);
    } else {
        __builtin_nontemporal_store(u32x2{v[0], v[1]}, (u32x2*)dst);
        if (full) __builtin_nontemporal_store(u32x2{v[2], v[3]}, (u32x2*)(dst + 4));
    }
}

// Tile order and the deal of tiles to workgroups (shared by the plain and the
// routed persistent kernels).  Logical tiles a = 0 .. nA-1 (the 1-byte-operand
// tiles) are ordered in bands of 8 M-tiles walked along N, so 32 consecutive
// tiles form an 8 x 4 block.  They are dealt in rounds: in a round every
// taking workgroup gets one tile, and with G a multiple of 8 workgroup
// b = 8j + x (on XCD x) takes position x * G/8 + j, so each XCD gets 32
// consecutive tiles -- one 8 x 4 block, whose A and B panels its CUs share in
// that XCD's L2.  W8A16 tiles of a routed launch (nF of them, each worth `skip`
// 1-byte tiles: 2 for a 256 x 256 tile, 1 for a 256 x 128 half) are dealt
// first, round robin: workgroups b < rF get qF + 1, the others qF.  The first
// `skip` rounds of 1-byte tiles then go only to workgroups b >= rF, which levels
// the load (a static version of what the hardware dispatcher does for one-tile
// grids).  A grid of one partial round (fewer tiles than workgroups, no W8A16
// tiles) gives each XCD ceil(n / 8) consecutive tiles instead, so that its
// tiles load every XCD's L2 and CUs alike rather than filling the first XCDs
// and leaving the others idle (the routed q/k/v, o and down projections at config
// 4's shapes with INT8 + FP8 rows, 160-170, 136 and 136 tiles of 256 x 256:
// 31.7 -> 28.4, 33.4 -> 30.5 and 69.4 -> 57.5 us).  The last, partial round of a longer grid keeps the full rounds'
// positions: spread there, config 4's gate|up grids measured 2-5% slower.
struct TileDeal {
    int tiles_m, tiles_n, nA, b, G, rF, P, first_round, skip;
    // the rounds of G from logical tile r0 on: `full` full ones, then a partial
    // one of `rem` tiles; this workgroup's position in a full round and in that one
    // (spread over the XCDs where it is the grid's only round)
    int r0, full, rem, pfull, plast;
    __device__ __forceinline__ TileDeal(int tm_count, int tn_count, int nF, int bb, int GG, int sk = 2)
        : tiles_m(tm_count), tiles_n(tn_count), nA(tm_count * tn_count), b(bb), G(GG), skip(sk) {
        rF = nF % G;
        P = G - rF;                                   // workgroups in the first `skip` rounds
        first_round = (rF != 0 && b < rF) ? skip : 0; // heavier workgroups skip those rounds
        r0 = rF == 0 ? 0 : skip * P;
        const int left = max(nA - r0, 0);
        full = left / G;
        rem = left - full * G;
        pfull = pos_in(G);
        plast = rF == 0 && full == 0 ? pos_in(rem) : pfull;
    }
    // Position of this workgroup in a round of n tiles in which all G take part
    // (n >= G: a full round): 0 .. n-1 for the workgroups that take a tile, G for
    // the others.  A full round gives XCD x positions x * G/8 .. +G/8-1; a
    // partial one q = ceil(n / 8) positions per XCD (pairs: q rounded up to even
    // where G/8 allows, so that positions 2i and 2i + 1 -- the two halves of a
    // tile -- share an XCD).
    __device__ __forceinline__ int pos_in(int n, bool pairs = false) const {
        const int per = G >> 3;
        if ((G & 7) != 0) return b;
        int q = n >= G ? per : (max(n, 0) + 7) >> 3;
        if (pairs && (q & 1) && q < per) ++q;
        const int j = b >> 3, p = (b & 7) * q + j;
        return j < q && p < n ? p : G;
    }
    // Position for a halved last round of n2 = 2 rem halves (one per workgroup,
    // positions 0 .. G-1): spread where that round is the grid's only one.
    __device__ __forceinline__ int half_pos(int n2, bool only) const { return only ? pos_in(n2, true) : pfull; }
    __device__ __forceinline__ int tile_index(int round) const {
        if (rF != 0 && round < skip) return round * P + (b - rF);
        const int r = rF == 0 ? round : round - skip;
        return r0 + r * G + (r < full ? pfull : plast);
    }
    __device__ __forceinline__ int count() const {
        // rounds first_round, first_round+1, ... while tile_index(round) < nA
        const int n = full + (plast < rem ? 1 : 0);   // rem == 0: plast == G
        if (rF == 0) return n;
        int k = 0;
        if (first_round == 0) {
            for (int r = 0; r < skip; ++r) k += tile_index(r) < nA;
            if (k < skip) return k;
        }
        return k + n;
    }
    // logical tile a -> (tm, tn): bands of 8 M-tiles, M fastest within a band
    __device__ __forceinline__ void coords(int a, int& tm, int& tn) const {
        const int band = a / (8 * tiles_n);
        const int m_first = band * 8;
        const int gsz = min(tiles_m - m_first, 8);
        const int r = a - band * 8 * tiles_n;
        tm = m_first + r % gsz;
        tn = r / gsz;
    }
};
