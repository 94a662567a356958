// ee_gemm_seq.h -- tile sequences of the persistent 256-row-tile GEMMs (the
// 8-wave and the 4-wave pipelines share them): which tiles a workgroup runs,
// in which order, for plain and routed grids.
#pragma once
#include "ee_gemm_dev.h"

#define T2M 256                           // rows of a tile

// Tiles of an un-routed GEMM for workgroup b of G (TileDeal: 8 x 4 blocks per XCD),
// at most `cap` rounds of them.
template <int TN>
struct Seq256 {
    static constexpr bool ROUTED = false, GATHER = false;
    TileDeal d;
    int cap;
    __device__ __forceinline__ Seq256(const EeGemmArgs& g, int b, int G, int cap_ = 0x7fffffff)
        : d((g.M + T2M - 1) / T2M, (g.N + TN - 1) / TN, 0, b, G), cap(cap_) {}
    __device__ __forceinline__ int count() const { return min(d.count(), cap); }
    __device__ __forceinline__ void coords(int i, int& tm, int& tn) const {
        d.coords(d.tile_index(d.first_round + i), tm, tn);
    }
};
// One 256 x 128 tile (tm, tn in 128-column units), or none.
struct Seq256Half {
    static constexpr bool ROUTED = false, GATHER = false;
    int n, tm, tn;
    __device__ __forceinline__ int count() const { return n; }
    __device__ __forceinline__ void coords(int, int& tm_, int& tn_) const {
        tm_ = tm;
        tn_ = tn;
    }
};

// logical tile a of a tiles_m x tiles_n grid -> (tm, tn): bands of 8 M-tiles, M fastest
EE_DEV void band_coords(int a, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int band = a / (8 * tiles_n);
    const int m_first = band * 8;
    const int gsz = min(tiles_m - m_first, 8);
    const int r = a - band * 8 * tiles_n;
    tm = m_first + r % gsz;
    tn = r / gsz;
}

// The 1-byte tiles lo .. hi-1 of this workgroup's deal (INT8 or FP8 phase).
struct SeqR1 {
    static constexpr bool ROUTED = true, GATHER = false;   // codes sit at their partition slots
    const TileDeal& d;
    int lo, n, T0, T1, nN;
    __device__ __forceinline__ int count() const { return n; }
    __device__ __forceinline__ void coords(int i, int& tm, int& tn) const {
        const int a = d.tile_index(d.first_round + lo + i);
        if (a < T0 * nN) band_coords(a, T0, nN, tm, tn);
        else band_coords(a - T0 * nN, T1, nN, tm, tn);
    }
};
// One routed 256 x 128 half of a 1-byte tile (tm, tn in 128-column units), or none.
struct SeqR1Half {
    static constexpr bool ROUTED = true, GATHER = false;
    int n, tm, tn;
    __device__ __forceinline__ int count() const { return n; }
    __device__ __forceinline__ void coords(int, int& tm_, int& tn_) const {
        tm_ = tm;
        tn_ = tn;
    }
};
// The FP16 tiles f = b, b + G, ... < nF: M-tile f % T2, N-tile f / T2.
struct SeqRF {
    static constexpr bool ROUTED = true, GATHER = true;    // fp16 rows gathered from x through a_idx
    int b, G, n, T2;
    __device__ __forceinline__ int count() const { return n; }
    __device__ __forceinline__ void coords(int i, int& tm, int& tn) const {
        const int f = b + i * G;
        tm = f % T2;
        tn = f / T2;
    }
};
