// route.hip -- per-row precision routing and row gather/scatter for gfx950.
//
// ee_route: tier[r] = 0 (INT8) if H[r] < tau_low, 1 (FP8) if H[r] < tau_high,
// else 2 (FP16) -- the dispatcher's strict comparisons (EE/python/
// dispatch.py:74-79), applied per row.  H is binary32 compared in double
// against double thresholds, exactly as `.item()` against Python floats.
// idx receives a stable partition of the row indices: the INT8 rows in
// ascending order, then the FP8 rows, then the FP16 rows; counts[3] their
// sizes.
//
// eek_route: one 1024-thread workgroup; thread t takes rows 4t .. 4t+3 of each
// chunk of 4096.  Pass 1 computes the tiers (heads == 1: from h; heads == 0:
// tier[] already holds them) and the totals; pass 2 places each chunk's rows:
// a thread's count of each tier (0..4) is split into three bits, and one
// ballot per bit gives, through mbcnt, the count of that tier in the lower
// lanes; wave totals go through LDS.  Up to 4096 rows (one chunk) the two
// passes are one: the wave totals give the tier totals as well, and the tiers
// stay in registers.
// eek_route_heads_tier: with heads > 1 the routed value of row r = b * seq + s
// is the mean over heads of h[b, :, s] (per-head attention-row entropies;
// summed in head order, then divided).  One thread per row over the whole
// grid writes tier[], then eek_route (heads == 0) partitions the rows: two
// launches instead of one workgroup walking every head of every row.
#include "../common/ee_device.h"

EE_DEV int route_tier(float h, double tl, double th) {
    const double d = (double)h;
    return d < tl ? 0 : (d < th ? 1 : 2);
}

EE_DEV uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

#define RT_RPT 4                        // rows per thread per chunk
#define RT_CHUNK (1024 * RT_RPT)

// Tiers of rows r0 .. r0+3 (3 past the end): from h (heads == 1) or tier[].
EE_DEV void route_load(const EeRouteArgs& a, int64_t r0, int (&t)[RT_RPT]) {
    if (a.heads == 1) {
        float hv[RT_RPT];
#pragma unroll
        for (int k = 0; k < RT_RPT; ++k) hv[k] = r0 + k < a.rows ? a.h[r0 + k] : 0.0f;
#pragma unroll
        for (int k = 0; k < RT_RPT; ++k) {
            t[k] = r0 + k < a.rows ? route_tier(hv[k], a.tau_low, a.tau_high) : 3;
            if (r0 + k < a.rows) a.tier[r0 + k] = t[k];
        }
    } else {
#pragma unroll
        for (int k = 0; k < RT_RPT; ++k) t[k] = r0 + k < a.rows ? a.tier[r0 + k] : 3;
    }
}

// This thread's rows of each tier among the lower lanes of its wave (pos) and
// the wave's totals (tot, lane-uniform), from n[q] <= 4 rows per tier.
EE_DEV void route_wave_scan(const int (&n)[3], int32_t (&pos)[3], int32_t (&tot)[3]) {
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        uint32_t below = 0, all = 0;
#pragma unroll
        for (int b = 0; b < 3; ++b) {                 // n[q] <= 4: three bits
            const uint64_t m = __ballot((n[q] >> b) & 1);
            below += lanes_below(m) << b;
            all += (uint32_t)__popcll(m) << b;
        }
        pos[q] = (int32_t)below;
        tot[q] = (int32_t)all;
    }
}

// idx entries of this thread's rows, in row order, from its first position per tier.
EE_DEV void route_place(const EeRouteArgs& a, int64_t r0, const int (&t)[RT_RPT], int32_t (&pos)[3]) {
#pragma unroll
    for (int k = 0; k < RT_RPT; ++k) {
        if (t[k] < 3) {
            const int32_t p = t[k] == 0 ? pos[0] : (t[k] == 1 ? pos[1] : pos[2]);
            a.idx[p] = (int32_t)(r0 + k);
            if (t[k] == 0) ++pos[0];
            else if (t[k] == 1) ++pos[1];
            else ++pos[2];
        }
    }
}

// rows <= 4096: one load, one barrier.
EE_DEV void route_chunk1(const EeRouteArgs& a, int32_t (*wsum)[3], int tid, int lane, int w) {
    const int64_t r0 = (int64_t)tid * RT_RPT;
    int t[RT_RPT];
    route_load(a, r0, t);
    int n[3] = {0, 0, 0};
#pragma unroll
    for (int k = 0; k < RT_RPT; ++k)
        if (t[k] < 3) n[t[k]]++;
    int32_t pos[3], tot[3];
    route_wave_scan(n, pos, tot);
    if (lane == 0) {
        wsum[w][0] = tot[0];
        wsum[w][1] = tot[1];
        wsum[w][2] = tot[2];
    }
    __syncthreads();
    int32_t total[3] = {0, 0, 0}, before[3] = {0, 0, 0};
    for (int i = 0; i < 16; ++i) {
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            total[q] += wsum[i][q];
            if (i < w) before[q] += wsum[i][q];
        }
    }
    if (tid < 3) a.counts[tid] = total[tid];
    pos[0] += before[0];
    pos[1] += total[0] + before[1];
    pos[2] += total[0] + total[1] + before[2];
    route_place(a, r0, t, pos);
}

extern "C" __global__ void __launch_bounds__(1024) eek_route(EeRouteArgs a) {
    __shared__ int32_t wsum[16][3];
    __shared__ int32_t base[3];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (a.rows <= RT_CHUNK) {
        route_chunk1(a, wsum, tid, lane, w);
        return;
    }

    // pass 1: tiers and totals per tier
    int32_t c[3] = {0, 0, 0};
    for (int64_t c0 = 0; c0 < a.rows; c0 += RT_CHUNK) {
        const int64_t r0 = c0 + (int64_t)tid * RT_RPT;
        int t[RT_RPT];
        route_load(a, r0, t);
#pragma unroll
        for (int k = 0; k < RT_RPT; ++k)
            if (t[k] < 3) c[t[k]]++;
    }
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        const int32_t v = wave_sum_i32(c[t]);
        if (lane == 0) wsum[w][t] = v;
    }
    __syncthreads();
    if (tid < 3) {
        int32_t tot = 0;
        for (int i = 0; i < 16; ++i) tot += wsum[i][tid];
        a.counts[tid] = tot;
        wsum[0][tid] = tot;  // read below after the barrier
    }
    __syncthreads();
    if (tid == 0) {
        base[0] = 0;
        base[1] = wsum[0][0];
        base[2] = wsum[0][0] + wsum[0][1];
    }
    __syncthreads();

    // pass 2: stable scatter, one chunk per step (tier[] of this thread's rows
    // was written by this thread in pass 1, or by the previous launch)
    for (int64_t c0 = 0; c0 < a.rows; c0 += RT_CHUNK) {
        const int64_t r0 = c0 + (int64_t)tid * RT_RPT;
        int t[RT_RPT];
        int n[3] = {0, 0, 0};
#pragma unroll
        for (int k = 0; k < RT_RPT; ++k) {
            t[k] = r0 + k < a.rows ? a.tier[r0 + k] : 3;
            if (t[k] < 3) n[t[k]]++;
        }
        int32_t pos[3], tot[3];
        route_wave_scan(n, pos, tot);
        if (lane == 0) {
            wsum[w][0] = tot[0];
            wsum[w][1] = tot[1];
            wsum[w][2] = tot[2];
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            int32_t before = base[q];
            for (int i = 0; i < w; ++i) before += wsum[i][q];
            pos[q] += before;
        }
        route_place(a, r0, t, pos);
        __syncthreads();
        if (tid < 3) {
            int32_t add = 0;
            for (int i = 0; i < 16; ++i) add += wsum[i][tid];
            base[tid] += add;
        }
        __syncthreads();
    }
}

// Tiers of rows routed on the mean over heads (heads > 1), one thread per row.
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_route_heads_tier(EeRouteArgs a) {
    const int64_t r = (int64_t)blockIdx.x * EE_BLOCK + threadIdx.x;
    if (r >= a.rows) return;
    const int64_t b = r / a.seq, sq = r % a.seq;
    const float* hp = a.h + b * a.heads * a.seq + sq;
    // ascending sum, one rounded division; the loads go out 32 at a time
    float sum = 0.0f;
    int j = 0;
    for (; j + 32 <= a.heads; j += 32) {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = hp[(int64_t)(j + u) * a.seq];
#pragma unroll
        for (int u = 0; u < 32; ++u) sum += v[u];
    }
    for (; j < a.heads; ++j) sum += hp[(int64_t)j * a.seq];
    a.tier[r] = route_tier(sum / (float)a.heads, a.tau_low, a.tau_high);
}

// Row gather/scatter through a routing partition.  scatter == 0:
// dst[r] = src[idx[off + r]]; scatter == 1: dst[idx[off + r]] = src[r];
// r < counts[tier] (or < rows without counts).  One wave per row, 16-byte
// moves when rows are 16-byte aligned, byte moves otherwise.
extern "C" __global__ void __launch_bounds__(EE_BLOCK) eek_row_copy(EeRowCopyArgs a) {
    const int lane = lane_id();
    const int64_t r = (int64_t)blockIdx.x * 4 + wave_id();
    const int64_t rows = a.counts ? (int64_t)a.counts[a.tier] : a.rows;
    if (r >= rows) return;
    const int64_t off = a.counts ? tier_offset(a.counts, a.tier) : 0;
    const int64_t j = a.idx ? (int64_t)a.idx[off + r] : r;
    const uint8_t* s = a.src + (a.scatter ? r : j) * a.ld_src;
    uint8_t* d = a.dst + (a.scatter ? j : r) * a.ld_dst;
    const bool vec = ((((uintptr_t)s) | ((uintptr_t)d) | (uintptr_t)a.row_bytes) & 15u) == 0;
    if (vec) {
        for (int64_t c = (int64_t)lane * 16; c < a.row_bytes; c += 64 * 16)
            *(u32x4*)(d + c) = *(const u32x4*)(s + c);
    } else {
        for (int64_t c = lane; c < a.row_bytes; c += 64) d[c] = s[c];
    }
}
