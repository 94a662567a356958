// route.hip -- per-row precision routing and row gather/scatter for gfx950.
//
// ee_route: tier[r] = 0 (INT8) if H[r] < tau_low, 1 (FP8) if H[r] < tau_high,
// else 2 (FP16) -- the dispatcher's strict comparisons (EE/python/
// dispatch.py:74-79), applied per row.  H is binary32 compared in double
// against double thresholds, exactly as `.item()` against Python floats.
// idx receives a stable partition of the row indices: the INT8 rows in
// ascending order, then the FP8 rows, then the FP16 rows; counts[3] their
// sizes.  One 1024-thread workgroup; positions come from wave ballots
// (mbcnt = popcount of the lower lanes' votes) and a scan of 16 wave totals.
// With heads > 1 the routed value of row r = b * seq + s is the mean over
// heads of h[b, :, s] (per-head attention-row entropies; summed in head order,
// then divided), so the caller needs no separate reduction.
#include "../common/ee_device.h"

EE_DEV int route_tier(float h, double tl, double th) {
    const double d = (double)h;
    return d < tl ? 0 : (d < th ? 1 : 2);
}

EE_DEV uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

extern "C" __global__ void __launch_bounds__(1024) eek_route(EeRouteArgs a) {
    __shared__ int32_t wsum[16][3];
    __shared__ int32_t base[3];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    // pass 1: tiers and totals per tier
    int32_t c[3] = {0, 0, 0};
    for (int64_t r = tid; r < a.rows; r += 1024) {
        float hv;
        if (a.heads == 1) {
            hv = a.h[r];
        } else {
            // mean over heads: ascending sum, one rounded division.  The loads
            // go out 32 at a time before the adds: one workgroup walks every
            // row, so a load-add chain would pay one memory latency per head
            // (36 us instead of 10.6 us for [8, 32, 512]).
            const int64_t b = r / a.seq, sq = r % a.seq;
            const float* hp = a.h + b * a.heads * a.seq + sq;
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
            hv = sum / (float)a.heads;
        }
        const int t = route_tier(hv, a.tau_low, a.tau_high);
        a.tier[r] = t;
        c[t]++;
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

    // pass 2: stable scatter, 1024 rows per step
    for (int64_t r0 = 0; r0 < a.rows; r0 += 1024) {
        const int64_t r = r0 + tid;
        const int t = (r < a.rows) ? a.tier[r] : 3;  // written by this thread in pass 1
        uint32_t pos = 0;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const uint64_t m = __ballot(t == k);
            if (t == k) pos = lanes_below(m);
            if (lane == 0) wsum[w][k] = __popcll(m);
        }
        __syncthreads();
        if (t < 3) {
            int32_t before = base[t];
            for (int i = 0; i < w; ++i) before += wsum[i][t];
            a.idx[before + (int32_t)pos] = (int32_t)r;
        }
        __syncthreads();
        if (tid < 3) {
            int32_t add = 0;
            for (int i = 0; i < 16; ++i) add += wsum[i][tid];
            base[tid] += add;
        }
        __syncthreads();
    }
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
