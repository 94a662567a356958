// probe.hip -- hardware probes for gfx950: the rates that bound the GEMM
// kernels, measured on the box by bench.py beside the kernels themselves.
//
//   eek_probe_stream    direct-to-LDS loads (global_load_lds_dwordx4) of L2-resident
//                       data into a 4-stage LDS ring: operand bytes per clock per CU,
//                       the stream every tile of the GEMMs is fed by
//   eek_probe_lds       ds_read_b128, 8 reads in flight per wave, conflict-free:
//                       fragment-read bytes per clock per CU
//   eek_probe_mfma_i8   v_mfma_i32_32x32x32_i8, four independent accumulators per
//                       wave, two waves per SIMD: clocks per MFMA
//   eek_probe_mfma_f8   v_mfma_scale_f32_32x32x64_f8f6f4, the same way
//   eek_probe_frag_*    the GEMMs' inner loop without their memory stream: each
//                       wave reads its fragments of a 64 x 64 block from LDS
//                       (random operands from src) and runs the MFMAs on them,
//                       as 32x32 MFMAs (i8 32x32x32, f16 32x32x16) or as the
//                       16x16 ones of the same work (i8 16x16x64, f16 16x16x32):
//                       clocks per iteration and, over a run long enough for the
//                       power limit to settle, the shader clock each holds
//
// Workgroups of 512 threads (8 waves, two per SIMD, as the GEMM kernels).
// Thread 0 reads s_memtime (shader clock) and s_memrealtime (100 MHz) after a
// barrier before the timed loop and after one behind it; the host turns them
// into rates and the clock frequency.
#include "../common/ee_device.h"
#include "../common/ee_gemm_dev.h"

#define PR_THREADS 512
#define PR_STAGE 32768                    // bytes of one ring stage (a 128 x 128 C0 tile's K stage)

EE_DEV void probe_times(const EeProbeArgs& a, int slot, uint64_t mt, uint64_t rt) {
    a.times[(int64_t)blockIdx.x * 4 + slot] = mt;
    a.times[(int64_t)blockIdx.x * 4 + 2 + slot] = rt;
}

// Workgroup b streams window b % 8 of src (the 8 XCDs each keep their window in
// L2 after the first pass) or, with own_window, window b (nothing shared: the
// stream comes from the MALL or HBM): per stage, wave w loads 1 KB groups 4w ..
// 4w+3, at most three of its stages in flight -- 96 KB per CU, as the GEMMs' rings
// hold -- (the ring slot a stage reuses was loaded four stages earlier, which
// the wait after the previous stage has retired).
extern "C" __global__ void __launch_bounds__(PR_THREADS) eek_probe_stream(EeProbeArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t ring[4 * PR_STAGE];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint8_t* win = a.src + (int64_t)(a.own_window ? blockIdx.x : (blockIdx.x & 7)) * a.window + lane * 16;
    const int nstage = (int)(a.window / PR_STAGE);
    const uint32_t lds0 = lds_addr(ring);
    __syncthreads();
    if (t == 0) probe_times(a, 0, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    for (int k = 0; k < a.iters; ++k) {
        const uint8_t* st = win + (int64_t)(k % nstage) * PR_STAGE;
        const uint32_t slot = lds0 + (uint32_t)((k & 3) * PR_STAGE);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int grp = wave * 4 + q;
            dma16(st + grp * 1024, slot + grp * 1024);
        }
        WAITCNT_VM(12);
    }
    WAITCNT_VM(0);
    __syncthreads();
    if (t == 0) probe_times(a, 1, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    a.sink[(int64_t)blockIdx.x * PR_THREADS + t] = *(const uint32_t*)(ring + t * 16);
}

// Wave w reads 1 KB at byte w * 1 KB of each 8 KB of a 64 KB region, lane l 16 bytes
// at 16 l: every 16-lane pass of a read covers the 64 banks once.
extern "C" __global__ void __launch_bounds__(PR_THREADS) eek_probe_lds(EeProbeArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t s[65536];
    const int t = threadIdx.x;
    for (int i = t * 16; i < 65536; i += PR_THREADS * 16) *(u32x4*)(s + i) = u32x4{(uint32_t)i, 1u, 2u, 3u};
    const uint32_t base = lds_addr(s) + (uint32_t)((t & 63) * 16 + (t >> 6) * 1024);
    u32x4 acc = {0u, 0u, 0u, 0u};
    __syncthreads();
    if (t == 0) probe_times(a, 0, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    for (int k = 0; k < a.iters; ++k) {
        u32x4 v0, v1, v2, v3, v4, v5, v6, v7;
        asm volatile(
            "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:8192\n\tds_read_b128 %2, %8 offset:16384\n\t"
            "ds_read_b128 %3, %8 offset:24576\n\tds_read_b128 %4, %8 offset:32768\n\tds_read_b128 %5, %8 offset:40960\n\t"
            "ds_read_b128 %6, %8 offset:49152\n\tds_read_b128 %7, %8 offset:57344\n\ts_waitcnt lgkmcnt(0)"
            : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3), "=v"(v4), "=v"(v5), "=v"(v6), "=v"(v7)
            : "v"(base)
            : "memory");
        acc ^= v0 ^ v1 ^ v2 ^ v3 ^ v4 ^ v5 ^ v6 ^ v7;
    }
    __syncthreads();
    if (t == 0) probe_times(a, 1, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    a.sink[(int64_t)blockIdx.x * PR_THREADS + t] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

extern "C" __global__ void __launch_bounds__(PR_THREADS) eek_probe_mfma_i8(EeProbeArgs a) {
    const int t = threadIdx.x;
    const i32x4 x = {t, t + 1, t + 2, t + 3}, y = {3 * t, t, 7, t};
    i32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    __syncthreads();
    if (t == 0) probe_times(a, 0, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    for (int k = 0; k < a.iters; ++k) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(y, x, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, x, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(y, y, c3, 0, 0, 0);
    }
    __syncthreads();
    if (t == 0) probe_times(a, 1, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    a.sink[(int64_t)blockIdx.x * PR_THREADS + t] = (uint32_t)(c0[0] ^ c1[5] ^ c2[10] ^ c3[15]);
}

// e4m3 operands of modest magnitude (bytes 0x30-0x3f: 0.5 .. 0.94), so the sums stay finite.
extern "C" __global__ void __launch_bounds__(PR_THREADS) eek_probe_mfma_f8(EeProbeArgs a) {
    const int t = threadIdx.x;
    const int u = 0x30303030 | ((t & 15) * 0x01010101);
    const i32x8 x = {u, u, u, u, u, u, u, u}, y = {u ^ 0x01010101, u, u, u, u, u, u, u};
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    __syncthreads();
    if (t == 0) probe_times(a, 0, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    for (int k = 0; k < a.iters; ++k) {
        c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(x, y, c0, 0, 0, 0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(y, x, c1, 0, 0, 0, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(x, x, c2, 0, 0, 0, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(y, y, c3, 0, 0, 0, 0, 0, 0);
    }
    __syncthreads();
    if (t == 0) probe_times(a, 1, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    a.sink[(int64_t)blockIdx.x * PR_THREADS + t] =
        __builtin_bit_cast(uint32_t, c0[0] + c1[5] + c2[10] + c3[15]);
}

// Fragment loops.  Iteration k: each wave reads 8 16-byte fragments per lane
// (1 KB apart, at 4 KB k + 512 wave + 16 lane modulo the 64 KB the workgroup
// copied from src block b % 16) and issues MFMAs over a 64 x 64 block worth
// 2 * 64 * 64 * 64 int8 ops or 2 * 64 * 64 * 32 f16 flops: 8 32x32 or 16 16x16.
__device__ __forceinline__ i32x4 frag_rd(const uint8_t* s, uint32_t o) { return *(const i32x4*)(s + (o & 0xFFF0u)); }

template <int V>
__device__ __forceinline__ void probe_frag(const EeProbeArgs& a) {
    __shared__ __attribute__((aligned(1024))) uint8_t s[65536];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint8_t* blk = a.src + (int64_t)(blockIdx.x & 15) * 65536;
    for (int i = t * 16; i < 65536; i += PR_THREADS * 16) *(i32x4*)(s + i) = *(const i32x4*)(blk + i);
    __syncthreads();
    const uint32_t lb = (uint32_t)(lane * 16 + wave * 512);
    uint32_t out = 0;
    if (t == 0) probe_times(a, 0, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    if constexpr (V == 0) {                           // i8 32x32x32: K 64 per iteration
        i32x16 c[2][2] = {};
        for (int k = 0; k < a.iters; ++k) {
            const uint32_t o = lb + (uint32_t)k * 4096u;
            i32x4 x[2][2], y[2][2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    x[h][i] = frag_rd(s, o + (h * 4 + i) * 1024);
                    y[h][i] = frag_rd(s, o + (h * 4 + 2 + i) * 1024);
                }
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) c[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x[h][i], y[h][j], c[i][j], 0, 0, 0);
        }
        out = (uint32_t)(c[0][0][0] ^ c[0][1][3] ^ c[1][0][7] ^ c[1][1][15]);
    } else if constexpr (V == 1) {                    // i8 16x16x64: K 64
        i32x4 c[4][4] = {};
        for (int k = 0; k < a.iters; ++k) {
            const uint32_t o = lb + (uint32_t)k * 4096u;
            i32x4 x[4], y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = frag_rd(s, o + i * 1024);
                y[i] = frag_rd(s, o + (4 + i) * 1024);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) c[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[i], y[j], c[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) out ^= (uint32_t)c[i][j][(i + j) & 3];
    } else if constexpr (V == 2) {                    // f16 32x32x16: K 32
        f32x16 c[2][2] = {};
        for (int k = 0; k < a.iters; ++k) {
            const uint32_t o = lb + (uint32_t)k * 4096u;
            f16x8 x[2][2], y[2][2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    x[h][i] = __builtin_bit_cast(f16x8, frag_rd(s, o + (h * 4 + i) * 1024));
                    y[h][i] = __builtin_bit_cast(f16x8, frag_rd(s, o + (h * 4 + 2 + i) * 1024));
                }
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) c[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x[h][i], y[h][j], c[i][j], 0, 0, 0);
        }
        out = __float_as_uint(c[0][0][0] + c[0][1][3] + c[1][0][7] + c[1][1][15]);
    } else {                                          // f16 16x16x32: K 32
        f32x4 c[4][4] = {};
        for (int k = 0; k < a.iters; ++k) {
            const uint32_t o = lb + (uint32_t)k * 4096u;
            f16x8 x[4], y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = __builtin_bit_cast(f16x8, frag_rd(s, o + i * 1024));
                y[i] = __builtin_bit_cast(f16x8, frag_rd(s, o + (4 + i) * 1024));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) c[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[i], y[j], c[i][j], 0, 0, 0);
        }
        float f = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) f += c[i][j][(i + j) & 3];
        out = __float_as_uint(f);
    }
    __syncthreads();
    if (t == 0) probe_times(a, 1, __builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime());
    a.sink[(int64_t)blockIdx.x * PR_THREADS + t] = out;
}
extern "C" __global__ void __launch_bounds__(PR_THREADS) eek_probe_frag_i8_32(EeProbeArgs a) { probe_frag<0>(a); }
extern "C" __global__ void __launch_bounds__(PR_THREADS) eek_probe_frag_i8_16(EeProbeArgs a) { probe_frag<1>(a); }
extern "C" __global__ void __launch_bounds__(PR_THREADS) eek_probe_frag_f16_32(EeProbeArgs a) { probe_frag<2>(a); }
extern "C" __global__ void __launch_bounds__(PR_THREADS) eek_probe_frag_f16_16(EeProbeArgs a) { probe_frag<3>(a); }
