// ee_kernel_args.h -- kernel argument blocks shared by the gfx950 code objects
// and the host launcher.  Every kernel takes exactly one of these structs by
// value; the launcher passes it through hipModuleLaunchKernel's kernelParams.
// Plain C layout (pointers and fixed-width integers only) so the host and the
// device compilers agree on every offset.
#pragma once
#include <stdint.h>

#include "entropy_engine.h"  // tier, quantiser-mode and GEMM-kind constants

#define EE_WAVE 64
#define EE_BLOCK 256

// Row softmax + Shannon entropy.
struct EeSoftmaxArgs {
    const uint16_t* x;    // fp16 logits, rows of S, row stride ld_x (elements)
    uint16_t* p;          // fp16 probabilities (nullable: entropy only)
    float* h;             // f32 entropy per row
    int32_t* tier;        // optional per-row precision tier (nullable)
    int64_t rows;
    int64_t ld_x;
    int64_t ld_p;
    int32_t S;
    int32_t causal;       // 1: column c of row r is kept iff c <= r % S
    double tau_low;       // tier thresholds, used when tier != nullptr
    double tau_high;
};

// Per-row activation quantisation (optionally gathering routed rows);
// mode is one of EE_QUANT_* (entropy_engine.h).
struct EeQuantArgs {
    const uint16_t* x;      // fp16 [*, K] activations, row stride ld_x
    void* codes;            // int8 / e4m3 codes [rows, K], row stride ld_c
    float* scale;           // f32 per output row
    const int32_t* idx;     // optional source-row list (routing partition)
    const int32_t* counts;  // optional device row counts per tier; output row
                            // r goes to slot off + r (off = rows of lower tiers)
    int64_t M;              // rows (upper bound when counts != nullptr)
    int64_t K;
    int64_t ld_x;
    int64_t ld_c;
    int32_t mode;
    int32_t tier;           // which counts[] entry / idx segment (routing)
    const uint32_t* tmax;   // EE_QUANT_F8_TENSOR: per-block |x| maxima (fp16 bits)
    int32_t n_tmax;         //   and their count
};

// Per-block max |x| over fp16 rows (first pass of the per-tensor FP8 scale).
struct EeAbsmaxArgs {
    const uint16_t* x;      // fp16 [M, K], row stride ld_x
    uint32_t* out;          // [gridDim.x] max |x| as fp16 bits (NaN propagates)
    int64_t M;
    int64_t K;
    int64_t ld_x;
};

// Tiled GEMM on MFMA.  C[m, n] = sum_k A[m, k] * B[n, k]  (B packed K-contiguous).
// kind (template argument of the kernel) is one of EE_GEMM_* (entropy_engine.h).
struct EeGemmArgs {
    const void* a;          // [M, K] int8 / e4m3 / fp16, row stride lda (elements)
    const void* b;          // [N, K] same element type, row stride ldb
    uint16_t* c;            // fp16 [*, N], row stride ldc
    int32_t* acc;           // optional int32 accumulators (I8 only), row stride ldc
    const float* a_scale;   // [M] (I8, F8)
    const float* b_scale;   // [N] (I8, F8)
    const int32_t* a_idx;   // optional: A row m is a[a_idx[off + m]] (else a[off + m])
    const int32_t* c_idx;   // optional: C row m is c[c_idx[off + m]]
    const int32_t* counts;  // optional device row counts per tier (M bound);
                            // off = counts[0] + .. + counts[tier-1], else 0
    int64_t lda;
    int64_t ldb;
    int64_t ldc;
    int32_t M;              // rows (upper bound when counts != nullptr)
    int32_t N;
    int32_t K;
    int32_t tier;
    int32_t swiglu;         // 1: B is gate|up interleaved in blocks of 32 rows (rows 64k .. 64k+31 =
                            // gate 32k .., rows 64k+32 .. 64k+63 = up 32k ..); C receives
                            // act [*, N/2] = fp16(fp16(silu(gate)) * up) instead of [*, N]
};

// The routed linear's tier GEMMs in one launch (eek_gemm_routed): t[k] is the
// EE_GEMM_I8 / F8 / F16 argument block of tier k (all with the same counts);
// mt_max = M-tile slots of the grid; f16_w8 picks the FP16 tier's pipeline so
// that its f32 summation order is the one ee_gemm uses.
struct EeRoutedGemmArgs {
    EeGemmArgs t[3];
    int32_t mt_max;
    int32_t f16_w8;         // 1: the FP16 tier runs the 8-wave pipeline (as ee_gemm does)
    int32_t f16_half_cus;   // > 0: FP16 tiles may run as 128 x 64 halves on this many CUs (eek_gemm_routed)
    int32_t pad_;
};

// Internal quantiser mode of the routed linear: partition slots below counts[0]
// get EE_QUANT_I8_DISPATCH codes, the next counts[1] slots EE_QUANT_F8_ROW codes.
#define EE_QUANT_ROUTED_I8_F8 16

// Per-row routing: tier + stable partition of row indices.
struct EeRouteArgs {
    const float* h;         // [rows], or with heads > 1 [rows / seq, heads, seq]: row r = b * seq + s
                            // routes on the mean over heads of h[b, :, s]
    int32_t* tier;          // [rows]
    int32_t* idx;           // [rows]: rows of tier 0, then tier 1, then tier 2
    int32_t* counts;        // [3]
    int64_t rows;
    double tau_low;
    double tau_high;
    int32_t heads;          // 1: h is per row; 0 (eek_route): tier[] already holds the tiers
    int32_t seq;
};

// Weight preparation (offline, once per layer).
struct EeWeightArgs {
    const void* src;        // see each kernel
    void* dst;
    void* dst2;
    const float* scale;
    int64_t R;              // rows of src
    int64_t C;              // columns of src
    int64_t ld_src;
    int64_t ld_dst;
};

// Row copy (gather / scatter through a routing partition).
struct EeRowCopyArgs {
    const uint8_t* src;
    uint8_t* dst;
    const int32_t* idx;
    const int32_t* counts;
    int64_t rows;           // upper bound
    int64_t row_bytes;
    int64_t ld_src;         // bytes
    int64_t ld_dst;         // bytes
    int32_t tier;
    int32_t scatter;        // 0: dst[r] = src[idx[r]]; 1: dst[idx[r]] = src[r]
};

// MLP activation (eek_silu_mul): act[m, j] = silu(gu[m, j]) * gu[m, F + j], fp16.
struct EeSiluMulArgs {
    const uint16_t* gu;     // fp16 [M, 2F]: gate | up halves, or (interleave) blocks of 32 alternating; row stride ld_gu
    uint16_t* act;          // fp16 [M, F], row stride ld_act
    int64_t M;
    int64_t F;
    int64_t ld_gu;
    int64_t ld_act;
    int32_t vec;            // 1: F, strides and pointers allow 16-byte accesses
    int32_t interleave;     // 1: gate of column j at 64*(j/32) + j%32, up 32 columns later
};

// eek_interleave_rows: dst row 64k + r = src row 32k + r, dst row 64k + 32 + r =
// src row F + 32k + r (r < 32) -- gate rows then up rows into blocks of 32.
struct EeInterleaveArgs {
    const uint8_t* src;
    uint8_t* dst;
    int64_t F;              // rows per half (a multiple of 32)
    int64_t row_bytes;      // a multiple of 4
    int64_t ld_src_bytes, ld_dst_bytes;
};

// eek_add_rmsnorm: one wave per row of D fp16 values (D % 8 == 0, D <= 4096).
struct EeRmsNormArgs {
    const uint16_t* x;      // fp16 [T, D], row stride ld_x
    const uint16_t* y;      // optional fp16 [T, D] added to x first (NULL: none), row stride ld_y
    const uint16_t* w;      // fp16 [D] weight
    uint16_t* x_out;        // fp16 [T, D]: x + y (only written when y != NULL), row stride ld_xo
    uint16_t* n_out;        // fp16 [T, D]: the normalised rows, row stride ld_n
    int64_t T;
    int64_t D;
    int64_t ld_x, ld_y, ld_xo, ld_n;
    float eps;
    float inv_d;            // f32(1 / D)
};

struct EeRmsNormRouteArgs {
    EeRmsNormArgs n;        // as eek_add_rmsnorm; launch row i is source row idx[i]
    const int32_t* idx;     // routing partition, slot -> row (T entries)
    const int32_t* counts;  // rows per tier: slots [0, c0) INT8, [c0, c0 + c1) FP8, the rest FP16
    uint8_t* codes;         // [T, D] codes of the INT8 and FP8 slots, row stride ld_c
    float* scale;           // [T] scales of those slots
    int64_t ld_c;
};

// eek_qkv_rope: rotary embedding of q and k and the head-major layouts.
struct EeQkvRopeArgs {
    const uint16_t* qkv;    // fp16 [B*S, (Hq + 2*Hkv) * d]: q heads, k heads, v heads; row stride ld
    const uint16_t* cos_t;  // fp16 [S, d]
    const uint16_t* sin_t;  // fp16 [S, d]
    uint16_t* q;            // fp16 [B, Hq, S, d]
    uint16_t* k;            // fp16 [B, Hkv, S, d]
    uint16_t* v;            // fp16 [B, Hkv, S, d]
    int64_t ld;
    int32_t B, S, Hq, Hkv, d;
    float q_scale;          // q is stored as fp16(rope(q) * q_scale); 1 stores rope(q)
    int32_t v_t;            // 1: v is V^T [B, Hkv, d, S], each 16-key group stored as keys 0-3, 8-11, 4-7, 12-15
};

// Fused causal attention + row entropy (attention.hip), head_dim 64.
struct EeAttnArgs {
    const uint16_t* q;      // fp16 [B, Hq, S, 64], carrying the 1/sqrt(64) scaling
    const uint16_t* k;      // fp16 [B, Hkv, S, 64]
    const uint16_t* vt;     // fp16 [B, Hkv, 64, S], key order of eek_qkv_rope's v_t layout
    uint16_t* out;          // fp16 [B*S, ld_out]: token-major, query head h at columns 64h .. 64h + 63
    float* h;               // f32 [B, Hq, S]: entropy of each probability row
    int64_t ld_out;
    int32_t B, S, Hq, Hkv;
    int32_t W;              // query heads (waves) per workgroup: 2 or 4, dividing Hq / Hkv
};

