/*
 * entropy_engine.h -- C ABI of the MI355X (gfx950) entropy-gated precision path.
 *
 * A host library (libentropy_engine.so) that loads gfx950 code objects
 * (*.hsaco, listed in entropy_engine_meta.json) with hipModuleLoadData and
 * launches them with hipModuleLaunchKernel.  It replaces the reference's
 * CubinEngine (.cubin + CUDA Driver API, EE/csrc/engine.cpp) and the Triton
 * launchers of EE/python/kernels.py.
 *   EE = "entropy-engine (1)/entropy-engine" in the reference tree.
 *
 * Conventions
 *  - Every call returns 0 (EE_OK) or a negative ee_status; the message of the
 *    last failure on the calling thread is ee_last_error().
 *  - All argument checks run before any HIP call, so a rejected call has no
 *    side effect on the device.
 *  - The caller owns every buffer (inputs, outputs, workspaces); the engine
 *    owns only its loaded modules.  Pointers are device pointers on the
 *    engine's device; "stream" is a hipStream_t (NULL = default stream).
 *    Calls are asynchronous on that stream.
 *  - fp16 tensors are passed as raw 16-bit storage; e4m3 codes as bytes (OCP
 *    e4m3fn, max 448).  Leading dimensions are in elements.
 *  - An ee_engine is immutable after creation: launches from several threads
 *    are safe; create/destroy must not overlap its use.
 */
#ifndef ENTROPY_ENGINE_H
#define ENTROPY_ENGINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EE_ABI_VERSION 1

typedef struct ee_engine ee_engine;
typedef struct ee_module_engine ee_module_engine;
typedef void* ee_stream_t; /* hipStream_t */

typedef enum {
    EE_OK = 0,
    EE_ERR_INVALID_ARG = -1, /* bad pointer, size, stride, alignment or dtype contract */
    EE_ERR_IO = -2,          /* code object / meta file cannot be opened or read */
    EE_ERR_META = -3,        /* meta JSON malformed or missing a key */
    EE_ERR_HIP = -4,         /* a HIP runtime call failed */
    EE_ERR_UNSUPPORTED = -5, /* shape outside what the kernels implement */
    EE_ERR_NOT_FOUND = -6    /* kernel symbol missing from the code objects */
} ee_status;

/* Precision tiers: EE/python/dispatch.py:32-36 (PrecisionTier). */
enum { EE_TIER_INT8 = 0, EE_TIER_FP8 = 1, EE_TIER_FP16 = 2 };

/* Activation quantiser modes. */
enum {
    EE_QUANT_I8_DISPATCH = 0, /* EE/python/kernels.py:336-338: fp16 scale, truncating cast   */
    EE_QUANT_I8_ENGINE = 1,   /* EE/test_cubin.py:93-103: f32 scale, round + clamp(+-127)    */
    EE_QUANT_F8_ROW = 2,      /* EE/python/kernels.py:361,144,159-160: e4m3 codes per row    */
    EE_QUANT_F8_TENSOR = 3    /* one e4m3 scale per tensor: ee_quant_tensor_f8 only           */
};

/* GEMM kinds (the three tiers). */
enum {
    EE_GEMM_I8 = 0,  /* EE/python/kernels.py:50-110  int8 x int8 -> int32 -> fp16 */
    EE_GEMM_F8 = 1,  /* EE/python/kernels.py:118-180 e4m3 x e4m3 -> f32 -> fp16   */
    EE_GEMM_F16 = 2, /* EE/python/kernels.py:192-246 fp16 x fp16 (W8A16 weights pre-dequantised) -> fp16 */
    EE_GEMM_W8A16 = 3 /* the same tier from int8 codes + f32 scales, dequantised in the kernel as
                         kernels.py:215,233 do in SRAM: w = fp16(fp16(b) * fp16(scale[n])) */
};

const char* ee_last_error(void);
int ee_abi_version(void);

/* ---- engine lifetime ------------------------------------------------------
 * Replaces load_cubin + CubinEngine construction (EE/csrc/engine.cpp:23-44,
 * 73-104).  lib_dir holds entropy_engine_meta.json and the *.hsaco files it
 * names; modules are loaded on the current device.  destroy unloads them
 * (the reference leaks its CUmodule). */
int ee_engine_create(const char* lib_dir, ee_engine** out);
int ee_engine_destroy(ee_engine* eng);
/* Tuning knobs (0 = automatic): "se_wpr" waves per softmax row (1..8),
 * "se_rpw" softmax rows per wave for short rows (1, 2, 4),
 * "se_nt" non-temporal loads of the softmax logits in the 2-, 4- and 8-wave
 * row layouts (1 off, 2 on; automatic: on where the logits and probabilities
 * together exceed the 256 MiB Infinity Cache),
 * "quant_wpr" waves per quantiser row (1,2,4);
 * "routed_unfused" = 1 makes ee_routed_linear use its five-launch sequence for
 * every K (for comparisons); "gemm_variant" = 1 runs every GEMM on the
 * loader-wave pipeline, 2 on the 8-wave pipeline where one exists (INT8 and
 * W8A16); automatic: the loader-wave pipeline.  INT8 results are identical
 * either way.  Every FP16-tier kernel sums K in one f32
 * order (slice after slice), whatever the shape, tile size or routing, except
 * the 8-wave form (gemm_variant = 2), which splits K between wave pairs; the
 * routed linear follows ee_gemm's choice.
 * "gemm_persist": INT8 / FP8 GEMMs with more tiles than CUs (and the routed
 * linear's tier grid) run as persistent grids, one workgroup per CU walking
 * its tiles with the stage ring running across tile boundaries; 1 turns that
 * off, n >= 2 forces it with min(n, tiles) workgroups.  Same bits either way.
 * "gemm_tile": 256 x 256-tile persistent kernels for plain GEMMs whose
 * 128 x 128 grid has more tiles than CUs, and for routed linears where the
 * 256 x 256 grid takes at most 1/2.1 of the 128 x 128 grid's rounds of the CUs
 * (automatic; same bits); 128 forbids them, 256 forces them at every size.
 * "gemm_tile_n": the width of those 256-row tiles: automatic (plain GEMMs take
 * 256 x 128 where 256 x 256 tiles would keep at most half the CUs busy; the
 * routed grid stays at 256), or 128 / 256 forced.  Same bits either way.
 * "gemm_waves": the pipeline of those 256-row tiles, plain and routed: 8 waves
 * (each a 128 x 64 block) or 4 waves (each a 128 x 128 block, accumulators in
 * AGPRs; tiles of at least two K stages); 0 automatic (4 where it applies).
 * Same bits either way. */
int ee_engine_set_option(ee_engine* eng, const char* key, int64_t value);
int ee_engine_device(const ee_engine* eng);
/* Name of the last kernel the calling thread launched through an ee_* entry
 * point ("" before the first).  A diagnostic with no counterpart in the
 * reference: tests use it to check which pipeline the launcher picked. */
const char* ee_last_kernel(void);

/* ---- a1/a2: fused softmax + entropy ---------------------------------------
 * Replaces fused_softmax_entropy_kernel + launcher (EE/python/kernels.py:
 * 264-312, 416-450).  x: fp16 [rows, S] (row stride ld_x); p: fp16 probs
 * [rows, S] (row stride ld_p) or NULL for entropy only; h: f32 [rows].
 * causal: keep column c of row r iff c <= r % S (the reference's [B,H,S,S]
 * rows).  tier: optional int32 [rows] = routing tier of h (strict compares
 * against tau_low/tau_high in double, EE/python/dispatch.py:74-79). */
int ee_softmax_entropy(ee_engine* eng, const void* x, void* p, float* h, int64_t rows, int32_t S,
                       int64_t ld_x, int64_t ld_p, int32_t causal, int32_t* tier, double tau_low,
                       double tau_high, ee_stream_t stream);

/* ---- a9/a11/a15: activation quantisers -------------------------------------
 * Replaces the PyTorch quantiser ops of triton_int8_gemm / triton_fp8_gemm
 * (EE/python/kernels.py:336-338, 361 + in-kernel :144,159-160) and the
 * CubinEngine test's quantiser (EE/test_cubin.py:93-103).
 * x fp16 [M, K] -> codes (int8 or e4m3 bytes) [M, K] (row stride ld_c) + f32 scale [M].
 * Routed form: with counts != NULL, rows r < counts[tier] are read from
 * x[idx[off + r]] and written to codes/scale slot off + r, where
 * off = counts[0] + ... + counts[tier-1]; M is then the upper bound. */
int ee_quant_act(ee_engine* eng, const void* x, int64_t M, int64_t K, int64_t ld_x, int32_t mode,
                 void* codes, int64_t ld_c, float* scale, const int32_t* idx, const int32_t* counts,
                 int32_t tier, ee_stream_t stream);

/* ---- a7: offline weight quantisation ----------------------------------------
 * Replaces quantize_weights_int8 (EE/python/dispatch.py:43-48).  w: fp16
 * nn.Linear weight [N, K]; writes int8 codes in GEMM operand order [N, K]
 * (row stride ld_c) and f32 per-channel scale [N].  ee_transpose_i8 turns the
 * codes into the reference's [K, N] buffer. */
int ee_quant_weight_i8(ee_engine* eng, const void* w, int64_t N, int64_t K, int64_t ld_w,
                       int8_t* codes_nk, int64_t ld_c, float* scale, ee_stream_t stream);

/* ---- FP8 e4m3 with one scale per tensor ------------------------------------
 * No counterpart in the reference, whose FP8 tier scales per row
 * (EE/python/kernels.py:361); benchmark config 1 ("FP8 e4m3 with per-tensor
 * amax scaling") names this scheme.  For x fp16 [M, K] (activations, or an
 * nn.Linear weight [N, K]):
 *   amax = max |x|;  s = amax / 448 (f32 division) if 0 < amax < inf, else 1;
 *   code = e4m3_rne_sat(f32(x) * f32(1 / s)).
 * Every scale[r] (r < M) receives s, so the FP8 GEMM applies it unchanged.
 * Two launches: per-block partial maxima into ws (EE_TENSOR_WS_FLOATS floats
 * of caller workspace), then the quantiser, which reduces them itself. */
#define EE_TENSOR_WS_FLOATS 1024
int ee_quant_tensor_f8(ee_engine* eng, const void* x, int64_t M, int64_t K, int64_t ld_x, uint8_t* codes,
                       int64_t ld_c, float* scale, float* ws, ee_stream_t stream);

/* dst[c, r] = src[r, c] for int8 [R, C]. */
int ee_transpose_i8(ee_engine* eng, const int8_t* src, int64_t R, int64_t C, int64_t ld_src,
                    int8_t* dst, int64_t ld_dst, ee_stream_t stream);
/* FP8 tier weight codes e4m3(fp16(b)) of int8 codes (EE/python/kernels.py:166). */
int ee_pack_b_f8(ee_engine* eng, const int8_t* codes_nk, int64_t N, int64_t K, int64_t ld_src,
                 uint8_t* dst, int64_t ld_dst, ee_stream_t stream);
/* W8A16 tier weights fp16(fp16(b) * fp16(scale[n])) (EE/python/kernels.py:215,233). */
int ee_pack_b_f16(ee_engine* eng, const int8_t* codes_nk, const float* scale, int64_t N, int64_t K,
                  int64_t ld_src, void* dst, int64_t ld_dst, ee_stream_t stream);

/* ---- a10/a12/a14: the tier GEMMs --------------------------------------------
 * Replaces gemm_{int8,fp8,fp16}_kernel and their launchers (EE/python/
 * kernels.py:50-246, 330-409).  C[m, n] = sum_k A[m, k] * B[n, k]:
 *   a: [M, K] int8 codes (I8), e4m3 codes (F8) or fp16 (F16), row stride lda;
 *   b_nk: [N, K] same element type (weights in operand order), row stride ldb;
 *   c: fp16, row stride ldc; a_scale [M], b_scale [N] f32 (I8/F8 only).
 *   acc_out: optional int32 accumulators (I8 only), row stride ldc.
 * Routed form: counts != NULL bounds M by counts[tier]; A row m is
 * a[a_idx[off+m]] if a_idx else a[off+m]; a_scale at off+m; C row m is
 * c[c_idx[off+m]] if c_idx else c[m].
 * Contract: K * elem_size, lda * elem_size, ldb * elem_size multiples of 16
 * bytes; a, b, b_scale 16-byte aligned; N and ldc multiples of 4; c 8-byte
 * aligned.  K * elem_size a multiple of 128 selects the pipelined kernels. */
int ee_gemm(ee_engine* eng, int32_t kind, const void* a, int64_t lda, const void* b_nk, int64_t ldb,
            void* c, int64_t ldc, const float* a_scale, const float* b_scale, int32_t M, int32_t N,
            int32_t K, const int32_t* a_idx, const int32_t* c_idx, const int32_t* counts, int32_t tier,
            int32_t* acc_out, ee_stream_t stream);

/* ---- a4/a6: per-row routing -------------------------------------------------
 * New with no reference function: the reference picks one tier per call
 * (EE/python/dispatch.py:68-82).  tier[r] by the same strict compares;
 * idx = stable partition [INT8 rows | FP8 rows | FP16 rows]; counts[3]. */
int ee_route(ee_engine* eng, const float* h, int64_t rows, double tau_low, double tau_high,
             int32_t* tier, int32_t* idx, int32_t* counts, ee_stream_t stream);
/* The same on the mean over heads of per-head row entropies h [B, heads, S]
 * (ee_attention_causal's entropy output): row r = b * S + s is routed on
 * (h[b, 0, s] + ... + h[b, heads - 1, s]) / heads, summed in head order.  The
 * reference routes on the mean of its attention entropies over heads and
 * queries (EE/python/dispatch.py:243-245, one value per call); this keeps one
 * value per token. */
int ee_route_heads(ee_engine* eng, const float* h, int32_t B, int32_t heads, int32_t S, double tau_low,
                   double tau_high, int32_t* tier, int32_t* idx, int32_t* counts, ee_stream_t stream);

/* Row gather (scatter = 0: dst[r] = src[idx[off+r]]) or scatter
 * (scatter = 1: dst[idx[off+r]] = src[r]) for r < counts[tier] (or rows). */
int ee_row_copy(ee_engine* eng, const void* src, int64_t ld_src_bytes, void* dst, int64_t ld_dst_bytes,
                int64_t rows, int64_t row_bytes, const int32_t* idx, const int32_t* counts, int32_t tier,
                int32_t scatter, ee_stream_t stream);

/* ---- routed linear: entropy-gated GEMM over a mixed batch -------------------
 * One tier per row: INT8 rows quantised (EE_QUANT_I8_DISPATCH) and run on the
 * I8 GEMM, FP8 rows on the F8 GEMM, FP16 rows on the W8A16 GEMM, outputs
 * scattered back to their rows; no host synchronisation.  idx/counts come
 * from ee_route.  ws_codes: bytes [M, K] (row stride K), ws_scale: f32 [M].
 * b_i8 / b_f8 / b_f16: the three weight operands [N, K] (row stride K).
 * K % 128 == 0: two launches -- one quantiser for the INT8 and FP8 rows, then
 * the three tier GEMMs in one grid (an M-tile never mixes tiers).  Other K
 * (a multiple of 16): five launches, each tier's quantiser and GEMM in turn.
 * Both produce the same bits. */
int ee_routed_linear(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                     const int32_t* idx, const int32_t* counts, const int8_t* b_i8, const uint8_t* b_f8,
                     const void* b_f16, const float* b_scale, void* c, int64_t ldc, void* ws_codes,
                     float* ws_scale, ee_stream_t stream);

/* ---- fused MLP: the engine EE/test_engine.py:17-26 calls ----------------------
 * The reference's test constructs entropy_engine_cuda.EntropyMLPEngine(gate_w,
 * up_w, down_w, tau_low, tau_high) and calls .forward(hidden, entropy), but
 * EE/csrc/engine.cpp:202-216 never defines it; its baseline is
 * F.linear(F.silu(F.linear(x, gate_w)) * F.linear(x, up_w), down_w) under the
 * dispatcher's tier choice (EE/test_engine.py:33-39).  These entry points are
 * that engine with every linear on the tier GEMMs above, as the Llama block
 * gates its MLP (EE/python/dispatch.py:199-203).
 *
 * ee_silu_mul: act[m, f] = fp16( fp16(silu(g)) * u ) with g = gu[m, f],
 * u = gu[m, F + f] (gate columns, then up columns, as one [M, 2F] row); the
 * two roundings of torch's fp16 F.silu(g) * u. */
int ee_silu_mul(ee_engine* eng, const void* gu, int64_t ld_gu, void* act, int64_t ld_act, int64_t M,
                int64_t F, ee_stream_t stream);

/* ---- the Llama block's elementwise work around the gated linears -----------
 * ee_add_rmsnorm replaces the residual add + LlamaRMSNorm pair of the block
 * the reference wraps (EE/python/dispatch.py:150-247 calls the HF layer's
 * norms around its dispatched MLP): s = fp16(x + y) (y may be NULL: s = x; when
 * given, s is also written to x_out), then n = fp16(w * fp16(f32(s) *
 * rsqrt(mean(f32(s)^2) + eps))).  One row per wave; D % 8 == 0, D <= 4096.
 * The mean sums in another order than torch's reduction (last-bit effects). */
int ee_add_rmsnorm(ee_engine* eng, const void* x, int64_t ld_x, const void* y, int64_t ld_y, const void* w,
                   void* x_out, int64_t ld_xo, void* n_out, int64_t ld_n, int64_t T, int64_t D, float eps,
                   ee_stream_t stream);

/* ee_add_rmsnorm over the rows of a routing partition (idx/counts from ee_route
 * or ee_route_heads), processed in slot order, that also writes the routed
 * linear's INT8 and FP8 operands: slot i (source row idx[i]) of the INT8 slots
 * [0, counts[0]) and FP8 slots [counts[0], counts[0] + counts[1]) gets its
 * codes in codes + i * ld_c (D bytes) and its scale in scale[i] -- the bits
 * ee_routed_linear's quantiser would write from n_out (the quantisers of
 * EE/python/kernels.py:336-338 and :361).  FP16 slots get n_out only: the
 * INT8 and FP8 slots' rows of n_out are left unwritten (their normalised
 * values reach the GEMM as those codes).  x_out is written for every row, as
 * by ee_add_rmsnorm.  With ee_routed_gemm this removes the quantiser's launch,
 * its read of n_out, and the write of n_out for the quantised rows.
 * No reference counterpart: the reference quantises inside each GEMM wrapper
 * (EE/python/kernels.py:336-338, 361).  ld_c % 8 == 0, codes 8-byte aligned. */
int ee_add_rmsnorm_route(ee_engine* eng, const void* x, int64_t ld_x, const void* y, int64_t ld_y, const void* w,
                         void* x_out, int64_t ld_xo, void* n_out, int64_t ld_n, int64_t T, int64_t D, float eps,
                         const int32_t* idx, const int32_t* counts, void* codes, int64_t ld_c, float* scale,
                         ee_stream_t stream);

/* Rotary embedding of the q and k heads of a fused q|k|v projection output
 * ([B*S, (Hq + 2*Hkv)*d], row stride ld) into head-major q [B, Hq, S, d],
 * k and v [B, Hkv, S, d]: x*cos + rotate_half(x)*sin with each op rounded to
 * fp16, as the HF Llama attention the reference wraps computes it; cos/sin
 * fp16 [S, d].  q is stored scaled by q_scale (1: unscaled).  d % 16 == 0;
 * B*S*(Hq + Hkv)*d/16 work items plus the v chunks must stay below 2^31
 * (EE_ERR_UNSUPPORTED otherwise). */
int ee_qkv_rope(ee_engine* eng, const void* qkv, int64_t ld, const void* cos_t, const void* sin_t, void* q, void* k,
                void* v, int32_t B, int32_t S, int32_t Hq, int32_t Hkv, int32_t d, float q_scale,
                ee_stream_t stream);
/* The same with v written transposed for ee_attention_causal: vt [B, Hkv, d, S],
 * row (b, h, j) holding v[.., j] of every token, and within each group of 16
 * tokens the order 0-3, 8-11, 4-7, 12-15.  S % 16 == 0.  No counterpart in
 * the reference (a layout of this build's fused attention). */
int ee_qkv_rope_vt(ee_engine* eng, const void* qkv, int64_t ld, const void* cos_t, const void* sin_t, void* q,
                   void* k, void* vt, int32_t B, int32_t S, int32_t Hq, int32_t Hkv, int32_t d, float q_scale,
                   ee_stream_t stream);

/* Causal grouped-query attention fused with the Shannon entropy of its
 * probability rows: for batch b, query head h (kv head h / (Hq / Hkv)) and
 * query s, over keys c <= s, x_c = fp16(q . k_c), p = softmax(x),
 * out = fp16(sum p_c v_c) and H = ln Z - sum p_c (x_c - max x) -- the HF
 * Llama attention whose probabilities EE/python/dispatch.py:243-245 takes the
 * entropy of, with the entropy of softmax_entropy (EE/python/kernels.py:
 * 264-312), without materialising the S x S scores.  q [B, Hq, S, d] already
 * scaled (ee_qkv_rope's q_scale), k [B, Hkv, S, d], vt from ee_qkv_rope_vt;
 * out fp16 [B*S, ld_out] token-major (head h at columns h*d ..), h f32
 * [B, Hq, S].  d == 64, S % 64 == 0, Hq / Hkv even.  Results agree with the unfused path
 * (fp16 scores, ee_softmax_entropy, a product with v) to fp16 rounding: the
 * probabilities here are fp16(e^(x - m_running)) normalised at the end. */
int ee_attention_causal(ee_engine* eng, const void* q, const void* k, const void* vt, void* out, int64_t ld_out,
                        float* h, int32_t B, int32_t S, int32_t Hq, int32_t Hkv, int32_t d, ee_stream_t stream);

/* Weight preparation: gate_w, up_w fp16 [F, H] and down_w fp16 [H, F] (the
 * nn.Linear layout, EE/test_engine.py:12-14) quantised per output channel as
 * quantize_weights_int8 does (EE/python/dispatch.py:43-48), into the caller's
 * buffers: gu_* hold the [2F, H] operand (gate rows 0..F-1, up rows F..2F-1)
 * as int8 codes, e4m3 codes, W8A16 fp16 weights and f32 scales [2F], with gate
 * and up rows interleaved in blocks of 32 (the SwiGLU layout below); dn_* the
 * [H, F] down operand and scales [H].  All 16-byte aligned, row stride = K.
 * F % 32 == 0. */
int ee_mlp_prepare(ee_engine* eng, const void* gate_w, const void* up_w, const void* down_w, int64_t H,
                   int64_t F, int64_t ld_gate, int64_t ld_up, int64_t ld_down, int8_t* gu_i8, uint8_t* gu_f8,
                   void* gu_f16, float* gu_scale, int8_t* dn_i8, uint8_t* dn_f8, void* dn_f16, float* dn_scale,
                   ee_stream_t stream);

/* Workspace bytes ee_mlp_forward needs for M rows (routed != 0: per-row
 * tiers); -1 for a bad shape. */
int64_t ee_mlp_workspace_bytes(int64_t M, int64_t H, int64_t F, int32_t routed);

/* out[M, H] = down( silu(gate(x)) * up(x) ) for x fp16 [M, H].
 * h_rows == NULL: one tier for the call from `entropy` by the dispatcher's
 * strict compares (EE/python/dispatch.py:74-79): INT8 = per-row int8
 * activations (EE_QUANT_I8_DISPATCH) on the I8 GEMM, FP8 = per-row e4m3 on
 * the F8 GEMM, FP16 = W8A16; the intermediate is re-quantised by the same
 * tier before the down GEMM, as a separate dispatched linear would.
 * h_rows != NULL (f32 [M]): one tier per row (ee_route), both linears on
 * ee_routed_linear; `entropy` is ignored.  No host synchronisation, no
 * allocation; workspace 256-byte aligned, ws_bytes >= ee_mlp_workspace_bytes.
 * The gate|up GEMM writes silu(gate) * up directly (SwiGLU epilogue) when H
 * allows the pipelined kernels (H % 128 == 0); otherwise it stores gate|up and
 * a separate pass applies the activation -- the same bits either way.
 * Contract: H % 16 == 0; F % 32 == 0; ld_x multiple of 8; ldo multiple of 4. */
int ee_mlp_forward(ee_engine* eng, const void* x, int64_t ld_x, int64_t M, int64_t H, int64_t F,
                   const int8_t* gu_i8, const uint8_t* gu_f8, const void* gu_f16, const float* gu_scale,
                   const int8_t* dn_i8, const uint8_t* dn_f8, const void* dn_f16, const float* dn_scale,
                   double entropy, const float* h_rows, double tau_low, double tau_high, void* out, int64_t ldo,
                   void* workspace, int64_t ws_bytes, ee_stream_t stream);

/* ---- SwiGLU forms: the gate|up projection of a Llama MLP with its activation -
 * The block the reference gates computes down(silu(gate(x)) * up(x))
 * (EE/python/dispatch.py:199-203, EE/test_engine.py:35).  With gate and up
 * as one operand whose rows are interleaved in blocks of 32 (rows 64k..64k+31
 * = gate rows 32k.., rows 64k+32..64k+63 = up rows 32k..; ee_interleave_gate_up
 * builds it from gate rows followed by up rows), the GEMM epilogue pairs each
 * gate output with its up output and writes act [M, N/2] =
 * fp16(fp16(silu(gate)) * up) -- the same bits as the plain GEMM followed by
 * ee_silu_mul, without the [M, N] intermediate.  N % 64 == 0; K * element
 * size % 128 == 0 (the pipelined kernels); act 16-byte aligned, ld_act % 8 == 0. */
int ee_gemm_swiglu(ee_engine* eng, int32_t kind, const void* a, int64_t lda, const void* b_nk, int64_t ldb, void* act,
                   int64_t ld_act, const float* a_scale, const float* b_scale, int32_t M, int32_t N, int32_t K,
                   const int32_t* a_idx, const int32_t* c_idx, const int32_t* counts, int32_t tier,
                   ee_stream_t stream);
int ee_routed_linear_swiglu(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                            const int32_t* idx, const int32_t* counts, const int8_t* b_i8, const uint8_t* b_f8,
                            const void* b_f16, const float* b_scale, void* act, int64_t ld_act, void* ws_codes,
                            float* ws_scale, ee_stream_t stream);

/* ---- allocation-free routed linear ----------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): ee_routed_linear without the ws_codes / ws_scale
 * workspace.  The codes and scales live in a device array of the library
 * (EE_NOALLOC_MAX_CODE_BYTES + 4 * EE_NOALLOC_MAX_ROWS bytes, one copy per
 * GPU, held until the process ends), resolved once per device when an engine
 * is created.  Nothing is allocated and nothing synchronises.  Limits:
 * M <= EE_NOALLOC_MAX_ROWS and M * K <= EE_NOALLOC_MAX_CODE_BYTES, else
 * EE_ERR_UNSUPPORTED.  Every call on one GPU shares the array: calls that
 * overlap on one GPU (other streams, other threads) race.  Same results as
 * ee_routed_linear. */
#define EE_NOALLOC_MAX_ROWS 16384
#define EE_NOALLOC_MAX_CODE_BYTES (32 * 1024 * 1024)
int ee_routed_linear_noalloc(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                             const int32_t* idx, const int32_t* counts, const int8_t* b_i8, const uint8_t* b_f8,
                             const void* b_f16, const float* b_scale, void* c, int64_t ldc, ee_stream_t stream);
/* ee_routed_linear and ee_routed_linear_swiglu without their quantiser: the
 * INT8 and FP8 slots' codes [M, K] (row stride K) and scales [M] were written
 * beforehand, by ee_add_rmsnorm_route (the same bits as the quantiser).  x is
 * still read for the FP16 slots.  One launch; K % 128 == 0. */
int ee_routed_gemm(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                   const int32_t* idx, const int32_t* counts, const int8_t* b_i8, const uint8_t* b_f8,
                   const void* b_f16, const float* b_scale, void* c, int64_t ldc, const void* codes,
                   const float* scale, ee_stream_t stream);
int ee_routed_gemm_swiglu(ee_engine* eng, const void* x, int64_t ld_x, int32_t M, int32_t K, int32_t N,
                          const int32_t* idx, const int32_t* counts, const int8_t* b_i8, const uint8_t* b_f8,
                          const void* b_f16, const float* b_scale, void* act, int64_t ld_act, const void* codes,
                          const float* scale, ee_stream_t stream);
/* Rows 0..F-1 (gate) and F..2F-1 (up) of src into the interleaved order above
 * (any row payload: int8 codes, e4m3 codes, fp16 weights, or 4-byte scales with
 * row_bytes = 4).  F % 32 == 0; not in place. */
int ee_interleave_gate_up(ee_engine* eng, const void* src, int64_t ld_src_bytes, void* dst, int64_t ld_dst_bytes,
                          int64_t F, int64_t row_bytes, ee_stream_t stream);

/* ---- CubinEngine counterpart (EE/csrc/engine.cpp:64-216) --------------------
 * One code object + one GEMM function, launched on the caller's stream (the
 * reference launched on the NULL stream, engine.cpp:160).  create mirrors the
 * constructor (engine.cpp:73-104; num_warps counts wave64s); from_metadata
 * reads "shared", "num_warps", "BLOCK_M", "BLOCK_N" from a meta JSON
 * (engine.cpp:168-199).  forward mirrors engine.cpp:106-166 but takes B in
 * operand order [N, K] and a caller-allocated fp16 C [M, N]. */
int ee_module_engine_create(const char* code_object_path, const char* func_name, int32_t shared_mem,
                            int32_t num_warps, int32_t block_m, int32_t block_n, ee_module_engine** out);
int ee_module_engine_from_metadata(const char* code_object_path, const char* meta_json_path,
                                   const char* func_name, ee_module_engine** out);
int ee_module_engine_info(const ee_module_engine* me, int32_t* shared_mem, int32_t* num_warps,
                          int32_t* block_m, int32_t* block_n);
int ee_module_engine_forward(ee_module_engine* me, const int8_t* a, int64_t lda, const int8_t* b_nk,
                             int64_t ldb, void* c, int64_t ldc, const float* a_scale, const float* b_scale,
                             int32_t M, int32_t N, int32_t K, ee_stream_t stream);
int ee_module_engine_destroy(ee_module_engine* me);

#ifdef __cplusplus
}
#endif
#endif /* ENTROPY_ENGINE_H */
