/*
 * qmm.h — C ABI of libqmm.so, the MI355X (gfx950) quantized-weight matmul library.
 *
 * Each entry point replaces one family of the reference's Loom kernels, keeping its argument order and buffer
 * layouts (paths relative to the reference root, S/ = skills/loom-port-llm/starter/). The reference boundary is
 * the `kernel.launch @name[grid](args)` contract its generators emit; here the kernel-name parameters (format, K,
 * mode, token group) become explicit arguments and every call takes the HIP stream it is enqueued on.
 *
 * Conventions
 *   - Pointers are caller-owned device pointers (no allocation happens inside any entry point except where a
 *     workspace size function says so); weights are the raw GGUF block bytes.
 *   - Calls are asynchronous on `stream` (a hipStream_t, NULL = the default stream) and return QMM_OK (0) or a
 *     negative qmm_status after host-side validation; a nonzero return means nothing was launched.
 *   - Outputs are written in full; with `accumulate` / QMM_GEMM_ACC the kernel reads and adds to them.
 */
#ifndef QMM_H
#define QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *qmm_stream_t; /* hipStream_t */

enum qmm_status {
  QMM_OK = 0,
  QMM_ERR_FORMAT = -1,    /* unsupported weight format for this entry point */
  QMM_ERR_SHAPE = -2,     /* a size violates a divisibility / range precondition */
  QMM_ERR_ALIGN = -3,     /* a pointer is not aligned as the kernel requires */
  QMM_ERR_NULL = -4,      /* a required pointer is NULL */
  QMM_ERR_RANGE = -5,     /* an enum or small integer argument is out of range (E, top-k, gating, ...) */
  QMM_ERR_DTYPE = -6,     /* unsupported activation / output dtype */
  QMM_ERR_LAUNCH = -7,    /* the HIP launch itself failed */
  QMM_ERR_WORKSPACE = -8  /* workspace too small */
};

/* QMM_MXFP4T: MXFP4 in MFMA-tiled planes (qmm_tile_mxfp4), the grouped GEMM's fast weight layout.
 * QMM_Q4_KT: Q4_K in the lane-ordered tiled layout (qmm_tile_q4k), the int8-activation decode GEMV's fast layout.
 * QMM_Q6_K: GGUF Q6_K (210 bytes per 256 values; ffn_down of the Q4_K_M files), read in place from a 4-byte aligned
 *           tensor (its super-blocks start on even addresses).
 * QMM_Q4_0T: Q4_0 in the lane-ordered tiled layout (qmm_tile_q40), the int8-activation decode GEMV's fast layout. */
enum qmm_format {
  QMM_Q4_0 = 0, QMM_Q4_K = 1, QMM_MXFP4 = 2, QMM_MXFP4S = 3, QMM_MXFP4T = 4, QMM_Q4_KT = 5, QMM_Q6_K = 6, QMM_Q4_0T = 7
};
/* A gate/up pair whose up matrix has another format than the gate matrix (the reference's "GATE+UP" formats, e.g. a
 * Q4_K_M layer with a Q4_K gate and a Q6_K up: g_gemm_{fmt}_{fmt2}_swiglu S/gen_gemm.py:535-547, g_moe_ggu_{fg}_{fu}
 * S/gen_moe.py:1126-1141, g_moe_gu_{fg}_{fu} S/gen_moe.py:535-552): pass QMM_GATE_UP(gate format, up format) as the
 * `fmt` of a call that computes silu(gate) * up (qmm_mv_swiglu, qmm_gemm in QMM_GEMM_SWIGLU mode, qmm_moe_expert_mv
 * and qmm_moe_grouped in mode 0, qmm_moe_routed). The high byte holds the up format + 1; a plain format (high byte 0)
 * is both matrices' format. */
#define QMM_GATE_UP(gate, up) ((gate) | (((up) + 1) << 8))
enum qmm_dtype {
  QMM_F32 = 0,
  QMM_F16 = 1,
  QMM_BF16 = 2,
  QMM_MXFP8 = 3, /* E4M3 codes + E8M0 per 32 */
  QMM_Q8 = 4     /* planar Q8_1: int8 codes [rows, K], then at byte rows*K f32 (f16-rounded d, code sum) per 32 */
};
enum qmm_gemm_mode { QMM_GEMM_STORE = 0, QMM_GEMM_ACC = 1, QMM_GEMM_SWIGLU = 2 };
enum qmm_act { QMM_ACT_SILU = 0, QMM_ACT_SWIGLU_OAI = 1 };
enum qmm_moe_flags { QMM_MOE_Q8 = 1 /* the decode chain on Q8_1 activations (the reference's MOE_Q8) */ };

/* Library version (major*10000 + minor*100 + patch) and the text of a status code. */
int qmm_version(void);
const char *qmm_strerror(int status);

/* Bytes of one weight row of K values: K / values_per_block * bytes_per_block
 * (replaces S/gen_llm.py:182-183 row_bytes; S/formats.py:5-19 FMT/SB). Returns 0 for an invalid (fmt, k). */
int64_t qmm_row_bytes(int fmt, int64_t k);

/* Bit-exact dequantization of `rows` rows of K values to f32 [rows, K]
 * (the values @g_q4_0_values S/quant_values.loom:386-408, @g_q4_k_values S/gen_llm.py:288-326,
 *  @g_mxfp4_values S/gen_llm.py:786-841 and @g_mxfp4s_values S/gen_llm.py:844-895 produce).
 * w: weight bytes; ws: the E8M0 scale plane for QMM_MXFP4S / QMM_MXFP4T, else NULL (QMM_MXFP4T: rows % 32 == 0,
 * K % 64 == 0; QMM_Q4_KT: rows % 16 == 0, K % 256 == 0; QMM_Q4_0T: rows % 16 == 0, K % 512 == 0). */
int qmm_dequant(int fmt, const void *w, const void *ws, int64_t rows, int64_t k, float *out, qmm_stream_t stream);

/* Decode matrix-vector product, the g_mv_{fmt}_k{K}[_t{TG}][_r{R}] family
 * (S/gen_llm.py:1159-1378 `_mv`, launch args S/gen_llm.py:1187-1197):
 *   y[t, r] = (accumulate ? y[t, r] : 0) + sum_k x[t, k] * W[r, k]   for t < tokens, r < n, fp32 accumulation.
 * x: [tokens, k] of x_dtype (QMM_F32 as the reference, or QMM_BF16); w: n rows of qmm_row_bytes(fmt, k) bytes;
 * ws: scale plane for QMM_MXFP4S else NULL; y: f32 [tokens, n]. Every token is computed with the same arithmetic
 * whatever `tokens` is, so a multi-token call equals one-token calls bit for bit. fmt QMM_Q4_0T: the Q4_0 weights in
 * the tiled layout of qmm_tile_q40 (n % 16 == 0, K = 512 U NW with U <= 3, NW <= 8), per block d (sum q x - 8 sum x)
 * in f32 (the reference's f32 Q4_0 decode up to f32 rounding). */
int qmm_mv(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype,
           const void *w, const void *ws, float *y, qmm_stream_t stream);

/* Decode swiglu matvec, g_mv_{fmt}_k{K}_swiglu[_t{TG}] (S/gen_llm.py:1159-1197; launch args (n, tokens, accumulate,
 * x, w, w2, y)): y[t, r] = (accumulate ? y[t, r] : 0) + silu(sum_k x[t, k] W[r, k]) * (sum_k x[t, k] W2[r, k]),
 * silu(g) = g / (1 + e^-g), fp32 accumulation. fmt QMM_Q4_0 / QMM_Q4_K / QMM_Q6_K / QMM_MXFP4 (the reference has no
 * swiglu matvec on split planes), or QMM_GATE_UP(gate, up) of two of them; w (gate) and w2 (up) [n, k]; x f32 / bf16
 * [tokens, k]; y f32 [tokens, n]. */
int qmm_mv_swiglu(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype,
                  const void *w, const void *w2, float *y, qmm_stream_t stream);

/* Q8_1 activation quantizer, g_quant_q8 (S/gen_llm.py:684-749; llama.cpp quantize_q8_1): per group of 32 values
 * d = amax / 127, q = sign(x/d) floor(|x/d| + 1/2) (0 when d = 0). x: f32 or bf16 [rows, k], k % 32 == 0; xq: the
 * planar buffer (QMM_Q8) of rows * k code bytes followed by rows * k / 32 f32 pairs (f16-rounded d, sum of codes),
 * 16-byte aligned. */
int qmm_quant_q8(int64_t rows, int64_t k, const void *x, int x_dtype, void *xq, qmm_stream_t stream);

/* Decode matrix-vector product on Q8_1 activations, the g_mv_{fmt}_k{K}[_t{TG}]_q8[_r{R}] family
 * (S/gen_llm.py:1288-1301, iq_dot :1024-1071; the reference's default decode path): per 32-value group an exact
 * integer dot di of weight codes and activation codes, then for Q4_K (di d sc_g - xs dmin m_g) da and for Q4_0
 * (d da) di with codes q - 8, summed in f32. fmt QMM_Q4_K (k % 256 == 0) or QMM_Q4_0 (k % 64 == 0). x: the planar
 * buffer of qmm_quant_q8 (x_dtype QMM_Q8) for tokens rows, or -- Q4_K with k = 4096 or 8192 only -- f32 / bf16
 * [tokens, k] rows, quantized inside the kernel exactly as qmm_quant_q8 does (same result bit for bit). y: f32
 * [tokens, n]. A multi-token call equals one-token calls bit for bit.
 * fmt QMM_Q4_KT: the weights in the tiled layout of qmm_tile_q4k (n % 16 == 0, K % 512 == 0, K / 512 a multiple of
 * at most 4 of a count of at most 8 waves); x planar Q8_1 or f32 / bf16 rows for every such K. For K = 4096 the
 * results equal the QMM_Q4_K call's bit for bit. fmt QMM_Q4_0T: the Q4_0 weights in the tiled layout of qmm_tile_q40,
 * the same shapes and activations as QMM_Q4_KT, per block (d da) (di - 8 xs) with di the dot of the codes q: the
 * QMM_Q4_0 call's sum, in the tiled kernel's summation order. */
int qmm_mv_q8(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype,
              const void *w, float *y, qmm_stream_t stream);

/* The two-matrix decode matvecs on Q8_1 activations (S/gen_llm.py:1159-1197, int8 variants; the reference's default
 * decode path for the FFN gate / up and for attention q + gate):
 *   g_mv_{fmt}_k{K}_swiglu[_t{TG}]_q8[_r{R}], launch args (n, tokens, accumulate, x, w, w2, y):
 *       y[t, r] = (accumulate ? y[t, r] : 0) + silu(g) u,   silu(g) = g / (1 + e^-g)
 *   g_mv_{fmt}_k{K}_pair[_t{TG}]_q8[_r{R}], launch args (n, tokens, accumulate, x, w, w2, y, y2):
 *       y[t, r] (+)= g,  y2[t, r] (+)= u
 * with g = x W^T and u = x W2^T computed as qmm_mv_q8 computes one matrix (per 32-value group an exact int32 dot of
 * codes, f32 fixups, the same reductions), so each is bit for bit the one-matrix kernel's of the same layout and K
 * (for GGUF Q4_K at K = 4096 / 8192 that is the tiled layout's, since the one-matrix GGUF call takes its K-sliced
 * kernel there). fmt QMM_Q4_KT / QMM_Q4_0T: W and W2 in the tiled layout of qmm_tile_q4k / qmm_tile_q40, x planar
 * Q8_1 or f32 / bf16 rows
 * (quantized in the kernel exactly as qmm_quant_q8 does); QMM_Q4_K / QMM_Q4_0 / QMM_Q6_K (GGUF): x planar Q8_1.
 * W, W2: [n, k]; y, y2: f32 [tokens, n]. A multi-token call equals one-token calls bit for bit. */
int qmm_mv_swiglu_q8(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype,
                     const void *w, const void *w2, float *y, qmm_stream_t stream);
int qmm_mv_pair_q8(int fmt, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype,
                   const void *w, const void *w2, float *y, float *y2, qmm_stream_t stream);

/* Prefill GEMM, the g_gemm_{fmt}_{store|acc|swiglu}[_m128|_m256] family
 * (S/gen_gemm.py:535-703, :706, :1224; launch args S/gen_gemm.py:549-556):
 *   store:  Y = (X W^T) * inv[row]        acc: Y += (X W^T) * inv[row]
 *   swiglu: Y = silu((X W^T) inv) * ((X W2^T) inv)
 * x: f16 [rows, k] (x_dtype QMM_F16), the reference's row-scaled x16 from qmm_row_scale_f16; scales: f32 [rows, 2]
 * with inv = scales[row, 1] (the reference's (2^-e, 2^e) pairs), or NULL for inv = 1; y: [rows, n] of y_dtype
 * (QMM_F32 as the reference, or QMM_BF16, rounded to nearest even). fp32 accumulation. K % 256 == 0. Weights are
 * dequantized to f16 as the reference stages them: Q4_K fma_f16(f16(q), f16(d sc), f16(-dmin m)); Q6_K (fmt
 * QMM_Q6_K, S/gen_gemm.py:369-444) fma_f16(f16(q), f16(d sc), f16(-32 d sc)) with q the unsigned 6-bit code; Q4_0
 * (fmt QMM_Q4_0, the reference's native Q4_0 staging S/moe_q4_0.py:11-38, S/gen_gemm.py:40-45) f16(q - 8) * d with
 * one f16 rounding, i.e. f16(d (q - 8)) for every finite d. MXFP4 weights go through qmm_gemm_mxfp4.
 * fmt QMM_Q4_KT: Q4_K in the tiled layout of qmm_tile_q4k (the int8 decode GEMV's; n % 16 == 0, K % 512 == 0), the
 * results equal the QMM_Q4_K call's on the GGUF blocks bit for bit, so one weight copy serves decode and prefill (the
 * reference's single weight view, S/gen_llm.py:5364-5371).
 * QMM_GEMM_SWIGLU: w is the gate matrix and w2 the up matrix (both [n, k]); silu(g) = g / (1 + e^-g); with
 * fmt = QMM_GATE_UP(gate, up) (Q4_K, Q6_K, Q4_0) the two matrices are in their own formats, g_gemm_{fmt}_{fmt2}_swiglu
 * (S/gen_gemm.py:535-547, :696-700).
 * Skip-padding (the reference's default GEMM_SKIP_PADDING): with scales, a 64-row tile whose rows all have
 * scales[row, 0] == 0 (padding rows of qmm_row_scale_f16_live) does no work and its y rows are not written. */
int qmm_gemm(int fmt, int mode, int64_t rows, int64_t k, int64_t n, const void *x, int x_dtype, const float *scales,
             const void *w, const void *w2, void *y, int y_dtype, qmm_stream_t stream);

/* Prefill GEMM on MXFP4 weights, the g_gemm_mxfp4s_{store|swiglu}_f8_m256 family (S/gen_mxfp4s.py:50-101; launch args
 * (rows, k, n, x, scales, w, ws [, w2, w2s], y)), on the gfx950 scaled f8f6f4 MFMA:
 *   store: Y = X8 W^T      acc: Y += X8 W^T      swiglu: Y = silu(X8 W^T) (X8 W2^T)
 * x: the MXFP8 activation of qmm_quant_mxfp8, E4M3 codes u8 [rows, k] with x_scales its E8M0 plane u8 [rows, k/32]
 * (one scale per 32 values, applied by the MFMA; the reference's gfx12 kernel scales fp8 rows by one power of two
 * each). fmt QMM_MXFP4S: w nibble plane [n, k/2], ws E8M0 plane [n, k/32]; QMM_MXFP4T: the MFMA-tiled planes of
 * qmm_tile_mxfp4 (n % 32 == 0). k % 64 == 0, k <= 12288. y: [rows, n] of y_dtype (QMM_F32, or QMM_BF16 rounded to
 * nearest even). fp32 accumulation. GGUF MXFP4 blocks go through qmm_repack_mxfp4 once at load. */
int qmm_gemm_mxfp4(int fmt, int mode, int64_t rows, int64_t k, int64_t n, const void *x, const void *x_scales,
                   const void *w, const void *ws, const void *w2, const void *ws2, void *y, int y_dtype,
                   qmm_stream_t stream);

/* MoE router top-k from logits, g_moe_route / g_moe_route_tr after the router matvec
 * (S/gen_moe.py:116-252, :255-500; llama.cpp gating: 1 softmax, 2 sigmoid, 3 softmax over the picked logits):
 *   ids i32 [tokens, KU] = the top-KU experts by score (ties to the lower id), wts f32 [tokens, KU].
 * logits f32 [tokens, E]; bias f32 [E] or NULL (gating 2: selection bias; gating 3: added to the logits);
 * norm != 0 divides the weights by max(sum, 6.103515625e-05); scale multiplies them. E <= 256, KU <= 8. */
int qmm_moe_topk(const float *logits, int64_t tokens, int E, int KU, int gating, int norm, float scale,
                 const float *bias, int32_t *ids, float *wts, qmm_stream_t stream);

/* qmm_moe_topk together with the activation operand of the grouped gate/up GEMM, for the token rows x (bf16
 * [tokens, H], H <= 4096): the reference's prefill chain issues the route (g_moe_route, S/gen_moe.py:116-500) and
 * the operand (g_row_scale_f16, S/gen_llm.py:1843-1915, for GGUF experts; the MXFP8 quantization for MXFP4 experts)
 * as separate kernels (S/gen_llm.py:5373-5376); both are per token, so one wave per token does both here (no
 * counterpart as one kernel in the reference). ids / wts as qmm_moe_topk; op_dtype QMM_F16: xo f16 [tokens, H] and
 * xo_scales f32 [tokens, 2] as qmm_row_scale_f16 (H % 8 == 0); QMM_MXFP8: xo E4M3 codes u8 [tokens, H] and
 * xo_scales E8M0 u8 [tokens, H / 32] as qmm_quant_mxfp8 (H % 32 == 0). Every output equals the separate calls'
 * bit for bit. */
int qmm_moe_topk_operand(const float *logits, int64_t tokens, int E, int KU, int gating, int norm, float scale,
                         const float *bias, int32_t *ids, float *wts, int64_t H, const void *x, int x_dtype,
                         int op_dtype, void *xo, void *xo_scales, qmm_stream_t stream);

/* The router with its matvec, g_moe_route / g_moe_route_tr / g_moe_route_tr_live (S/gen_moe.py:116-500; launch
 * S/gen_llm.py:5373, :5380): logits f32 [tokens, E] = x W^T (fp32 accumulation; x f32 or bf16 [tokens, H], W the
 * router weight ffn_gate_inp f32 or bf16 [E, H], H % 4 == 0), then qmm_moe_topk on them. logits is the caller's
 * buffer and holds the logits afterwards. info (i32 [tokens, 4]) or NULL: tokens with info[t, 2] == 0 are padding
 * of the epoch (_live) and get no ids or weights (qmm_moe_bucket with the same info never reads them). */
int qmm_moe_route(int64_t tokens, int64_t H, int E, int KU, int gating, int norm, float scale, const void *x,
                  int x_dtype, const void *w, int w_dtype, const float *bias, const int32_t *info, float *logits,
                  int32_t *ids, float *wts, qmm_stream_t stream);

/* Shared-expert gate, g_moe_shared_gate (S/gen_moe.py:780-823): sg f32 [tokens] = sigmoid(x[t] . w), x f32 or bf16
 * [tokens, H], w (ffn_gate_inp_shexp) f32 or bf16 [H], H % 4 == 0, fp32 accumulation. */
int qmm_moe_shared_gate(int64_t tokens, int64_t H, const void *x, int x_dtype, const void *w, int w_dtype, float *sg,
                        qmm_stream_t stream);

/* Per-expert output scale folded into the combine weights, g_moe_wscale (S/gen_moe.py:1010-1045; ffn_down_exps.scale):
 * wts[t, k] *= scale[clamp(ids[t, k], 0, E - 1)]. ids i32 / wts f32 [tokens, KU], scale f32 [E]. */
int qmm_moe_wscale(int64_t tokens, int KU, int E, const int32_t *ids, const float *scale, float *wts,
                   qmm_stream_t stream);

/* MoE bucket / permute, g_moe_bucket (S/gen_moe.py:829-955; scratch sizes S/gen_llm.py:5388-5432):
 * assignments a = t*KU + k of live tokens (info[t, 2] != 0; info i32 [tokens, 4] or NULL = all live) grouped by
 * expert into 64-row tiles in expert-id order, assignments in ascending a inside each expert's segment.
 *   tile_info i32 [max_tiles, 2] = (expert, rows) or (-1, 0); rowmap i32 [max_tiles*64] = assignment or -1;
 *   pos i32 [tokens*KU] = row or -1.   max_tiles >= tokens*KU/64 + E. */
int qmm_moe_bucket(int64_t tokens, int KU, int E, int64_t max_tiles, const int32_t *info, const int32_t *ids,
                   int32_t *tile_info, int32_t *rowmap, int32_t *pos, qmm_stream_t stream);

/* Decode expert matvecs, g_moe_gu_{fmt}[_fused]_k{H}_r{R} / g_moe_dn_{fmt}_k{FE}_r{R}
 * (S/gen_moe.py:535-727; launch args :564):
 *   gu (mode 0): act[a] = act_fn(Wg[e] x[a/KU], Wu[e] x[a/KU])      e = ids[a], a < assignments
 *   dn (mode 1): ys[a]  = Wd[e] x[a]
 * n: output width (FE for gu, H for dn); k: input width. w: expert tensor [E, n, k] (gu: gate; fused != 0: one
 * [E, 2n, k] tensor, each expert's n gate rows then its n up rows, w2 ignored); w2: up tensor [E, n, k] for gu.
 * bias: for gu f32 [E, n] gate bias and bias2 up bias; for dn bias [E, n]; NULL = none. x: [rows, k] of x_dtype
 * (gu: rows = assignments/KU tokens; dn: rows = assignments). y: f32 [assignments, n]. gu with two tensors may take
 * fmt = QMM_GATE_UP(gate, up) of GGUF formats (g_moe_gu_{fg}_{fu}, S/gen_moe.py:535-552, :643-649). */
int qmm_moe_expert_mv(int fmt, int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                      int64_t assignments, const int32_t *ids, const void *x, int x_dtype, const void *w,
                      const void *w2, const float *bias, const float *bias2, float *y, qmm_stream_t stream);

/* The decode expert matvecs on Q8_1 activations, g_moe_gu_{fmt}[_fused]_q8_k{H}_r{R} / g_moe_dn_{fmt}_q8_k{FE}_r{R}
 * (S/gen_moe.py:535-727 with int8 activations; the reference's default MOE_Q8 decode chain, S/gen_llm.py:5290-5303,
 * :5381-5383: the router input quantized once, the gate/up output quantized by qmm_quant_q8 before the down matvec):
 *   gu (mode 0): act[a] = act_fn(Wg[e] xq[a/KU], Wu[e] xq[a/KU])      e = clamp(ids[a], 0, E - 1)
 *   dn (mode 1): ys[a]  = Wd[e] xq[a]
 * with each product computed as qmm_mv_q8 computes it (exact int32 group dots, f32 fixups). fmt QMM_Q4_K / QMM_Q4_0 /
 * QMM_Q6_K; weights as qmm_moe_expert_mv (fused: one [E, 2n, k] gate_up tensor). x: the planar Q8_1 buffer of
 * qmm_quant_q8 over x_rows rows (gu: the assignments / KU tokens; dn: the assignments). bias / bias2 as
 * qmm_moe_expert_mv (the reference builds this path without expert biases), NULL = none. y: f32 [assignments, n]. */
int qmm_moe_expert_mv_q8(int fmt, int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                         int64_t assignments, const int32_t *ids, const void *x, const void *w, const void *w2,
                         const float *bias, const float *bias2, float *y, qmm_stream_t stream);

/* The reference's opt-in int8 decode of MXFP4 split planes (MXFP4S_Q8, S/formats.py:26-28): the int8 matvecs of
 * qmm_mv_q8 / qmm_mv_swiglu_q8 / qmm_mv_pair_q8 (mode 0 / 1 / 2; g_mv_mxfp4s_k{K}[_swiglu|_pair][_t{TG}]_q8,
 * S/gen_llm.py:1159-1197, :1288-1301) and of qmm_moe_expert_mv_q8 for mxfp4s weights, whose scale planes have no
 * place in those signatures. Per 32-value block: signed codes c = 2 x the E2M1 values (0 1 2 3 4 6 8 12 and
 * negatives) and d = 2^(e - 128) from the E8M0 byte (@g_mxfp4s_icodes, S/gen_mxfp4s.py:1113-1160), the exact integer
 * dot sum c q with the Q8_1 codes, then (d da) di (iq_dot, S/gen_llm.py:1047-1049). w / w2: nibble planes [n, k/2]
 * (byte j: values 2j low, 2j+1 high); ws / ws2: E8M0 planes [n, k/32]; k % 64 == 0. x: the planar Q8_1 buffer of
 * qmm_quant_q8 (x_dtype QMM_Q8). y (and y2, pair): f32 [tokens, n]. */
int qmm_mv_mxfp4s_q8(int mode, int64_t k, int64_t n, int64_t tokens, int accumulate, const void *x, int x_dtype,
                     const void *w, const void *ws, const void *w2, const void *ws2, float *y, float *y2,
                     qmm_stream_t stream);
/* The decode expert matvecs of qmm_moe_expert_mv_q8 on mxfp4s experts: w / ws the [E, n, k] planes (fused gate_up:
 * [E, 2n, k] planes, expert e's n gate rows then its n up rows, in both planes), w2 / ws2 the up planes when not
 * fused. */
int qmm_moe_expert_mv_mxfp4s_q8(int mode, int fused, int act, int64_t k, int64_t n, int E, int KU,
                                int64_t assignments, const int32_t *ids, const void *x, const void *w, const void *ws,
                                const void *w2, const void *ws2, const float *bias, const float *bias2, float *y,
                                qmm_stream_t stream);

/* qmm_moe_expert_mv for MXFP4 split planes (the reference's mxfp4s expert tensors, S/gen_llm.py:844-895):
 * w / w2 are nibble planes [E, rows, k/2] and ws / ws2 their E8M0 scale planes [E, rows, k/32]; with fused != 0
 * w and ws hold each expert's n gate rows then its n up rows and w2 / ws2 are ignored. */
int qmm_moe_expert_mv_split(int mode, int fused, int act, int64_t k, int64_t n, int E, int KU, int64_t assignments,
                            const int32_t *ids, const void *x, int x_dtype, const void *w, const void *ws,
                            const void *w2, const void *ws2, const float *bias, const float *bias2, float *y,
                            qmm_stream_t stream);

/* qmm_moe_expert_mv for MXFP4 in MFMA-tiled planes (QMM_MXFP4T from qmm_tile_mxfp4, each expert tensor tiled as
 * [E rows, k]), the planes the grouped prefill GEMM reads, so one weight copy serves decode and prefill (no reference
 * counterpart for the layout; the products are g_moe_gu_* / g_moe_dn_* on mxfp4s, S/gen_moe.py:535-727): w / w2 the
 * tile planes, ws / ws2 their scale groups; fused as qmm_moe_expert_mv_split (expert e's n gate rows then its n up
 * rows in one tiled tensor). n % 32 == 0, k % 64 == 0, assignments <= 65535. Per 32-value block the split-plane
 * kernel's arithmetic (fp4 x activation pairs in f32, times the E8M0 scale); the blocks are summed in another order
 * (the rel-L2 bar against the oracle holds, not bit equality with the split-plane call). A multi-token call equals
 * one-token calls bit for bit. */
int qmm_moe_expert_mv_tiled(int mode, int fused, int act, int64_t k, int64_t n, int E, int KU, int64_t assignments,
                            const int32_t *ids, const void *x, int x_dtype, const void *w, const void *ws,
                            const void *w2, const void *ws2, const float *bias, const float *bias2, float *y,
                            qmm_stream_t stream);

/* Grouped expert GEMM over bucketed rows, g_moe_ggu_{fmt}[_fused]_k{H} / g_moe_gdn_{fmt}_k{FE}
 * (S/gen_moe.py:1126-1228). The name fields (fmt, mode gu / dn, fused, the activation, E and KU, which the reference
 * compiles into the kernel) come first, then the launch arguments in the reference's order
 * (max_rows, k, n, xrows, tile_info, rowmap, x16, scales, w [, w2] [, biases], y) (S/gen_llm.py:5376-5378), with the
 * split-plane scale planes beside their nibble planes:
 *   gu (mode 0): act[r] = act_fn(Wg[e] x[t] inv + bias[e], Wu[e] x[t] inv + bias2[e]),  t = rowmap[r]/KU
 *   dn (mode 1): ys[r]  = Wd[e] x[r] inv + bias[e]                                      (x rows sorted)
 * for every row r of every 64-row tile whose expert e = tile_info[tile, 0] >= 0; rows with rowmap[r] == -1 and the
 * rows of unused tiles are not written (the combine reads only the rows pos names). Weights as qmm_moe_expert_mv: w [E, n, k] (gu: gate;
 * fused != 0: [E, 2n, k], each expert's n gate rows then its n up rows; w2 the up tensor otherwise).
 *   QMM_Q4_K:   x is the row-scaled f16 operand (x_dtype QMM_F16) from qmm_row_scale_f16 with its scales f32
 *               [x_rows, 2] in x_scales (inv = scales[row, 1]); K % 256 == 0; f16 MFMA, weights staged as
 *               fma_f16(f16(q), f16(d sc), f16(-dmin m)).
 *   QMM_Q4_KT:  as QMM_Q4_K with the weights in the tiled layout of qmm_tile_q4k (each expert's [n, k] tiled as
 *               part of the [E n, k] tensor: n % 16 == 0): for K <= 4096 read by the narrow kernel as contiguous
 *               1 KB streams at every row count (the same staging, the products summed in another order), beyond
 *               that (K % 512 == 0) by the 64-row tile kernel at its tiled addresses, whose results then equal the
 *               QMM_Q4_K call's bit for bit (no counterpart in the reference: a load-time layout).
 *   QMM_Q6_K:   as QMM_Q4_K with Q6_K weights (staged as qmm_gemm stages them); g_moe_gdn_q6_k of the Q4_K_M
 *               expert layout (Q4_K gate / up, Q6_K down).
 *   QMM_Q4_0:   as QMM_Q4_K with Q4_0 weights, staged f16(d (q - 8)) (specialize_grouped, S/moe_q4_0.py:41-61).
 *   QMM_GATE_UP(gate, up) of QMM_Q4_K / QMM_Q6_K / QMM_Q4_0: gu with two tensors, each in its own format
 *               (g_moe_ggu_{fg}_{fu}, S/gen_moe.py:1126-1141).
 *   QMM_MXFP4S: weights in split planes, ws / ws2 the E8M0 planes [E, rows, k/32]; x is MXFP8 (x_dtype
 *               QMM_MXFP8) from qmm_quant_mxfp8: E4M3 codes u8 [x_rows, k] with x_scales u8 [x_rows, k/32];
 *               K % 64 == 0; scaled f8f6f4 MFMA, inv = 1.
 *   QMM_MXFP4T: as QMM_MXFP4S with the weights in MFMA-tiled planes from qmm_tile_mxfp4 (each expert's [rows, k]
 *               tiled on its own: n % 32 == 0; a fused gate_up expert tiles as 2n rows); the same results bit for
 *               bit, read as contiguous 1 KB streams (no counterpart in the reference: a load-time layout).
 * max_rows: rows of the sorted outputs, max_tiles * 64 (a multiple of 64). x_rows: rows of x (gu: tokens; dn: >=
 * max_rows). y: f32 [max_rows, n].
 * bias / bias2: the per-expert output biases f32 [E, n] (gpt-oss ffn_{gate,up,down}_exps.bias, _gemm_bias_act
 * S/gen_moe.py:958-1007), added after the row inverse and before the activation; NULL = none (bias2: gu only). */
int qmm_moe_grouped(int fmt, int mode, int fused, int act, int E, int KU, int64_t max_rows, int64_t k, int64_t n,
                    int64_t x_rows, const int32_t *tile_info, const int32_t *rowmap, const void *x, int x_dtype,
                    const void *x_scales, const void *w, const void *ws, const void *w2, const void *ws2,
                    const float *bias, const float *bias2, float *y, qmm_stream_t stream);

/* The gate/up grouped GEMM (mode 0 of qmm_moe_grouped, MXFP4 weights) with the MXFP8 quantization of its output
 * fused into the epilogue (no reference counterpart: the reference writes act f32 and its next kernel reads it back).
 * codes u8 [max_rows, n] and scales u8 [max_rows, n/32] are exactly qmm_quant_mxfp8(act, tile_info) of the
 * act qmm_moe_grouped would write (the down GEMM's A operand), bit for bit; rows of unused tiles are not written,
 * dead rows come out as codes 0 and scale byte 0. fmt QMM_MXFP4S or QMM_MXFP4T; n % 32 == 0; codes 16-byte
 * aligned. Other arguments as qmm_moe_grouped. */
int qmm_moe_grouped_mxfp8(int fmt, int fused, int act, int E, int KU, int64_t max_rows, int64_t k, int64_t n,
                          int64_t x_rows, const int32_t *tile_info, const int32_t *rowmap, const void *x,
                          const void *x_scales, const void *w, const void *ws, const void *w2, const void *ws2,
                          const float *bias, const float *bias2, uint8_t *codes, uint8_t *scales,
                          qmm_stream_t stream);

/* Row-scaled f16 producer, g_row_scale_f16[_tiles] (S/gen_llm.py:1843-1915, S/gen_moe.py:503-527):
 * per row e = clamp(exponent(max|x|) - 13, 0, 100), x16 = f16(x * 2^-e), scales = (2^-e, 2^e).
 * tile_info (i32 [rows/64, 2]) or NULL: only the first tile_info[t, 1] rows of each tile t with an expert are
 * converted (the bucket fills tiles from the top); the other rows are skipped. x: [rows, k] of x_dtype
 * (QMM_F32 as the reference, or QMM_BF16). This is the A operand qmm_gemm takes. */
int qmm_row_scale_f16(int64_t rows, int64_t k, const void *x, int x_dtype, float *scales, void *x16,
                      const int32_t *tile_info, qmm_stream_t stream);

/* qmm_row_scale_f16 over listed rows only: for i < n, row rows[i] (skipped when < 0) of x [.., k] is scaled and
 * written where qmm_row_scale_f16 writes it (x16 / scales at that row). With the bucket's pos as the list these are
 * the rows g_row_scale_f16_tiles (S/gen_moe.py:503-527) scales, by a grid over the assignments instead of over every
 * tile row. k % 8 == 0, k <= 8192, x and x16 16-byte aligned. */
int qmm_row_scale_f16_rows(int64_t n, const int32_t *rows, int64_t k, const void *x, int x_dtype, float *scales,
                           void *x16, qmm_stream_t stream);

/* g_row_scale_f16_live (S/gen_llm.py:1915-1937): qmm_row_scale_f16 over an epoch's rows, where a padding row
 * (info i32 [rows, 4] with info[row, 2] == 0) gets scale and inverse 0 and zero f16 values without its x row being
 * read. qmm_gemm skips a 64-row tile whose rows all have scale 0 (GEMM_SKIP_PADDING, S/gen_gemm.py:2188-2220). */
int qmm_row_scale_f16_live(int64_t rows, const int32_t *info, int64_t k, const void *x, int x_dtype, float *scales,
                           void *x16, qmm_stream_t stream);

/* MXFP8 activation quantizer, the A operand of the gfx950 scaled MFMA (no reference counterpart: the reference's
 * fp8 producers, S/gen_mxfp4s.py:852-969, quantize with a per-row power-of-two scale for gfx12 WMMA). One E8M0
 * scale per 32 values along K (OCP MX):  s = clamp(floor(log2(amax_32)) - 7, -127, 127),
 * codes = E4M3_RNE(x * 2^-s), scales = s + 127. x: [rows, k] of x_dtype (QMM_F32 / QMM_BF16), k % 32 == 0.
 * tile_info (i32 [rows/64, 2]) or NULL: rows of unused tiles are skipped. codes u8 [rows, k], scales u8 [rows, k/32]. */
int qmm_quant_mxfp8(int64_t rows, int64_t k, const void *x, int x_dtype, const int32_t *tile_info, uint8_t *codes,
                    uint8_t *scales, qmm_stream_t stream);

/* One-time weight preparation: GGUF MXFP4 17-byte blocks -> split planes (the reference's mxfp4s layout,
 * S/formats.py:12-15): nibbles u8 [rows, k/2] (byte j = elements 2j low nibble, 2j+1 high nibble) and
 * E8M0 scales u8 [rows, k/32]. Bit-exact: every code and exponent is kept. */
int qmm_repack_mxfp4(const void *w, int64_t rows, int64_t k, uint8_t *nibbles, uint8_t *scales, qmm_stream_t stream);

/* One-time weight preparation for the int8-activation decode GEMV and the grouped expert GEMMs (no reference
 * counterpart: the reference reads the GGUF blocks as they are): GGUF Q4_K rows [rows, k] -> the tiled layout
 * QMM_Q4_KT. Each block of 16 rows keeps its bytes in its own range, cut into units of 512 values (two super-blocks
 * a row), 4608 bytes each: the 32 16-byte headers ([f16 d][f16 dmin][12 scale bytes]) of super-block sb of row r at
 * 16 (2 r + sb), then four 1 KB code planes, plane q holding at 16 l (l = 4 r + 2 sb + h) code bytes 16 (4 h + q)
 * .. +15 of that super-block. When k % 512 == 256 the row block ends in a half unit of 2304 bytes (the rows' last
 * super-blocks): the 16 headers at 16 r, then four 512-byte planes, plane q holding at 16 (2 r + h) code bytes
 * 16 (4 h + q) .. +15. A byte permutation (same size); qmm_dequant(QMM_Q4_KT) gives the GGUF values bit for bit.
 * rows % 16 == 0, k % 256 == 0 (the decode GEMV takes k % 512 == 0). */
int qmm_tile_q4k(const void *w, int64_t rows, int64_t k, void *w_t, qmm_stream_t stream);

/* The same preparation for GGUF Q4_0 rows (no reference counterpart: the reference's @g_q4_0 matvecs read the 18-byte
 * blocks in place, S/gen_llm.py:536-552) -> QMM_Q4_0T, units of 16 rows x 512 values, 4608 bytes: at 16 (2 r + sb)
 * the eight f16 d of blocks 8 sb .. 8 sb + 7 of row r, then four 1 KB code planes, plane q holding at 16 l
 * (l = 4 r + 2 sb + h) bytes 16 (4 h + q) .. +15 of the 128 code bytes of those eight blocks, whose byte 32 p + i
 * holds code i of block 2 p in its low nibble and code i of block 2 p + 1 in its high nibble. A permutation of codes
 * and scales (same size); qmm_dequant(QMM_Q4_0T) gives the GGUF values bit for bit. rows % 16 == 0, k % 512 == 0. */
int qmm_tile_q40(const void *w, int64_t rows, int64_t k, void *w_t, qmm_stream_t stream);

/* One-time weight preparation for the grouped GEMM (no reference counterpart: the reference reads the split planes
 * of S/formats.py:12-15 as they are): split planes (nibbles [rows, k/2], scales [rows, k/32]) -> MFMA-tiled planes.
 * nib_t [rows/32][k/64][64 lanes][16 B]: tile (row block rb, chunk c) holds at lane l = 32 h + i the 16 nibble bytes
 * of row 32 rb + i, values 64 c + 32 h .. 64 c + 32 h + 31 (the E2M1 operand of lane l of the scaled MFMA);
 * sc_t [rows/32][ceil(k/256)][64 lanes][4 B]: byte q of lane l in group g is the E8M0 scale of that lane's block
 * in chunk 4 g + q (0 past K). A byte permutation: qmm_dequant(QMM_MXFP4T) gives the split planes' values bit for
 * bit. rows % 32 == 0, k % 64 == 0; nib_t has rows * k / 2 bytes, sc_t qmm_mxfp4t_scale_bytes(rows, k). */
int qmm_tile_mxfp4(const void *nibbles, const void *scales, int64_t rows, int64_t k, void *nib_t, void *sc_t,
                   qmm_stream_t stream);
int64_t qmm_mxfp4t_scale_bytes(int64_t rows, int64_t k);

/* MoE combine, g_moe_combine / g_moe_combine_sorted (S/gen_moe.py:730-762, :1231-1280):
 *   y[t, c] = fma(w[t,KU-1], v[KU-1], ... fma(w[t,0], v[0], accumulate ? y[t, c] : 0))
 * with v[k] = ys[row(t,k), c], row = pos[t*KU+k] (pos != NULL; -1 gives 0) or t*KU+k (pos == NULL).
 * ys f32 [rows, H]; wts f32 [tokens, KU]; y f32 [tokens, H]. */
int qmm_moe_combine(int64_t tokens, int64_t rows, int64_t H, int KU, const float *ys, const int32_t *pos,
                    const float *wts, int accumulate, float *y, qmm_stream_t stream);

/* The combine of a layer with gated shared experts, shared_gated (S/gen_moe.py:765-779): y[t] holds the shared
 * experts' output, y[t] = sg[t] y[t] + sum_k w[t,k] ys[row(t,k)] (the product first, then the fma chain in k
 * order). sg f32 [tokens] from qmm_moe_shared_gate; other arguments as qmm_moe_combine. */
int qmm_moe_combine_gated(int64_t tokens, int64_t rows, int64_t H, int KU, const float *ys, const int32_t *pos,
                          const float *wts, const float *sg, float *y, qmm_stream_t stream);

/* The decode chain's routing and gate/up expert matvecs in one launch: g_moe_route (S/gen_moe.py:116-500) over given
 * logits followed by g_moe_gu_{fmt}[_fused]_k{H}_r{R} (S/gen_moe.py:535-727, launch :564), the reference's first
 * decode commands (S/gen_llm.py:5373-5381), fused. The routing arguments as qmm_moe_topk (ids / wts are written as
 * it writes them), then the gate/up matvec's as qmm_moe_expert_mv_split with mode 0 (fmt any qmm_moe_expert_mv
 * format, QMM_MXFP4S with its scale planes ws / ws2, or QMM_MXFP4T with its tiled planes; w2 / ws2 ignored when
 * fused): act[a] for the tokens * KU assignments, each workgroup ranking its token's logits itself. Equal bit for bit
 * to qmm_moe_topk then qmm_moe_expert_mv[_split|_tiled](mode 0). */
int qmm_moe_topk_expert_mv(const float *logits, int64_t tokens, int E, int KU, int gating, int norm, float scale,
                           const float *router_bias, int32_t *ids, float *wts, int fmt, int fused, int act, int64_t k,
                           int64_t n, const void *x, int x_dtype, const void *w, const void *ws, const void *w2,
                           const void *ws2, const float *bias, const float *bias2, float *y, qmm_stream_t stream);

/* The decode chain's down expert matvecs and combine in one launch: g_moe_dn_{fmt}_k{FE}_r{R} (S/gen_moe.py:535-727,
 * launch :564) followed by g_moe_combine (S/gen_moe.py:730-762), the reference's last two decode commands
 * (S/gen_llm.py:5381-5385), fused; the ys buffer between them is not written.
 *   y[t, c] = fma(wts[t,KU-1], ys[t*KU+KU-1, c], ... fma(wts[t,0], ys[t*KU, c], y0)),
 *   ys[a] = Wd[e] x[a] + bias[e] (e = clamp(ids[a], 0, E - 1)),  y0 = sg ? sg[t] y[t, c] : accumulate ? y[t, c] : 0
 * equal bit for bit to qmm_moe_expert_mv[_split](mode 1) then qmm_moe_combine[_gated] (pos NULL). fmt as
 * qmm_moe_expert_mv plus QMM_MXFP4S (ws its scale planes [E, n, k/32]; ignored otherwise) and QMM_MXFP4T (tiled
 * planes, ws their scale groups; then each ys row is qmm_moe_expert_mv_tiled's); w [E, n, k]; x [tokens*KU,
 * k] f32 / bf16 (the gate/up output); ids i32 / wts f32 [tokens, KU]; bias f32 [E, n] or NULL; sg f32 [tokens] or
 * NULL; y f32 [tokens, n]. tokens <= 65535. */
int qmm_moe_expert_mv_combine(int fmt, int64_t k, int64_t n, int E, int KU, int64_t tokens, const int32_t *ids,
                              const float *wts, const void *x, int x_dtype, const void *w, const void *ws,
                              const float *bias, int accumulate, const float *sg, float *y, qmm_stream_t stream);

/* The routed experts of one MoE layer as one call: the command sequence of the reference's moe_routed
 * (S/gen_llm.py:5324-5385) on one stream, its intermediates (the buffers of moe_alloc, S/gen_llm.py:5388-5432) in the
 * caller's workspace of at least qmm_moe_routed_workspace_size bytes (256-byte aligned):
 *   tokens >= 64 (prefill): qmm_moe_route / qmm_moe_topk, [qmm_moe_wscale], qmm_moe_bucket, the activation operand
 *     (qmm_row_scale_f16 for GGUF formats, qmm_quant_mxfp8 for MXFP4 planes), the grouped gate/up GEMM
 *     (qmm_moe_grouped / qmm_moe_grouped_mxfp8), its output's operand, the grouped down GEMM, qmm_moe_combine;
 *   tokens < 64 (decode): route, [wscale], the gate/up and down expert matvecs (qmm_moe_expert_mv[_split|_tiled], or with
 *     flags QMM_MOE_Q8 qmm_quant_q8 + qmm_moe_expert_mv_q8 for both), qmm_moe_combine over the assignments; on f32 /
 *     bf16 activations the down matvecs and the combine run as qmm_moe_expert_mv_combine, and with given logits,
 *     E <= 64 and tokens * KU <= 8 the routing and the gate/up matvecs as qmm_moe_topk_expert_mv.
 * Results equal those of the separate calls bit for bit. Names as in those calls: fmt the gate / up format (GGUF
 * Q4_K / Q6_K / Q4_0 / MXFP4, split MXFP4S, tiled MXFP4T, or Q4_KT for prefill; or QMM_GATE_UP(gate, up) of GGUF
 * formats with two tensors, without QMM_MOE_Q8), fmt_down the down tensor's (-1: fmt, a pair's gate format); x f32 /
 * bf16 [tokens, H]; logits f32 [tokens, E], or NULL to route with w_router [E, H] (f32 / bf16); router_bias and
 * down_scale (f32 [E]) or NULL; ws_* the split / tiled scale planes; bias_* the expert biases or NULL; y f32
 * [tokens, H] is written, or added to (accumulate), or with sg (f32 [tokens], the shared gate) y = sg y + routed. */
int qmm_moe_routed(int fmt, int fmt_down, int fused, int act, int gating, int norm, float scale, int flags, int E,
                   int KU, int64_t tokens, int64_t H, int64_t FE, const void *x, int x_dtype, const float *logits,
                   const void *w_router, int w_router_dtype, const float *router_bias, const float *down_scale,
                   const void *w_gate, const void *ws_gate, const void *w_up, const void *ws_up, const void *w_down,
                   const void *ws_down, const float *bias_gate, const float *bias_up, const float *bias_down,
                   const float *sg, int accumulate, float *y, void *workspace, int64_t workspace_bytes,
                   qmm_stream_t stream);
/* Workspace bytes qmm_moe_routed needs (router != 0: routing from w_router, which keeps the logits there), or -1
 * for a combination it does not run. */
int64_t qmm_moe_routed_workspace_size(int fmt, int flags, int E, int KU, int64_t tokens, int64_t H, int64_t FE,
                                      int router);

/* qmm_moe_routed without a workspace argument and without any allocation: no counterpart in the reference (its
 * command programs allocate every buffer up front); it is for callers that cannot allocate device memory -- code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. The intermediates live in one
 * static device array of 16 MiB per GPU (held until the process ends), enough for the decode chain of a model with
 * H + FE <= 8192 and top-8 routing on given logits at up to 63 tokens on f32 / bf16 activations, and up to 48 tokens
 * with QMM_MOE_Q8 (its Q8_1 buffers take the rest); a call needing more returns QMM_ERR_WORKSPACE before launching anything (use
 * qmm_moe_routed). Calls that overlap on one GPU (two streams or host threads) share the array and race. Arguments
 * and results as qmm_moe_routed. */
int qmm_moe_routed_static(int fmt, int fmt_down, int fused, int act, int gating, int norm, float scale, int flags,
                          int E, int KU, int64_t tokens, int64_t H, int64_t FE, const void *x, int x_dtype,
                          const float *logits, const void *w_router, int w_router_dtype, const float *router_bias,
                          const float *down_scale, const void *w_gate, const void *ws_gate, const void *w_up,
                          const void *ws_up, const void *w_down, const void *ws_down, const float *bias_gate,
                          const float *bias_up, const float *bias_down, const float *sg, int accumulate, float *y,
                          qmm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QMM_H */
