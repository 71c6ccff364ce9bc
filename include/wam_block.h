/*
 * wam_block.h - C ABI of the MI355X (gfx950) Wan DiT block library
 * (libwam_block.so).
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream handle
 * (passed as void*; NULL is the null stream).  No torch or C++ types cross
 * this boundary.  All tensors are dense row-major.  Activations are bf16
 * (2-byte bfloat16); weights are in nn.Linear layout [N_out, K_in], so a
 * projection computes Y = X * W^T + b.
 *
 * Error behaviour: every int-returning entry point returns WAM_OK (0) on
 * success and a negative WAM_ERR_* code otherwise; wam_last_error() then
 * holds a message for the calling thread.  Shape/contract violations are
 * detected on the host before anything is launched (the reference raises
 * RuntimeError from TORCH_CHECK at the same points:
 * 算子研究/wam_ops/optimized/csrc/block.cu:320-330).
 *
 * Reference interfaces replaced (paths relative to the reference repo):
 *   wam_block_forward      <- ext.forward(weights[27], x, context, temb, freq,
 *                             cache[5], candidate_rows, update, eps[7], debug,
 *                             fused_ffn1, mode)
 *                             算子研究/wam_ops/optimized/csrc/block.cu:317-340,348-351
 *                             and the whole-layer variant
 *                             算子研究/wam_ops/optimized/csrc/whole_layer.cu:1080-1237
 *   wam_prepare_context    <- WholeLayerBlock.prepare_context(context, precompute=True)
 *                             算子研究/wam_ops/optimized/whole_layer.py:41-67
 *   wam_linear             <- linear(x, w, b) (cuBLASLt, bias epilogue)
 *                             算子研究/wam_ops/baseline/csrc/gemm.h:35-76, plus the
 *                             residual/GELU kernels fused into its epilogue
 *                             算子研究/wam_ops/baseline/csrc/block.cu:90-102,119-129
 *   wam_ln_modulate        <- norm(x, g, b, eps, rms=false) + table_kernel +
 *                             modulation_kernel
 *                             算子研究/wam_ops/baseline/csrc/block.cu:42-89
 *   wam_rms_rope           <- norm(x, g, {}, eps, rms=true) + rope_kernel
 *                             算子研究/wam_ops/baseline/csrc/block.cu:42-58,103-118
 *   wam_attention          <- sdpa(q, k, v) over [history || own] KV
 *                             算子研究/wam_ops/optimized/csrc/attention_tiles.cu:195-274,
 *                             with the pool read through a slot list instead of
 *                             pack_kernel (baseline/csrc/block.cu:213-224)
 *   wam_kv_layout          <- layout_kernel (slot compaction, eviction, new-slot
 *                             bookkeeping) 算子研究/wam_ops/baseline/csrc/block.cu:133-200
 *   wam_kv_commit          <- private_kernel 算子研究/wam_ops/baseline/csrc/block.cu:201-212
 * Model input/output around the block loop (WanTransformer3DModel.forward,
 * 投机采样/wam-p0-worktree/wan_va/modules/model.py:1060-1116; the reference
 * runs these as torch ops, it has no native kernels for them):
 *   wam_patchify           <- rearrange of the latents before patch_embedding_mlp /
 *                             action_embedder (model.py:1060-1071)
 *   wam_timestep_embedding <- condition_embedder.timesteps_proj (diffusers
 *                             Timesteps, model.py:216-218,233)
 *   wam_rows_linear        <- time_embedder / time_proj / action_proj_out linears
 *                             on few rows (model.py:219-222,234-239,1109)
 *   wam_rope_freqs         <- WanRotaryPosEmbed.forward (model.py:276-286)
 *   (norm_out + modulation is wam_ln_modulate with a one-vector temb;
 *    patch_embedding_mlp, text_embedder and proj_out are wam_linear)
 */
#ifndef WAM_BLOCK_H
#define WAM_BLOCK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WAM_ABI_VERSION 1

enum {
  WAM_OK = 0,
  WAM_ERR_ARG = -1,   /* contract violation detected on the host */
  WAM_ERR_HIP = -2,   /* a HIP runtime call failed */
  WAM_ERR_STATE = -3  /* a device-side contract check failed (see *_info) */
};

/* Element types; zero (a memset struct) means bf16. */
enum { WAM_BF16 = 0, WAM_F32 = 1, WAM_FP8 = 2 /* OCP e4m3 (e4m3fn) */,
       WAM_I64 = 3, WAM_F64 = 4 /* grid ids of wam_rope_freqs only */,
       WAM_FP8_MX = 5 /* e4m3 values with one e8m0 exponent per 32 consecutive
                        values of a row (an OCP MX block): value = q * 2^(e - 127) */ };

/* Epilogues of wam_linear. */
enum {
  WAM_EPI_BIAS = 0,          /* y = bf16(acc + b)                              */
  WAM_EPI_BIAS_GELU = 1,     /* y = bf16(gelu_tanh(acc + b))                   */
  WAM_EPI_BIAS_GATE_RES = 2, /* y = bf16(res + (acc + b) * gate[row, col])     */
  WAM_EPI_BIAS_RES = 3       /* y = bf16(res + (acc + b))                      */
};

/* Modulation source: mod[b, t, i, :] = table[i, :] + temb[b, r(t), i, :]
 * (model.py:751-759; i = 0 shift, 1 scale, 2 gate, 3 c_shift, 4 c_scale,
 * 5 c_gate).  temb is [B, L, mods, D].  L == 1 (per sample), L == tokens
 * (per token, the reference's timestep_proj), or any divisor of tokens: row
 * r(t) = t / (tokens / L) then serves tokens / L consecutive tokens (one
 * latent frame: the reference repeats each frame's timestep over the frame's
 * tokens, model.py:1078-1086, so per-frame rows give the same values).
 * mods == 6, or mods == 1 for one vector that serves every index i (the
 * output head: scale_shift_table[2, D] + temb[B, L, D], model.py:1096). */
typedef struct {
  const void* table; /* [6, D] (or [2, D] for the output head) */
  int table_dtype;   /* WAM_F32 | WAM_BF16 */
  const void* temb;  /* [B, L, mods, D] */
  int temb_dtype;    /* WAM_F32 | WAM_BF16 */
  int temb_len;      /* L: 1, tokens, or a divisor of tokens */
  int tokens;        /* tokens per batch row (M) */
  int temb_mods;     /* mods: 6 (0 is read as 6) or 1 */
} wam_modulation;

/* ---------------------------------------------------------------- linear */
typedef struct {
  const void* a;     /* [M, K] bf16, row stride lda (elements) */
  int64_t lda;
  int M, K;
  int n_seg;         /* 1..3 output segments (QKV runs as one launch) */
  int seg_n;         /* columns per segment */
  const void* w[3];  /* [seg_n, K] bf16 (or fp8, w_dtype) each, row stride ldw elements */
  int64_t ldw;
  const void* bias[3]; /* [seg_n] bf16 each, or NULL */
  void* out[3];      /* [M, seg_n] bf16 each, row stride ldo */
  int64_t ldo;
  int epilogue;      /* WAM_EPI_* */
  const void* res;   /* residual [M, seg_n], row stride ldr */
  int64_t ldr;
  int res_dtype;     /* WAM_BF16 | WAM_F32 */
  int out_dtype;     /* WAM_BF16 | WAM_F32 (f32 only for the residual epilogues) |
                        WAM_FP8_MX (below) */
  wam_modulation gate; /* gate row = mod[b, t, gate_index] for row m = b*tokens+t */
  int gate_index;
  /* Weight storage.  WAM_BF16, or WAM_FP8: e4m3 weights with one fp32 scale
   * per output column (w_scale[s][n], typically absmax/448 of the bf16 row):
   * acc = sum_k a[m,k] * fp8(w[n,k]) is scaled by w_scale[n] before the bias.
   * This is the fp8-weight / bf16-activation FFN variant; the reference has
   * no fp8 path. */
  int w_dtype;
  const float* w_scale[3];
  /* Optional workspace for the split-K tail: when the 256x256 tiles leave
   * a partial last round, the remaining output columns may run split over k
   * with fp32 partial sums here (at least wam_linear_workspace_bytes(M,
   * seg_n, n_seg, K) bytes), or, without it, as smaller tiles.  Not in the
   * reference (cuBLASLt picks its own algorithm and workspace). */
  void* workspace; int64_t workspace_bytes;
  /* Optional q/k-norm epilogue (WAM_EPI_BIAS only): the across-heads RMSNorm
   * and RoPE of model.py:609-623 (replacing the separate norm_q/norm_k + rope
   * passes, baseline/csrc/block.cu:103-118), split so that a 256-column tile
   * can apply them.  For each segment s with norm_ssq[s] != NULL, with
   * y = bf16(acc + b) of row m:
   *   norm_ssq[s][m * ceil(seg_n / 256) + c / 256] = sum of y^2 over the 256
   *     columns of group c / 256 (fp32),
   *   out = bf16(rope(y * norm_gamma[s]))  (bf16 gamma [seg_n]; rotation of
   *     pairs (2j, 2j+1) of every norm_head_dim-wide head by
   *     norm_freq[fb, t, j], complex64 [norm_freq_batch, norm_tokens,
   *     norm_head_dim / 2], row m = b * norm_tokens + t; no rotation when
   *     norm_freq is NULL).
   * The 1/rms factor rsqrt(sum of the row's norm_ssq / seg_n + eps) is left
   * to the consumer (wam_attention's q_ssq; the rotation is linear, so it
   * commutes with that factor).  Not in the reference, whose norm is a
   * separate row pass. */
  float* norm_ssq[3]; const void* norm_gamma[3];
  const void* norm_freq; int norm_freq_batch, norm_tokens, norm_head_dim;
  /* Activation storage.  WAM_BF16, or WAM_FP8: a is e4m3 [M, K] (lda in
   * elements = bytes) with one fp32 scale per row (a_scale[m], e.g. absmax/448
   * from wam_quantize_fp8_rows), and the product runs on the fp8 MFMA:
   * y = sum_k fp8(a[m,k]) fp8(w[n,k]) * a_scale[m] * w_scale[n] + b[n].
   * Needs fp8 weights, WAM_EPI_BIAS or WAM_EPI_BIAS_GELU, one segment of
   * whole 256-column tiles and K a multiple of 128.  Not in the reference
   * (an fp8-activation variant of the FFN).
   * WAM_FP8_MX: a is e4m3 [M, K] with e8m0 exponents a_block_scale [M, K / 32]
   * (bytes, row stride K / 32): y = sum_k q[m,k] 2^(e[m,k/32]-127) fp8(w[n,k])
   * * w_scale[n] + b[n], the exponents applied by the MFMA itself.  Needs fp8
   * weights, WAM_EPI_BIAS, WAM_EPI_BIAS_GATE_RES or WAM_EPI_BIAS_RES with a
   * bf16 output, one segment of whole 256-column tiles and K a multiple of
   * 128. */
  int a_dtype; const float* a_scale;
  const void* a_block_scale;
  /* out_dtype WAM_FP8_MX (a_dtype WAM_FP8, WAM_EPI_BIAS or WAM_EPI_BIAS_GELU):
   * out[0] is e4m3 [M, seg_n] (ldo in bytes) and out_block_scale [M, seg_n /
   * 32] the e8m0 exponent of each row's 32-column blocks, the smallest with
   * max |y| <= 448 * 2^(e - 127) over the block; q = e4m3(y * 2^(127 - e)),
   * round to nearest even.  The FFN1 -> FFN2 hand-over of the fp8 FFN. */
  void* out_block_scale;
} wam_linear_args;

int wam_linear(const wam_linear_args* args, void* stream);
int64_t wam_linear_workspace_bytes(int M, int N, int n_seg, int K);

/* Per-row fp8 quantization of a bf16 matrix w [rows, cols] (row stride ldw):
 * scale[r] = max_c |w[r,c]| / 448 (1 for an all-zero row) and
 * q[r, c] = e4m3(w[r,c] * (448 / max_c |w[r,c]|)) (fp32 product with the
 * row's fp32 reciprocal factor; factor 1 for an all-zero row), round to
 * nearest even (q row stride cols).
 * Prepares the fp8 weights of wam_linear (w_dtype = WAM_FP8).  No counterpart
 * in the reference, which has no fp8 path. */
int wam_quantize_fp8_rows(const void* w, int rows, int cols, int64_t ldw, void* q, float* scale,
                          void* stream);

/* ----------------------------------------------------------- LayerNorm */
/* y = bf16(LN(x) * (1 + mod[shift+1]) + mod[shift])   when affine == 0
 * y = bf16(LN(x) * gamma + beta)                      when affine == 1
 * LN without affine parameters, fp32 statistics, eps. */
typedef struct {
  const void* x; /* [rows, D] bf16 or f32 (x_dtype) */
  void* y;       /* [rows, D] bf16 */
  int rows, D;
  int x_dtype;   /* WAM_BF16 | WAM_F32 */
  float eps;
  int affine;
  const void* gamma; const void* beta; int gb_dtype; /* affine == 1 */
  wam_modulation mod; int shift_index;              /* affine == 0 */
  /* Optional e4m3 copy of y (no counterpart in the reference; the fp8
   * activations of wam_linear): y8 [rows, D] bytes and y8_scale [rows] fp32
   * with y8_scale[r] = max_d |y[r,d]| / 448 (1 for an all-zero row) and
   * y8[r,d] = e4m3(y[r,d] * (448 / max_d |y[r,d]|)) rounded to nearest even
   * (as wam_quantize_fp8_rows), y being the
   * bf16 result (the same bytes wam_quantize_fp8_rows makes of it).  With y8
   * set, y may be NULL (no bf16 output). */
  void* y8; float* y8_scale;
} wam_ln_args;

int wam_ln_modulate(const wam_ln_args* args, void* stream);

/* ------------------------------------------------------ RMSNorm + RoPE */
/* For each of up to two tensors (q, k): y = rope(x * rsqrt(mean(x^2)+eps) * g)
 * over the full D-wide row (RMSNorm across heads, model.py:325-330,609-612),
 * RoPE pairs (2j, 2j+1) of every head rotated by freq[bf, t, j]
 * (model.py:614-623).  In place is allowed (y == x). */
typedef struct {
  const void* x[2]; void* y[2]; const void* gamma[2]; float eps[2];
  int64_t ldx, ldy; /* row strides (elements) */
  int n_tensors;    /* 1 or 2 */
  int rows, D, head_dim;
  const void* freq; /* complex64 [Bf, tokens, head_dim/2] or NULL (no RoPE) */
  int freq_batch, tokens;
} wam_rms_rope_args;

int wam_rms_rope(const wam_rms_rope_args* args, void* stream);

/* ------------------------------------------------------------ attention */
/* O[b, i, h, :] = softmax_j(Q[b,i,h,:] . K_j / sqrt(hd)) V_j over the key list
 *   j <  n_hist : pool row pool_rows[b] (or b), slot slots[j]
 *   j >= n_hist : own key (j - n_hist) of own batch row kv_rows[b] (or b)
 * Slots address rows within one pool row block: slots[j] * pool_rstride <
 * pool_bstride (a [Bp, P, H, 128] pool has pool_bstride = P * pool_rstride).
 * n_hist is read from device memory (n_hist_dev) so the host never waits for
 * the slot compaction.  Non-causal, like model.py:37-40. */
typedef struct {
  const void* q; int64_t q_bstride, q_rstride;  /* elements */
  void* o; int64_t o_bstride, o_rstride;
  int B, Mq, H, head_dim;
  const void* pool_k; const void* pool_v;
  int64_t pool_bstride, pool_rstride; int pool_batch;
  const int32_t* slots; const int32_t* n_hist_dev;
  const int64_t* pool_rows;
  const void* k; const void* v; int64_t kv_bstride, kv_rstride; int Mk;
  const int64_t* kv_rows; int kv_batch;
  float scale;
  /* Optional workspace for key-range splits of the last dispatch round
   * (used when the query grid alone would leave CUs idle): at least
   * wam_attention_workspace_bytes(B, Mq, H, max_keys) bytes, or NULL to run
   * unsplit.  max_keys: host-side upper bound of Mk + n_hist (0 = Mk), used
   * only to plan the split.  Not in the reference (its FlashAttention call
   * chooses splits internally). */
  void* workspace; int64_t workspace_bytes; int max_keys;
  /* Optional per-query RMS factor, for queries written by wam_linear's norm
   * epilogue: when q_ssq != NULL, query row r = b * Mq + i is taken as
   * Q[b, i] * rsqrt(sum_{t < q_ssq_n} q_ssq[r * q_ssq_n + t] / q_norm_dim
   * + q_eps), applied to its scores (which are linear in Q).  q_ssq_n <= 16.
   * The reference normalises Q in a separate pass (model.py:609-612). */
  const float* q_ssq; int q_ssq_n; int q_norm_dim; float q_eps;
  /* Optional device int (kv_layout's info[2]): when it holds s >= 0, the
   * history is slots s, s + 1, ..., s + n_hist - 1 in that order, i.e.
   * slots[j] == s + j, and the kernel reads the pool rows at that base
   * without the slot list; -1 (or a NULL pointer) reads them through slots.
   * No counterpart in the reference, which gathers the valid rows. */
  const int32_t* hist_base_dev;
} wam_attention_args;

int wam_attention(const wam_attention_args* args, void* stream);
int64_t wam_attention_workspace_bytes(int B, int Mq, int H, int max_keys);
/* wam_attention without a workspace, and without any device allocation: no
 * counterpart in the reference.  For callers that cannot allocate (code under
 * HIP graph capture, serving loops that forbid hipMalloc).  args->workspace
 * must be NULL and workspace_bytes 0; the key-range split's partial results
 * go to a static 64 MiB device array of the library (one per GPU, held until
 * the process ends).  A call whose own key-range split (the plan this call
 * would run, with the query tile this call would use) needs more than 64 MiB
 * of partials is refused with WAM_ERR_ARG.  wam_attention_workspace_bytes
 * may report more than that plan needs (it covers every query tile), so it
 * is an upper bound, not the test.  Calls that overlap on one GPU share the
 * array and race. */
int wam_attention_noalloc(const wam_attention_args* args, void* stream);

/* ------------------------------------------------------------- KV pool */
/* Device-side bookkeeping of the original-mode KV pool (model.py:547-593):
 *  candidate == 0: evict the oldest ids while fewer than `tokens` slots are
 *    free (ties by ascending slot), take the first `tokens` free slots, give
 *    them id = max(valid id) + 1 and is_pred = (update == 1), and set their
 *    mask to (update != 0) (update 0 is the temporary write whose mask
 *    restore_cache clears again).
 *  candidate == 1: read only.
 * Always: hist_slots = the valid slots before the new ones, in ascending
 * order, and n_hist their count.  info[0] = n_hist, info[1] = error code
 * (0 ok, 2 invalid candidate row), info[2] = hist_slots[0] when the history
 * is one run of consecutive slots (hist_slots[j] == hist_slots[0] + j), else
 * -1 (attention's hist_base_dev).  Runs as one workgroup; no host sync. */
typedef struct {
  uint8_t* mask; int64_t* ids; uint8_t* is_pred; int pool;
  int tokens; int update; int candidate;
  const int64_t* rows; int batch; int pool_batch;
  int32_t* hist_slots; int32_t* new_slots; int32_t* info;
} wam_kv_layout_args;

int wam_kv_layout(const wam_kv_layout_args* args, void* stream);

/* Copy the new K/V rows [B, tokens, D] (row stride ld) to pool[b, new_slots[t]]. */
typedef struct {
  const void* k; const void* v; int64_t ld;
  void* pool_k; void* pool_v; int64_t pool_bstride, pool_rstride;
  const int32_t* new_slots; int B, tokens, D;
} wam_kv_commit_args;

int wam_kv_commit(const wam_kv_commit_args* args, void* stream);

/* ---------------------------------------------------------------- block */
/* Weights in the reference order (optimized/native.py:35-49):
 *  0 scale_shift_table [1,6,D] (f32|bf16)   1,2 norm2 weight/bias (f32|bf16, or NULL)
 *  3..10 attn1 to_q w,b  to_k w,b  to_v w,b  to_out[0] w,b
 *  11,12 attn1 norm_q.weight, norm_k.weight
 *  13..20 attn2 to_q, to_k, to_v, to_out[0] (w,b)   21,22 attn2 norm_q, norm_k
 *  23,24 ffn.net[0].proj w,b    25,26 ffn.net[2] w,b
 * eps = [norm1, norm2, norm3, attn1.q, attn1.k, attn2.q, attn2.k]. */
typedef struct {
  const void* w[27];
  int table_dtype; int norm2_dtype;
  int dim, heads, head_dim, ffn_dim;
  float eps[7];
  /* Optional fp8 FFN (no counterpart in the reference): when ffn_fp8[0] is
   * set, FFN1 uses e4m3 weights ffn_fp8[0] [ffn_dim, dim] with per-row scales
   * ffn_scale[0], and FFN2 ffn_fp8[1] [dim, ffn_dim] with ffn_scale[1]
   * (wam_quantize_fp8_rows of w[23] and w[25]); the biases stay w[24], w[26]. */
  const void* ffn_fp8[2];
  const float* ffn_scale[2];
  /* With ffn_fp8 set: ffn_act_fp8 = 1 also quantizes FFN1's input per row
   * (LayerNorm 3 writes e4m3 rows with absmax/448 scales, as wam_ln_args.y8)
   * and runs FFN1 on the fp8 MFMA (wam_linear a_dtype = WAM_FP8).
   * ffn_act_fp8 = 2 in addition has FFN1 write the GELU output as MX e4m3
   * (out_dtype WAM_FP8_MX: one e8m0 exponent per row and 32 columns) and runs
   * FFN2 on it (a_dtype WAM_FP8_MX): both FFN GEMMs on the fp8 MFMA.  Needs
   * ffn_dim to be a multiple of 256.  Workspace: the layout always holds the
   * e4m3 rows and their scales; the MX hidden layer fits in the bf16 one's
   * bytes. */
  int ffn_act_fp8;
} wam_block_weights;

#define WAM_DEBUG_SLOTS 28
/* debug[i] (if non-NULL) receives a copy of intermediate i:
 *  0 modulated1 [R,D]  1 self_q_rope [R,D]  2 self_k_rope [R,D]  3 self_v [R,D]
 *  4 self_attention [R,D]  5 residual1 [R,D] f32  6 norm2 [R,D]  7 cross_q [R,D]
 *  8 cross_k [Bc*Lc,D]  9 cross_v [Bc*Lc,D]  10 cross_attention [R,D]
 *  11 residual2 [R,D] f32  12 modulated3 [R,D]  13 gelu [R,F]  14 output [R,D]
 *  15 self_q_linear [R,D]  16 self_k_linear [R,D]  17 self_q_norm [R,D]
 *  18 self_k_norm [R,D] (RMSNorm before RoPE)  19 self_out [R,D] (to_out before
 *  the gate)  20 cross_q_linear [R,D]  21 cross_k_linear [Bc*Lc,D] (only when
 *  the call projects the context; untouched with precomputed cross K/V)
 *  22 cross_out [R,D]  23 ffn1 [R,F] (before GELU)  24 ffn2 [R,D] (before the
 *  gate)  25 norm1 [R,D]  26 norm3 [R,D] (LayerNorm before the modulation)
 *  27 modulation [B,L,6,D] f32 (table + temb)
 * (all bf16 except the residual-stream tensors, which the block keeps in
 * fp32 between the input and the output, and the modulation).  Slots 15-27
 * are the reference's remaining named intermediates
 * (optimized/csrc/whole_layer.cu:1203-1209); the fused kernels do not
 * materialise them, so the block computes them with extra launches when
 * they are requested. */

typedef struct {
  const wam_block_weights* weights;
  int B, M;                     /* batch rows and tokens per row; R = B*M */
  const void* x;                /* [B, M, D] bf16 */
  const void* context;          /* [Bc, Lc, D] bf16; may be NULL when cross_k/v given */
  int context_batch, context_len;
  const int64_t* context_rows;  /* [B] context row per batch row, or NULL (= b) */
  wam_modulation mod;           /* table = weights->w[0] */
  const void* freq;             /* complex64 [Bf, M, head_dim/2] or NULL */
  int freq_batch;
  /* original-mode KV pool; cache_k == NULL means no cache */
  void* cache_k; void* cache_v; int64_t* cache_id; uint8_t* cache_mask;
  uint8_t* cache_is_pred; int cache_batch; int pool;
  const int64_t* candidate_rows; /* [B] or NULL */
  int update;
  /* precomputed cross K/V [Bc, Lc, D] (already RMS-normed K); NULL = compute */
  const void* cross_k; const void* cross_v;
  void* out;                    /* [B, M, D] bf16 (or fp32, out_dtype) */
  void* workspace; size_t workspace_bytes;
  void** debug;                 /* NULL or WAM_DEBUG_SLOTS pointers */
  void* timer;                  /* NULL or a wam_timer */
  /* WAM_BF16 (0, the reference's output) or WAM_F32: the final gated
   * residual x2 + f * c_gate before its bf16 rounding, i.e. the block's
   * arithmetic without the output's own rounding (a parity diagnostic; the
   * reference block returns bf16). */
  int out_dtype;
} wam_block_args;

size_t wam_block_workspace_bytes(int B, int M, int dim, int ffn_dim,
                                 int context_batch, int context_len, int pool);
int wam_block_forward(const wam_block_args* args, void* stream);

/* Cross K = RMS(ctx Wk^T + bk) * g, V = ctx Wv^T + bv for the context rows
 * (attn2 of model.py:777-782), written to k_out/v_out [rows, D]. */
int wam_prepare_context(const wam_block_weights* weights, const void* context,
                        int rows, void* k_out, void* v_out, void* stream);

/* ------------------------------------------------- model input / output */
/* Patch rearrange of the latents (model.py:1064-1069, and 1060-1062 with a
 * 1x1x1 patch for the action latents):
 *   out[b*L + (f*Hp + h)*Wp + w, (c*p1 + i)*p2*p3 + j*p3 + k]
 *       = x[b, c, f*p1 + i, h*p2 + j, w*p3 + k]
 * with L = Fp*Hp*Wp = (F/p1)(H/p2)(W/p3).  x is [B, C, F, H, W] bf16,
 * contiguous; out is [B*L, k_pad] bf16 and columns C*p1*p2*p3 .. k_pad-1 are
 * zero, so a following wam_linear runs with K = k_pad (a multiple of 64)
 * against weights zero-padded to k_pad columns. */
typedef struct {
  const void* x;
  void* out;
  int B, C, F, H, W;
  int p1, p2, p3;
  int k_pad;
} wam_patchify_args;

int wam_patchify(const wam_patchify_args* args, void* stream);

/* Sinusoidal timestep embedding, diffusers 0.36.0 get_timestep_embedding as
 * Timesteps(dim, flip_sin_to_cos, downscale_freq_shift) calls it
 * (model.py:216-218): freq_i = exp(-ln(max_period) * i / (dim/2 - shift)),
 * fp32, i < dim/2; out[r] = [cos(t_r freq), sin(t_r freq)] when
 * flip_sin_to_cos, else [sin, cos]. */
typedef struct {
  const float* t;   /* [rows] */
  int rows, dim;    /* dim even */
  int flip_sin_to_cos;
  float shift;      /* downscale_freq_shift */
  float max_period; /* 10000 */
  void* out;        /* [rows, dim] */
  int out_dtype;    /* WAM_F32 | WAM_BF16 */
} wam_timestep_args;

int wam_timestep_embedding(const wam_timestep_args* args, void* stream);

/* Linear over few rows on the vector ALUs (weight-streaming, any N and K):
 *   out[r, n] = act_out(sum_k act_in(x[r, k]) * w[n, k] + bias[n])
 * For the condition embedder, whose rows are one per (sample, frame)
 * timestep: time_embedder.linear_1 + SiLU, linear_2 (fp32 weights, the
 * model's _keep_in_fp32_modules), time_proj(SiLU(temb)); and action_proj_out
 * (N = 30).  Rounding follows torch's per-op dtypes: act_in(x) is rounded to
 * x's dtype (the input SiLU uses a hardware exp2/reciprocal, a few fp32 ulp);
 * with act_out the pre-activation is rounded to the output dtype first.
 * Accumulation is fp32.  Rows are processed 8 at a time, so the weights are
 * read ceil(R / 8) times: use wam_linear for many rows. */
enum { WAM_ACT_NONE = 0, WAM_ACT_SILU = 1 };
typedef struct {
  const void* x; int x_dtype; int64_t ldx;  /* [R, K] WAM_F32 | WAM_BF16 */
  const void* w; int w_dtype; int64_t ldw;  /* [N, K] WAM_F32 | WAM_BF16 */
  const void* bias; int bias_dtype;         /* [N] or NULL */
  void* out; int out_dtype; int64_t ldo;    /* [R, N] */
  int R, N, K;
  int act_in, act_out;                      /* WAM_ACT_* */
} wam_rows_linear_args;

int wam_rows_linear(const wam_rows_linear_args* args, void* stream);

/* 3D RoPE frequencies (WanRotaryPosEmbed.forward, model.py:276-286):
 * head_dim splits into f/h/w dims hd - 2*(hd/3), hd/3, hd/3 (44/42/42 for
 * 128); pair j of axis a with dim d_a has base 1 / theta^(2j / d_a) (float64),
 * angle = float(grid[b, a, l] * base) and out[b, l, pair] = (cos, sin) of it,
 * complex64.  grid is [B, G >= 3, L] (rows frame, height, width, ...), dtype
 * WAM_I64, WAM_F32 or WAM_F64. */
typedef struct {
  const void* grid; int grid_dtype;
  int64_t grid_bstride, grid_rstride, grid_lstride; /* elements */
  int B, L, head_dim;
  double theta;
  void* out;  /* complex64 [B, L, head_dim/2] */
} wam_rope_freq_args;

int wam_rope_freqs(const wam_rope_freq_args* args, void* stream);

/* --------------------------------------------------------------- timing */
/* Stage timer: pairs of HIP events recorded on the launch stream around
 * selected stages of wam_block_forward. */
enum {
  WAM_STAGE_LN1 = 0, WAM_STAGE_QKV, WAM_STAGE_RMS_ROPE, WAM_STAGE_KV_LAYOUT,
  WAM_STAGE_SELF_ATTN, WAM_STAGE_SELF_OUT, WAM_STAGE_LN2, WAM_STAGE_CROSS_Q,
  WAM_STAGE_CROSS_KV, WAM_STAGE_CROSS_ATTN, WAM_STAGE_CROSS_OUT, WAM_STAGE_LN3,
  WAM_STAGE_FFN1, WAM_STAGE_FFN2, WAM_STAGE_KV_COMMIT, WAM_N_STAGES
};
void* wam_timer_create(int capacity, uint32_t stage_mask);
void wam_timer_reset(void* timer);
/* Synchronises the recorded events; fills up to max (stage, ms) records. */
int wam_timer_read(void* timer, int32_t* stages, float* ms, int max);
void wam_timer_destroy(void* timer);

/* ------------------------------------------------------------ measurement */
/* MFMA throughput probe (no counterpart in the reference: it measures the
 * roofline denominators that the benchmark reports beside the vendor peaks).
 * Launches one kernel on `stream` in which every wave issues `iters` rounds of
 * independent MFMAs of the given kind (two waves per SIMD on every CU) and
 * stores one float per thread to `sink` (2 x CUs x 256 floats).  *flop is the
 * kernel's FLOP count; time it with events on the same stream. */
enum {
  WAM_PEAK_BF16_32 = 0, /* v_mfma_f32_32x32x16_bf16 */
  WAM_PEAK_BF16_16 = 1, /* v_mfma_f32_16x16x32_bf16 */
  WAM_PEAK_FP8_32 = 2,  /* v_mfma_scale_f32_32x32x64_f8f6f4, e4m3 x e4m3, unit scales */
  WAM_PEAK_FP8_16 = 3   /* v_mfma_scale_f32_16x16x128_f8f6f4, e4m3 x e4m3, unit scales */
};
int wam_mfma_peak(int kind, int iters, void* sink, int64_t sink_bytes, double* flop, void* stream);

/* ---------------------------------------------------------------- misc */
const char* wam_last_error(void);
int wam_abi_version(void);
/* sizeof() of the argument struct named `name` (0 if unknown), so bindings
 * can check their struct layout against the library's. */
size_t wam_abi_struct_size(const char* name);

#ifdef __cplusplus
}
#endif
#endif /* WAM_BLOCK_H */
