// Whole DiT block: the stage sequence of WanTransformerBlock.forward
// (model.py:741-794) as a stream of fused HIP kernels on the caller's stream.
//
//   h1  = LN(x) * (1 + scale) + shift                       ln_modulate
//   qkv = h1 [Wq|Wk|Wv]^T + b                               one GEMM launch
//   q,k = rope(RMS(q) g_q), rope(RMS(k) g_k)                rms_rope (in place)
//   [pool bookkeeping]                                       kv_layout
//   a1  = attention(q, [history || k], [history || v])       attention
//   x1  = x + (a1 Wo^T + bo) * gate                          GEMM + gated residual
//   [commit new K/V to the pool, update 1/2]                 kv_commit
//   n2  = LN(x1) g2 + b2                                     ln_modulate (affine)
//   cq  = RMS(n2 Wq2^T + bq2) g                              GEMM + norm epilogue
//                                                            (y g + sums of squares;
//                                                            1/rms applied in attention)
//   ck, cv from context (or precomputed by prepare_context)  GEMM + rms_rope
//   x2  = x1 + (attention(cq, ck, cv) Wo2^T + bo2)           attention + GEMM + residual
//   h3  = LN(x2) * (1 + c_scale) + c_shift                   ln_modulate
//   u   = gelu_tanh(h3 W1^T + b1)                            GEMM + GELU
//   out = x2 + (u W2^T + b2) * c_gate                        GEMM + gated residual
//
// Intermediates live in one caller-provided workspace; the library never
// allocates device memory.  The reference runs the same sequence as
// 算子研究/wam_ops/baseline/csrc/block.cu:262-310.
#include <stdio.h>
#include <string.h>
#include <vector>
#include "wam_common.h"

namespace wam {

int linear(const wam_linear_args*, hipStream_t);
int mx_dequant_bf16(const void* q, const void* e, void* y, int rows, int cols, hipStream_t s);
int ln_modulate(const wam_ln_args*, hipStream_t);
int rms_rope(const wam_rms_rope_args*, hipStream_t);
int attention(const wam_attention_args*, hipStream_t);
int64_t attention_workspace_bytes(int B, int Mq, int H, int64_t max_keys);
int64_t linear_workspace_bytes(int M, int seg_n, int n_seg, int K);
bool linear_norm_in_epilogue(int M, int seg_n, int n_seg, int K, int64_t ws_bytes, bool rope);
int kv_layout(const wam_kv_layout_args*, hipStream_t);
int kv_commit(const wam_kv_commit_args*, hipStream_t);

static thread_local char g_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

// ------------------------------------------------------------------ timer
struct Timer {
  int capacity = 0, count = 0;
  uint32_t mask = 0;
  std::vector<hipEvent_t> ev;
  std::vector<int32_t> stage;
};

struct Scope {
  Timer* t; int stage; hipStream_t s; bool on;
  Scope(void* timer, int st, hipStream_t str) : t(static_cast<Timer*>(timer)), stage(st), s(str) {
    on = t && (t->mask >> st & 1u) && t->count < t->capacity;
    if (on) (void)hipEventRecord(t->ev[2 * t->count], s);
  }
  ~Scope() {
    if (on) {
      (void)hipEventRecord(t->ev[2 * t->count + 1], s);
      t->stage[t->count++] = stage;
    }
  }
};

// -------------------------------------------------------------- workspace
static size_t align_up(size_t v) { return (v + 255) & ~size_t(255); }

struct Layout {
  size_t h, h8, h8s, qkv, attn, x1, x2, ck, cv, act, slots, newslots, info, ssq, zeros, split, split_bytes, total;
};

static Layout layout(int B, int M, int D, int F, int Bc, int Lc, int pool) {
  Layout L{};
  const size_t R = (size_t)B * M;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align_up(bytes); return o; };
  L.h = take(R * D * 2);
  // e4m3 rows of the LayerNorm-3 output and their scales (fp8 FFN1 input).
  L.h8 = take(R * D);
  L.h8s = take(R * 4);
  L.qkv = take(R * 3 * D * 2);
  L.attn = take(R * D * 2);
  L.x1 = take(R * D * 4);  // residual stream kept in fp32
  L.x2 = take(R * D * 4);
  L.ck = take((size_t)Bc * Lc * D * 2);
  L.cv = take((size_t)Bc * Lc * D * 2);
  L.act = take(R * F * 2);
  L.slots = take((size_t)(pool > 0 ? pool : 1) * 4);
  L.newslots = take((size_t)(M > 0 ? M : 1) * 4);
  L.info = take(16);
  // Per-row sums of squares of the cross queries per 256-column group (the
  // q-norm epilogue of the projection).
  L.ssq = take(R * (size_t)((D + 255) / 256) * 4);
  // A zero modulation (table [2, D] and one vector per batch row) for the
  // unmodulated LayerNorm debug outputs.
  L.zeros = take(((size_t)B + 2) * D * 4);
  // Partial results of the self attention's key-range splits (own keys + the
  // pool), the cross attention's (context keys) and the split-K GEMM tails.
  // One region: the kernels that use it run one after another on the stream.
  const int64_t need[] = {attention_workspace_bytes(B, M, D / 128, (int64_t)M + (pool > 0 ? pool : 0)),
                          attention_workspace_bytes(B, M, D / 128, Lc),
                          linear_workspace_bytes((int)R, D, 1, D),   // self_out, cross_q, cross_out
                          linear_workspace_bytes((int)R, F, 1, D),   // FFN1
                          linear_workspace_bytes((int)R, D, 1, F)};  // FFN2
  int64_t most = 0;
  for (int64_t n : need) most = n > most ? n : most;
  L.split_bytes = (size_t)most;
  L.split = take(L.split_bytes);
  L.total = off;
  return L;
}

__global__ void cast_f32_bf16_kernel(const float* x, bf16* y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    y[i] = static_cast<bf16>(x[i]);
}

static int cast_f32_bf16(const float* x, bf16* y, int64_t n, hipStream_t s) {
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(cast_f32_bf16_kernel, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256),
                     0, s, x, y, n);
  WAM_LAUNCHED("cast_f32_bf16_kernel");
  return WAM_OK;
}

__global__ void fill_zero_kernel(float* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0.f;
}

// modulation[b, l, i, d] = table[i, d] + temb[b, l, i, d] in fp32 (the
// reference's `modulation` intermediate, model.py:751-759).
__global__ void modulation_table_kernel(wam_modulation m, int D, int64_t n, float* out) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int d = (int)(e % D);
    const int i = (int)((e / D) % 6);
    const float t = m.table_dtype == WAM_F32 ? static_cast<const float*>(m.table)[i * D + d]
                                             : static_cast<float>(static_cast<const bf16*>(m.table)[i * D + d]);
    const float u = m.temb_dtype == WAM_F32 ? static_cast<const float*>(m.temb)[e]
                                            : static_cast<float>(static_cast<const bf16*>(m.temb)[e]);
    out[e] = t + u;
  }
}

static int copy_debug(void** dbg, int slot, const void* src, size_t bytes, hipStream_t s) {
  if (dbg && dbg[slot]) WAM_HIP(hipMemcpyAsync(dbg[slot], src, bytes, hipMemcpyDeviceToDevice, s));
  return WAM_OK;
}

static int check_weights(const wam_block_weights* w) {
  WAM_REQUIRE(w != nullptr, "block: null weights");
  WAM_REQUIRE(w->head_dim == 128 && w->heads >= 1 && w->dim == w->heads * w->head_dim,
              "block: dim=%d must equal heads(%d) x head_dim(128)", w->dim, w->heads);
  WAM_REQUIRE(w->dim % 128 == 0 && w->ffn_dim % 128 == 0 && w->dim <= 4096,
              "block: dim=%d / ffn_dim=%d must be multiples of 128 (dim <= 4096)", w->dim, w->ffn_dim);
  WAM_REQUIRE(w->w[0] != nullptr, "block: scale_shift_table (weight 0) missing");
  for (int i = 3; i < 27; ++i)
    WAM_REQUIRE(w->w[i] != nullptr, "block: weight %d missing", i);
  WAM_REQUIRE((w->w[1] == nullptr) == (w->w[2] == nullptr), "block: norm2 weight/bias must both be set or both empty");
  WAM_REQUIRE(w->table_dtype == WAM_F32 || w->table_dtype == WAM_BF16, "block: table dtype");
  WAM_REQUIRE(w->norm2_dtype == WAM_F32 || w->norm2_dtype == WAM_BF16, "block: norm2 dtype");
  WAM_REQUIRE(!w->ffn_fp8[0] || (w->ffn_fp8[1] && w->ffn_scale[0] && w->ffn_scale[1]),
              "block: fp8 FFN needs both weights and both scale vectors");
  WAM_REQUIRE(w->ffn_act_fp8 >= 0 && w->ffn_act_fp8 <= 2, "block: ffn_act_fp8 must be 0, 1 or 2");
  WAM_REQUIRE(!w->ffn_act_fp8 || (w->ffn_fp8[0] && w->ffn_dim % 256 == 0),
              "block: fp8 FFN activations need the fp8 FFN weights and ffn_dim %% 256 == 0 (ffn_dim=%d)",
              w->ffn_dim);
  return WAM_OK;
}

static void gemm_args(wam_linear_args& g, const void* a, int64_t lda, int M, int K, int N,
                      const void* w, const void* b, void* out, int64_t ldo) {
  memset(&g, 0, sizeof(g));
  g.a = a; g.lda = lda; g.M = M; g.K = K; g.n_seg = 1; g.seg_n = N;
  g.w[0] = w; g.ldw = K; g.bias[0] = b; g.out[0] = out; g.ldo = ldo;
  g.epilogue = WAM_EPI_BIAS;
}

// Cross K/V of the context rows: k = RMS(ctx Wk^T + bk) g, v = ctx Wv^T + bv.
static int context_kv(const wam_block_weights* W, const void* ctx, int rows, void* k, void* v,
                      hipStream_t s, void* k_linear_debug = nullptr) {
  const int D = W->dim;
  wam_linear_args g;
  gemm_args(g, ctx, D, rows, D, D, W->w[15], W->w[16], k, D);
  g.n_seg = 2; g.w[1] = W->w[17]; g.bias[1] = W->w[18]; g.out[1] = v;
  WAM_TRY(linear(&g, s));
  if (k_linear_debug)
    WAM_HIP(hipMemcpyAsync(k_linear_debug, k, (size_t)rows * D * 2, hipMemcpyDeviceToDevice, s));
  wam_rms_rope_args r{};
  r.x[0] = k; r.y[0] = k; r.gamma[0] = W->w[22]; r.eps[0] = W->eps[6];
  r.ldx = D; r.ldy = D; r.n_tensors = 1; r.rows = rows; r.D = D; r.head_dim = W->head_dim;
  return rms_rope(&r, s);
}

static int block_forward(const wam_block_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr, "block: null args");
  WAM_TRY(check_weights(a->weights));
  const wam_block_weights* W = a->weights;
  const int B = a->B, M = a->M, D = W->dim, F = W->ffn_dim, H = W->heads;
  const int R = B * M;
  WAM_REQUIRE(B >= 1 && M >= 1, "block: empty input B=%d M=%d", B, M);
  WAM_REQUIRE(a->x && a->out, "block: null x/out");
  WAM_REQUIRE(a->out_dtype == WAM_BF16 || a->out_dtype == WAM_F32, "block: out_dtype %d", a->out_dtype);
  WAM_REQUIRE(a->out_dtype == WAM_BF16 || !a->debug, "block: debug outputs need the bf16 output");
  WAM_TRY(check_modulation(a->mod, R, "block"));
  WAM_REQUIRE(a->mod.tokens == M && a->mod.temb_mods != 1, "block: temb must be [B, L, 6, D] over M tokens");
  const bool precomputed = a->cross_k && a->cross_v;
  WAM_REQUIRE(a->context_batch >= 1 && a->context_len >= 1, "block: context shape");
  WAM_REQUIRE(precomputed || a->context, "block: context or precomputed cross K/V required");
  if (!a->context_rows) WAM_REQUIRE(a->context_batch == 1 || a->context_batch == B,
                                    "block: context batch %d vs B=%d", a->context_batch, B);
  const bool cache = a->cache_k != nullptr;
  const bool candidate = a->candidate_rows != nullptr;
  WAM_REQUIRE(!candidate || cache, "candidate verification requires existing read-only KV");
  WAM_REQUIRE(!candidate || a->update == 0, "candidate verification requires update_cache=0");
  if (cache) {
    WAM_REQUIRE(a->cache_v && a->cache_id && a->cache_mask && a->cache_is_pred && a->pool >= 1,
                "block: cache needs k, v, id, mask, is_pred");
    WAM_REQUIRE(candidate || a->cache_batch == B, "block: cache batch %d must equal B=%d",
                a->cache_batch, B);
    WAM_REQUIRE(candidate || M <= a->pool, "block: %d tokens exceed the pool of %d", M, a->pool);
    WAM_REQUIRE(a->update >= 0 && a->update <= 2, "block: update must be 0, 1 or 2");
  }
  const Layout L = layout(B, M, D, F, a->context_batch, a->context_len, cache ? a->pool : 0);
  WAM_REQUIRE(a->workspace && a->workspace_bytes >= L.total,
              "block: workspace of %zu bytes is smaller than the %zu required",
              a->workspace_bytes, L.total);
  char* ws = static_cast<char*>(a->workspace);
  void* split_ws = L.split_bytes ? ws + L.split : nullptr;
  const int64_t split_bytes = (int64_t)L.split_bytes;
  bf16* h = reinterpret_cast<bf16*>(ws + L.h);
  uint8_t* h8 = reinterpret_cast<uint8_t*>(ws + L.h8);
  float* h8s = reinterpret_cast<float*>(ws + L.h8s);
  bf16* qkv = reinterpret_cast<bf16*>(ws + L.qkv);
  bf16* attn = reinterpret_cast<bf16*>(ws + L.attn);
  float* x1 = reinterpret_cast<float*>(ws + L.x1);
  float* x2 = reinterpret_cast<float*>(ws + L.x2);
  bf16* act = reinterpret_cast<bf16*>(ws + L.act);
  // The MX hidden layer (ffn_act_fp8 = 2): e4m3 [R, F] at act, its e8m0
  // exponents [R, F / 32] right after (within the bf16 layer's bytes).
  uint8_t* act_mx = reinterpret_cast<uint8_t*>(ws + L.act) + (size_t)R * F;
  int32_t* slots = reinterpret_cast<int32_t*>(ws + L.slots);
  int32_t* newslots = reinterpret_cast<int32_t*>(ws + L.newslots);
  int32_t* info = reinterpret_cast<int32_t*>(ws + L.info);
  float* qssq = reinterpret_cast<float*>(ws + L.ssq);
  const size_t rowb = (size_t)R * D * 2;
  // Cross-attention query norm: the projection's epilogue writes y g and the
  // row's sums of squares, attention applies 1/rms (no row pass), when the
  // projection runs as one launch of the four-wave kernel or as one round of
  // 320-row tiles (6240 rows); other tilings would run the norm as a pass
  // anyway, and the row pass is as fast.  A debug call runs
  // the same kernels; its copies of the projection (before the norm) and of
  // the normalised queries come from extra debug-only launches.  (For the
  // self-attention queries the same fusion measured even: the QKV
  // epilogue's cost matched the half of the q/k row pass it removes.)
  const bool qnorm_fused = linear_norm_in_epilogue(R, D, 1, D, split_bytes, false);
  const int qparts = (D + 255) / 256;

  wam_modulation mod = a->mod;
  mod.table = W->w[0];
  mod.table_dtype = W->table_dtype;

  // 1. LN1 + modulation (shift 0, scale 1).
  {
    Scope sc(a->timer, WAM_STAGE_LN1, s);
    wam_ln_args l{};
    l.x = a->x; l.y = h; l.rows = R; l.D = D; l.eps = W->eps[0]; l.affine = 0;
    l.mod = mod; l.shift_index = 0;
    WAM_TRY(ln_modulate(&l, s));
  }
  WAM_TRY(copy_debug(a->debug, 0, h, rowb, s));
  // Debug only: the reference's unfused intermediates (slots 15-27), each
  // by an extra launch where the fused kernels do not materialise it.
  auto dbg = [&](int i) -> void* { return a->debug ? a->debug[i] : nullptr; };
  float* zeros = reinterpret_cast<float*>(ws + L.zeros);
  auto plain_ln = [&](const void* x, int x_dtype, float eps, void* y) -> int {
    // LayerNorm without modulation: a zero table [2, D] and zero vectors
    wam_ln_args l{};
    l.x = x; l.x_dtype = x_dtype; l.y = y; l.rows = R; l.D = D; l.eps = eps; l.affine = 0;
    l.mod.table = zeros; l.mod.table_dtype = WAM_F32; l.mod.temb = zeros + 2 * D; l.mod.temb_dtype = WAM_F32;
    l.mod.temb_len = 1; l.mod.tokens = M; l.mod.temb_mods = 1; l.shift_index = 0;
    return ln_modulate(&l, s);
  };
  auto plain_linear = [&](const void* x, int K, int N, int wi, int wf8, void* y) -> int {
    // bias epilogue only, with the same weights as the fused launch
    wam_linear_args g;
    gemm_args(g, x, K, R, K, N, W->w[wi], W->w[wi + 1], y, N);
    if (wf8 >= 0 && W->ffn_fp8[0]) {
      g.w[0] = W->ffn_fp8[wf8]; g.w_dtype = WAM_FP8; g.w_scale[0] = W->ffn_scale[wf8];
    }
    if (wf8 == 0 && W->ffn_act_fp8) {
      g.a = h8; g.a_dtype = WAM_FP8; g.a_scale = h8s;  // the fused FFN1's own input
    }
    if (wf8 == 1 && W->ffn_act_fp8 == 2) {
      // FFN2's own MX input
      g.a = act; g.lda = F; g.a_dtype = WAM_FP8_MX; g.a_block_scale = act_mx;
    }
    g.workspace = split_ws; g.workspace_bytes = split_bytes;
    return linear(&g, s);
  };
  if (dbg(25) || dbg(26)) {
    const int64_t nz = ((int64_t)B + 2) * D;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((nz + 255) / 256)), dim3(256), 0, s, zeros, nz);
    WAM_LAUNCHED("fill_zero_kernel");
  }
  if (dbg(25)) WAM_TRY(plain_ln(a->x, WAM_BF16, W->eps[0], dbg(25)));
  if (dbg(27)) {
    const int64_t n = (int64_t)B * mod.temb_len * 6 * D;
    hipLaunchKernelGGL(modulation_table_kernel, dim3((unsigned)((n + 255) / 256 < 16384 ? (n + 255) / 256 : 16384)),
                       dim3(256), 0, s, mod, D, n, static_cast<float*>(dbg(27)));
    WAM_LAUNCHED("modulation_table_kernel");
  }
  // 2. Q|K|V projection as one launch into the packed [R, 3D] buffer.
  {
    Scope sc(a->timer, WAM_STAGE_QKV, s);
    wam_linear_args g;
    gemm_args(g, h, D, R, D, D, W->w[3], W->w[4], qkv, 3 * D);
    g.n_seg = 3;
    g.w[1] = W->w[5]; g.bias[1] = W->w[6]; g.out[1] = qkv + D;
    g.w[2] = W->w[7]; g.bias[2] = W->w[8]; g.out[2] = qkv + 2 * D;
    g.workspace = split_ws; g.workspace_bytes = split_bytes;
    WAM_TRY(linear(&g, s));
  }
  for (int i = 0; i < 2; ++i) {
    if (dbg(15 + i))
      WAM_HIP(hipMemcpy2DAsync(dbg(15 + i), D * 2, qkv + i * D, 3 * D * 2, D * 2, R, hipMemcpyDeviceToDevice, s));
    if (dbg(17 + i)) {
      wam_rms_rope_args r{};
      r.x[0] = qkv + i * D; r.y[0] = dbg(17 + i); r.gamma[0] = W->w[11 + i]; r.eps[0] = W->eps[3 + i];
      r.ldx = 3 * D; r.ldy = D; r.n_tensors = 1; r.rows = R; r.D = D; r.head_dim = W->head_dim;
      WAM_TRY(rms_rope(&r, s));
    }
  }
  // 3. q/k RMSNorm across heads + RoPE, in place.
  {
    Scope sc(a->timer, WAM_STAGE_RMS_ROPE, s);
    wam_rms_rope_args r{};
    r.x[0] = qkv; r.y[0] = qkv; r.gamma[0] = W->w[11]; r.eps[0] = W->eps[3];
    r.x[1] = qkv + D; r.y[1] = qkv + D; r.gamma[1] = W->w[12]; r.eps[1] = W->eps[4];
    r.ldx = 3 * D; r.ldy = 3 * D; r.n_tensors = 2; r.rows = R; r.D = D;
    r.head_dim = W->head_dim;
    r.freq = a->freq; r.freq_batch = a->freq_batch; r.tokens = M;
    WAM_TRY(rms_rope(&r, s));
  }
  if (a->debug) {
    for (int i = 0; i < 3; ++i)
      if (a->debug[1 + i])
        WAM_HIP(hipMemcpy2DAsync(a->debug[1 + i], D * 2, qkv + i * D, 3 * D * 2, D * 2, R,
                                 hipMemcpyDeviceToDevice, s));
  }
  // 4. Pool bookkeeping.
  if (cache) {
    Scope sc(a->timer, WAM_STAGE_KV_LAYOUT, s);
    wam_kv_layout_args k{};
    k.mask = a->cache_mask; k.ids = a->cache_id; k.is_pred = a->cache_is_pred; k.pool = a->pool;
    k.tokens = M; k.update = a->update; k.candidate = candidate ? 1 : 0;
    k.rows = a->candidate_rows; k.batch = B; k.pool_batch = a->cache_batch;
    k.hist_slots = slots; k.new_slots = newslots; k.info = info;
    WAM_TRY(kv_layout(&k, s));
  }
  // 5. Self attention over [history || own].
  {
    Scope sc(a->timer, WAM_STAGE_SELF_ATTN, s);
    wam_attention_args t{};
    t.q = qkv; t.q_bstride = (int64_t)M * 3 * D; t.q_rstride = 3 * D;
    t.o = attn; t.o_bstride = (int64_t)M * D; t.o_rstride = D;
    t.B = B; t.Mq = M; t.H = H; t.head_dim = W->head_dim;
    if (cache) {
      t.pool_k = a->cache_k; t.pool_v = a->cache_v;
      t.pool_rstride = D; t.pool_bstride = (int64_t)a->pool * D; t.pool_batch = a->cache_batch;
      t.slots = slots; t.n_hist_dev = info; t.pool_rows = a->candidate_rows;
      t.hist_base_dev = info + 2;
    }
    t.k = qkv + D; t.v = qkv + 2 * D; t.kv_bstride = (int64_t)M * 3 * D; t.kv_rstride = 3 * D;
    t.Mk = M; t.kv_batch = B;
    t.max_keys = M + (cache ? a->pool : 0);
    t.scale = 1.0f / sqrtf((float)W->head_dim);
    t.workspace = L.split_bytes ? ws + L.split : nullptr; t.workspace_bytes = (int64_t)L.split_bytes;
    WAM_TRY(attention(&t, s));
  }
  WAM_TRY(copy_debug(a->debug, 4, attn, rowb, s));
  // 6. New K/V into the pool for committed updates.
  if (cache && !candidate && a->update != 0) {
    Scope sc(a->timer, WAM_STAGE_KV_COMMIT, s);
    wam_kv_commit_args c{};
    c.k = qkv + D; c.v = qkv + 2 * D; c.ld = 3 * D;
    c.pool_k = a->cache_k; c.pool_v = a->cache_v;
    c.pool_bstride = (int64_t)a->pool * D; c.pool_rstride = D;
    c.new_slots = newslots; c.B = B; c.tokens = M; c.D = D;
    WAM_TRY(kv_commit(&c, s));
  }
  // 7. Output projection + gated residual (gate 2).
  {
    Scope sc(a->timer, WAM_STAGE_SELF_OUT, s);
    wam_linear_args g;
    gemm_args(g, attn, D, R, D, D, W->w[9], W->w[10], x1, D);
    g.epilogue = WAM_EPI_BIAS_GATE_RES; g.res = a->x; g.ldr = D; g.gate = mod; g.gate_index = 2;
    g.out_dtype = WAM_F32;
    g.workspace = split_ws; g.workspace_bytes = split_bytes;
    WAM_TRY(linear(&g, s));
  }
  WAM_TRY(copy_debug(a->debug, 5, x1, rowb * 2, s));
  if (dbg(19)) WAM_TRY(plain_linear(attn, D, D, 9, -1, dbg(19)));
  // 8. norm2 (affine LayerNorm), or without cross_attn_norm the bf16 cast
  //    of the residual stream that the identity norm2 passes through.
  const bf16* n2 = h;
  {
    Scope sc(a->timer, WAM_STAGE_LN2, s);
    if (W->w[1]) {
      wam_ln_args l{};
      l.x = x1; l.x_dtype = WAM_F32; l.y = h; l.rows = R; l.D = D; l.eps = W->eps[1]; l.affine = 1;
      l.gamma = W->w[1]; l.beta = W->w[2]; l.gb_dtype = W->norm2_dtype;
      WAM_TRY(ln_modulate(&l, s));
    } else {
      WAM_TRY(cast_f32_bf16(x1, h, (int64_t)R * D, s));
    }
  }
  WAM_TRY(copy_debug(a->debug, 6, n2, rowb, s));
  // 9. Cross Q = RMS(n2 Wq2^T + b) g  (into the q third of the qkv buffer).
  bf16* cq = qkv;
  {
    Scope sc(a->timer, WAM_STAGE_CROSS_Q, s);
    wam_linear_args g;
    gemm_args(g, n2, D, R, D, D, W->w[13], W->w[14], cq, D);
    g.workspace = split_ws; g.workspace_bytes = split_bytes;
    if (qnorm_fused) { g.norm_ssq[0] = qssq; g.norm_gamma[0] = W->w[21]; }
    WAM_TRY(linear(&g, s));
    if (!qnorm_fused) {
      WAM_TRY(copy_debug(a->debug, 20, cq, rowb, s));
      wam_rms_rope_args r{};
      r.x[0] = cq; r.y[0] = cq; r.gamma[0] = W->w[21]; r.eps[0] = W->eps[5];
      r.ldx = D; r.ldy = D; r.n_tensors = 1; r.rows = R; r.D = D; r.head_dim = W->head_dim;
      WAM_TRY(rms_rope(&r, s));
    }
  }
  if (qnorm_fused) {
    // debug only: the projection before its norm, and the normalised queries
    // as the reference forms them (the projection, then the RMS row pass:
    // bf16(y rsqrt(mean y^2 + eps) g), one rounding)
    if (dbg(20)) WAM_TRY(plain_linear(n2, D, D, 13, -1, dbg(20)));
    if (dbg(7)) {
      WAM_TRY(plain_linear(n2, D, D, 13, -1, dbg(7)));
      wam_rms_rope_args r{};
      r.x[0] = dbg(7); r.y[0] = dbg(7); r.gamma[0] = W->w[21]; r.eps[0] = W->eps[5];
      r.ldx = D; r.ldy = D; r.n_tensors = 1; r.rows = R; r.D = D; r.head_dim = W->head_dim;
      WAM_TRY(rms_rope(&r, s));
    }
  } else {
    WAM_TRY(copy_debug(a->debug, 7, cq, rowb, s));
  }
  // 10. Cross K/V: precomputed or from the context.
  const void* ck = a->cross_k;
  const void* cv = a->cross_v;
  const size_t ctxb = (size_t)a->context_batch * a->context_len * D * 2;
  if (!precomputed) {
    Scope sc(a->timer, WAM_STAGE_CROSS_KV, s);
    WAM_TRY(context_kv(W, a->context, a->context_batch * a->context_len, ws + L.ck, ws + L.cv, s, dbg(21)));
    ck = ws + L.ck;
    cv = ws + L.cv;
  }
  WAM_TRY(copy_debug(a->debug, 8, ck, ctxb, s));
  WAM_TRY(copy_debug(a->debug, 9, cv, ctxb, s));
  // 11. Cross attention.
  {
    Scope sc(a->timer, WAM_STAGE_CROSS_ATTN, s);
    wam_attention_args t{};
    t.q = cq; t.q_bstride = (int64_t)M * D; t.q_rstride = D;
    t.o = attn; t.o_bstride = (int64_t)M * D; t.o_rstride = D;
    t.B = B; t.Mq = M; t.H = H; t.head_dim = W->head_dim;
    t.k = ck; t.v = cv; t.kv_bstride = (int64_t)a->context_len * D; t.kv_rstride = D;
    t.Mk = a->context_len; t.kv_batch = a->context_batch;
    t.kv_rows = a->context_rows;
    t.max_keys = a->context_len;
    t.scale = 1.0f / sqrtf((float)W->head_dim);
    t.workspace = L.split_bytes ? ws + L.split : nullptr; t.workspace_bytes = (int64_t)L.split_bytes;
    if (qnorm_fused) { t.q_ssq = qssq; t.q_ssq_n = qparts; t.q_norm_dim = D; t.q_eps = W->eps[5]; }
    WAM_TRY(attention(&t, s));
  }
  WAM_TRY(copy_debug(a->debug, 10, attn, rowb, s));
  // 12. Cross output projection + plain residual.
  {
    Scope sc(a->timer, WAM_STAGE_CROSS_OUT, s);
    wam_linear_args g;
    gemm_args(g, attn, D, R, D, D, W->w[19], W->w[20], x2, D);
    g.epilogue = WAM_EPI_BIAS_RES; g.res = x1; g.ldr = D; g.res_dtype = WAM_F32;
    g.out_dtype = WAM_F32;
    g.workspace = split_ws; g.workspace_bytes = split_bytes;
    WAM_TRY(linear(&g, s));
  }
  WAM_TRY(copy_debug(a->debug, 11, x2, rowb * 2, s));
  if (dbg(22)) WAM_TRY(plain_linear(attn, D, D, 19, -1, dbg(22)));
  if (dbg(26)) WAM_TRY(plain_ln(x2, WAM_F32, W->eps[2], dbg(26)));
  // 13. LN3 + modulation (c_shift 3, c_scale 4).
  {
    Scope sc(a->timer, WAM_STAGE_LN3, s);
    wam_ln_args l{};
    l.x = x2; l.x_dtype = WAM_F32; l.y = h; l.rows = R; l.D = D; l.eps = W->eps[2]; l.affine = 0;
    l.mod = mod; l.shift_index = 3;
    if (W->ffn_act_fp8) {
      // e4m3 rows for the fp8 FFN1; the bf16 rows only when a debug copy reads them
      l.y8 = h8; l.y8_scale = h8s;
      if (!dbg(12)) l.y = nullptr;
    }
    WAM_TRY(ln_modulate(&l, s));
  }
  WAM_TRY(copy_debug(a->debug, 12, h, rowb, s));
  if (dbg(23)) WAM_TRY(plain_linear(h, D, F, 23, 0, dbg(23)));
  // 14. FFN1 + GELU(tanh).
  {
    Scope sc(a->timer, WAM_STAGE_FFN1, s);
    wam_linear_args g;
    gemm_args(g, h, D, R, D, F, W->w[23], W->w[24], act, F);
    g.epilogue = WAM_EPI_BIAS_GELU;
    if (W->ffn_fp8[0]) {
      g.w[0] = W->ffn_fp8[0]; g.w_dtype = WAM_FP8; g.w_scale[0] = W->ffn_scale[0];
    }
    if (W->ffn_act_fp8) {
      g.a = h8; g.a_dtype = WAM_FP8; g.a_scale = h8s;
    }
    if (W->ffn_act_fp8 == 2) {
      // e4m3 hidden layer with e8m0 exponents per 32 columns, FFN2's MX input
      g.out_dtype = WAM_FP8_MX; g.out_block_scale = act_mx;
    }
    g.workspace = split_ws; g.workspace_bytes = split_bytes;
    WAM_TRY(linear(&g, s));
  }
  if (W->ffn_act_fp8 == 2) {
    if (dbg(13)) WAM_TRY(mx_dequant_bf16(act, act_mx, dbg(13), R, F, s));
  } else {
    WAM_TRY(copy_debug(a->debug, 13, act, (size_t)R * F * 2, s));
  }
  if (dbg(24)) WAM_TRY(plain_linear(act, F, D, 25, 1, dbg(24)));
  // 15. FFN2 + gated residual (c_gate 5).
  {
    Scope sc(a->timer, WAM_STAGE_FFN2, s);
    wam_linear_args g;
    gemm_args(g, act, F, R, F, D, W->w[25], W->w[26], a->out, D);
    g.epilogue = WAM_EPI_BIAS_GATE_RES; g.res = x2; g.ldr = D; g.res_dtype = WAM_F32;
    if (W->ffn_fp8[0]) {
      g.w[0] = W->ffn_fp8[1]; g.w_dtype = WAM_FP8; g.w_scale[0] = W->ffn_scale[1];
    }
    if (W->ffn_act_fp8 == 2) {
      g.a_dtype = WAM_FP8_MX; g.a_block_scale = act_mx;
    }
    g.gate = mod; g.gate_index = 5;
    g.out_dtype = a->out_dtype;
    g.workspace = split_ws; g.workspace_bytes = split_bytes;
    WAM_TRY(linear(&g, s));
  }
  WAM_TRY(copy_debug(a->debug, 14, a->out, rowb, s));
  return WAM_OK;
}

}  // namespace wam

extern "C" {

const char* wam_last_error(void) { return wam::g_error; }
int wam_abi_version(void) { return WAM_ABI_VERSION; }

size_t wam_abi_struct_size(const char* name) {
  if (!name) return 0;
  if (!strcmp(name, "wam_modulation")) return sizeof(wam_modulation);
  if (!strcmp(name, "wam_linear_args")) return sizeof(wam_linear_args);
  if (!strcmp(name, "wam_ln_args")) return sizeof(wam_ln_args);
  if (!strcmp(name, "wam_rms_rope_args")) return sizeof(wam_rms_rope_args);
  if (!strcmp(name, "wam_attention_args")) return sizeof(wam_attention_args);
  if (!strcmp(name, "wam_kv_layout_args")) return sizeof(wam_kv_layout_args);
  if (!strcmp(name, "wam_kv_commit_args")) return sizeof(wam_kv_commit_args);
  if (!strcmp(name, "wam_block_weights")) return sizeof(wam_block_weights);
  if (!strcmp(name, "wam_block_args")) return sizeof(wam_block_args);
  if (!strcmp(name, "wam_patchify_args")) return sizeof(wam_patchify_args);
  if (!strcmp(name, "wam_timestep_args")) return sizeof(wam_timestep_args);
  if (!strcmp(name, "wam_rows_linear_args")) return sizeof(wam_rows_linear_args);
  if (!strcmp(name, "wam_rope_freq_args")) return sizeof(wam_rope_freq_args);
  return 0;
}

size_t wam_block_workspace_bytes(int B, int M, int dim, int ffn_dim, int context_batch,
                                 int context_len, int pool) {
  return wam::layout(B, M, dim, ffn_dim, context_batch, context_len, pool).total;
}

int wam_block_forward(const wam_block_args* args, void* stream) {
  return wam::block_forward(args, static_cast<hipStream_t>(stream));
}

int wam_prepare_context(const wam_block_weights* weights, const void* context, int rows,
                        void* k_out, void* v_out, void* stream) {
  WAM_TRY(wam::check_weights(weights));
  WAM_REQUIRE(context && k_out && v_out && rows >= 1, "prepare_context: null tensor or empty context");
  return wam::context_kv(weights, context, rows, k_out, v_out, static_cast<hipStream_t>(stream));
}

void* wam_timer_create(int capacity, uint32_t stage_mask) {
  if (capacity < 1) return nullptr;
  auto* t = new wam::Timer();
  t->capacity = capacity;
  t->mask = stage_mask;
  t->ev.resize(2 * (size_t)capacity);
  t->stage.resize(capacity);
  for (auto& e : t->ev) {
    if (hipEventCreate(&e) != hipSuccess) {
      wam::set_error("hipEventCreate failed");
      delete t;
      return nullptr;
    }
  }
  return t;
}

void wam_timer_reset(void* timer) {
  if (timer) static_cast<wam::Timer*>(timer)->count = 0;
}

int wam_timer_read(void* timer, int32_t* stages, float* ms, int max) {
  auto* t = static_cast<wam::Timer*>(timer);
  WAM_REQUIRE(t != nullptr, "timer: null");
  const int n = t->count < max ? t->count : max;
  for (int i = 0; i < n; ++i) {
    WAM_HIP(hipEventSynchronize(t->ev[2 * i + 1]));
    float v = 0.f;
    WAM_HIP(hipEventElapsedTime(&v, t->ev[2 * i], t->ev[2 * i + 1]));
    stages[i] = t->stage[i];
    ms[i] = v;
  }
  return n;
}

void wam_timer_destroy(void* timer) {
  auto* t = static_cast<wam::Timer*>(timer);
  if (!t) return;
  for (auto& e : t->ev) (void)hipEventDestroy(e);
  delete t;
}

}  // extern "C"
