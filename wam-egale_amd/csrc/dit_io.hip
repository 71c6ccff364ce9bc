// Model input/output around the block loop (WanTransformer3DModel.forward,
// 投机采样/wam-p0-worktree/wan_va/modules/model.py:1060-1116):
//
//   patchify        the latents' patch rearrange ahead of patch_embedding_mlp /
//                   action_embedder (model.py:1060-1071); the projection itself
//                   is wam_linear on the gathered rows.
//   timestep        diffusers' sinusoidal timestep embedding (Timesteps,
//                   model.py:216-218,233).
//   rows_linear     the condition embedder's few-row linears (time_embedder,
//                   time_proj; model.py:219-222,234-239) and action_proj_out.
//   rope_freqs      WanRotaryPosEmbed.forward (model.py:276-286).
//
// All of these are small next to one block (kilobytes to a few megabytes of
// HBM traffic, or one pass over the condition embedder's weights); they are
// written to be bandwidth-reasonable and exact, not tuned.
#include <math.h>
#include "wam_common.h"

namespace wam {

// ---------------------------------------------------------------- patchify
// One thread per (sample, channel, token), tokens fastest, so that a wave's
// reads walk along the latent rows; each thread writes its p1*p2*p3 output
// columns.  The thread of channel 0 also zeroes the row's padding columns.
__global__ __launch_bounds__(256) void patchify_kernel(wam_patchify_args a, int Fp, int Hp, int Wp) {
  const int L = Fp * Hp * Wp;
  const int64_t total = (int64_t)a.B * a.C * L;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int tok = (int)(i % L);
  const int64_t bc = i / L;
  const int c = (int)(bc % a.C);
  const int64_t b = bc / a.C;
  const int wi = tok % Wp, hi = (tok / Wp) % Hp, fi = tok / (Wp * Hp);
  const int P = a.p1 * a.p2 * a.p3;
  const bf16* src = static_cast<const bf16*>(a.x) + (b * a.C + c) * (int64_t)a.F * a.H * a.W;
  bf16* row = static_cast<bf16*>(a.out) + (b * L + tok) * (int64_t)a.k_pad;
  bf16* dst = row + (int64_t)c * P;
  for (int i1 = 0; i1 < a.p1; ++i1)
    for (int j = 0; j < a.p2; ++j)
      for (int k = 0; k < a.p3; ++k) {
        const int64_t s = ((int64_t)(fi * a.p1 + i1) * a.H + (hi * a.p2 + j)) * a.W + (wi * a.p3 + k);
        dst[(i1 * a.p2 + j) * a.p3 + k] = src[s];
      }
  if (c == 0)
    for (int col = a.C * P; col < a.k_pad; ++col) row[col] = static_cast<bf16>(0.f);
}

int patchify(const wam_patchify_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr && a->x && a->out, "wam_patchify: null args");
  WAM_REQUIRE(a->B >= 1 && a->C >= 1 && a->F >= 1 && a->H >= 1 && a->W >= 1 && a->p1 >= 1 &&
              a->p2 >= 1 && a->p3 >= 1, "wam_patchify: empty shape");
  WAM_REQUIRE(a->F % a->p1 == 0 && a->H % a->p2 == 0 && a->W % a->p3 == 0,
              "wam_patchify: F/H/W (%d/%d/%d) must be multiples of the patch (%d/%d/%d)", a->F, a->H,
              a->W, a->p1, a->p2, a->p3);
  const int64_t K = (int64_t)a->C * a->p1 * a->p2 * a->p3;
  WAM_REQUIRE(a->k_pad >= K, "wam_patchify: k_pad %d < C*p1*p2*p3 = %lld", a->k_pad, (long long)K);
  const int Fp = a->F / a->p1, Hp = a->H / a->p2, Wp = a->W / a->p3;
  const int64_t L = (int64_t)Fp * Hp * Wp;
  const int64_t threads = (int64_t)a->B * a->C * L;
  WAM_REQUIRE(L < (1ll << 31) && threads < (1ll << 40), "wam_patchify: too large");
  hipLaunchKernelGGL(patchify_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, *a, Fp, Hp,
                     Wp);
  WAM_LAUNCHED("patchify_kernel");
  return WAM_OK;
}

// --------------------------------------------------------------- timestep
// One thread per (row, frequency).  The frequency and the argument are formed
// in fp32 exactly as the reference's op sequence does (fp32 exponent, fp32
// product); exp, sin and cos are evaluated in fp64 and rounded once.
__global__ __launch_bounds__(256) void timestep_kernel(wam_timestep_args a, float neg_log_period) {
  const int half = a.dim / 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)a.rows * half) return;
  const int64_t r = i / half;
  const int j = (int)(i % half);
  const float e = (neg_log_period * (float)j) / ((float)half - a.shift);
  const float freq = (float)exp((double)e);
  const float arg = a.t[r] * freq;
  const float sv = (float)sin((double)arg), cv = (float)cos((double)arg);
  const int64_t base = r * a.dim;
  const int64_t pc = base + (a.flip_sin_to_cos ? j : half + j);
  const int64_t ps = base + (a.flip_sin_to_cos ? half + j : j);
  if (a.out_dtype == WAM_F32) {
    float* o = static_cast<float*>(a.out);
    o[pc] = cv;
    o[ps] = sv;
    if (j == 0 && (a.dim & 1)) o[base + a.dim - 1] = 0.f;
  } else {
    bf16* o = static_cast<bf16*>(a.out);
    o[pc] = static_cast<bf16>(cv);
    o[ps] = static_cast<bf16>(sv);
    if (j == 0 && (a.dim & 1)) o[base + a.dim - 1] = static_cast<bf16>(0.f);
  }
}

int timestep_embedding(const wam_timestep_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr && a->t && a->out, "wam_timestep_embedding: null args");
  WAM_REQUIRE(a->rows >= 0 && a->dim >= 2, "wam_timestep_embedding: rows %d dim %d", a->rows, a->dim);
  WAM_REQUIRE(a->out_dtype == WAM_F32 || a->out_dtype == WAM_BF16, "wam_timestep_embedding: out dtype");
  WAM_REQUIRE(a->max_period > 0.f && (float)(a->dim / 2) != a->shift, "wam_timestep_embedding: period/shift");
  if (a->rows == 0) return WAM_OK;
  const int64_t n = (int64_t)a->rows * (a->dim / 2);
  const float nl = (float)(-log((double)a->max_period));
  hipLaunchKernelGGL(timestep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, *a, nl);
  WAM_LAUNCHED("timestep_kernel");
  return WAM_OK;
}

// ------------------------------------------------------------ rows_linear
// Weight streaming: each wave owns kRlOut consecutive outputs (weight rows)
// and up to kRlRows rows of x.  Lane l reads the 8-element pieces
// k = 8l + 512j of its weight rows (16-byte loads, 1 KB per wave instruction,
// straight from HBM) and of the x rows, and keeps the kRlRows x kRlOut
// partial dot products in registers; one DPP reduction per output at the end.
//
// Without an input activation the x rows are read from L2 by every wave and
// a workgroup is 4 independent waves.  With one (SiLU), act_in(x) is formed
// once per workgroup of 8 waves into LDS, kRlSeg columns at a time, so the
// activation is not recomputed per wave.
constexpr int kRlRows = 8, kRlOut = 4, kRlSeg = 2048;

__device__ inline float silu(float v) { return v / (1.f + expf(-v)); }
// SiLU of an input element: v * rcp(1 + 2^(-v log2 e)); a few ulp of fp32,
// below the bf16 rounding that follows for bf16 inputs.
__device__ inline float silu_fast(float v) {
  return v * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-v * kLog2e));
}
__device__ inline float round_to(float v, int dtype) {
  return dtype == WAM_BF16 ? static_cast<float>(static_cast<bf16>(v)) : v;
}

template <bool VEC>
__device__ inline void rl_load8(const void* p, int dtype, int64_t off, int left, float out[8]) {
  if (VEC) {
    ld8_f32(p, dtype, off, out);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = e < left ? ld_scalar(p, dtype, off + e) : 0.f;
  }
}

template <bool VEC>
__device__ inline void rl_weights(const wam_rows_linear_args& a, int n0, int nc, int k, float wv[kRlOut][8]) {
#pragma unroll
  for (int c = 0; c < kRlOut; ++c) {
    if (c < nc) {
      rl_load8<VEC>(a.w, a.w_dtype, (int64_t)(n0 + c) * a.ldw + k, a.K - k, wv[c]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) wv[c][e] = 0.f;
    }
  }
}

__device__ inline void rl_fma(float acc[kRlRows][kRlOut], int r, const float xv[8], const float wv[kRlOut][8]) {
#pragma unroll
  for (int c = 0; c < kRlOut; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][c] += xv[e] * wv[c][e];
}

__device__ inline void rl_store(const wam_rows_linear_args& a, float acc[kRlRows][kRlOut], int lane, int n0,
                                int r0, int nr, int nc) {
  // Lane r * kRlOut + c keeps the sum of output (r, c).
  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < kRlRows; ++r)
#pragma unroll
    for (int c = 0; c < kRlOut; ++c) {
      const float v = wave_sum(acc[r][c]);
      if (lane == r * kRlOut + c) mine = v;
    }
  const int r = lane / kRlOut, c = lane % kRlOut;
  if (lane >= kRlRows * kRlOut || r >= nr || c >= nc) return;
  const int n = n0 + c;
  float v = mine;
  if (a.bias) v += ld_scalar(a.bias, a.bias_dtype, n);
  if (a.act_out == WAM_ACT_SILU) v = silu(round_to(v, a.out_dtype));
  const int64_t o = (int64_t)(r0 + r) * a.ldo + n;
  if (a.out_dtype == WAM_F32) static_cast<float*>(a.out)[o] = v;
  else static_cast<bf16*>(a.out)[o] = static_cast<bf16>(v);
}

template <bool VEC>
__global__ __launch_bounds__(256) void rows_linear_kernel(wam_rows_linear_args a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * kRlOut;
  const int r0 = blockIdx.y * kRlRows;
  if (n0 >= a.N) return;  // whole wave; nothing below synchronises
  const int nr = min(kRlRows, a.R - r0), nc = min(kRlOut, a.N - n0);
  float acc[kRlRows][kRlOut];
#pragma unroll
  for (int r = 0; r < kRlRows; ++r)
#pragma unroll
    for (int c = 0; c < kRlOut; ++c) acc[r][c] = 0.f;
  for (int k = lane * 8; k < a.K; k += 512) {
    float wv[kRlOut][8];
    rl_weights<VEC>(a, n0, nc, k, wv);
#pragma unroll
    for (int r = 0; r < kRlRows; ++r) {
      if (r >= nr) continue;
      float xv[8];
      rl_load8<VEC>(a.x, a.x_dtype, (int64_t)(r0 + r) * a.ldx + k, a.K - k, xv);
      rl_fma(acc, r, xv, wv);
    }
  }
  rl_store(a, acc, lane, n0, r0, nr, nc);
}

// With act_in: 8 waves share act_in(x) staged in LDS (fp32, rounded to x's dtype).
template <bool VEC>
__global__ __launch_bounds__(512) void rows_linear_act_kernel(wam_rows_linear_args a) {
  __shared__ __attribute__((aligned(16))) float xs[kRlRows][kRlSeg];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 8 + wave) * kRlOut;
  const int r0 = blockIdx.y * kRlRows;
  const int nr = min(kRlRows, a.R - r0), nc = max(0, min(kRlOut, a.N - n0));
  float acc[kRlRows][kRlOut];
#pragma unroll
  for (int r = 0; r < kRlRows; ++r)
#pragma unroll
    for (int c = 0; c < kRlOut; ++c) acc[r][c] = 0.f;
  for (int seg = 0; seg < a.K; seg += kRlSeg) {
    const int len = min(kRlSeg, a.K - seg);
    __syncthreads();  // the previous segment is no longer read
    for (int i = threadIdx.x * 8; i < kRlRows * kRlSeg; i += 512 * 8) {
      const int r = i / kRlSeg, k = i % kRlSeg;
      float v[8];
      if (r < nr && k < len) {
        rl_load8<VEC>(a.x, a.x_dtype, (int64_t)(r0 + r) * a.ldx + seg + k, len - k, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = round_to(silu_fast(v[e]), a.x_dtype);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
      }
      *reinterpret_cast<float4*>(&xs[r][k]) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(&xs[r][k + 4]) = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
    if (nc == 0) continue;  // wave past N: keeps joining the barriers
    for (int k = lane * 8; k < len; k += 512) {
      float wv[kRlOut][8];
      rl_weights<VEC>(a, n0, nc, seg + k, wv);
#pragma unroll
      for (int r = 0; r < kRlRows; ++r) {
        if (r >= nr) continue;
        const float4 p = *reinterpret_cast<const float4*>(&xs[r][k]);
        const float4 q = *reinterpret_cast<const float4*>(&xs[r][k + 4]);
        const float xv[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
        rl_fma(acc, r, xv, wv);
      }
    }
  }
  if (nc > 0) rl_store(a, acc, lane, n0, r0, nr, nc);
}

static bool fd(int d) { return d == WAM_F32 || d == WAM_BF16; }

int rows_linear(const wam_rows_linear_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr && a->x && a->w && a->out, "wam_rows_linear: null args");
  WAM_REQUIRE(a->R >= 0 && a->N >= 1 && a->K >= 1, "wam_rows_linear: shape R=%d N=%d K=%d", a->R, a->N,
              a->K);
  WAM_REQUIRE(fd(a->x_dtype) && fd(a->w_dtype) && fd(a->out_dtype) && (!a->bias || fd(a->bias_dtype)),
              "wam_rows_linear: dtypes must be WAM_F32 or WAM_BF16");
  WAM_REQUIRE(a->ldx >= a->K && a->ldw >= a->K && a->ldo >= a->N, "wam_rows_linear: strides");
  WAM_REQUIRE((a->act_in == WAM_ACT_NONE || a->act_in == WAM_ACT_SILU) &&
              (a->act_out == WAM_ACT_NONE || a->act_out == WAM_ACT_SILU), "wam_rows_linear: activation");
  if (a->R == 0) return WAM_OK;
  WAM_REQUIRE(a->N <= (1 << 30) && (a->R + kRlRows - 1) / kRlRows <= 65535, "wam_rows_linear: too large");
  // 16-byte vector loads need 8-element chunks that start 16-byte aligned.
  const auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool vec = a->K % 8 == 0 && a->ldx % 8 == 0 && a->ldw % 8 == 0 && al(a->x) && al(a->w);
  const bool act = a->act_in != WAM_ACT_NONE;
  const int per_wg = kRlOut * (act ? 8 : 4);
  const dim3 grid((unsigned)((a->N + per_wg - 1) / per_wg), (unsigned)((a->R + kRlRows - 1) / kRlRows));
  if (act) {
    if (vec) hipLaunchKernelGGL(rows_linear_act_kernel<true>, grid, dim3(512), 0, s, *a);
    else hipLaunchKernelGGL(rows_linear_act_kernel<false>, grid, dim3(512), 0, s, *a);
  } else {
    if (vec) hipLaunchKernelGGL(rows_linear_kernel<true>, grid, dim3(256), 0, s, *a);
    else hipLaunchKernelGGL(rows_linear_kernel<false>, grid, dim3(256), 0, s, *a);
  }
  WAM_LAUNCHED("rows_linear_kernel");
  return WAM_OK;
}

// ------------------------------------------------------------- rope_freqs
// One thread per (sample, token, pair).  The angle is the float rounding of
// the float64 product, as the reference forms it; cos and sin are evaluated in
// fp64 and rounded once.
__global__ __launch_bounds__(256) void rope_freq_kernel(wam_rope_freq_args a, int fdim, int hdim) {
  const int P = a.head_dim / 2, nf = fdim / 2, nh = hdim / 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)a.B * a.L * P) return;
  const int p = (int)(i % P);
  const int64_t bl = i / P;
  const int64_t l = bl % a.L, b = bl / a.L;
  int axis, j, d;
  if (p < nf) { axis = 0; j = p; d = fdim; }
  else if (p < nf + nh) { axis = 1; j = p - nf; d = hdim; }
  else { axis = 2; j = p - nf - nh; d = hdim; }
  const int64_t gi = b * a.grid_bstride + axis * a.grid_rstride + l * a.grid_lstride;
  double g;
  if (a.grid_dtype == WAM_I64) g = (double)static_cast<const int64_t*>(a.grid)[gi];
  else if (a.grid_dtype == WAM_F64) g = static_cast<const double*>(a.grid)[gi];
  else g = (double)static_cast<const float*>(a.grid)[gi];
  const double base = 1.0 / pow(a.theta, (double)(2 * j) / (double)d);
  const float ang = (float)(g * base);
  static_cast<float2*>(a.out)[i] = make_float2((float)cos((double)ang), (float)sin((double)ang));
}

int rope_freqs(const wam_rope_freq_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr && a->grid && a->out, "wam_rope_freqs: null args");
  WAM_REQUIRE(a->grid_dtype == WAM_I64 || a->grid_dtype == WAM_F32 || a->grid_dtype == WAM_F64,
              "wam_rope_freqs: grid dtype %d", a->grid_dtype);
  WAM_REQUIRE(a->B >= 0 && a->L >= 0 && a->head_dim >= 6 && a->head_dim % 2 == 0 && a->theta > 0,
              "wam_rope_freqs: shape");
  const int hdim = a->head_dim / 3, fdim = a->head_dim - 2 * hdim;
  WAM_REQUIRE(fdim / 2 + 2 * (hdim / 2) == a->head_dim / 2,
              "wam_rope_freqs: head_dim %d does not split into whole f/h/w pairs", a->head_dim);
  const int64_t n = (int64_t)a->B * a->L * (a->head_dim / 2);
  if (n == 0) return WAM_OK;
  hipLaunchKernelGGL(rope_freq_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, *a, fdim, hdim);
  WAM_LAUNCHED("rope_freq_kernel");
  return WAM_OK;
}

}  // namespace wam

extern "C" int wam_patchify(const wam_patchify_args* args, void* stream) {
  return wam::patchify(args, static_cast<hipStream_t>(stream));
}
extern "C" int wam_timestep_embedding(const wam_timestep_args* args, void* stream) {
  return wam::timestep_embedding(args, static_cast<hipStream_t>(stream));
}
extern "C" int wam_rows_linear(const wam_rows_linear_args* args, void* stream) {
  return wam::rows_linear(args, static_cast<hipStream_t>(stream));
}
extern "C" int wam_rope_freqs(const wam_rope_freq_args* args, void* stream) {
  return wam::rope_freqs(args, static_cast<hipStream_t>(stream));
}
