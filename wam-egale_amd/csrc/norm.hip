// Row-reduction kernels: LayerNorm fused with AdaLN modulation, and the
// across-heads RMSNorm fused with 3D RoPE.  One wave64 owns one row; the row
// stays in registers between the statistics and the normalisation, so each
// row is read from HBM once and written once.
//
// LayerNorm+modulate follows model.py:761-763 / 786-788 (norm1/norm3:
// FP32LayerNorm without affine, then x*(1+scale)+shift, cast to bf16) and
// model.py:775-776 (norm2: FP32LayerNorm with fp32 affine).  The reference's
// native equivalents are norm/modulation_kernel/table_kernel in
// 算子研究/wam_ops/baseline/csrc/block.cu:42-89.
//
// RMSNorm+RoPE follows model.py:609-623: RMSNorm over the full D-wide row
// (all heads), times the affine weight, then the complex rotation of pair
// (2j, 2j+1) of every head by freq[t, j]; baseline/csrc/block.cu:103-118.
#include "wam_common.h"

namespace wam {

// ------------------------------------------------------------- LayerNorm
// One wave per row, 8 rows per workgroup.  The per-column vectors the rows
// multiply and add (1 + scale and shift of the modulation, or gamma and beta)
// are the same for every row of a sample: when the workgroup's rows share
// them, they are formed once into LDS (fp32) and every wave reads them there.
// Loaded per wave instead, they were 8x the bytes of the bf16 row itself.
constexpr int kLnWaves = 8;
constexpr int kLnMaxD = 4096;

template <int CH, bool XF32>
__device__ inline void ln_load_row(const void* x, int64_t row, int D, int lane, float v[CH][8]) {
  const int nch = D >> 3;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + c * 64;
    if (ch < nch) {
      ld8_f32(x, XF32 ? WAM_F32 : WAM_BF16, row * D + ch * 8, v[c]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[c][e] = 0.f;
    }
  }
}

// mul/add of 8 columns at ch*8 for token row `row`, from global memory.
__device__ inline void ln_coeffs(const wam_ln_args& a, int64_t row, int ch, float mul[8], float add[8]) {
  if (a.affine) {
    ld8_f32(a.gamma, a.gb_dtype, ch * 8, mul);
    ld8_f32(a.beta, a.gb_dtype, ch * 8, add);
  } else {
    ld_mod8(a.mod, a.D, row, a.shift_index, ch * 8, add);
    ld_mod8(a.mod, a.D, row, a.shift_index + 1, ch * 8, mul);
#pragma unroll
    for (int e = 0; e < 8; ++e) mul[e] += 1.f;
  }
}

// Q8: the bf16 rows are also written as e4m3 with one fp32 scale per row,
// scale = max |bf16 row| / 448 (1 for an all-zero row), q = e4m3(y * (448 /
// max)) rounded to nearest even (one division per row): what the row
// quantizer of the fp8 GEMM makes of the bf16 output, without reading it
// back.
template <int CH, bool XF32, bool Q8>
__global__ __launch_bounds__(64 * kLnWaves) void ln_modulate_kernel(wam_ln_args a) {
  __shared__ __attribute__((aligned(16))) float s_mul[kLnMaxD];
  __shared__ __attribute__((aligned(16))) float s_add[kLnMaxD];
  const int lane = threadIdx.x & 63;
  const int64_t first = (int64_t)blockIdx.x * kLnWaves;
  const int64_t last = min(first + kLnWaves, (int64_t)a.rows) - 1;
  const int64_t row = first + (threadIdx.x >> 6);
  const int D = a.D, nch = D >> 3;
  // Do all rows of this workgroup use the same coefficients?
  const bool shared = a.affine != 0 || temb_row(a.mod, first) == temb_row(a.mod, last);
  if (shared) {
    for (int ch = threadIdx.x; ch < nch; ch += 64 * kLnWaves) {
      float mul[8], add[8];
      ln_coeffs(a, first, ch, mul, add);
      *reinterpret_cast<float4*>(s_mul + ch * 8) = make_float4(mul[0], mul[1], mul[2], mul[3]);
      *reinterpret_cast<float4*>(s_mul + ch * 8 + 4) = make_float4(mul[4], mul[5], mul[6], mul[7]);
      *reinterpret_cast<float4*>(s_add + ch * 8) = make_float4(add[0], add[1], add[2], add[3]);
      *reinterpret_cast<float4*>(s_add + ch * 8 + 4) = make_float4(add[4], add[5], add[6], add[7]);
    }
    __syncthreads();
  }
  if (row >= a.rows) return;
  float v[CH][8];
  ln_load_row<CH, XF32>(a.x, row, D, lane, v);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) s += v[c][e];
  const float mean = wave_sum(s) / D;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (lane + c * 64 < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) { const float d = v[c][e] - mean; q += d * d; }
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / D + a.eps);
  bf16* y = static_cast<bf16*>(a.y) + row * D;
  float mx = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + c * 64;
    if (ch >= nch) continue;
    float mul[8], add[8];
    if (shared) {
      const float4 m0 = *reinterpret_cast<const float4*>(s_mul + ch * 8);
      const float4 m1 = *reinterpret_cast<const float4*>(s_mul + ch * 8 + 4);
      const float4 a0 = *reinterpret_cast<const float4*>(s_add + ch * 8);
      const float4 a1 = *reinterpret_cast<const float4*>(s_add + ch * 8 + 4);
      mul[0] = m0.x; mul[1] = m0.y; mul[2] = m0.z; mul[3] = m0.w;
      mul[4] = m1.x; mul[5] = m1.y; mul[6] = m1.z; mul[7] = m1.w;
      add[0] = a0.x; add[1] = a0.y; add[2] = a0.z; add[3] = a0.w;
      add[4] = a1.x; add[5] = a1.y; add[6] = a1.z; add[7] = a1.w;
    } else {
      ln_coeffs(a, row, ch, mul, add);
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = static_cast<bf16>((v[c][e] - mean) * rstd * mul[e] + add[e]);
    if (!Q8 || a.y) st_bf16x8(y + ch * 8, o);
    if (Q8) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[c][e] = static_cast<float>(o[e]);
        mx = fmaxf(mx, fabsf(v[c][e]));
      }
    }
  }
  if (Q8) {
    const float amax = wave_max(mx);
    const float sc = amax > 0.f ? amax / 448.0f : 1.0f;
    const float inv = amax > 0.f ? 448.0f / amax : 1.0f;
    uint8_t* q = static_cast<uint8_t*>(a.y8) + row * D;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int ch = lane + c * 64;
      if (ch >= nch) continue;
      int lo = 0, hi = 0;
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[c][0] * inv, v[c][1] * inv, lo, false);
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[c][2] * inv, v[c][3] * inv, lo, true);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[c][4] * inv, v[c][5] * inv, hi, false);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[c][6] * inv, v[c][7] * inv, hi, true);
      *reinterpret_cast<u32x2*>(q + ch * 8) = u32x2{(unsigned)lo, (unsigned)hi};
    }
    if (lane == 0) a.y8_scale[row] = sc;
  }
}

template <bool XF32, bool Q8>
static void launch_ln(const wam_ln_args* a, hipStream_t s) {
  const dim3 grid((unsigned)((a->rows + kLnWaves - 1) / kLnWaves)), block(64 * kLnWaves);
  const int ch = (a->D / 8 + 63) / 64;
  if (ch <= 1) hipLaunchKernelGGL((ln_modulate_kernel<1, XF32, Q8>), grid, block, 0, s, *a);
  else if (ch <= 2) hipLaunchKernelGGL((ln_modulate_kernel<2, XF32, Q8>), grid, block, 0, s, *a);
  else if (ch <= 3) hipLaunchKernelGGL((ln_modulate_kernel<3, XF32, Q8>), grid, block, 0, s, *a);
  else if (ch <= 6) hipLaunchKernelGGL((ln_modulate_kernel<6, XF32, Q8>), grid, block, 0, s, *a);
  else hipLaunchKernelGGL((ln_modulate_kernel<8, XF32, Q8>), grid, block, 0, s, *a);
}

int ln_modulate(const wam_ln_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr, "wam_ln_modulate: null args");
  WAM_REQUIRE(a->rows >= 0 && a->D > 0 && a->D % 8 == 0 && a->D <= 4096,
              "wam_ln_modulate: D=%d must be a multiple of 8 and <= 4096", a->D);
  WAM_REQUIRE(a->x && (a->y || a->y8), "wam_ln_modulate: null x/y");
  WAM_REQUIRE(!a->y8 || a->y8_scale, "wam_ln_modulate: y8 needs y8_scale");
  WAM_REQUIRE(a->x_dtype == WAM_BF16 || a->x_dtype == WAM_F32, "wam_ln_modulate: x dtype");
  if (a->affine) {
    WAM_REQUIRE(a->gamma && a->beta, "wam_ln_modulate: affine needs gamma and beta");
  } else {
    WAM_TRY(check_modulation(a->mod, a->rows, "wam_ln_modulate"));
    WAM_REQUIRE((a->shift_index == 0 || a->shift_index == 3) && (a->mod.temb_mods != 1 || a->shift_index == 0),
                "wam_ln_modulate: shift index %d (0 with a one-vector temb and a [2, D] table)",
                a->shift_index);
  }
  if (a->rows == 0) return WAM_OK;
  const bool q8 = a->y8 != nullptr;
  if (a->x_dtype == WAM_F32) q8 ? launch_ln<true, true>(a, s) : launch_ln<true, false>(a, s);
  else q8 ? launch_ln<false, true>(a, s) : launch_ln<false, false>(a, s);
  WAM_LAUNCHED("ln_modulate_kernel");
  return WAM_OK;
}

// ------------------------------------------------------- RMSNorm + RoPE
template <int CH>
__global__ __launch_bounds__(256) void rms_rope_kernel(wam_rms_rope_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (job >= (int64_t)a.rows * a.n_tensors) return;
  const int tsel = (int)(job % a.n_tensors);
  const int64_t row = job / a.n_tensors;
  const int D = a.D, nch = D >> 3;
  const bf16* x = static_cast<const bf16*>(tsel ? a.x[1] : a.x[0]) + row * a.ldx;
  bf16* y = static_cast<bf16*>(tsel ? a.y[1] : a.y[0]) + row * a.ldy;
  const bf16* g = static_cast<const bf16*>(tsel ? a.gamma[1] : a.gamma[0]);
  const float eps = tsel ? a.eps[1] : a.eps[0];
  float v[CH][8];
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + c * 64;
    if (ch < nch) {
      bf16x8 t = ld_bf16x8(x + ch * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) { v[c][e] = static_cast<float>(t[e]); q += v[c][e] * v[c][e]; }
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / D + eps);
  const float2* f = nullptr;
  if (a.freq) {
    int64_t b, t;
    split_row(row, a.tokens, b, t);
    const int64_t fb = a.freq_batch == 1 ? 0 : b;
    f = static_cast<const float2*>(a.freq) + (fb * a.tokens + t) * (a.head_dim / 2);
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + c * 64;
    if (ch >= nch) continue;
    const int d0 = ch * 8;
    bf16x8 gv = ld_bf16x8(g + d0);
    float n[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) n[e] = v[c][e] * rstd * static_cast<float>(gv[e]);
    if (f) {
      const int j0 = (d0 % a.head_dim) >> 1;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float2 z = f[j0 + (e >> 1)];
        const float re = n[e], im = n[e + 1];
        n[e] = re * z.x - im * z.y;
        n[e + 1] = re * z.y + im * z.x;
      }
    }
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = static_cast<bf16>(n[e]);
    st_bf16x8(y + d0, o);
  }
}

int rms_rope(const wam_rms_rope_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr, "wam_rms_rope: null args");
  WAM_REQUIRE(a->n_tensors == 1 || a->n_tensors == 2, "wam_rms_rope: n_tensors must be 1 or 2");
  WAM_REQUIRE(a->D > 0 && a->D % 8 == 0 && a->D <= 4096, "wam_rms_rope: D=%d unsupported", a->D);
  WAM_REQUIRE(a->ldx % 8 == 0 && a->ldy % 8 == 0 && a->ldx >= a->D && a->ldy >= a->D,
              "wam_rms_rope: row strides must be >= D and 16-byte aligned");
  for (int i = 0; i < a->n_tensors; ++i)
    WAM_REQUIRE(a->x[i] && a->y[i] && a->gamma[i], "wam_rms_rope: null tensor %d", i);
  if (a->freq) {
    WAM_REQUIRE(a->head_dim > 0 && a->head_dim % 8 == 0 && a->D % a->head_dim == 0,
                "wam_rms_rope: head_dim=%d must divide D and be a multiple of 8", a->head_dim);
    WAM_REQUIRE(a->tokens > 0 && a->rows % a->tokens == 0 && a->freq_batch >= 1 &&
                (a->freq_batch == 1 || a->freq_batch == a->rows / a->tokens),
                "wam_rms_rope: freq batch %d / tokens %d contract", a->freq_batch, a->tokens);
  }
  if (a->rows == 0) return WAM_OK;
  const int64_t jobs = (int64_t)a->rows * a->n_tensors;
  const dim3 grid((unsigned)((jobs + 3) / 4)), block(256);
  const int ch = (a->D / 8 + 63) / 64;
  if (ch <= 1) hipLaunchKernelGGL(rms_rope_kernel<1>, grid, block, 0, s, *a);
  else if (ch <= 2) hipLaunchKernelGGL(rms_rope_kernel<2>, grid, block, 0, s, *a);
  else if (ch <= 3) hipLaunchKernelGGL(rms_rope_kernel<3>, grid, block, 0, s, *a);
  else if (ch <= 6) hipLaunchKernelGGL(rms_rope_kernel<6>, grid, block, 0, s, *a);
  else hipLaunchKernelGGL(rms_rope_kernel<8>, grid, block, 0, s, *a);
  WAM_LAUNCHED("rms_rope_kernel");
  return WAM_OK;
}

}  // namespace wam

extern "C" int wam_ln_modulate(const wam_ln_args* args, void* stream) {
  return wam::ln_modulate(args, static_cast<hipStream_t>(stream));
}
extern "C" int wam_rms_rope(const wam_rms_rope_args* args, void* stream) {
  return wam::rms_rope(args, static_cast<hipStream_t>(stream));
}
