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
//
// No global load of these kernels sits inside a branch: the compiler waits
// for a load in a branch before the branch ends, so a row read chunk by
// chunk under `if (chunk < D / 8)` cost one memory round trip per chunk
// (4680 x 3072 bf16 rows: 16.2 us against 12.8 us with the loads issued
// together).  Chunks are clamped to the row and masked afterwards instead.
constexpr int kLnWaves = 8;
constexpr int kLnMaxD = 4096;  // one coefficient chunk per thread: D / 8 <= 64 * kLnWaves

// Raw words of a lane's chunks of one row (chunk lane + 64 c of the row's
// D / 8 chunks of 8 values): one 16-byte word per bf16 chunk, two per fp32
// chunk.
template <int CH, bool XF32>
struct LnRow {
  u32x4 w[CH][XF32 ? 2 : 1];
};

// Issues the loads of a lane's chunks of row `row`, all in flight at once.
template <int CH, bool XF32>
__device__ inline LnRow<CH, XF32> ln_issue_row(const void* x, int64_t row, int D, int lane) {
  LnRow<CH, XF32> r;
  // a buffer resource over the row (its base in scalar registers, one offset
  // register per load); chunks past the row's end read zeros
  constexpr int EB = XF32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(static_cast<const char*>(x) + row * D * EB, (uint32_t)D * EB);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int off = (lane + c * 64) * 8 * EB;
    r.w[c][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    if constexpr (XF32)
      r.w[c][XF32 ? 1 : 0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, 0));
  }
  return r;
}

// fp32 values of chunk c of the lane; a chunk past the row's end is zeros
// (selects, not a branch).
template <int CH, bool XF32>
__device__ inline void ln_widen_chunk(const LnRow<CH, XF32>& r, int c, int nch, int lane, float v[8]) {
  const bool in = lane + c * 64 < nch;
  u32x4 a = r.w[c][0], b = r.w[c][XF32 ? 1 : 0];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = in ? a[e] : 0u;
    b[e] = in ? b[e] : 0u;
  }
  widen8(XF32, a, b, v);
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

// The sources of a workgroup's shared coefficients: add = s0 + s1, mul = s2 +
// s3 (+ 1 with modulation), with their element types.  Affine: beta, beta,
// gamma, gamma, the second of each pair not added.
struct LnSources {
  const char* p[4];
  int f32[4];
};
__device__ inline LnSources ln_sources(const wam_ln_args& a, int64_t row) {
  LnSources s;
  if (a.affine) {
    s.p[0] = s.p[1] = static_cast<const char*>(a.beta);
    s.p[2] = s.p[3] = static_cast<const char*>(a.gamma);
    s.f32[0] = s.f32[1] = s.f32[2] = s.f32[3] = a.gb_dtype == WAM_F32;
  } else {
    const wam_modulation& m = a.mod;
    const int64_t trow = temb_row(m, row);
    const int tb = m.table_dtype == WAM_F32 ? 4 : 2, eb = m.temb_dtype == WAM_F32 ? 4 : 2;
    s.p[0] = static_cast<const char*>(m.table) + (int64_t)a.shift_index * a.D * tb;
    s.p[1] = static_cast<const char*>(m.temb) + temb_off(m, trow, a.shift_index, a.D, 0) * eb;
    s.p[2] = static_cast<const char*>(m.table) + (int64_t)(a.shift_index + 1) * a.D * tb;
    s.p[3] = static_cast<const char*>(m.temb) + temb_off(m, trow, a.shift_index + 1, a.D, 0) * eb;
    s.f32[0] = s.f32[2] = tb == 4;
    s.f32[1] = s.f32[3] = eb == 4;
  }
  return s;
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
  const int64_t row = first + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int D = a.D, nch = D >> 3;
  // Do all rows of this workgroup use the same coefficients?
  const bool shared = a.affine != 0 || temb_row(a.mod, first) == temb_row(a.mod, last);
  // Load order: this thread's coefficient chunk (when shared), then its row,
  // so that the coefficients are formed while the row is in flight.
  const int fch = min((int)threadIdx.x, nch - 1);
  u32x4 cw[4][2];
  int cf32[4] = {0, 0, 0, 0};
  if (shared) {
    const LnSources src = ln_sources(a, first);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(src.p[i], (uint32_t)D * (src.f32[i] ? 4 : 2));
      const int off = fch * (src.f32[i] ? 32 : 16);
      cw[i][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
      cw[i][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + (src.f32[i] ? 16 : 0), 0, 0));
      cf32[i] = src.f32[i];
    }
  }
  // (a row past the end reads the last row and stores nothing)
  const LnRow<CH, XF32> raw = ln_issue_row<CH, XF32>(a.x, min(row, (int64_t)a.rows - 1), D, lane);
  if (shared) {
    float c[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) widen8(cf32[i] != 0, cw[i][0], cw[i][1], c[i]);
    if ((int)threadIdx.x < nch) {
      float mul[8], add[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        add[e] = a.affine ? c[0][e] : c[0][e] + c[1][e];
        mul[e] = a.affine ? c[2][e] : (c[2][e] + c[3][e]) + 1.f;
      }
      *reinterpret_cast<float4*>(s_mul + threadIdx.x * 8) = make_float4(mul[0], mul[1], mul[2], mul[3]);
      *reinterpret_cast<float4*>(s_mul + threadIdx.x * 8 + 4) = make_float4(mul[4], mul[5], mul[6], mul[7]);
      *reinterpret_cast<float4*>(s_add + threadIdx.x * 8) = make_float4(add[0], add[1], add[2], add[3]);
      *reinterpret_cast<float4*>(s_add + threadIdx.x * 8 + 4) = make_float4(add[4], add[5], add[6], add[7]);
    }
    __syncthreads();
  }
  if (row >= a.rows) return;
  // The row stays in its raw words (24 registers per lane for a bf16 row of
  // 3072) and is widened again in each pass.
  float v[8];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    ln_widen_chunk<CH, XF32>(raw, c, nch, lane, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) s += v[e];
  }
  const float mean = wave_sum(s) / D;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const bool in = lane + c * 64 < nch;
    ln_widen_chunk<CH, XF32>(raw, c, nch, lane, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = in ? v[e] - mean : 0.f;
      q += d * d;
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / D + a.eps);
  bf16* y = static_cast<bf16*>(a.y) + row * D;
  float mx = 0.f;
  bf16x8 ob[Q8 ? CH : 1];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + c * 64;
    const bool in = ch < nch;
    const int cc = in ? ch : nch - 1;
    float mul[8], add[8];
    if (shared) {
      const float4 m0 = *reinterpret_cast<const float4*>(s_mul + cc * 8);
      const float4 m1 = *reinterpret_cast<const float4*>(s_mul + cc * 8 + 4);
      const float4 a0 = *reinterpret_cast<const float4*>(s_add + cc * 8);
      const float4 a1 = *reinterpret_cast<const float4*>(s_add + cc * 8 + 4);
      mul[0] = m0.x; mul[1] = m0.y; mul[2] = m0.z; mul[3] = m0.w;
      mul[4] = m1.x; mul[5] = m1.y; mul[6] = m1.z; mul[7] = m1.w;
      add[0] = a0.x; add[1] = a0.y; add[2] = a0.z; add[3] = a0.w;
      add[4] = a1.x; add[5] = a1.y; add[6] = a1.z; add[7] = a1.w;
    } else {
      ln_coeffs(a, row, cc, mul, add);
    }
    ln_widen_chunk<CH, XF32>(raw, c, nch, lane, v);
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = static_cast<bf16>((v[e] - mean) * rstd * mul[e] + add[e]);
    if (in && (!Q8 || a.y)) st_bf16x8(y + ch * 8, o);
    if constexpr (Q8) {
      ob[c] = o;
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = in ? fmaxf(mx, fabsf(static_cast<float>(o[e]))) : mx;
    }
  }
  if constexpr (Q8) {
    const float amax = wave_max(mx);
    const float sc = amax > 0.f ? amax / 448.0f : 1.0f;
    const float inv = amax > 0.f ? 448.0f / amax : 1.0f;
    uint8_t* q8 = static_cast<uint8_t*>(a.y8) + row * D;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int ch = lane + c * 64;
      float w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = static_cast<float>(ob[c][e]) * inv;
      int lo = 0, hi = 0;
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(w[0], w[1], lo, false);
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(w[2], w[3], lo, true);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(w[4], w[5], hi, false);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(w[6], w[7], hi, true);
      if (ch < nch) *reinterpret_cast<u32x2*>(q8 + ch * 8) = u32x2{(unsigned)lo, (unsigned)hi};
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
  const int64_t job = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (job >= (int64_t)a.rows * a.n_tensors) return;
  const int tsel = (int)(job % a.n_tensors);
  const int64_t row = job / a.n_tensors;
  const int D = a.D, nch = D >> 3;
  const bf16* x = static_cast<const bf16*>(tsel ? a.x[1] : a.x[0]) + row * a.ldx;
  bf16* y = static_cast<bf16*>(tsel ? a.y[1] : a.y[0]) + row * a.ldy;
  const bf16* g = static_cast<const bf16*>(tsel ? a.gamma[1] : a.gamma[0]);
  const float eps = tsel ? a.eps[1] : a.eps[0];
  // The row's chunks and gamma's (buffer loads: chunks past the row's end
  // read zeros), all issued before any is used and none inside a branch,
  // then the rotation factors.
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)D * 2), rg = make_rsrc(g, (uint32_t)D * 2);
  u32x4 xr[CH], gr[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int off = (lane + c * 64) * 16;
    xr[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
    gr[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0));
  }
  // RoPE factors of the lane's columns: a lane's chunks lie 512 columns apart,
  // so when the head size divides 512 they sit at the same place in their
  // heads and one set of 4 pairs serves all of them.
  const float2* f = nullptr;
  if (a.freq) {
    int64_t b, t;
    split_row(row, a.tokens, b, t);
    const int64_t fb = a.freq_batch == 1 ? 0 : b;
    f = static_cast<const float2*>(a.freq) + (fb * a.tokens + t) * (a.head_dim / 2);
  }
  const bool same = 512 % a.head_dim == 0;
  float2 fz[4] = {};
  if (f && same) {
    const float2* fp = f + (((lane * 8) % a.head_dim) >> 1);
#pragma unroll
    for (int e = 0; e < 4; ++e) fz[e] = fp[e];
  }
  float v[CH][8];
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    u32x4 w = xr[c];
    const bool in = lane + c * 64 < nch;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = in ? w[e] : 0u;
    widen8(false, w, w, v[c]);
#pragma unroll
    for (int e = 0; e < 8; ++e) q += v[c][e] * v[c][e];
  }
  const float rstd = rsqrtf(wave_sum(q) / D + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = lane + c * 64;
    if (ch >= nch) continue;
    const int d0 = ch * 8;
    float gv[8];
    widen8(false, gr[c], gr[c], gv);
    float n[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) n[e] = v[c][e] * rstd * gv[e];
    auto rotate = [&](const float2 (&z)[4]) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float re = n[e], im = n[e + 1];
        n[e] = re * z[e >> 1].x - im * z[e >> 1].y;
        n[e + 1] = re * z[e >> 1].y + im * z[e >> 1].x;
      }
    };
    if (f && same) {
      rotate(fz);
    } else if (f) {
      const float2* fp = f + ((d0 % a.head_dim) >> 1);
      const float2 z[4] = {fp[0], fp[1], fp[2], fp[3]};
      rotate(z);
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
