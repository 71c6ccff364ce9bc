// bf16 GEMM on CDNA4 MFMA with fused projection epilogues.
//
//   Y[m, n] = epilogue( sum_k A[m, k] * W[n, k] + b[n] )
//
// A is the activation [M, K] and W an nn.Linear weight [N, K]; both are
// K-contiguous, so both MFMA operands are read from LDS as 16-byte K-runs.
// The product is formed transposed (D = W * A^T) so that every lane of a
// 32x32 accumulator tile owns one output row m and runs of 4 consecutive
// columns n, which the epilogue stores as 8-byte vectors.
//
// Reference stages fused here: the cuBLASLt bias GEMM
// (算子研究/wam_ops/baseline/csrc/gemm.h:35-76), GELU-tanh on the FFN1 output
// (baseline/csrc/block.cu:119-129), the gated residual
// x + y * gate (block.cu:90-102, gate 2 and 5) and the plain bf16 residual
// add of cross attention (model.py:783).
#include "wam_common.h"

namespace wam {

struct LinearParams {
  const bf16* a; int64_t lda; int M, K;
  int seg_n, n_tiles_per_seg, m_tiles, n_tiles;
  const bf16* w[3]; int64_t ldw;
  const bf16* bias[3];
  void* out[3]; int64_t ldo;
  int epi;
  const void* res; int64_t ldr; int res_f32, out_f32;
  wam_modulation gate; int gate_index;
};

template <int BM_, int BN_, int BK_, int WGM_, int WGN_>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_;
  static constexpr int kWaves = WGM * WGN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int KCH = BK / 8;                 // 16-byte chunks per row
  static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int ROWS_PER_PASS = kThreads / KCH;
  static constexpr int A_LD = BM / ROWS_PER_PASS, B_LD = BN / ROWS_PER_PASS;
  static_assert(BM % ROWS_PER_PASS == 0 && BN % ROWS_PER_PASS == 0, "load split");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
};

// Byte offset of 16-byte chunk `c` of LDS row `r`; the XOR spreads the 32
// rows read by one MFMA operand fetch over distinct bank groups.
template <int KCH>
__device__ inline int lds_off(int r, int c) {
  return (r * KCH + (c ^ (r & (KCH - 1)))) * 16;
}

__device__ inline void ld_mod4(const wam_modulation& m, int D, int64_t row, int idx,
                               int d, float out[4]) {
  const int64_t b = row / m.tokens, t = row - b * m.tokens;
  const int64_t trow = b * m.temb_len + (m.temb_len == 1 ? 0 : t);
  const int64_t toff = (trow * 6 + idx) * (int64_t)D + d;
  const int64_t tab = (int64_t)idx * D + d;
  if (m.table_dtype == WAM_F32) {
    float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(m.table) + tab);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else {
    bf16x4 v = *reinterpret_cast<const bf16x4*>(static_cast<const bf16*>(m.table) + tab);
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = static_cast<float>(v[e]);
  }
  if (m.temb_dtype == WAM_F32) {
    float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(m.temb) + toff);
    out[0] += v.x; out[1] += v.y; out[2] += v.z; out[3] += v.w;
  } else {
    bf16x4 v = *reinterpret_cast<const bf16x4*>(static_cast<const bf16*>(m.temb) + toff);
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] += static_cast<float>(v[e]);
  }
}

template <class C, int EPI>
__global__ __launch_bounds__(C::kThreads, 1) void gemm_bf16_kernel(LinearParams p) {
  __shared__ __attribute__((aligned(16))) char smem[2 * C::STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WGN, wn = wave % C::WGN;

  // Tile order: XCD-contiguous ranges, then groups of 8 m-tiles swept along n
  // so that one XCD's L2 holds a few A row-panels and W column-panels.
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  constexpr int G = 8;
  const int per_group = G * p.n_tiles;
  const int group = tile / per_group, in_group = tile - group * per_group;
  const int first_m = group * G;
  const int gsize = min(p.m_tiles - first_m, G);
  const int tm = __builtin_amdgcn_readfirstlane(first_m + in_group % gsize);
  const int tn = __builtin_amdgcn_readfirstlane(in_group / gsize);
  const int seg = __builtin_amdgcn_readfirstlane(tn / p.n_tiles_per_seg);
  const int n0 = (tn - seg * p.n_tiles_per_seg) * C::BN;
  const int m0 = tm * C::BM;

  const bf16* __restrict__ A = p.a;
  const bf16* wseg = seg == 0 ? p.w[0] : (seg == 1 ? p.w[1] : p.w[2]);
  const bf16* __restrict__ W = wseg + (int64_t)n0 * p.ldw;

  // Global -> register staging through buffer resources: thread owns chunk
  // (tid % KCH) of rows tid / KCH + i * ROWS_PER_PASS.  Rows past M fall
  // outside the A resource and load as zeros.
  const int lc = tid % C::KCH, lr = tid / C::KCH;
  const uint32_t a_bytes = (uint32_t)(p.M - m0) * (uint32_t)p.lda * 2u;
  const __amdgpu_buffer_rsrc_t ra_src = make_rsrc(A + (int64_t)m0 * p.lda, a_bytes);
  const __amdgpu_buffer_rsrc_t rb_src = make_rsrc(W, (uint32_t)((int64_t)C::BN * p.ldw * 2));
  const int a_voff = (lr * (int)p.lda + lc * 8) * 2;
  const int b_voff = (lr * (int)p.ldw + lc * 8) * 2;
  const int a_step = C::ROWS_PER_PASS * (int)p.lda * 2;
  const int b_step = C::ROWS_PER_PASS * (int)p.ldw * 2;

  bf16x8 ra[C::A_LD], rb[C::B_LD];
  auto gload = [&](int kt) {
    const int ko = kt * C::BK * 2;
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) ra[i] = buf_ld16(ra_src, a_voff + i * a_step + ko);
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) rb[i] = buf_ld16(rb_src, b_voff + i * b_step + ko);
  };
  auto lstore = [&](int stage) {
    char* base = smem + stage * C::STAGE;
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i)
      st_bf16x8(base + lds_off<C::KCH>(lr + i * C::ROWS_PER_PASS, lc), ra[i]);
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i)
      st_bf16x8(base + C::A_BYTES + lds_off<C::KCH>(lr + i * C::ROWS_PER_PASS, lc), rb[i]);
  };

  f32x16 acc[C::TN][C::TM];
#pragma unroll
  for (int j = 0; j < C::TN; ++j)
#pragma unroll
    for (int i = 0; i < C::TM; ++i) acc[j][i] = f32x16{};

  const int nk = p.K / C::BK;
  gload(0);
  lstore(0);
  __syncthreads();

  const int half = lane >> 5, l32 = lane & 31;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    const char* abase = smem + cur * C::STAGE;
    const char* bbase = abase + C::A_BYTES;
#pragma unroll
    for (int ks = 0; ks < C::BK / 16; ++ks) {
      const int c = ks * 2 + half;
      bf16x8 fa[C::TM], fb[C::TN];
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
        fa[i] = ld_bf16x8(abase + lds_off<C::KCH>(wm * C::WTM + i * 32 + l32, c));
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
        fb[j] = ld_bf16x8(bbase + lds_off<C::KCH>(wn * C::WTN + j * 32 + l32, c));
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j], fa[i], acc[j][i], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue.  acc[j][i][4g + e] holds Y[m, n + e] with
  //   m = m0 + wm*WTM + i*32 + l32,  n = n0 + wn*WTN + j*32 + 8g + 4*half.
  void* out = seg == 0 ? p.out[0] : (seg == 1 ? p.out[1] : p.out[2]);
  const bf16* __restrict__ bias = seg == 0 ? p.bias[0] : (seg == 1 ? p.bias[1] : p.bias[2]);
#pragma unroll
  for (int i = 0; i < C::TM; ++i) {
    const int m = m0 + wm * C::WTM + i * 32 + l32;
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * C::WTN + j * 32 + 8 * g + 4 * half;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = acc[j][i][4 * g + e];
        if (bias) {
          bf16x4 bv = *reinterpret_cast<const bf16x4*>(bias + n);
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] += static_cast<float>(bv[e]);
        }
        if constexpr (EPI == WAM_EPI_BIAS_GELU) {
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = gelu_tanh(y[e]);
        } else if constexpr (EPI == WAM_EPI_BIAS_GATE_RES || EPI == WAM_EPI_BIAS_RES) {
          float rv[4];
          const int64_t ro = (int64_t)m * p.ldr + n;
          if (p.res_f32) {
            const float4 t = *reinterpret_cast<const float4*>(static_cast<const float*>(p.res) + ro);
            rv[0] = t.x; rv[1] = t.y; rv[2] = t.z; rv[3] = t.w;
          } else {
            const bf16x4 t = *reinterpret_cast<const bf16x4*>(static_cast<const bf16*>(p.res) + ro);
#pragma unroll
            for (int e = 0; e < 4; ++e) rv[e] = static_cast<float>(t[e]);
          }
          if constexpr (EPI == WAM_EPI_BIAS_GATE_RES) {
            float gt[4];
            ld_mod4(p.gate, p.seg_n, m, p.gate_index, n, gt);
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = rv[e] + y[e] * gt[e];
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = rv[e] + y[e];
          }
          if (p.out_f32) {
            *reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)m * p.ldo + n) =
                make_float4(y[0], y[1], y[2], y[3]);
            continue;
          }
        }
        bf16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(y[e]);
        *reinterpret_cast<bf16x4*>(static_cast<bf16*>(out) + (int64_t)m * p.ldo + n) = o;
      }
    }
  }
}

using CfgBig = GemmCfg<256, 256, 64, 2, 2>;
using CfgMid = GemmCfg<128, 128, 64, 2, 2>;

template <class C>
static int launch_gemm(LinearParams& p, hipStream_t s) {
  p.n_tiles_per_seg = p.seg_n / C::BN;
  p.m_tiles = (p.M + C::BM - 1) / C::BM;
  const int grid = p.m_tiles * p.n_tiles;
  switch (p.epi) {
    case WAM_EPI_BIAS:
      hipLaunchKernelGGL((gemm_bf16_kernel<C, WAM_EPI_BIAS>), dim3(grid), dim3(C::kThreads), 0, s, p);
      break;
    case WAM_EPI_BIAS_GELU:
      hipLaunchKernelGGL((gemm_bf16_kernel<C, WAM_EPI_BIAS_GELU>), dim3(grid), dim3(C::kThreads), 0, s, p);
      break;
    case WAM_EPI_BIAS_GATE_RES:
      hipLaunchKernelGGL((gemm_bf16_kernel<C, WAM_EPI_BIAS_GATE_RES>), dim3(grid), dim3(C::kThreads), 0, s, p);
      break;
    default:
      hipLaunchKernelGGL((gemm_bf16_kernel<C, WAM_EPI_BIAS_RES>), dim3(grid), dim3(C::kThreads), 0, s, p);
      break;
  }
  WAM_LAUNCHED("gemm_bf16_kernel");
  return WAM_OK;
}

int linear(const wam_linear_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr, "wam_linear: null args");
  WAM_REQUIRE(a->n_seg >= 1 && a->n_seg <= 3, "wam_linear: n_seg must be 1..3 (got %d)", a->n_seg);
  WAM_REQUIRE(a->M >= 1 && a->K >= 1 && a->seg_n >= 1, "wam_linear: empty shape M=%d K=%d N=%d",
              a->M, a->K, a->seg_n);
  WAM_REQUIRE(a->K % 64 == 0, "wam_linear: K=%d must be a multiple of 64", a->K);
  WAM_REQUIRE(a->seg_n % 128 == 0, "wam_linear: N=%d must be a multiple of 128", a->seg_n);
  WAM_REQUIRE(a->lda % 8 == 0 && a->ldw % 8 == 0 && a->ldo % 4 == 0,
              "wam_linear: row strides must keep 16-byte alignment");
  WAM_REQUIRE(a->a != nullptr, "wam_linear: null activation");
  WAM_REQUIRE((int64_t)a->M * a->lda * 2 < (int64_t)1 << 31 && (int64_t)a->seg_n * a->ldw * 2 < (int64_t)1 << 31,
              "wam_linear: operands above 2 GiB are not supported");
  for (int i = 0; i < a->n_seg; ++i)
    WAM_REQUIRE(a->w[i] != nullptr && a->out[i] != nullptr, "wam_linear: null weight/out %d", i);
  WAM_REQUIRE(a->epilogue >= WAM_EPI_BIAS && a->epilogue <= WAM_EPI_BIAS_RES,
              "wam_linear: unknown epilogue %d", a->epilogue);
  WAM_REQUIRE((a->res_dtype == WAM_BF16 || a->res_dtype == WAM_F32) &&
              (a->out_dtype == WAM_BF16 || a->out_dtype == WAM_F32), "wam_linear: dtype codes");
  if (a->epilogue == WAM_EPI_BIAS_GATE_RES || a->epilogue == WAM_EPI_BIAS_RES)
    WAM_REQUIRE(a->res != nullptr && a->ldr % 4 == 0, "wam_linear: residual missing");
  else
    WAM_REQUIRE(a->out_dtype == WAM_BF16, "wam_linear: fp32 output only for residual epilogues");
  if (a->epilogue == WAM_EPI_BIAS_GATE_RES) {
    WAM_REQUIRE(a->gate.table && a->gate.temb && a->gate.tokens > 0 &&
                (a->gate.temb_len == 1 || a->gate.temb_len == a->gate.tokens) &&
                a->gate_index >= 0 && a->gate_index < 6 && a->M % a->gate.tokens == 0,
                "wam_linear: gate modulation contract");
  }
  LinearParams p{};
  p.a = static_cast<const bf16*>(a->a); p.lda = a->lda; p.M = a->M; p.K = a->K;
  p.seg_n = a->seg_n; p.ldw = a->ldw; p.ldo = a->ldo; p.epi = a->epilogue;
  for (int i = 0; i < 3; ++i) {
    const int j = i < a->n_seg ? i : 0;
    p.w[i] = static_cast<const bf16*>(a->w[j]);
    p.bias[i] = static_cast<const bf16*>(a->bias[j]);
    p.out[i] = a->out[j];
  }
  p.res = a->res; p.ldr = a->ldr;
  p.res_f32 = a->res_dtype == WAM_F32;
  p.out_f32 = a->out_dtype == WAM_F32;
  p.gate = a->gate; p.gate_index = a->gate_index;
  // Big tiles when the grid still covers the chip; otherwise 128x128.
  const bool big = a->seg_n % 256 == 0 &&
                   (int64_t)((a->M + 255) / 256) * (a->seg_n / 256) * a->n_seg >= 200;
  if (big) {
    p.n_tiles = a->n_seg * (a->seg_n / CfgBig::BN);
    return launch_gemm<CfgBig>(p, s);
  }
  p.n_tiles = a->n_seg * (a->seg_n / CfgMid::BN);
  return launch_gemm<CfgMid>(p, s);
}

}  // namespace wam

extern "C" int wam_linear(const wam_linear_args* args, void* stream) {
  return wam::linear(args, static_cast<hipStream_t>(stream));
}
