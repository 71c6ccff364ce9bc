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
#include <string.h>
#include <type_traits>
#include "wam_common.h"

namespace wam {

struct LinearParams {
  const bf16* a; int64_t lda; int M, K;
  int seg_n, n_tiles_per_seg, m_tiles, n_tiles, n_seg_count;
  const void* w[3]; int64_t ldw;      // ldw in elements of the weight dtype
  const bf16* bias[3];
  void* out[3]; int64_t ldo;
  int epi;
  const void* res; int64_t ldr; int res_f32, out_f32;
  wam_modulation gate; int gate_index;
  const float* wscale[3];  // per-output-column fp32 scales of fp8 weights (else unused)
  int mod_d;   // row length of the modulation table (the full output width)
  int n_off;   // column of this launch's first output column in that table
  // Split-K launches (one segment): k range kp of k_split writes its raw fp32
  // sums to part[kp][m][n] (row stride seg_n); gemm_splitk_reduce_kernel adds
  // the ranges in order and applies the epilogue.
  int k_split;
  float* part;
  // q/k-norm epilogue (kEpiBiasNorm): per segment, the sums of squares of
  // the bf16 outputs per 256-column group (row stride ssq_ld), the gamma the
  // outputs are multiplied by, and the RoPE table (nfreq, or none).
  float* ssq[3]; const bf16* ngamma[3];
  const float2* nfreq; int nfreq_batch, ntokens, nhd, ssq_ld;
  // fp8 e4m3 activations (the fp8 MFMA mode): A is [M, K] bytes with one
  // fp32 scale per row
  const float* ascale;
  // MX activations: A is e4m3 [M, K] with one e8m0 exponent per row and 32
  // consecutive k (abscale, row stride K / 32 bytes); MX output: out[0] is
  // e4m3 [M, seg_n] (row stride ldo bytes) with one e8m0 exponent per row and
  // 32 consecutive columns (oscale, row stride seg_n / 32 bytes).
  const uint8_t* abscale;
  uint8_t* oscale;
};

constexpr int kEpiPartial = 100;   // kernel epilogue of a split-K range: raw fp32 sums
constexpr int kEpiBiasNorm = 101;  // bias, then the q/k-norm epilogue (four-wave kernel; eight-wave without RoPE)

template <int BM_, int BN_, int BK_, int WGM_, int WGN_, int STAGES_, int BLOCKS_ = 1, int SCHED_ = 0,
          int WB_ = 2, int SPLIT_ = 1>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_, STAGES = STAGES_;
  static constexpr int WB = WB_;          // bytes per weight element: 2 (bf16) or 1 (fp8 e4m3)
  static constexpr bool kW4 = false;
  // SPLIT > 1: a stage's loads are issued in SPLIT parts, one at the barrier
  // and the others before the MFMAs of the next k-step's first sub-steps, so
  // the load issue does not stall the waves all at once.  With two stages
  // the later parts have most of a k-step to land before the next barrier.
  static constexpr int SPLIT = SPLIT_;
  static constexpr int BLOCKS = BLOCKS_;  // resident workgroups per CU
  static constexpr int EPI_ROWS = 1 << 30;  // cap on the epilogue's fp32 rows per stage buffer
  static constexpr int SCHED = SCHED_;    // 2: all DS reads of the next k-step, then this
                                          // step's MFMAs; 0: the compiler's order
  static constexpr int kWaves = WGM * WGN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int KCH = BK / 8;                     // 16-byte chunks per LDS row
  static constexpr int ROW_BYTES = BK * 2;
  static constexpr int W_ROW_BYTES = BK * WB;
  static constexpr int KCH_W = W_ROW_BYTES / 16;         // 16-byte chunks per LDS weight row
  static constexpr int A_BYTES = BM * ROW_BYTES, B_BYTES = BN * W_ROW_BYTES;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int ROWS_PER_LOAD = 1024 / ROW_BYTES;    // A rows per wave-wide 16 B/lane load
  static constexpr int W_ROWS_PER_LOAD = 1024 / W_ROW_BYTES;
  static constexpr int A_LOADS = BM / ROWS_PER_LOAD, W_LOADS = BN / W_ROWS_PER_LOAD;
  static constexpr int LOADS = A_LOADS + W_LOADS;          // per stage, whole workgroup
  static constexpr int LOADS_PER_WAVE = LOADS / kWaves;
  static_assert(KCH == 8 || KCH == 4, "BK must be 64 or 32");
  static_assert(WB == 2 || (WB == 1 && BK == 64), "fp8 weights use 64-deep k-steps");
  static_assert(A_LOADS % kWaves == 0 && W_LOADS % kWaves == 0 && kWaves % 2 == 0,
                "loads per wave: A then W");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  static_assert(STAGES >= 2 && BLOCKS * (STAGES * STAGE + (5 - STAGES) * 1024) <= 160 * 1024, "LDS budget");
  static_assert(SPLIT == 1 || (STAGES >= 2 && LOADS_PER_WAVE % SPLIT == 0 && SPLIT - 1 <= BK / 16 - 1),
                "split load issue");
};

// Byte offset of logical 16-byte chunk `c` of LDS row `r`.  The gfx950 LDS
// has 64 banks of 4 bytes (256 bytes per cycle), and a ds_read_b128 serves 16
// lanes per cycle.  An MFMA operand fetch reads 32 consecutive rows at one
// logical chunk, so any 16 consecutive rows must land on 16 distinct 16-byte
// bank slots: rows sharing a 256-byte bank line (2 rows of 128 bytes, 4 of 64)
// are separated by the XOR of the row's index within its bank-line group.
template <int KCH>
__device__ inline int lds_off(int r, int c) {
  if constexpr (KCH == 8) return r * 128 + ((c ^ ((r >> 1) & 7)) << 4);
  else return r * 64 + ((c ^ ((r >> 2) & 3)) << 4);
}

__device__ inline void ld_mod4(const wam_modulation m, int D, int64_t row, int idx,
                               int d, float out[4]) {
  const int64_t toff = temb_off(m, temb_row(m, row), idx, D, d);
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

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Issue the direct-to-LDS loads of k-tile `kt` into LDS stage `stage`.  Load
// g (0 <= g < LOADS) fills the 1 KB LDS block g, i.e. rows ROWS_PER_LOAD*g ..
// +ROWS_PER_LOAD of the stacked [A rows; W rows] tile.  Wave w issues loads
// g = w + i * kWaves; whether a load reads A or W depends on i only, so the
// unrolled sequence has no branches.  a_lane / b_lane already include the
// swizzle term of the wave's block parity (the wave count is even).
template <class C, int NPARTS = 1>
__device__ __forceinline__ void issue_stage(char* base, i32x4 ra, i32x4 rb, int wave, int a_lane,
                                            int b_lane, int a_pitch, int b_pitch, int kt, int part = 0) {
  const int ko = kt * C::BK * 2, ko_w = kt * C::BK * C::WB;
  constexpr int A_ITERS = C::A_LOADS / C::kWaves;
  constexpr int PER = C::LOADS_PER_WAVE / NPARTS;
#pragma unroll
  for (int ip = 0; ip < PER; ++ip) {
    const int i = part * PER + ip;  // part is a constant wherever the caller is unrolled
    const int g = wave + i * C::kWaves;
    char* dst = base + g * 1024;
    if (i < A_ITERS)
      asm_ld16_lds(ra, dst, a_lane + g * C::ROWS_PER_LOAD * a_pitch + ko);
    else
      asm_ld16_lds(rb, dst, b_lane + (g - C::A_LOADS) * C::W_ROWS_PER_LOAD * b_pitch + ko_w);
  }
}

// MFMA operand fragments of one 16-deep k-step (logical chunk c of each row).
template <class C>
__device__ __forceinline__ void fetch_frags(const char* abase, const char* bbase, int wm, int wn,
                                            int l32, int c, bf16x8 (&fa)[C::TM], bf16x8 (&fb)[C::TN]) {
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
    fa[i] = ld_bf16x8(abase + lds_off<C::KCH>(wm * C::WTM + i * 32 + l32, c));
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    const int r = wn * C::WTN + j * 32 + l32;
    if constexpr (C::WB == 2) {
      fb[j] = ld_bf16x8(bbase + lds_off<C::KCH>(r, c));
    } else {
      // 8 fp8 weights (8 bytes: half c & 1 of 16-byte chunk c >> 1 of a
      // 64-byte row), widened exactly to bf16; the per-column scale is
      // applied to the accumulator in the epilogue.
      const u32x2 q = *reinterpret_cast<const u32x2*>(bbase + lds_off<4>(r, c >> 1) + (c & 1) * 8);
      fb[j] = fp8x8_to_bf16x8(q);
    }
  }
}

// The epilogue of 4 consecutive outputs (m, n..n+3) from their fp32 sums v:
// fp8 column scale, bias, then GELU-tanh, or the (gated) residual with an
// fp32 or bf16 output.  The caller loads the residual rv (fp32) of the
// residual epilogues.  With gate_held the gate of these columns is
// gate_pre (every row the caller handles reads the same modulation row);
// otherwise it is read for row m.
template <int EPI, int WB>
__device__ __forceinline__ void epi_apply(const LinearParams& p, void* out, int m, int n, const f32x4 v,
                                          const float (&bv)[4], const float (&wsc)[4],
                                          const float (&gate_pre)[4], bool gate_held, const float (&rv)[4]) {
  float y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = WB == 1 ? v[e] * wsc[e] + bv[e] : v[e] + bv[e];
  if constexpr (EPI == WAM_EPI_BIAS_GELU) {
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = gelu_tanh(y[e]);
  } else if constexpr (EPI == WAM_EPI_BIAS_GATE_RES || EPI == WAM_EPI_BIAS_RES) {
    if constexpr (EPI == WAM_EPI_BIAS_GATE_RES) {
      float gt[4];
      if (gate_held) {
#pragma unroll
        for (int e = 0; e < 4; ++e) gt[e] = gate_pre[e];
      } else {
        ld_mod4(p.gate, p.mod_d, m, p.gate_index, n + p.n_off, gt);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = rv[e] + y[e] * gt[e];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = rv[e] + y[e];
    }
    if (p.out_f32) {
      *reinterpret_cast<float4*>(static_cast<float*>(out) + (int64_t)m * p.ldo + n) =
          make_float4(y[0], y[1], y[2], y[3]);
      return;
    }
  }
  bf16x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(y[e]);
  *reinterpret_cast<bf16x4*>(static_cast<bf16*>(out) + (int64_t)m * p.ldo + n) = o;
}

template <class C, int EPI, int RF32 = 0>
__global__ __launch_bounds__(C::kThreads, C::BLOCKS) void gemm_bf16_kernel(LinearParams p) {
  // One __shared__ object per pipeline stage: the compiler tracks the
  // direct-to-LDS loads per object, so reading one stage while another is
  // being filled needs no wait on the outstanding loads.
  __shared__ __attribute__((aligned(1024))) char lds0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char lds1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) char lds2[C::STAGES > 2 ? C::STAGE : 16];
  __shared__ __attribute__((aligned(1024))) char lds3[C::STAGES > 3 ? C::STAGE : 16];
  __shared__ __attribute__((aligned(1024))) char lds4[C::STAGES > 4 ? C::STAGE : 16];
  static_assert(C::STAGES <= 5, "at most five stage objects");
#define WAM_GEMM_BUF(st) ((st) == 0 ? lds0 : (st) == 1 ? lds1 : (st) == 2 ? lds2 : (st) == 3 ? lds3 : lds4)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / C::WGN, wn = wave % C::WGN;

  // Tile order: XCD-contiguous ranges, then groups of 8 m-tiles swept along n
  // so that one XCD's L2 holds a few A row-panels and W column-panels.
  int tile = xcd_remap(blockIdx.x, gridDim.x);
  int kp = 0;  // k range of a split-K launch: pieces are (k range, tile), tiles fastest
  if constexpr (EPI == kEpiPartial) {
    const int tiles = p.m_tiles * p.n_tiles;
    kp = __builtin_amdgcn_readfirstlane(tile / tiles);
    tile -= kp * tiles;
  }
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

  const bf16* A = p.a;
  const char* wseg = static_cast<const char*>(seg == 0 ? p.w[0] : (seg == 1 ? p.w[1] : p.w[2]));
  const char* W = wseg + (int64_t)n0 * p.ldw * C::WB;

  // Direct-to-LDS staging.  Load g (0 <= g < LOADS) of a stage fills the
  // 1 KB LDS block g, i.e. rows ROWS_PER_LOAD*g .. +ROWS_PER_LOAD of the
  // stacked [A rows; W rows] tile; lane L lands at byte 16 L of that block,
  // which is physical chunk L % KCH of row L / KCH, so it fetches the logical
  // chunk that the swizzle maps there.  Rows of A past M fall outside the
  // buffer resource and load as zeros.
  // A split-K range starts kb k-tiles in: both resources start there, and
  // their byte bounds shrink by the same amount.
  int nk = p.K / C::BK, kb = 0;
  if constexpr (EPI == kEpiPartial) {
    kb = (int)((int64_t)kp * nk / p.k_split);
    nk = (int)((int64_t)(kp + 1) * nk / p.k_split) - kb;
  }
  const uint32_t ka = (uint32_t)kb * C::BK * 2u, kw = (uint32_t)kb * C::BK * C::WB;
  const uint32_t a_bytes = (uint32_t)(p.M - m0) * (uint32_t)p.lda * 2u;
  const i32x4 ra = make_rsrc4(A + (int64_t)m0 * p.lda + (int64_t)kb * C::BK, a_bytes - ka);
  // Weight rows past N (a partial last n-tile) load as zeros.
  const int n_rows = min(C::BN, p.seg_n - n0);
  const i32x4 rb = make_rsrc4(W + kw, (uint32_t)((int64_t)n_rows * p.ldw * C::WB) - kw);
  const int lrow = lane / C::KCH, pchunk = lane % C::KCH;
  // The swizzle term of row r = ROWS_PER_LOAD * g + lrow: for 128-byte rows
  // (8 rows per block) it depends on the parity of g, for 64-byte rows (16
  // rows per block) on lrow only.  With an even wave count every block a wave
  // loads has the wave's parity.
  const int r1 = C::ROWS_PER_LOAD + lrow;
  const int chunk0 = C::KCH == 8 ? (pchunk ^ ((lrow >> 1) & 7)) : (pchunk ^ ((lrow >> 2) & 3));
  const int chunk1 = C::KCH == 8 ? (pchunk ^ ((r1 >> 1) & 7)) : (pchunk ^ ((r1 >> 2) & 3));
  const int lchunk = (wave & 1) ? chunk1 : chunk0;
  const int a_lane = (lrow * (int)p.lda + lchunk * 8) * 2;
  const int a_pitch = (int)p.lda * 2, b_pitch = (int)p.ldw * C::WB;
  int b_lane;
  if constexpr (C::WB == 2) {
    b_lane = lrow * b_pitch + lchunk * 16;
  } else {
    // 64-byte weight rows, 16 per block: the swizzle term (r >> 2) & 3 of row
    // r = 16 g + lane / 4 depends on the lane only.
    const int wrow = lane >> 2, wch = (lane & 3) ^ ((wrow >> 2) & 3);
    b_lane = wrow * b_pitch + wch * 16;
  }

  // The epilogue's per-column operands are loaded before the k loop, so that
  // their latency is not at the end of the tile.
  constexpr int RPO_FIT = (C::STAGE / (C::BN * 4)) / 32 * 32;
  constexpr int RPO = RPO_FIT < C::EPI_ROWS ? RPO_FIT : C::EPI_ROWS;  // fp32 rows per buffer
  static_assert(RPO >= 32, "a stage buffer must hold 32 fp32 rows of the tile");
  constexpr int ROUND = RPO * C::STAGES;                 // rows staged per round
  constexpr int NROUNDS = (C::BM + ROUND - 1) / ROUND;
  constexpr int QPR = C::BN / 4;                         // 16-byte chunks per fp32 row
  constexpr int RPI = 64 / QPR;                          // rows per wave-wide access
  static_assert(QPR == 64 || QPR == 32, "BN must be 256 or 128");
  constexpr int ROW_B = C::BN * 4;
  void* out = seg == 0 ? p.out[0] : (seg == 1 ? p.out[1] : p.out[2]);
  const bf16* __restrict__ bias = seg == 0 ? p.bias[0] : (seg == 1 ? p.bias[1] : p.bias[2]);
  const int q = lane % QPR;  // this lane's chunk of a row in the read phase
  const int n = n0 + 4 * q;
  const bool n_ok = n < p.seg_n;  // N is a multiple of 4: a lane's 4 columns are all in or all out
  float bv[4] = {0.f, 0.f, 0.f, 0.f};
  if (bias && n_ok) {
    const bf16x4 t = *reinterpret_cast<const bf16x4*>(bias + n);
#pragma unroll
    for (int e = 0; e < 4; ++e) bv[e] = static_cast<float>(t[e]);
  }
  float wsc[4] = {1.f, 1.f, 1.f, 1.f};
  if constexpr (C::WB == 1) {
    const float* ws = seg == 0 ? p.wscale[0] : (seg == 1 ? p.wscale[1] : p.wscale[2]);
    const float4 t = n_ok ? *reinterpret_cast<const float4*>(ws + n) : make_float4(1.f, 1.f, 1.f, 1.f);
    wsc[0] = t.x; wsc[1] = t.y; wsc[2] = t.z; wsc[3] = t.w;
  }
  f32x16 acc[C::TN][C::TM];
#pragma unroll
  for (int j = 0; j < C::TN; ++j)
#pragma unroll
    for (int i = 0; i < C::TM; ++i) acc[j][i] = f32x16{};

  const int half = lane >> 5, l32 = lane & 31;
  constexpr int KSTEPS = C::BK / 16;
  constexpr int MF = C::TM * C::TN, R = C::TM + C::TN;
  static_assert(KSTEPS % 2 == 0, "fragment double buffer alternates per k-step");

  // Prologue: all STAGES buffers in flight, wait for the first.
#pragma unroll
  for (int st = 0; st < C::STAGES; ++st)
    if (st < nk) issue_stage<C>(WAM_GEMM_BUF(st), ra, rb, wave, a_lane, b_lane, a_pitch, b_pitch, st);
  if (nk >= C::STAGES) wait_vmcnt<(C::STAGES - 1) * C::LOADS_PER_WAVE>();
  else wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();

  bf16x8 fa[2][C::TM], fb[2][C::TN];
  fetch_frags<C>(lds0, lds0 + C::A_BYTES, wm, wn, l32, half, fa[0], fb[0]);

  // The k loop is unrolled by STAGES so that every buffer reference is to a
  // fixed __shared__ object.
  for (int kt0 = 0; kt0 < nk; kt0 += C::STAGES) {
#pragma unroll
    for (int st = 0; st < C::STAGES; ++st) {
      const int kt = kt0 + st;
      if (kt >= nk) break;
      const char* abase = WAM_GEMM_BUF(st);
      const char* bbase = abase + C::A_BYTES;
      // k-steps 0 .. KSTEPS-2: read the next step's fragments, then this
      // step's MFMAs.
#pragma unroll
      for (int ks = 0; ks + 1 < KSTEPS; ++ks) {
        if constexpr (C::SPLIT > 1) {
          // the remaining parts of the loads issued at the previous barrier
          // (tile kt - 1 + STAGES into the previous stage's buffer)
          if (ks + 1 < C::SPLIT && kt >= 1 && kt - 1 + C::STAGES < nk)
            issue_stage<C, C::SPLIT>(WAM_GEMM_BUF((st + C::STAGES - 1) % C::STAGES), ra, rb, wave, a_lane,
                                     b_lane, a_pitch, b_pitch, kt - 1 + C::STAGES, ks + 1);
        }
        fetch_frags<C>(abase, bbase, wm, wn, l32, (ks + 1) * 2 + half, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
#pragma unroll
          for (int i = 0; i < C::TM; ++i)
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[ks & 1][j], fa[ks & 1][i], acc[j][i],
                                                                0, 0, 0);
        if constexpr (C::SCHED == 2) {
          __builtin_amdgcn_sched_group_barrier(0x100, R, 0);   // all DS reads of step ks+1
          __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);  // then the MFMAs of step ks
        }
      }
      // Every LDS read of this stage is done (the last step's fragments are
      // in registers), so the barrier goes here: the next stage's data is
      // then visible, this stage's buffer can be refilled, and the next
      // stage's first reads overlap this stage's last MFMAs.
      if (kt + 1 < nk) {
        if (kt + C::STAGES - 1 < nk) wait_vmcnt<(C::STAGES - 2) * C::LOADS_PER_WAVE>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (kt + C::STAGES < nk)
          issue_stage<C, C::SPLIT>(WAM_GEMM_BUF(st), ra, rb, wave, a_lane, b_lane, a_pitch, b_pitch,
                                   kt + C::STAGES, 0);
        const char* na = WAM_GEMM_BUF((st + 1) % C::STAGES);
        fetch_frags<C>(na, na + C::A_BYTES, wm, wn, l32, half, fa[0], fb[0]);
      }
      constexpr int LAST = (KSTEPS - 1) & 1;
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[LAST][j], fa[LAST][i], acc[j][i], 0, 0, 0);
    }
  }

  // Epilogue, staged through LDS.  The accumulators are in MFMA layout (a
  // lane holds one row and 4 columns per fragment), which would make every
  // global store and residual read touch 32 rows at 16 bytes each.  Instead
  // the fp32 tile goes to the (now idle) stage buffers, RPO rows per buffer,
  // and is read back row-wise: a wave covers whole rows, so bias, modulation,
  // residual and output accesses are contiguous and fill whole cache lines.
  // Rows are 16-byte chunks XOR-swizzled by (row & 15), which keeps both the
  // column-wise writes and the row-wise reads free of bank conflicts.
  // The residual of a round's rows is loaded into registers before the round
  // is staged through LDS (16 bytes per row chunk: 4 fp32, or 4 bf16 in the
  // low half), so the whole round's loads are in flight together.
  constexpr bool RES = EPI == WAM_EPI_BIAS_GATE_RES || EPI == WAM_EPI_BIAS_RES;
  constexpr int ITERS = ROUND / (C::kWaves * RPI);
  constexpr int RB = RF32 ? 4 : 2;  // residual bytes per element
  typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
  typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
  // The residual through a buffer resource over the tile's rows from column
  // n0 (rows past M read zeros), so the prefetch has no branch: a load inside
  // a branch, or a dtype chosen at run time, left the compiler waiting for
  // all memory operations (the previous rows' stores included) before every
  // row of the epilogue.
  const int rows_left = min(p.M - m0, C::BM);
  const __amdgpu_buffer_rsrc_t rres =
      RES ? make_rsrc(static_cast<const char*>(p.res) + ((int64_t)m0 * p.ldr + n0) * RB,
                      (uint32_t)((rows_left - 1) * (uint32_t)p.ldr + (uint32_t)min(C::BN, p.seg_n - n0)) * RB)
          : make_rsrc(p.a, 0u);
  std::conditional_t<RF32 != 0, u32x4v, u32x2v> rraw[RES ? ITERS : 1];
  auto res_prefetch = [&](int rd) {
    if constexpr (RES) {
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        const int row = rd * ROUND + (it * C::kWaves + wave) * RPI + lane / QPR;
        const int off = (row * (int)p.ldr + 4 * q) * RB;
        if constexpr (RF32)
          rraw[it] = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rres, off, 0, 0));
        else
          rraw[it] = __builtin_bit_cast(u32x2v, __builtin_amdgcn_raw_buffer_load_b64(rres, off, 0, 0));
      }
    }
  };
  res_prefetch(0);
  // The gate of this lane's 4 columns, loaded once per tile (after the k
  // loop, which has no registers to spare for it) when the tile's rows read
  // at most two consecutive modulation rows (one or two samples, or latent
  // frames): gate for the rows before gate_split, gate2 from there on.  Rows
  // that read more (one modulation row per token) load theirs per row.
  float gate[4] = {0.f, 0.f, 0.f, 0.f}, gate2[4] = {0.f, 0.f, 0.f, 0.f};
  bool gate_held = false;
  int gate_split = 0;  // first tile row served by the second modulation row
  if constexpr (EPI == WAM_EPI_BIAS_GATE_RES) {
    const int m_last = min(m0 + C::BM, p.M) - 1;
    const int64_t tr0 = temb_row(p.gate, m0), tr1 = temb_row(p.gate, m_last);
    gate_held = tr1 - tr0 <= 1;
    gate_split = (int)(temb_first_row(p.gate, tr1) - m0);
    // columns clamped into the row: both loads unconditional, in flight with
    // the residual's
    const int nc = min(n, p.seg_n - 4) + p.n_off;
    ld_mod4(p.gate, p.mod_d, m0, p.gate_index, nc, gate);
    ld_mod4(p.gate, p.mod_d, m_last, p.gate_index, nc, gate2);
  }
  // q-norm epilogue (no RoPE here): the gamma of the lane's 4 columns and the
  // segment's sums-of-squares array.  With 256-column tiles a wave holds one
  // whole row of the tile per pass, so a row's sum is one wave reduction.
  constexpr bool NORM = EPI == kEpiBiasNorm;
  static_assert(!NORM || C::BN == 256, "the q-norm epilogue needs 256-column tiles");
  float gm[4] = {1.f, 1.f, 1.f, 1.f};
  float* nssq = nullptr;
  if constexpr (NORM) {
    nssq = seg == 0 ? p.ssq[0] : (seg == 1 ? p.ssq[1] : p.ssq[2]);
    const bf16* g = seg == 0 ? p.ngamma[0] : (seg == 1 ? p.ngamma[1] : p.ngamma[2]);
    const bf16x4 tg = *reinterpret_cast<const bf16x4*>(g + min(n, p.seg_n - 4));
#pragma unroll
    for (int e = 0; e < 4; ++e) gm[e] = static_cast<float>(tg[e]);
  }
  // Every wave is done reading the last stage (its fragments are in
  // registers and consumed); only LDS operations are waited for, so the
  // residual loads stay in flight.
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int rd = 0; rd < NROUNDS; ++rd) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      const int r = wm * C::WTM + i * 32;  // first tile row of this fragment row (uniform)
      if (r / ROUND != rd) continue;
      const int obj = (r % ROUND) / RPO;
      char* buf = WAM_GEMM_BUF(obj);
      const int lr = r % RPO + l32;
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int qq = (wn * C::WTN + j * 32 + 8 * g) / 4 + half;
          const f32x4 v = {acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3]};
          *reinterpret_cast<f32x4*>(buf + lr * ROW_B + ((qq ^ (lr & 15)) << 4)) = v;
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS writes are done
    __builtin_amdgcn_s_barrier();
    // the round's residual rows have landed (one wait per round, which also
    // drains the previous round's stores)
    if constexpr (RES) wait_vmcnt<0>();
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int rr = (it * C::kWaves + wave) * RPI + lane / QPR;  // row within the round
      const int row = rd * ROUND + rr;
      const int m = m0 + row;
      if constexpr (NORM) {
        // y = bf16(acc + b) as the bias epilogue rounds it; the row's sum of
        // y^2 over the tile's 256 columns (every lane of the wave takes part
        // in the reduction); the stored value bf16(y * gamma), one rounding.
        const bool row_ok = row < C::BM && m < p.M;
        const int lrr = rr % RPO;
        const f32x4 v = *reinterpret_cast<const f32x4*>(WAM_GEMM_BUF(rr / RPO) + lrr * ROW_B + ((q ^ (lrr & 15)) << 4));
        bf16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(v[e] + bv[e]);
        const bf16x2 o01 = {o[0], o[1]}, o23 = {o[2], o[3]};
        const float ss = __builtin_amdgcn_fdot2_f32_bf16(o23, o23, __builtin_amdgcn_fdot2_f32_bf16(o01, o01, 0.f, false),
                                                         false);
        const float tot = wave_sum(row_ok && n_ok ? ss : 0.f);
        if (row_ok && lane == 0) nssq[(int64_t)m * p.ssq_ld + (n0 >> 8)] = tot;
        if (row_ok && n_ok) {
          bf16x4 t;
#pragma unroll
          for (int e = 0; e < 4; ++e) t[e] = static_cast<bf16>(static_cast<float>(o[e]) * gm[e]);
          *reinterpret_cast<bf16x4*>(static_cast<bf16*>(out) + (int64_t)m * p.ldo + n) = t;
        }
        continue;
      }
      if (row >= C::BM || m >= p.M || !n_ok) continue;
      const int obj = rr / RPO, lr = rr % RPO;
      const char* buf = WAM_GEMM_BUF(obj);
      const f32x4 v = *reinterpret_cast<const f32x4*>(buf + lr * ROW_B + ((q ^ (lr & 15)) << 4));
      if constexpr (EPI == kEpiPartial) {
        *reinterpret_cast<f32x4*>(p.part + ((int64_t)kp * p.M + m) * p.seg_n + n) = v;
      } else {
        float rv[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (RES) {
          const auto t = rraw[it];
          if constexpr (RF32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) rv[e] = __uint_as_float(t[e]);  // by value: a vector element has no address
          } else {
            rv[0] = __uint_as_float(t[0] << 16);
            rv[1] = __uint_as_float(t[0] & 0xffff0000u);
            rv[2] = __uint_as_float(t[1] << 16);
            rv[3] = __uint_as_float(t[1] & 0xffff0000u);
          }
        }
        float gsel[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) gsel[e] = row >= gate_split ? gate2[e] : gate[e];
        epi_apply<EPI, C::WB>(p, out, m, n, v, bv, wsc, gsel, gate_held, rv);
      }
    }
    if (rd + 1 < NROUNDS) {
      res_prefetch(rd + 1);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // this round's LDS reads are done
      __builtin_amdgcn_s_barrier();
    }
  }
#undef WAM_GEMM_BUF
}

// ---------------------------------------------------------------------------
// 256x256x64 tiles on four waves, one per SIMD.  Each wave owns a 128x128
// quarter of the tile (16 accumulators of 32x32, held in AGPRs), so a k-step
// reads 128 KB of MFMA operands from LDS; eight 128x64 waves read 192 KB.
// Global loads are staged through VGPRs in two register sets (the data of
// k-step d lives in set d % 2): during k-step t, set (t+1) % 2 is written to
// the free LDS stage and then reloaded with k-step t+3, so every load has
// about two k-steps to land.  The loads and the LDS writes are spread evenly
// over the k-step, about one per three MFMAs: issued in bursts, they fill the
// texture unit's address and command queues, and a wave that cannot issue a
// load cannot issue the MFMAs behind it either (4680x3072x14336:
// SQ_VMEM_TA_ADDR_FIFO_FULL 1.7e7 -> 4.5e5 cycles, k loop 369 -> 337 us).
struct CfgW4 {
  static constexpr int BM = 256, BN = 256, BK = 64, WB = 2, kThreads = 256;
  static constexpr bool kW4 = true;
};
// The same kernel on 224 x 256 tiles, the four waves side by side along n
// (224 x 64 each, 7 x 2 MFMA blocks): 4680 rows are 21 such tiles (0.5% of
// padding against 3.9% for 19 x 256), and a 3072-column GEMM then fills 252
// of the 256 CUs in one round of 7/8 of a 256-row tile's work.
struct CfgW4t224 {
  static constexpr int BM = 224, BN = 256, BK = 64, WB = 2, kThreads = 256;
  static constexpr bool kW4 = true;
};
// The same two tilings with fp8 e4m3 weights (widened to bf16 on the way
// into LDS; per-column scales in the epilogue).
struct CfgW4f8 {
  static constexpr int BM = 256, BN = 256, BK = 64, WB = 1, kThreads = 256;
  static constexpr bool kW4 = true;
};
struct CfgW4t224f8 {
  static constexpr int BM = 224, BN = 256, BK = 64, WB = 1, kThreads = 256;
  static constexpr bool kW4 = true;
};

// The NM MFMAs of one 16-deep sub-step with the NR fragment reads of the
// next sub-step, W LDS writes and V global loads spread evenly between them
// (NM = 16, NR = 8: one read after every second MFMA).
// (Counts above NM put two of a kind after some MFMAs.)
template <int MASK>
__device__ __forceinline__ void sched_n(int c) {
  if (c == 1) __builtin_amdgcn_sched_group_barrier(MASK, 1, 0);
  else if (c == 2) __builtin_amdgcn_sched_group_barrier(MASK, 2, 0);
  else if (c >= 3) __builtin_amdgcn_sched_group_barrier(MASK, 3, 0);
}
template <int W, int V, int NM, int NR>
__device__ __forceinline__ void w4_sched() {
  static_assert(NR <= 3 * NM && W <= 3 * NM && V <= 3 * NM, "at most 3 of a kind per MFMA");
#pragma unroll
  for (int q = 0; q < NM; ++q) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
    sched_n<0x100>(((q + 1) * NR) / NM - (q * NR) / NM);    // DS read
    sched_n<0x200>(((q + 1) * W) / NM - (q * W) / NM);      // DS write
    sched_n<0x020>(((q + 1) * V) / NM - (q * V) / NM);      // VMEM read
  }
}

// RF32 / OF32: the residual / output is fp32 (else bf16; OF32 = 2: e4m3 with
// e8m0 exponents per 32 columns, the MX output); compile-time so
// that the epilogue's loads and stores are branch-free.  TM: tile rows, 256
// (waves 2 x 2, 128 x 128 each) or 224 (waves 1 x 4, 224 x 64 each).
// WB: bytes per weight element, 2 (bf16) or 1 (fp8 e4m3 with per-column
// fp32 scales).  fp8 weight rows are 64 bytes per k-step: a thread loads 16
// of them (a quarter row) and widens them exactly to bf16 in registers as it
// writes the stage, so the LDS layout and the MFMA loop are those of bf16;
// the scale multiplies the fp32 sums in the epilogue.
// F8MM: A and W are both e4m3 (per-row and per-column fp32 scales) and the
// product runs on v_mfma_scale_f32_32x32x64_f8f6f4 with unit block scales.  A
// k-step is then 128 values = 128 bytes per row, so staging, LDS layout and
// epilogue are those of bf16 byte for byte; only the fragment reads (32 bytes
// per lane) and the MFMA differ.  AMX: A carries e8m0 exponents per row and
// 32 k instead of a row scale, applied as the MFMA's block scales.
template <int EPI, int RF32, int OF32, int TM, int WB = 2, bool F8MM = false, bool AMX = false>
__global__ __launch_bounds__(256, 1) void gemm_w4_kernel(LinearParams p) {
  static_assert(TM == 256 || TM == 224, "tile rows");
  static_assert(WB == 2 || WB == 1, "weight bytes");
  constexpr bool MXO = OF32 == 2;  // e4m3 output with e8m0 exponents per 32 columns
  static_assert(!F8MM || (WB == 2 && TM == 224), "fp8 MFMA: 224-row tiles");
  static_assert(!F8MM || AMX || EPI == WAM_EPI_BIAS || EPI == WAM_EPI_BIAS_GELU,
                "fp8 MFMA with per-row activation scales: bias or GELU epilogue");
  static_assert(!AMX || (F8MM && !MXO && EPI != WAM_EPI_BIAS_GELU), "MX activations: fp8 MFMA, bf16 output");
  static_assert(!MXO || (F8MM && !AMX && (EPI == WAM_EPI_BIAS || EPI == WAM_EPI_BIAS_GELU)),
                "MX output: fp8 MFMA with per-row activation scales, bias or GELU");
  constexpr int AE = F8MM ? 1 : 2;        // bytes per A element
  constexpr int WE = F8MM ? 1 : WB;       // bytes per W element
  constexpr int MB = TM == 256 ? 4 : 7;   // 32-row m-blocks per wave
  constexpr int NB = TM == 256 ? 4 : 2;   // 32-column n-blocks per wave
  constexpr int WGN = TM == 256 ? 2 : 4;  // waves along n
  constexpr int LA = TM / 32;             // A staging loads per thread and k-step
  constexpr int LW = WB == 2 ? 8 : 4;     // W staging loads per thread and k-step
  constexpr int NL = LA + LW;
  constexpr int WKB = F8MM ? 128 : 64 * WB;  // bytes of a weight row per k-step
  constexpr int NM = MB * NB, NR = MB + NB;  // MFMAs and fragment reads per sub-step
  __shared__ __attribute__((aligned(1024))) char L0[65536];
  __shared__ __attribute__((aligned(1024))) char L1[65536];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int half = lane >> 5, l32 = lane & 31;

  // Tile order: XCD-contiguous ranges, then groups of 8 m-tiles swept along n.
  int tile = xcd_remap(blockIdx.x, gridDim.x);
  int kp = 0;
  if constexpr (EPI == kEpiPartial) {
    const int tiles = p.m_tiles * p.n_tiles;
    kp = __builtin_amdgcn_readfirstlane(tile / tiles);
    tile -= kp * tiles;
  }
  constexpr int G = 8;
  const int per_group = G * p.n_tiles;
  const int group = tile / per_group, in_group = tile - group * per_group;
  const int first_m = group * G;
  const int gsize = min(p.m_tiles - first_m, G);
  const int tm = __builtin_amdgcn_readfirstlane(first_m + in_group % gsize);
  const int tn = __builtin_amdgcn_readfirstlane(in_group / gsize);
  const int seg = __builtin_amdgcn_readfirstlane(tn / p.n_tiles_per_seg);
  const int n0 = (tn - seg * p.n_tiles_per_seg) * 256;
  const int m0 = tm * TM;

  int nk = p.K / (F8MM ? 128 : 64), kb = 0;
  if constexpr (EPI == kEpiPartial) {
    kb = (int)((int64_t)kp * nk / p.k_split);
    nk = (int)((int64_t)(kp + 1) * nk / p.k_split) - kb;
  }
  // Buffer resources that move to k-tile kt: rows past M (A) or past the
  // segment's N (W) load as zeros through the bound.
  const char* wseg = static_cast<const char*>(seg == 0 ? p.w[0] : (seg == 1 ? p.w[1] : p.w[2]));
  const char* abase = reinterpret_cast<const char*>(p.a) + (int64_t)m0 * p.lda * AE + kb * 128;
  const char* bbase = wseg + (int64_t)n0 * p.ldw * WE + kb * WKB;
  const uint32_t abytes = (uint32_t)(p.M - m0) * (uint32_t)p.lda * (uint32_t)AE - (uint32_t)kb * 128u;
  const uint32_t bbytes =
      (uint32_t)min(256, p.seg_n - n0) * (uint32_t)p.ldw * (uint32_t)WE - (uint32_t)kb * (uint32_t)WKB;
  auto res_a = [&](int kt) { return make_rsrc(abase + kt * 128, abytes - (uint32_t)kt * 128u); };
  auto res_b = [&](int kt) { return make_rsrc(bbase + kt * WKB, bbytes - (uint32_t)kt * (uint32_t)WKB); };

  // Staging: load i (0..NL-1) of a thread is row 32 i + tid / 8 of A (i < LA)
  // or row 32 (i - LA) + tid / 8 of W, 16-byte chunk tid % 8.  Its LDS slot
  // is that row's chunk under the swizzle; (row >> 1) & 7 does not depend on i.
  // fp8 weights: W load j is row 64 j + tid / 4, bytes 16 (tid % 4) .. +16,
  // i.e. the bf16 chunks 2 (tid % 4) and 2 (tid % 4) + 1 of that row.
  const int lr = tid >> 3, lc = tid & 7;
  const int va = lr * (int)p.lda * AE + lc * 16;
  const int vb = WB == 2 ? lr * (int)p.ldw * WE + lc * 16 : (tid >> 2) * (int)p.ldw + (tid & 3) * 16;
  const int ra32 = 32 * (int)p.lda * AE, rb32 = (WB == 2 ? 32 : 64) * (int)p.ldw * WE;
  const int wofs = lds_off<8>(lr, lc);
  const int wofs8_0 = lds_off<8>(tid >> 2, 2 * (tid & 3)), wofs8_1 = lds_off<8>(tid >> 2, 2 * (tid & 3) + 1);
  typedef unsigned int u32x4s __attribute__((ext_vector_type(4)));
  u32x4s S0[NL], S1[NL];
  auto gload = [&](u32x4s* S, int kt, auto lo_c, auto hi_c) {
    constexpr int LO = decltype(lo_c)::value, HI = decltype(hi_c)::value;
    const __amdgpu_buffer_rsrc_t ra = res_a(kt), rb = res_b(kt);
#pragma unroll
    for (int i = LO; i < HI; ++i) {
      if (i < LA) S[i] = __builtin_bit_cast(u32x4s, __builtin_amdgcn_raw_buffer_load_b128(ra, va + i * ra32, 0, 0));
      else S[i] = __builtin_bit_cast(u32x4s, __builtin_amdgcn_raw_buffer_load_b128(rb, vb + (i - LA) * rb32, 0, 0));
    }
  };
  auto swrite = [&](u32x4s* S, char* buf, auto lo_c, auto hi_c) {
    constexpr int LO = decltype(lo_c)::value, HI = decltype(hi_c)::value;
#pragma unroll
    for (int i = LO; i < HI; ++i) {
      if (WB == 2 || i < LA) {
        *reinterpret_cast<u32x4s*>(buf + (i >= LA ? 32768 + (i - LA) * 4096 : i * 4096) + wofs) = S[i];
      } else {
        char* w = buf + 32768 + (i - LA) * 8192;
        *reinterpret_cast<bf16x8*>(w + wofs8_0) = fp8x8_to_bf16x8(u32x2{S[i][0], S[i][1]});
        *reinterpret_cast<bf16x8*>(w + wofs8_1) = fp8x8_to_bf16x8(u32x2{S[i][2], S[i][3]});
      }
    }
  };
  // LDS writes of staging slots [lo, hi): one per slot, two per fp8 W slot.
  constexpr auto dsw = [](int lo, int hi) {
    int n = 0;
    for (int i = lo; i < hi; ++i) n += (WB == 1 && i >= LA) ? 2 : 1;
    return n;
  };
  // The staging sets go to LDS and are reloaded in three parts over a k-step.
  constexpr int P1 = WB == 1 ? 5 : (NL == 16 ? 6 : 5), P2 = WB == 1 ? 9 : (NL == 16 ? 11 : 10);
  using I0 = std::integral_constant<int, 0>;
  using IP1 = std::integral_constant<int, P1>;
  using IP2 = std::integral_constant<int, P2>;
  using INL = std::integral_constant<int, NL>;

  f32x16 acc[NB][MB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[j][i] = f32x16{};
  if constexpr (F8MM) {
  // fp8 MFMA k loop.  One staging set (k-step t+1 written to the free stage
  // and reloaded with t+2 during step t: one step of lead) and two sub-steps
  // of 64 values per 128-byte k-step.  The MFMA's k = 64 are two blocks of
  // 32: block b is bytes 16 b .. 16 b + 15 of both lane halves, and its
  // block scale comes from lane half b (measured on the device).  A lane of
  // half h therefore takes logical chunks 4 s + h (block 2 s of the k-step)
  // and 4 s + 2 + h (block 2 s + 1), so that each MFMA block is one 32-value
  // block of the row.
  typedef int i32x8 __attribute__((ext_vector_type(8)));
  i32x8 ga[2][MB], gb[2][NB];
  const int rowa = (wm * 32 * MB + l32) * 128, rowb = 32768 + (wn * 32 * NB + l32) * 128;
  auto frag8 = [&](const char* p8, int s) {
    const int sw = (l32 >> 1) & 7, c = 4 * s + half;
    const u32x4s lo = *reinterpret_cast<const u32x4s*>(p8 + ((c ^ sw) << 4));
    const u32x4s hi = *reinterpret_cast<const u32x4s*>(p8 + (((c + 2) ^ sw) << 4));
    return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  // AMX: the e8m0 exponents of the A tile's rows for a k-step (4 bytes =
  // 4 blocks of 32 per row) ride with the stage, thread t loading row t
  // into bytes 28672 + 4 t (free: the A rows end at 28672, W starts at
  // 32768).  Lane half h supplies the scale of MFMA block h, i.e. of the
  // k-step's block 2 s + h: its rows' words shifted right by 8 h hold that
  // of sub-step 0 in byte 0 and that of sub-step 1 in byte 2, which the
  // MFMA's operand select picks.
  constexpr int kScl = 28672;
  const uint32_t ldsc = (uint32_t)p.K / 32u;  // exponent bytes per A row
  const __amdgpu_buffer_rsrc_t rsc =
      AMX ? make_rsrc(p.abscale + (int64_t)m0 * ldsc, (uint32_t)(p.M - m0) * ldsc) : make_rsrc(p.a, 0u);
  uint32_t ssc = 0;
  uint32_t scw[2][MB];
  auto rd8 = [&](const char* buf, int s, int f, int par) {
#pragma unroll
    for (int i = 0; i < MB; ++i) ga[f][i] = frag8(buf + rowa + i * 4096, s);
#pragma unroll
    for (int j = 0; j < NB; ++j) gb[f][j] = frag8(buf + rowb + j * 4096, s);
    if (AMX && s == 0) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
        scw[par][i] = *reinterpret_cast<const uint32_t*>(buf + kScl + (wm * 32 * MB + 32 * i + l32) * 4) >> (8 * half);
    }
  };
  auto mm8 = [&](int f, int par) {
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        if constexpr (AMX) {
          if (f == 0)
            acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(gb[f][j], ga[f][i], acc[j][i], 0, 0, 0, 127,
                                                                        0, (int)scw[par][i]);
          else
            acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(gb[f][j], ga[f][i], acc[j][i], 0, 0, 0, 127,
                                                                        2, (int)scw[par][i]);
        } else {
          acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(gb[f][j], ga[f][i], acc[j][i], 0, 0, 0, 127,
                                                                      0, 127);
        }
      }
  };
  auto gsc = [&](int kt) {
    if constexpr (AMX) ssc = __builtin_amdgcn_raw_buffer_load_b32(rsc, tid * (int)ldsc + kt * 4, 0, 0);
  };
  auto wsc8 = [&](char* buf) {
    if constexpr (AMX) *reinterpret_cast<uint32_t*>(buf + kScl + tid * 4) = ssc;
  };
  // Prologue: k-step 0 into L0, k-step 1 into the staging set.
  gload(S0, 0, I0{}, INL{});
  gsc(0);
  swrite(S0, L0, I0{}, INL{});
  wsc8(L0);
  gload(S0, min(1, nk - 1), I0{}, INL{});
  gsc(min(1, nk - 1));
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  rd8(L0, 0, 0, 0);
  // Step t: sub-step 0 from `cur` with the writes of k-step t+1 to `nxt` and
  // the loads of k-step t+2; the barrier; sub-step 1 with the reads of the
  // next step's sub-step 0 from `nxt`.  PAR = t % 2 picks the exponent words.
  auto kstep8 = [&](int t, char* cur, char* nxt, auto par_c) {
    constexpr int PAR = decltype(par_c)::value;
    rd8(cur, 1, 1, PAR);
    swrite(S0, nxt, I0{}, INL{});
    wsc8(nxt);
    gload(S0, min(t + 2, nk - 1), I0{}, INL{});
    gsc(min(t + 2, nk - 1));
    mm8(0, PAR);
    w4_sched<NL + (AMX ? 1 : 0), NL + (AMX ? 1 : 0), NM, NR * 2>();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    rd8(nxt, 0, 0, 1 - PAR);
    mm8(1, PAR);
    w4_sched<0, 0, NM, NR * 2 + (AMX ? MB : 0)>();
    __builtin_amdgcn_sched_barrier(0);
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  int t = 0;
  for (; t + 1 < nk; t += 2) {
    kstep8(t, L0, L1, P0{});
    kstep8(t + 1, L1, L0, P1{});
  }
  if (t < nk) kstep8(t, L0, L1, P0{});
  } else {
  // Fragments of a sub-step: rows wm*32*MB + 32 i + l32 of A and wn*32*NB +
  // 32 j + l32 of W at logical chunk 2 s + half; the swizzle term is
  // (l32 >> 1) & 7.
  bf16x8 fa[2][MB], fb[2][NB];
  const int rowa = (wm * 32 * MB + l32) * 128, rowb = 32768 + (wn * 32 * NB + l32) * 128;
  auto rd = [&](const char* buf, int s, int f) {
    const int xo = ((2 * s + half) ^ ((l32 >> 1) & 7)) << 4;
#pragma unroll
    for (int i = 0; i < MB; ++i) fa[f][i] = ld_bf16x8(buf + rowa + i * 4096 + xo);
#pragma unroll
    for (int j = 0; j < NB; ++j) fb[f][j] = ld_bf16x8(buf + rowb + j * 4096 + xo);
  };
  auto mm = [&](int f) {
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
        acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[f][j], fa[f][i], acc[j][i], 0, 0, 0);
  };

  // Prologue: k-tiles 0 and 1 into the register sets, k-tile 0 into L0, then
  // k-tile 2 into set 0.  Loads past the last k-tile repeat it: unconditional
  // register writes keep the staging sets out of control-flow merges, which
  // made the register allocator copy and spill them.
  gload(S0, 0, I0{}, INL{});
  gload(S1, min(1, nk - 1), I0{}, INL{});
  swrite(S0, L0, I0{}, INL{});
  gload(S0, min(2, nk - 1), I0{}, INL{});
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  rd(L0, 0, 0);

  // One k-step from `cur`; Snext holds k-step t+1 (written to `nxt`) and is
  // reloaded with k-step t+3.
  auto kstep = [&](int t, char* cur, char* nxt, u32x4s* Snext) {
    const int kt3 = min(t + 3, nk - 1);
    rd(cur, 1, 1);
    swrite(Snext, nxt, I0{}, IP1{});
    mm(0);
    w4_sched<dsw(0, P1), 0, NM, NR>();
    __builtin_amdgcn_sched_barrier(0);
    rd(cur, 2, 0);
    swrite(Snext, nxt, IP1{}, IP2{});
    gload(Snext, kt3, I0{}, IP1{});
    mm(1);
    w4_sched<dsw(P1, P2), P1, NM, NR>();
    __builtin_amdgcn_sched_barrier(0);
    rd(cur, 3, 1);
    swrite(Snext, nxt, IP2{}, INL{});
    gload(Snext, kt3, IP1{}, IP2{});
    mm(0);
    w4_sched<dsw(P2, NL), P2 - P1, NM, NR>();
    __builtin_amdgcn_sched_barrier(0);
    // Every wave has written its part of the next stage and read its last
    // fragments of this one.
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    rd(nxt, 0, 0);
    gload(Snext, kt3, IP2{}, INL{});
    mm(1);
    w4_sched<0, NL - P2, NM, NR>();
    __builtin_amdgcn_sched_barrier(0);
  };
  // Pairs of k-steps without a condition inside (a conditional second step
  // made the accumulators cross a control-flow merge and spill).
  int t = 0;
  for (; t + 1 < nk; t += 2) {
    kstep(t, L0, L1, S1);
    kstep(t + 1, L1, L0, S0);
  }
  if (t < nk) kstep(t, L0, L1, S1);
  }

  // ------------------------------------------------------------- epilogue
  // Two rounds of 128 rows through both stage buffers (1 KB fp32 rows, 16-byte
  // chunks XOR-swizzled by row & 15).  In round r every wave writes its
  // m-tiles 2r and 2r+1 (rows wm*128 + 64 r .. +64 of the tile) as whole
  // 4-float slices of the accumulators, then every thread reads back one
  // 16-byte chunk (4 columns) of 32 rows, so bias, gate, residual and output
  // accesses are whole contiguous rows.  Residual loads and output stores go
  // through buffer resources bounded at row M: rows past M read zeros and
  // their stores are dropped, so the epilogue has no per-row branches, and a
  // round's residual loads are all in flight during its LDS exchange.
  const int q = tid & 63;
  const int n = n0 + 4 * q;  // the W4 path takes whole 256-column tiles only
  float bv[4] = {0.f, 0.f, 0.f, 0.f};
  {
    const bf16* __restrict__ bias = seg == 0 ? p.bias[0] : (seg == 1 ? p.bias[1] : p.bias[2]);
    if (bias) {
      const bf16x4 tb = *reinterpret_cast<const bf16x4*>(bias + n);
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[e] = static_cast<float>(tb[e]);
    }
  }
  float wsc[4] = {1.f, 1.f, 1.f, 1.f};  // fp8 weight scales of the lane's columns
  if constexpr ((WB == 1 || F8MM) && EPI != kEpiPartial) {
    const float4 t = *reinterpret_cast<const float4*>((seg == 0 ? p.wscale[0] : (seg == 1 ? p.wscale[1] : p.wscale[2])) + n);
    wsc[0] = t.x; wsc[1] = t.y; wsc[2] = t.z; wsc[3] = t.w;
  }
  // The gate of the lane's 4 columns for the tile's rows when they read at
  // most two consecutive modulation rows (samples or latent frames): gate
  // before tile row gate_split, gate2 from there on; otherwise per row.
  float gate[4] = {0.f, 0.f, 0.f, 0.f}, gate2[4] = {0.f, 0.f, 0.f, 0.f};
  bool gate_held = false;
  int gate_split = 0;
  if constexpr (EPI == WAM_EPI_BIAS_GATE_RES) {
    const int m_last = min(m0 + TM, p.M) - 1;
    const int64_t tr0 = temb_row(p.gate, m0), tr1 = temb_row(p.gate, m_last);
    gate_held = tr1 - tr0 <= 1;
    gate_split = (int)(temb_first_row(p.gate, tr1) - m0);
    ld_mod4(p.gate, p.mod_d, m0, p.gate_index, n + p.n_off, gate);
    ld_mod4(p.gate, p.mod_d, m_last, p.gate_index, n + p.n_off, gate2);
  }
  constexpr bool RES = EPI == WAM_EPI_BIAS_GATE_RES || EPI == WAM_EPI_BIAS_RES;
  constexpr bool PART = EPI == kEpiPartial;
  constexpr int RB = RF32 ? 4 : 2;                 // residual bytes per element
  constexpr int OB = PART ? 4 : (MXO ? 1 : (OF32 ? 4 : 2));  // output bytes per element
  // Rows of this tile that exist (the resources start at row m0, so their
  // bounds cover at most TM rows and stay far below 2^32 bytes).
  const uint32_t rows_left = (uint32_t)min(p.M - m0, TM);
  // (without a residual the resource is a zero-length one over the output; never read)
  const __amdgpu_buffer_rsrc_t rres =
      RES ? make_rsrc(static_cast<const char*>(p.res) + ((int64_t)m0 * p.ldr + n0) * RB,
                      (uint32_t)((rows_left - 1) * (uint32_t)p.ldr + 256u) * RB)
          : make_rsrc(p.a, 0u);
  __amdgpu_buffer_rsrc_t rout;
  {
    char* obase;
    int64_t ld;
    if constexpr (PART) {
      obase = reinterpret_cast<char*>(p.part + ((int64_t)kp * p.M + m0) * p.seg_n + n0);
      ld = p.seg_n;
    } else {
      void* out = seg == 0 ? p.out[0] : (seg == 1 ? p.out[1] : p.out[2]);
      obase = static_cast<char*>(out) + ((int64_t)m0 * p.ldo + n0) * OB;
      ld = p.ldo;
    }
    rout = make_rsrc(obase, (uint32_t)((rows_left - 1) * (uint32_t)ld + 256u) * OB);
  }
  const int ld_out = PART ? p.seg_n : (int)p.ldo;
  // MX output exponents of this tile: rows m0.., the tile's 8 column blocks
  const __amdgpu_buffer_rsrc_t rmxs =
      MXO ? make_rsrc(p.oscale + (int64_t)m0 * (p.seg_n / 32) + n0 / 32,
                      (uint32_t)((rows_left - 1) * (uint32_t)(p.seg_n / 32) + 8u))
          : make_rsrc(p.a, 0u);
  typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
  typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
  // Tile row handled by pass ps (0..31) of round r: rows 64 r .. +64 of each
  // wave row (TM = 256), or rows 128 r .. +128 (TM = 224, whose second round
  // has 96 rows, passes 0..23).
  auto row_of = [&](int r, int ps) {
    const int rr = ps * 4 + (tid >> 6);
    return TM == 256 ? (rr >> 6) * 128 + 64 * r + (rr & 63) : 128 * r + rr;
  };
  // The same row from the wave-uniform wave index (scalar arithmetic).
  auto row_u = [&](int r, int ps) {
    const int rr = ps * 4 + wave;
    return TM == 256 ? (rr >> 6) * 128 + 64 * r + (rr & 63) : 128 * r + rr;
  };
  // q/k-norm epilogue of this segment: gamma of the lane's 4 columns, the
  // RoPE pair index of its first column, and the tile's 256-column group.
  constexpr bool NORM = EPI == kEpiBiasNorm;
  float* const nssq = NORM ? (seg == 0 ? p.ssq[0] : (seg == 1 ? p.ssq[1] : p.ssq[2])) : nullptr;
  const bool nrm = NORM && nssq != nullptr;
  const bool rope = nrm && p.nfreq != nullptr;
  float gm[4] = {1.f, 1.f, 1.f, 1.f};
  if (nrm) {
    const bf16* g = seg == 0 ? p.ngamma[0] : (seg == 1 ? p.ngamma[1] : p.ngamma[2]);
    const bf16x4 tg = *reinterpret_cast<const bf16x4*>(g + n);
#pragma unroll
    for (int e = 0; e < 4; ++e) gm[e] = static_cast<float>(tg[e]);
  }
  const int jp = rope ? (n % p.nhd) >> 1 : 0;
  const int gcol = n0 >> 8;
  // One round; r is a compile-time constant, so the pass loops below unroll
  // and the residual registers are never indexed at run time.
  // RoPE table row of tile row `row` (wave-uniform): the row itself, or the
  // row modulo the tokens of one sample when every sample shares the table.
  const int fmod = (NORM && p.nfreq_batch == 1 && p.ntokens < p.M) ? p.ntokens : 0;
  auto round = [&](auto r_c, auto nrm_c, auto rope_c) {
    constexpr int r = decltype(r_c)::value;
    constexpr bool NRM = decltype(nrm_c)::value, ROPE = decltype(rope_c)::value;
    constexpr int nps = (TM == 224 && r == 1) ? 24 : 32;
    u32x4v rraw[RES ? 32 : 1];
    if constexpr (RES) {
#pragma unroll
      for (int ps = 0; ps < nps; ++ps) {
        const int off = (row_of(r, ps) * (int)p.ldr + 4 * q) * RB;
        if constexpr (RF32) {
          rraw[ps] = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rres, off, 0, 0));
        } else {
          const u32x2v t2 = __builtin_bit_cast(u32x2v, __builtin_amdgcn_raw_buffer_load_b64(rres, off, 0, 0));
          rraw[ps] = u32x4v{t2[0], t2[1], 0u, 0u};
        }
      }
    }
    // The round's RoPE factors (two complex per lane and row), in flight
    // during the LDS exchange like the residual rows.
    float4 fr[ROPE ? 32 : 1];
    if constexpr (ROPE) {
      // Rows of the round are row_u(r, 0) + offsets below 256; with a shared
      // table one division per round, then at most one wrap per row when a
      // sample has >= 256 tokens.
      const int base = m0 + row_u(r, 0);
      // buffer loads: the lane's pair offset in the address, the (uniform)
      // row offset in the scalar offset
      const int hb = (p.nhd >> 1) * 8;
      const __amdgpu_buffer_rsrc_t rf =
          make_rsrc(p.nfreq, (uint32_t)(p.nfreq_batch == 1 ? p.ntokens : p.M) * (uint32_t)hb);
      auto ld = [&](int ps, int frow) {
        fr[ps] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rf, jp * 8, frow * hb, 0));
      };
      if (fmod == 0) {
#pragma unroll
        for (int ps = 0; ps < nps; ++ps) ld(ps, min(base + row_u(r, ps) - row_u(r, 0), p.M - 1));
      } else if (fmod >= 256) {
        const int tb = base % fmod;
#pragma unroll
        for (int ps = 0; ps < nps; ++ps) {
          const int t = tb + row_u(r, ps) - row_u(r, 0);
          ld(ps, t >= fmod ? t - fmod : t);
        }
      } else {
#pragma unroll
        for (int ps = 0; ps < nps; ++ps) ld(ps, (base + row_u(r, ps) - row_u(r, 0)) % fmod);
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    // The wave's m-blocks of this round, as 1 KB fp32 rows: TM = 256, blocks
    // 2r and 2r+1 into L0 (wave row 0) or L1 (wave row 1); TM = 224, blocks
    // 4r .. 4r+3 (of 7), two into each buffer.
#pragma unroll
    for (int ii = 0; ii < (TM == 256 ? 2 : 4); ++ii) {
      const int i = TM == 256 ? 2 * r + ii : 4 * r + ii;
      if (i >= MB) continue;
      char* buf = (TM == 256 ? wm : ii >> 1) ? L1 : L0;
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int lrw = (ii & 1) * 32 + l32;
            const int qq = wn * 8 * NB + j * 8 + 2 * g + half;
            f32x4 v;
            if (g == 0) v = __builtin_shufflevector(acc[j][i], acc[j][i], 0, 1, 2, 3);
            else if (g == 1) v = __builtin_shufflevector(acc[j][i], acc[j][i], 4, 5, 6, 7);
            else if (g == 2) v = __builtin_shufflevector(acc[j][i], acc[j][i], 8, 9, 10, 11);
            else v = __builtin_shufflevector(acc[j][i], acc[j][i], 12, 13, 14, 15);
            *reinterpret_cast<f32x4*>(buf + lrw * 1024 + ((qq ^ (lrw & 15)) << 4)) = v;
          }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int b8 = 0; b8 < nps / 8; ++b8) {
      f32x4 vv[8];
      float ssr[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      int xkeep = 0;  // MXO: the exponent of pass (lane & 7) of this batch, for lane's block
#pragma unroll
      for (int k8 = 0; k8 < 8; ++k8) {
        const int ps = b8 * 8 + k8;
        const int rr = ps * 4 + (tid >> 6);
        const char* buf = ps < 16 ? L0 : L1;
        const int lrw = rr & 63;
        vv[k8] = *reinterpret_cast<const f32x4*>(buf + lrw * 1024 + ((q ^ (lrw & 15)) << 4));
      }
#pragma unroll
      for (int k8 = 0; k8 < 8; ++k8) {
        const int ps = b8 * 8 + k8;
        const int row = row_of(r, ps);
        const int off = (row * ld_out + 4 * q) * OB;
        if constexpr (PART) {
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, vv[k8]), rout, off, 0, 0);
          continue;
        }
        float y[4];
        if constexpr (F8MM && AMX) {
          // the MX exponents were applied by the MFMA; the column scale here
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = vv[k8][e] * wsc[e] + bv[e];
        } else if constexpr (F8MM) {
          // row scale of the fp8 activations times the column scale
          const float sr = p.ascale[min(m0 + row, p.M - 1)];
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = vv[k8][e] * (sr * wsc[e]) + bv[e];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = WB == 1 ? vv[k8][e] * wsc[e] + bv[e] : vv[k8][e] + bv[e];
        }
        if constexpr (EPI == WAM_EPI_BIAS_GELU) {
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = gelu_tanh(y[e]);
        } else if constexpr (RES) {
          float rv[4];
          const u32x4v t4 = rraw[ps];
          if constexpr (RF32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) rv[e] = __uint_as_float(t4[e]);
          } else {
            rv[0] = __uint_as_float(t4[0] << 16);
            rv[1] = __uint_as_float(t4[0] & 0xffff0000u);
            rv[2] = __uint_as_float(t4[1] << 16);
            rv[3] = __uint_as_float(t4[1] & 0xffff0000u);
          }
          if constexpr (EPI == WAM_EPI_BIAS_GATE_RES) {
            float gt[4];
            if (gate_held) {
#pragma unroll
              for (int e = 0; e < 4; ++e) gt[e] = row >= gate_split ? gate2[e] : gate[e];
            } else {
              // rows past M read the last row's modulation (their stores are dropped)
              ld_mod4(p.gate, p.mod_d, min(m0 + row, p.M - 1), p.gate_index, n + p.n_off, gt);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = rv[e] + y[e] * gt[e];
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = rv[e] + y[e];
          }
        }
        if constexpr (MXO) {
          // e4m3 with one e8m0 exponent per 32 columns (8 lanes): the block's
          // largest |y| sets it, every value is scaled by an exact power of two
          const float amax = max8_lanes(fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3]))));
          const int X = mx_exponent(amax);
          const float inv = __uint_as_float((uint32_t)(127 - X) << 23);
          int pk = 0;
          pk = __builtin_amdgcn_cvt_pk_fp8_f32(y[0] * inv, y[1] * inv, pk, false);
          pk = __builtin_amdgcn_cvt_pk_fp8_f32(y[2] * inv, y[3] * inv, pk, true);
          __builtin_amdgcn_raw_buffer_store_b32((uint32_t)pk, rout, off, 0, 0);
          // every lane of the 8-lane group holds X; lane k8 of it keeps it for
          // one store of the batch's 8 rows x 8 blocks below
          xkeep = (q & 7) == k8 ? X + 127 : xkeep;
        } else if constexpr (OF32 && RES) {
          __builtin_amdgcn_raw_buffer_store_b128(u32x4v{__float_as_uint(y[0]), __float_as_uint(y[1]),
                                                        __float_as_uint(y[2]), __float_as_uint(y[3])},
                                                 rout, off, 0, 0);
        } else {
          bf16x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(y[e]);
          if constexpr (NRM) {
            // y = bf16(acc + b): its squares, then gamma and the rotation of
            // pairs (n, n+1), (n+2, n+3) in fp32, one rounding.
            float z[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) z[e] = static_cast<float>(o[e]);
            const bf16x2 o01 = {o[0], o[1]}, o23 = {o[2], o[3]};
            ssr[k8] = __builtin_amdgcn_fdot2_f32_bf16(o23, o23, __builtin_amdgcn_fdot2_f32_bf16(o01, o01, 0.f, false),
                                                      false);
#pragma unroll
            for (int e = 0; e < 4; ++e) z[e] *= gm[e];
            if constexpr (ROPE) {
              const float4 f = fr[ps];
              const float a0 = z[0] * f.x - z[1] * f.y, a1 = z[0] * f.y + z[1] * f.x;
              const float a2 = z[2] * f.z - z[3] * f.w, a3 = z[2] * f.w + z[3] * f.z;
              z[0] = a0; z[1] = a1; z[2] = a2; z[3] = a3;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(z[e]);
          }
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2v, o), rout, off, 0, 0);
        }
      }
      if constexpr (NRM) {
        // The 8 rows' sums over the wave's 256 columns: lane 16 g + 0 holds
        // rows 2 (g & 1) + 4 (g >> 1) + j of the batch in red[j].
        float red[2];
        wave_sum8(ssr, red);
        const int g = lane >> 4;
        if ((lane & 15) == 0) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int mrow = m0 + row_of(r, b8 * 8 + 2 * (g & 1) + 4 * (g >> 1) + j);
            if (mrow < p.M) nssq[(int64_t)mrow * p.ssq_ld + gcol] = red[j];
          }
        }
      }
      if constexpr (MXO) {
        const int xrow = row_of(r, b8 * 8 + (q & 7));
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)xkeep, rmxs, xrow * (int)(p.seg_n / 32) + (q >> 3), 0, 0);
      }
      // one batch of LDS reads live at a time
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Both rounds per variant: the norm variants are chosen once per tile (a
  // segment's tiles all take one), so no per-row branch remains.
  auto rounds = [&](auto nrm_c, auto rope_c) {
    round(std::integral_constant<int, 0>{}, nrm_c, rope_c);
    round(std::integral_constant<int, 1>{}, nrm_c, rope_c);
  };
  using F = std::false_type;
  using T = std::true_type;
  if constexpr (NORM) {
    if (rope) rounds(T{}, T{});
    else if (nrm) rounds(T{}, F{});
    else rounds(F{}, F{});
  } else {
    rounds(F{}, F{});
  }
}

// Tile configurations: BM x BN x BK, waves (M x N), LDS stages.
// 256x256: one workgroup per CU, the DS reads of a k-step grouped before its
// MFMAs, loads issued in two parts.  The smaller tiles serve grids that would
// not cover the chip with 256x256 tiles and the 128x128 tails.
using Cfg256x256w8t2 = GemmCfg<256, 256, 64, 2, 4, 2, 1, 2, 2, 2>;
// 320x256 tiles, eight waves of 160x64 (two stages of 72 KB, loads issued in
// three parts): 6240 rows are 20 such tiles, so a 3072-column GEMM is one
// round of 240 tiles on 256 CUs.  The epilogue stages 32 rows per buffer
// (five rounds of 64 rows): a round's residual rows then take 32 registers
// per lane next to the 160 accumulators (with 64 rows per buffer they took
// 64, and the gated-residual kernel spilled to scratch).
struct Cfg320x256w8 : GemmCfg<320, 256, 64, 2, 4, 2, 1, 2, 2, 3> {
  static constexpr int EPI_ROWS = 32;
};
using Cfg256x128w4 = GemmCfg<256, 128, 64, 2, 2, 3>;
using Cfg128x128w4 = GemmCfg<128, 128, 64, 2, 2, 3>;
// fp8 e4m3 weights on the small tiles (64-byte LDS weight rows widened at
// the fragment read); the big tiles run the four-wave kernel.
using Cfg128x128f8 = GemmCfg<128, 128, 64, 2, 2, 3, 1, 0, 1>;

// Sum of the k_split fp32 partial ranges of a split-K launch (in range
// order), then the launch's epilogue.  One thread per 4 consecutive outputs.
template <int EPI, int WB>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(LinearParams p) {
  const int q4 = p.seg_n / 4;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.M * q4) return;
  const int m = (int)(i / q4), n = (int)(i - (int64_t)m * q4) * 4;
  const int64_t plane = (int64_t)p.M * p.seg_n, at = (int64_t)m * p.seg_n + n;
  // The loads are issued before any is used and none inside a branch whose
  // body uses it (the compiler waits for such a load at the branch's end):
  // the first two ranges (a split launch has at least two), the bias through
  // a buffer resource (a null bias is a zero-length one: zeros), the scales
  // and the residual's raw words; the adds and widening come after.
  const f32x4 v0 = *reinterpret_cast<const f32x4*>(p.part + at);
  const f32x4 v1 = *reinterpret_cast<const f32x4*>(p.part + plane + at);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.bias[0], p.bias[0] ? (uint32_t)p.seg_n * 2u : 0u);
  const u32x2 braw = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rb, n * 2, 0, 0));
  float wsc[4] = {1.f, 1.f, 1.f, 1.f};
  if constexpr (WB == 1) {
    const float4 t = *reinterpret_cast<const float4*>(p.wscale[0] + n);
    wsc[0] = t.x; wsc[1] = t.y; wsc[2] = t.z; wsc[3] = t.w;
  }
  constexpr bool RES = EPI == WAM_EPI_BIAS_GATE_RES || EPI == WAM_EPI_BIAS_RES;
  u32x4 rraw = {0u, 0u, 0u, 0u};
  if constexpr (RES) {
    const int64_t ro = (int64_t)m * p.ldr + n;
    if (p.res_f32) {
      rraw = *reinterpret_cast<const u32x4*>(static_cast<const float*>(p.res) + ro);
    } else {
      const u32x2 t = *reinterpret_cast<const u32x2*>(static_cast<const bf16*>(p.res) + ro);
      rraw = u32x4{t[0], t[1], 0u, 0u};
    }
  }
  f32x4 v = v0 + v1;
  for (int r = 2; r < p.k_split; ++r) v += *reinterpret_cast<const f32x4*>(p.part + r * plane + at);
  float bv[4];
  bv[0] = __uint_as_float(braw[0] << 16);
  bv[1] = __uint_as_float(braw[0] & 0xffff0000u);
  bv[2] = __uint_as_float(braw[1] << 16);
  bv[3] = __uint_as_float(braw[1] & 0xffff0000u);
  const float no_gate[4] = {0.f, 0.f, 0.f, 0.f};
  float rv[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (RES) {
    if (p.res_f32) {
#pragma unroll
      for (int e = 0; e < 4; ++e) rv[e] = __uint_as_float(rraw[e]);
    } else {
      rv[0] = __uint_as_float(rraw[0] << 16);
      rv[1] = __uint_as_float(rraw[0] & 0xffff0000u);
      rv[2] = __uint_as_float(rraw[1] << 16);
      rv[3] = __uint_as_float(rraw[1] & 0xffff0000u);
    }
  }
  epi_apply<EPI, WB>(p, p.out[0], m, n, v, bv, wsc, no_gate, false, rv);
}

// The q/k-norm epilogue as a pass over a finished bias GEMM's bf16 output,
// for launches that do not end in the four-wave kernel: one wave per (row,
// 256-column group) of segment `seg`, the arithmetic of kEpiBiasNorm.
__global__ __launch_bounds__(256) void linear_norm_kernel(LinearParams p, int seg) {
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (job >= (int64_t)p.M * p.ssq_ld) return;
  const int m = (int)(job / p.ssq_ld), g = (int)(job - (int64_t)m * p.ssq_ld);
  const int n = g * 256 + 4 * lane;
  const bool ok = n < p.seg_n;  // seg_n is a multiple of 8: whole groups of 4
  bf16* out = static_cast<bf16*>(seg == 0 ? p.out[0] : (seg == 1 ? p.out[1] : p.out[2])) + (int64_t)m * p.ldo;
  float z[4] = {0.f, 0.f, 0.f, 0.f};
  if (ok) {
    const bf16x4 t = *reinterpret_cast<const bf16x4*>(out + n);
#pragma unroll
    for (int e = 0; e < 4; ++e) z[e] = static_cast<float>(t[e]);
  }
  const float ss = wave_sum(z[0] * z[0] + z[1] * z[1] + z[2] * z[2] + z[3] * z[3]);
  float* ssq = seg == 0 ? p.ssq[0] : (seg == 1 ? p.ssq[1] : p.ssq[2]);
  if (lane == 0) ssq[(int64_t)m * p.ssq_ld + g] = ss;
  if (!ok) return;
  const bf16x4 tg = *reinterpret_cast<const bf16x4*>((seg == 0 ? p.ngamma[0] : (seg == 1 ? p.ngamma[1] : p.ngamma[2])) + n);
#pragma unroll
  for (int e = 0; e < 4; ++e) z[e] *= static_cast<float>(tg[e]);
  if (p.nfreq) {
    const int frow = (p.nfreq_batch == 1 && p.ntokens < p.M) ? m % p.ntokens : m;
    const float4 f = *reinterpret_cast<const float4*>(p.nfreq + (int64_t)frow * (p.nhd >> 1) + ((n % p.nhd) >> 1));
    const float a0 = z[0] * f.x - z[1] * f.y, a1 = z[0] * f.y + z[1] * f.x;
    const float a2 = z[2] * f.z - z[3] * f.w, a3 = z[2] * f.w + z[3] * f.z;
    z[0] = a0; z[1] = a1; z[2] = a2; z[3] = a3;
  }
  bf16x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = static_cast<bf16>(z[e]);
  *reinterpret_cast<bf16x4*>(out + n) = o;
}

static int linear_norm_pass(const LinearParams& p, hipStream_t s) {
  const int64_t jobs = (int64_t)p.M * p.ssq_ld;
  for (int i = 0; i < p.n_seg_count; ++i) {
    if (!p.ssq[i]) continue;
    hipLaunchKernelGGL(linear_norm_kernel, dim3((unsigned)((jobs + 3) / 4)), dim3(256), 0, s, p, i);
    WAM_LAUNCHED("linear_norm_kernel");
  }
  return WAM_OK;
}

template <class C, int EPI>
static void launch_tiles(dim3 grid, const LinearParams& p, hipStream_t s) {
  if constexpr (C::kW4) {
    constexpr bool RES = EPI == WAM_EPI_BIAS_GATE_RES || EPI == WAM_EPI_BIAS_RES;
    if constexpr (RES) {
      if (p.res_f32 && p.out_f32)
        hipLaunchKernelGGL((gemm_w4_kernel<EPI, 1, 1, C::BM, C::WB>), grid, dim3(C::kThreads), 0, s, p);
      else if (p.res_f32)
        hipLaunchKernelGGL((gemm_w4_kernel<EPI, 1, 0, C::BM, C::WB>), grid, dim3(C::kThreads), 0, s, p);
      else if (p.out_f32)
        hipLaunchKernelGGL((gemm_w4_kernel<EPI, 0, 1, C::BM, C::WB>), grid, dim3(C::kThreads), 0, s, p);
      else
        hipLaunchKernelGGL((gemm_w4_kernel<EPI, 0, 0, C::BM, C::WB>), grid, dim3(C::kThreads), 0, s, p);
    } else {
      hipLaunchKernelGGL((gemm_w4_kernel<EPI, 0, 0, C::BM, C::WB>), grid, dim3(C::kThreads), 0, s, p);
    }
  } else {
    constexpr bool RES = EPI == WAM_EPI_BIAS_GATE_RES || EPI == WAM_EPI_BIAS_RES;
    if constexpr (RES) {
      if (p.res_f32) {
        hipLaunchKernelGGL((gemm_bf16_kernel<C, EPI, 1>), grid, dim3(C::kThreads), 0, s, p);
        return;
      }
    }
    hipLaunchKernelGGL((gemm_bf16_kernel<C, EPI, 0>), grid, dim3(C::kThreads), 0, s, p);
  }
}

template <class C>
static int launch_gemm(LinearParams& p, hipStream_t s) {
  WAM_REQUIRE(p.K % C::BK == 0 && (p.n_seg_count == 1 || p.seg_n % C::BN == 0) &&
              (!C::kW4 || p.seg_n % C::BN == 0),
              "wam_linear: N=%d / K=%d do not fit a %dx%dx%d tile", p.seg_n, p.K, C::BM, C::BN, C::BK);
  p.n_tiles_per_seg = (p.seg_n + C::BN - 1) / C::BN;
  p.m_tiles = (p.M + C::BM - 1) / C::BM;
  p.n_tiles = p.n_tiles_per_seg * p.n_seg_count;
  const int grid = p.m_tiles * p.n_tiles;
  if (p.k_split > 1) {
    WAM_REQUIRE(p.n_seg_count == 1 && p.part && p.k_split <= p.K / C::BK, "wam_linear: bad split-K launch");
    launch_tiles<C, kEpiPartial>(dim3(grid * p.k_split), p, s);
    WAM_LAUNCHED("gemm_bf16_kernel");
    const unsigned rblocks = (unsigned)(((int64_t)p.M * (p.seg_n / 4) + 255) / 256);
    switch (p.epi) {
      case WAM_EPI_BIAS:
        hipLaunchKernelGGL((gemm_splitk_reduce_kernel<WAM_EPI_BIAS, C::WB>), dim3(rblocks), dim3(256), 0, s, p);
        break;
      case WAM_EPI_BIAS_GELU:
        hipLaunchKernelGGL((gemm_splitk_reduce_kernel<WAM_EPI_BIAS_GELU, C::WB>), dim3(rblocks), dim3(256), 0, s,
                           p);
        break;
      case WAM_EPI_BIAS_GATE_RES:
        hipLaunchKernelGGL((gemm_splitk_reduce_kernel<WAM_EPI_BIAS_GATE_RES, C::WB>), dim3(rblocks), dim3(256), 0,
                           s, p);
        break;
      default:
        hipLaunchKernelGGL((gemm_splitk_reduce_kernel<WAM_EPI_BIAS_RES, C::WB>), dim3(rblocks), dim3(256), 0, s,
                           p);
        break;
    }
    WAM_LAUNCHED("gemm_splitk_reduce_kernel");
    return WAM_OK;
  }
  switch (p.epi) {
    case kEpiBiasNorm:
      if constexpr (C::kW4 || std::is_same_v<C, Cfg320x256w8>) {
        WAM_REQUIRE(C::kW4 || p.nfreq == nullptr, "wam_linear: the 320-row q-norm epilogue has no RoPE");
        launch_tiles<C, kEpiBiasNorm>(dim3(grid), p, s);
      } else {
        WAM_REQUIRE(false, "wam_linear: the q/k-norm epilogue runs in the four-wave or the 320-row kernel only");
      }
      break;
    case WAM_EPI_BIAS:
      launch_tiles<C, WAM_EPI_BIAS>(dim3(grid), p, s);
      break;
    case WAM_EPI_BIAS_GELU:
      launch_tiles<C, WAM_EPI_BIAS_GELU>(dim3(grid), p, s);
      break;
    case WAM_EPI_BIAS_GATE_RES:
      launch_tiles<C, WAM_EPI_BIAS_GATE_RES>(dim3(grid), p, s);
      break;
    default:
      launch_tiles<C, WAM_EPI_BIAS_RES>(dim3(grid), p, s);
      break;
  }
  WAM_LAUNCHED("gemm_bf16_kernel");
  return WAM_OK;
}

// 256x256 tiles run in whole-chip rounds (one workgroup per CU).  When the
// tile count is not a multiple of the CU count, the last round keeps CUs idle.
// The plan then runs the first `full` rounds' worth of whole output columns
// as the main launch and the remaining columns (the tail) one of two ways:
//   kind 1: 128x128 tiles over the whole chip; a round of them costs about
//           0.375 of a 256x256 tile's time (measured at K = 3072 and 14336);
//   kind 2: split-K: each 256x256 tail tile in ks k ranges (ks * tail tiles
//           <= CUs), fp32 partial sums in the caller's workspace, then one
//           reduce pass that applies the epilogue.  Cost per range 1/ks of a
//           tile, plus about 4 k-tiles of pipeline fill, plus the reduce
//           (a 256 KB partial per range at ~5 TB/s, against ~1.8 us per
//           64-deep k-tile of a 256x256 tile).
// Costs are in 256x256 tile times; the cheapest of one launch, kind 1 and
// kind 2 (when the workspace holds its partials) wins.  E.g. 6240 x 3072 x
// 14336: 250 tiles + 50 tail tiles in 5 ranges (1.25 vs 1.375 for kind 1).
struct GemmPlan {
  int kind;     // 0: one launch
  int n_main;   // 256-column tiles of the main launch
  int k_split;  // kind 2
};

static GemmPlan gemm_plan(int M, int seg_n, int n_seg, int K, int cus, int64_t ws_bytes) {
  const GemmPlan one{0, 0, 1};
  if (n_seg != 1 || seg_n % 256 != 0 || K % 64 != 0) return one;
  const int mt = (M + 255) / 256, nt = seg_n / 256;
  const int64_t tiles = (int64_t)mt * nt, full = tiles / cus;
  if (full < 1 || tiles % cus == 0) return one;
  const int n_main = (int)(full * cus / mt);
  if (n_main < 1 || n_main >= nt) return one;
  const int tail_cols = (nt - n_main) * 256;
  const int64_t tail_tiles = (int64_t)mt * (nt - n_main);
  const double nk = K / 64.0;
  double best = (double)((tiles + cus - 1) / cus);
  GemmPlan plan = one;
  const int64_t small = (int64_t)((M + 127) / 128) * (tail_cols / 128);
  const double cost1 = (double)full + (double)((small + cus - 1) / cus) * 0.375;
  if (cost1 < best - 1e-9) best = cost1, plan = GemmPlan{1, n_main, 1};
  const int64_t ks = cus / tail_tiles < 8 ? cus / tail_tiles : 8;
  if (ks >= 2 && ks <= nk) {
    const int64_t bytes = ks * M * (int64_t)tail_cols * 4;
    const double cost2 = (double)full + 1.0 / ks + 4.0 / nk + (double)(tail_tiles * ks) * 0.052 / (nk * 1.8);
    if (bytes <= ws_bytes && cost2 < best - 1e-9) best = cost2, plan = GemmPlan{2, n_main, (int)ks};
  }
  return plan;
}

static int64_t plan_workspace(const GemmPlan& g, int M, int seg_n) {
  return g.kind == 2 ? (int64_t)g.k_split * M * (int64_t)(seg_n - g.n_main * 256) * 4 : 0;
}

template <class CBig, class CSmall>
static int launch_big(LinearParams& p, int64_t ws_bytes, hipStream_t s) {
  const GemmPlan g = gemm_plan(p.M, p.seg_n, p.n_seg_count, p.K, device_cu_count(), p.part ? ws_bytes : 0);
  if (g.kind == 0) return launch_gemm<CBig>(p, s);
  LinearParams main = p;
  main.seg_n = g.n_main * 256;
  main.k_split = 1;
  WAM_TRY(launch_gemm<CBig>(main, s));
  LinearParams tail = p;
  const int64_t c0 = (int64_t)g.n_main * 256;
  tail.seg_n = p.seg_n - (int)c0;
  tail.n_off = p.n_off + (int)c0;
  tail.w[0] = static_cast<const char*>(p.w[0]) + c0 * p.ldw * CBig::WB;
  if (p.wscale[0]) tail.wscale[0] = p.wscale[0] + c0;
  tail.bias[0] = p.bias[0] ? p.bias[0] + c0 : nullptr;
  tail.out[0] = static_cast<char*>(p.out[0]) + c0 * (p.out_f32 ? 4 : 2);
  if (p.res) tail.res = static_cast<const char*>(p.res) + c0 * (p.res_f32 ? 4 : 2);
  if (g.kind == 1) {
    tail.k_split = 1;
    return launch_gemm<CSmall>(tail, s);
  }
  tail.k_split = g.k_split;
  return launch_gemm<CBig>(tail, s);
}

// Cost of a launch in 256x256-tile times: the 256-row plan (whole rounds,
// or rounds plus a tail, gemm_plan) against one launch of 224-row tiles,
// whose rounds take 7/8 as long.
static bool w4_t224_wins(int M, int seg_n, int n_seg, int K, int cus, int64_t ws_bytes) {
  const int64_t nt = (int64_t)(seg_n / 256) * n_seg;
  const int64_t t256 = (int64_t)((M + 255) / 256) * nt, t224 = (int64_t)((M + 223) / 224) * nt;
  double c256 = (double)((t256 + cus - 1) / cus);
  const GemmPlan g = gemm_plan(M, seg_n, n_seg, K, cus, ws_bytes);
  if (g.kind != 0) {
    // The plan's tail, in full-tile rounds: 0.4, as measured for the 128x128
    // tail of 4680 x 14336 x 3072 (35 us against 87 us per round of 256-row
    // tiles).  That shape then takes the 224-row tiles, whose partial fifth
    // round runs at a higher clock than the full ones.
    c256 = (double)(t256 / cus) + 0.4;
  }
  const double c224 = (double)((t224 + cus - 1) / cus) * (224.0 / 256.0);
  return c224 < c256 - 1e-9;
}

// One round of 320-row tiles, when that round is shorter than the 256-row
// plan (a round plus a tail) and the 224-row plan has lost already: 6240 x
// 3072 (240 tiles against 300 + a tail), measured alternating on one box:
// bias 114 -> 102 us, plain residual 129 -> 115, gated residual 141 -> 121,
// bias + q-norm pass 132 -> 118, and 6240 x 3072 x 14336 474 -> 463 us.
static bool t320_one_round(int M, int seg_n, int n_seg, int K, int cus, int64_t ws_bytes) {
  const int64_t nt = (int64_t)(seg_n / 256) * n_seg;
  const int64_t t320 = (int64_t)((M + 319) / 320) * nt, t256 = (int64_t)((M + 255) / 256) * nt;
  if (seg_n % 256 != 0 || t320 > cus) return false;
  if (gemm_plan(M, seg_n, n_seg, K, cus, ws_bytes).kind == 0) return false;
  return 320.0 / 256.0 < (double)(t256 / cus) + 0.4 - 1e-9;
}

// Whether linear() takes the 256x256 path for this shape.
static bool uses_big_tiles(int M, int seg_n, int n_seg) {
  const int64_t big_tiles = (int64_t)((M + 255) / 256) * (seg_n / 256) * n_seg;
  return seg_n % 256 == 0 && big_tiles >= 200;
}

int64_t linear_workspace_bytes(int M, int seg_n, int n_seg, int K) {
  if (M < 1 || seg_n < 1 || K < 1 || !uses_big_tiles(M, seg_n, n_seg)) return 0;
  return plan_workspace(gemm_plan(M, seg_n, n_seg, K, device_cu_count(), INT64_MAX), M, seg_n);
}

// Whether linear() applies the q/k-norm epilogue inside its one launch for
// this bf16 shape: the four-wave kernel, or one round of 320-row tiles when
// there is no RoPE (otherwise it runs the GEMM and then the norm pass, which
// costs about what a separate RMSNorm pass costs).
bool linear_norm_in_epilogue(int M, int seg_n, int n_seg, int K, int64_t ws_bytes, bool rope) {
  if (M < 1 || K % 64 != 0 || !uses_big_tiles(M, seg_n, n_seg)) return false;
  const int cus = device_cu_count();
  if (w4_t224_wins(M, seg_n, n_seg, K, cus, ws_bytes)) return true;
  if (t320_one_round(M, seg_n, n_seg, K, cus, ws_bytes)) return !rope;
  return gemm_plan(M, seg_n, n_seg, K, cus, ws_bytes).kind == 0;
}

int linear(const wam_linear_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr, "wam_linear: null args");
  WAM_REQUIRE(a->n_seg >= 1 && a->n_seg <= 3, "wam_linear: n_seg must be 1..3 (got %d)", a->n_seg);
  WAM_REQUIRE(a->M >= 1 && a->K >= 1 && a->seg_n >= 1, "wam_linear: empty shape M=%d K=%d N=%d",
              a->M, a->K, a->seg_n);
  WAM_REQUIRE(a->K % 64 == 0, "wam_linear: K=%d must be a multiple of 64", a->K);
  WAM_REQUIRE(a->seg_n % 8 == 0 && (a->n_seg == 1 || a->seg_n % 128 == 0),
              "wam_linear: N=%d must be a multiple of 8 (of 128 with several segments)", a->seg_n);
  WAM_REQUIRE(a->w_dtype == WAM_BF16 || a->w_dtype == WAM_FP8, "wam_linear: w_dtype %d", a->w_dtype);
  WAM_REQUIRE(a->a_dtype == WAM_BF16 || a->a_dtype == WAM_FP8 || a->a_dtype == WAM_FP8_MX,
              "wam_linear: a_dtype %d", a->a_dtype);
  const bool f8 = a->w_dtype == WAM_FP8;
  const bool a8 = a->a_dtype == WAM_FP8;
  const bool amx = a->a_dtype == WAM_FP8_MX;
  const bool mxo = a->out_dtype == WAM_FP8_MX;
  const int wb = f8 ? 1 : 2;
  WAM_REQUIRE((a->lda * (a8 || amx ? 1 : 2)) % 16 == 0 && (a->ldw * wb) % 16 == 0 && a->ldo % 4 == 0,
              "wam_linear: row strides must keep 16-byte alignment");
  WAM_REQUIRE(a->a != nullptr, "wam_linear: null activation");
  WAM_REQUIRE((int64_t)a->M * a->lda * 2 < (int64_t)1 << 31 && (int64_t)a->seg_n * a->ldw * wb < (int64_t)1 << 31,
              "wam_linear: operands above 2 GiB are not supported");
  // Epilogue addresses within one tile (up to 256 rows of fp32) are 32-bit.
  WAM_REQUIRE(a->ldo < ((int64_t)1 << 21) && a->ldr < ((int64_t)1 << 21),
              "wam_linear: output/residual row strides must be below 2^21 elements");
  for (int i = 0; i < a->n_seg; ++i) {
    WAM_REQUIRE(a->w[i] != nullptr && a->out[i] != nullptr, "wam_linear: null weight/out %d", i);
    WAM_REQUIRE(!f8 || a->w_scale[i] != nullptr, "wam_linear: fp8 weights need w_scale %d", i);
  }
  WAM_REQUIRE(a->epilogue >= WAM_EPI_BIAS && a->epilogue <= WAM_EPI_BIAS_RES,
              "wam_linear: unknown epilogue %d", a->epilogue);
  WAM_REQUIRE((a->res_dtype == WAM_BF16 || a->res_dtype == WAM_F32) &&
              (a->out_dtype == WAM_BF16 || a->out_dtype == WAM_F32 || mxo), "wam_linear: dtype codes");
  if (a->epilogue == WAM_EPI_BIAS_GATE_RES || a->epilogue == WAM_EPI_BIAS_RES)
    WAM_REQUIRE(a->res != nullptr && a->ldr % 4 == 0, "wam_linear: residual missing");
  else
    WAM_REQUIRE(a->out_dtype != WAM_F32, "wam_linear: fp32 output only for residual epilogues");
  WAM_REQUIRE(!mxo || (a8 && (a->epilogue == WAM_EPI_BIAS || a->epilogue == WAM_EPI_BIAS_GELU) &&
                       a->out_block_scale != nullptr),
              "wam_linear: an MX output needs fp8 activations with row scales, WAM_EPI_BIAS or "
              "WAM_EPI_BIAS_GELU, and out_block_scale");
  if (a->epilogue == WAM_EPI_BIAS_GATE_RES) {
    WAM_TRY(check_modulation(a->gate, a->M, "wam_linear"));
    WAM_REQUIRE(a->gate.temb_mods != 1 && a->gate_index >= 0 && a->gate_index < 6,
                "wam_linear: the gate reads a [.., 6, D] temb (index %d)", a->gate_index);
  }
  LinearParams p{};
  p.a = static_cast<const bf16*>(a->a); p.lda = a->lda; p.M = a->M; p.K = a->K;
  p.seg_n = a->seg_n; p.ldw = a->ldw; p.ldo = a->ldo; p.epi = a->epilogue;
  for (int i = 0; i < 3; ++i) {
    const int j = i < a->n_seg ? i : 0;
    p.w[i] = a->w[j];
    p.wscale[i] = f8 ? a->w_scale[j] : nullptr;
    p.bias[i] = static_cast<const bf16*>(a->bias[j]);
    p.out[i] = a->out[j];
  }
  p.res = a->res; p.ldr = a->ldr;
  p.res_f32 = a->res_dtype == WAM_F32;
  p.out_f32 = a->out_dtype == WAM_F32;
  p.gate = a->gate; p.gate_index = a->gate_index;
  p.n_seg_count = a->n_seg;
  p.mod_d = a->seg_n;
  p.n_off = 0;
  WAM_REQUIRE(a->workspace_bytes >= 0, "wam_linear: negative workspace_bytes");
  p.k_split = 1;
  p.part = static_cast<float*>(a->workspace);
  const int64_t ws_bytes = a->workspace ? a->workspace_bytes : 0;
  const bool norm = a->norm_ssq[0] || a->norm_ssq[1] || a->norm_ssq[2];
  if (norm) {
    WAM_REQUIRE(a->epilogue == WAM_EPI_BIAS && !f8 && a->out_dtype == WAM_BF16,
                "wam_linear: the q/k-norm epilogue needs WAM_EPI_BIAS, bf16 weights and a bf16 output");
    for (int i = 0; i < 3; ++i) {
      WAM_REQUIRE(!a->norm_ssq[i] || (i < a->n_seg && a->norm_gamma[i]),
                  "wam_linear: norm segment %d needs a gamma (and must exist)", i);
      p.ssq[i] = i < a->n_seg ? a->norm_ssq[i] : nullptr;
      p.ngamma[i] = i < a->n_seg ? static_cast<const bf16*>(a->norm_gamma[i]) : nullptr;
    }
    if (a->norm_freq) {
      WAM_REQUIRE(a->norm_head_dim > 0 && a->norm_head_dim % 4 == 0 && a->seg_n % a->norm_head_dim == 0,
                  "wam_linear: norm head_dim %d must be a multiple of 4 dividing N=%d", a->norm_head_dim,
                  a->seg_n);
      WAM_REQUIRE(a->norm_tokens >= 1 && a->M % a->norm_tokens == 0 &&
                  (a->norm_freq_batch == 1 || a->norm_freq_batch == a->M / a->norm_tokens),
                  "wam_linear: norm freq batch %d / tokens %d contract", a->norm_freq_batch, a->norm_tokens);
      WAM_REQUIRE(((uintptr_t)a->norm_freq & 15) == 0, "wam_linear: norm_freq must be 16-byte aligned");
      p.nfreq = static_cast<const float2*>(a->norm_freq);
      p.nfreq_batch = a->norm_freq_batch; p.ntokens = a->norm_tokens; p.nhd = a->norm_head_dim;
    }
    p.ssq_ld = (a->seg_n + 255) / 256;
  }
  const bool big = uses_big_tiles(a->M, a->seg_n, a->n_seg);
  if (a8 || amx) {
    WAM_REQUIRE(f8 && (amx ? a->a_block_scale != nullptr : a->a_scale != nullptr),
                "wam_linear: fp8 activations need fp8 weights and a_scale (a_block_scale for WAM_FP8_MX)");
    WAM_REQUIRE(!amx || ((uintptr_t)a->a_block_scale & 3) == 0,
                "wam_linear: a_block_scale must be 4-byte aligned (one word per row and 128 values)");
    if (a8)
      WAM_REQUIRE((a->epilogue == WAM_EPI_BIAS || a->epilogue == WAM_EPI_BIAS_GELU) && !norm,
                  "wam_linear: fp8 activations with row scales take WAM_EPI_BIAS or WAM_EPI_BIAS_GELU");
    else
      WAM_REQUIRE(a->epilogue != WAM_EPI_BIAS_GELU && !norm &&
                  (a->out_dtype == WAM_BF16 || (a->out_dtype == WAM_F32 && a->epilogue == WAM_EPI_BIAS_GATE_RES &&
                                                a->res_dtype == WAM_F32)),
                  "wam_linear: MX activations take WAM_EPI_BIAS, WAM_EPI_BIAS_GATE_RES or WAM_EPI_BIAS_RES "
                  "with a bf16 output (fp32 only for the gated fp32 residual)");
    WAM_REQUIRE(a->n_seg == 1 && a->seg_n % 256 == 0 && a->K % 128 == 0,
                "wam_linear: fp8 activations need one segment, N a multiple of 256 and K of 128 (N=%d K=%d)",
                a->seg_n, a->K);
    p.ascale = a->a_scale;
    p.abscale = static_cast<const uint8_t*>(a->a_block_scale);
    p.oscale = static_cast<uint8_t*>(a->out_block_scale);
    p.n_tiles_per_seg = a->seg_n / 256;
    p.m_tiles = (a->M + 223) / 224;
    p.n_tiles = p.n_tiles_per_seg;
    const dim3 grid((unsigned)(p.m_tiles * p.n_tiles));
    if (amx) {
      if (a->epilogue == WAM_EPI_BIAS)
        hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS, 0, 0, 224, 2, true, true>), grid, dim3(256), 0, s, p);
      else if (a->epilogue == WAM_EPI_BIAS_GATE_RES && p.res_f32 && p.out_f32)
        hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS_GATE_RES, 1, 1, 224, 2, true, true>), grid, dim3(256), 0, s, p);
      else if (a->epilogue == WAM_EPI_BIAS_GATE_RES && p.res_f32)
        hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS_GATE_RES, 1, 0, 224, 2, true, true>), grid, dim3(256), 0, s, p);
      else if (a->epilogue == WAM_EPI_BIAS_GATE_RES)
        hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS_GATE_RES, 0, 0, 224, 2, true, true>), grid, dim3(256), 0, s, p);
      else if (p.res_f32)
        hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS_RES, 1, 0, 224, 2, true, true>), grid, dim3(256), 0, s, p);
      else
        hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS_RES, 0, 0, 224, 2, true, true>), grid, dim3(256), 0, s, p);
    } else if (a->epilogue == WAM_EPI_BIAS) {
      if (mxo) hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS, 0, 2, 224, 2, true>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS, 0, 0, 224, 2, true>), grid, dim3(256), 0, s, p);
    } else {
      if (mxo) hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS_GELU, 0, 2, 224, 2, true>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((gemm_w4_kernel<WAM_EPI_BIAS_GELU, 0, 0, 224, 2, true>), grid, dim3(256), 0, s, p);
    }
    WAM_LAUNCHED("gemm_w4_kernel (fp8 MFMA)");
    return WAM_OK;
  }
  WAM_REQUIRE(!mxo, "wam_linear: an MX output needs fp8 activations with row scales");
  if (f8) {
    // fp8 weights: the four-wave kernel widens them to bf16 as it stages
    // them (FFN unit at 4680 rows, alternating runs on one box: 713-714 us
    // with the eight-wave kernel, 678 us with this one; bf16 679-680 us)
    if (big) {
      if (w4_t224_wins(a->M, a->seg_n, a->n_seg, a->K, device_cu_count(), ws_bytes))
        return launch_gemm<CfgW4t224f8>(p, s);
      return launch_big<CfgW4f8, Cfg128x128f8>(p, ws_bytes, s);
    }
    return launch_gemm<Cfg128x128f8>(p, s);
  }
  // Big tiles when the grid still covers the chip; otherwise smaller tiles.
  // The four-wave kernel has the faster k loop.  On 224-row tiles it wins
  // whenever those need fewer tile-times (4680 rows: QKV 240 -> 226 us,
  // 4680 x 3072 x 3072 78 -> 75 us, FFN2 335 -> 321 us, the gated-residual
  // projection 95 -> 92 us against the eight-wave kernel).  On 256-row tiles
  // its epilogue reads residual rows with one wave per SIMD, which costs more
  // than the loop gains when the loop is short (4680 and 6240 x 3072 x 3072
  // with the gated and plain residual epilogues: 4-12% slower than the
  // eight-wave kernel; every other block GEMM 0-10% faster).
  // With the q/k-norm epilogue, a launch that is one four-wave grid applies
  // it in its epilogue; any other runs the bias GEMM and then the norm pass.
  if (big) {
    const bool res = a->epilogue == WAM_EPI_BIAS_GATE_RES || a->epilogue == WAM_EPI_BIAS_RES;
    if (w4_t224_wins(a->M, a->seg_n, a->n_seg, a->K, device_cu_count(), ws_bytes)) {
      if (norm) p.epi = kEpiBiasNorm;
      return launch_gemm<CfgW4t224>(p, s);
    }
    if (t320_one_round(a->M, a->seg_n, a->n_seg, a->K, device_cu_count(), ws_bytes)) {
      if (norm && !p.nfreq) {
        p.epi = kEpiBiasNorm;
        return launch_gemm<Cfg320x256w8>(p, s);
      }
      WAM_TRY(launch_gemm<Cfg320x256w8>(p, s));
      return norm ? linear_norm_pass(p, s) : WAM_OK;
    }
    if (res && a->K <= 4096) return launch_big<Cfg256x256w8t2, Cfg128x128w4>(p, ws_bytes, s);
    if (norm && gemm_plan(p.M, p.seg_n, p.n_seg_count, p.K, device_cu_count(), p.part ? ws_bytes : 0).kind == 0) {
      p.epi = kEpiBiasNorm;
      return launch_gemm<CfgW4>(p, s);
    }
    WAM_TRY((launch_big<CfgW4, Cfg128x128w4>(p, ws_bytes, s)));
    return norm ? linear_norm_pass(p, s) : WAM_OK;
  }
  const int64_t mid_tiles = (int64_t)((a->M + 255) / 256) * (a->seg_n / 128) * a->n_seg;
  if (mid_tiles >= 200) WAM_TRY(launch_gemm<Cfg256x128w4>(p, s));
  else WAM_TRY(launch_gemm<Cfg128x128w4>(p, s));
  return norm ? linear_norm_pass(p, s) : WAM_OK;
}

// bf16 copy of an MX matrix (e4m3 q [rows, cols] with an e8m0 exponent per
// row and 32 columns): a debug view of the fp8 FFN's hidden layer.  Every
// e4m3 value times a power of two in bf16 range is a bf16 value (exact).
__global__ __launch_bounds__(256) void mx_dequant_bf16_kernel(const uint8_t* __restrict__ q,
                                                              const uint8_t* __restrict__ e, bf16* __restrict__ y,
                                                              int cols, int64_t n4) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const int64_t idx = i * 4, r = idx / cols;
  const int c = (int)(idx - r * cols);
  const uint32_t v = *reinterpret_cast<const uint32_t*>(q + idx);
  const float sc = __uint_as_float((uint32_t)e[r * (cols / 32) + c / 32] << 23);
  bf16x4 o;
  o[0] = static_cast<bf16>(__builtin_amdgcn_cvt_f32_fp8((int)v, 0) * sc);
  o[1] = static_cast<bf16>(__builtin_amdgcn_cvt_f32_fp8((int)v, 1) * sc);
  o[2] = static_cast<bf16>(__builtin_amdgcn_cvt_f32_fp8((int)v, 2) * sc);
  o[3] = static_cast<bf16>(__builtin_amdgcn_cvt_f32_fp8((int)v, 3) * sc);
  *reinterpret_cast<bf16x4*>(y + idx) = o;
}

int mx_dequant_bf16(const void* q, const void* e, void* y, int rows, int cols, hipStream_t s) {
  WAM_REQUIRE(rows >= 0 && cols % 32 == 0, "mx_dequant_bf16: cols=%d must be a multiple of 32", cols);
  const int64_t n4 = (int64_t)rows * cols / 4;
  if (n4 == 0) return WAM_OK;
  hipLaunchKernelGGL(mx_dequant_bf16_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                     static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(e), static_cast<bf16*>(y), cols,
                     n4);
  WAM_LAUNCHED("mx_dequant_bf16_kernel");
  return WAM_OK;
}

// Per-row fp8 e4m3 quantization: one workgroup per row.
__global__ __launch_bounds__(256) void quantize_fp8_rows_kernel(const bf16* __restrict__ w, int cols,
                                                                int64_t ldw, uint8_t* __restrict__ q,
                                                                float* __restrict__ scale) {
  __shared__ unsigned smax;
  const int r = blockIdx.x, tid = threadIdx.x;
  const bf16* row = w + (int64_t)r * ldw;
  if (tid == 0) smax = 0u;
  __syncthreads();
  float mx = 0.f;
  for (int c = tid * 8; c < cols; c += 256 * 8) {
    const bf16x8 v = ld_bf16x8(row + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(static_cast<float>(v[e])));
  }
  atomicMax(&smax, __float_as_uint(mx));  // non-negative floats order as their bits
  __syncthreads();
  const float amax = __uint_as_float(smax);
  const float sc = amax > 0.f ? amax / 448.0f : 1.0f;
  const float inv = amax > 0.f ? 448.0f / amax : 1.0f;  // one division per row
  uint8_t* qrow = q + (int64_t)r * cols;
  for (int c = tid * 8; c < cols; c += 256 * 8) {
    const bf16x8 v = ld_bf16x8(row + c);
    int lo = 0, hi = 0;
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(static_cast<float>(v[0]) * inv, static_cast<float>(v[1]) * inv, lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(static_cast<float>(v[2]) * inv, static_cast<float>(v[3]) * inv, lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(static_cast<float>(v[4]) * inv, static_cast<float>(v[5]) * inv, hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(static_cast<float>(v[6]) * inv, static_cast<float>(v[7]) * inv, hi, true);
    *reinterpret_cast<u32x2*>(qrow + c) = u32x2{(unsigned)lo, (unsigned)hi};
  }
  if (tid == 0) scale[r] = sc;
}

int quantize_fp8_rows(const void* w, int rows, int cols, int64_t ldw, void* q, float* scale, hipStream_t s) {
  WAM_REQUIRE(w && q && scale, "wam_quantize_fp8_rows: null pointer");
  WAM_REQUIRE(rows >= 1 && cols >= 8 && cols % 8 == 0 && ldw % 8 == 0 && ldw >= cols,
              "wam_quantize_fp8_rows: rows=%d cols=%d ldw=%lld (cols and ldw multiples of 8)", rows, cols,
              (long long)ldw);
  hipLaunchKernelGGL(quantize_fp8_rows_kernel, dim3(rows), dim3(256), 0, s, static_cast<const bf16*>(w), cols,
                     ldw, static_cast<uint8_t*>(q), scale);
  WAM_LAUNCHED("quantize_fp8_rows_kernel");
  return WAM_OK;
}

}  // namespace wam

extern "C" int wam_quantize_fp8_rows(const void* w, int rows, int cols, int64_t ldw, void* q, float* scale,
                                     void* stream) {
  return wam::quantize_fp8_rows(w, rows, cols, ldw, q, scale, static_cast<hipStream_t>(stream));
}

extern "C" int wam_linear(const wam_linear_args* args, void* stream) {
  return wam::linear(args, static_cast<hipStream_t>(stream));
}

extern "C" int64_t wam_linear_workspace_bytes(int M, int N, int n_seg, int K) {
  return wam::linear_workspace_bytes(M, N, n_seg, K);
}
