// Flash attention forward on CDNA4 MFMA, head_dim 128, bf16 in/out, fp32
// online softmax.  Keys come from two places: the KV pool, read through a
// slot list (history), and the projection output of this call (own keys).
//
// Math: softmax(Q K^T / sqrt(hd)) V per head, non-causal, as
// F.scaled_dot_product_attention in model.py:37-40; the online-softmax
// rescaling is the standard flash-attention recurrence (running max m, running
// sum l, O <- O * exp(m_old - m_new) + P V).
//
// Orientation.  S^T = K * Q^T is formed with v_mfma_f32_32x32x16_bf16, so a
// lane of the 32x32 accumulator owns ONE query (column) and 16 of the 32 keys
// (rows); the other 16 keys of that query sit in lane ^ 32.  Row statistics
// therefore need a single cross-half exchange.  O^T = V^T * P^T reuses the S^T
// registers as the B operand without any data movement: MFMA k-slot u of lane
// half h is key 8*(u/4) + 4*h + u%4 of the 16-key step, which is exactly the
// key order of the S^T accumulator; V^T is written to LDS in that same slot
// order.  The per-query rescale factor is then a per-lane scalar.
//
// The reference's native path uses FlashAttention-2 (CUDA) after packing the
// pool rows into a contiguous tensor (pack_kernel,
// 算子研究/wam_ops/baseline/csrc/block.cu:213-224); here the pool is read in
// place through the slot list.
#include <algorithm>
#include <mutex>
#include "wam_common.h"

namespace wam {

constexpr int kAttnHD = 128;
constexpr int kAttnKT = 64;                          // keys per LDS stage
constexpr int kAttnTile = kAttnKT * kAttnHD * 2;     // 16 KB per K or V tile
constexpr int kAttnStage = 2 * kAttnTile;            // K tile + V tile
constexpr int kAttnStages = 3;

// LDS layouts (64 banks x 4 bytes; 256-byte rows = one bank line).
// K [64 keys][128 d]: an S^T operand fetch reads 16 consecutive keys at one
// 16-byte chunk per cycle, so chunk XOR (key mod 16).
__device__ inline int k_off(int key, int c) { return key * 256 + ((c ^ (key & 15)) << 4); }
// V [64 keys][128 d] in natural layout: a transposed read fetches 4
// consecutive keys x 64 bytes per 32 lanes, so the 64-byte segment XOR
// (key mod 4).
__device__ inline int v_off(int key, int c) { return key * 256 + ((c ^ ((key & 3) << 2)) << 4); }

__device__ inline int clamp_row(int r, int n) { return r < 0 ? 0 : (r >= n ? n - 1 : r); }

// Per-query RMS factor of queries written by wam_linear's norm epilogue:
// rsqrt(sum of the row's q_ssq_n partial sums of squares / q_norm_dim + eps)
// for query row b * Mq + qi (clamped into range).  The RMSNorm across heads
// is model.py:609-612; the rotation after it is linear and commutes.  The
// pipelined kernel stages the partial sums through LDS instead (see there).
constexpr int kQssqMax = 16;
__device__ inline float q_rms_factor(const wam_attention_args& a, int b, int qi) {
  const float* p = a.q_ssq + ((int64_t)b * a.Mq + min(qi, a.Mq - 1)) * a.q_ssq_n;
  float s = 0.f;
  for (int t = 0; t < a.q_ssq_n; ++t) s += p[t];
  return rsqrtf(s / (float)a.q_norm_dim + a.q_eps);
}

// Workgroup: W waves x 32 queries of one (batch row, head).  Wave w owns
// queries q0 + 32 w .. +32 and keeps its Q fragments in registers.
// A unit is one (query tile, batch row, head), numbered query tile fastest.
// Workgroups 0 .. n_full-1 each run one whole unit (n_full = all units when
// nothing is split).  Each of the remaining units is split into n_split
// contiguous key ranges, one workgroup per range; those write their
// unnormalised O and their (max, sum) to `part`, and attention_combine_kernel
// merges them.  Whole units are dispatched first, so the splits fill the last
// dispatch round evenly.
template <int W>
__global__ __launch_bounds__(64 * W, 1) void attention_kernel(wam_attention_args a,
                                                              const int* __restrict__ slots, int n_full,
                                                              int n_split, float* __restrict__ part) {
  // One __shared__ object per stage: the compiler tracks direct-to-LDS loads
  // per object, so reading one stage while others are being filled does not
  // wait for those loads.
  __shared__ __attribute__((aligned(1024))) char lds0[kAttnStage];
  __shared__ __attribute__((aligned(1024))) char lds1[kAttnStage];
  __shared__ __attribute__((aligned(1024))) char lds2[kAttnStage];
  // Each wave's 32 query rows (8 KB), laid out like a K tile.
  __shared__ __attribute__((aligned(1024))) char ldsq[32 * W * kAttnHD * 2];
  static_assert(kAttnStages == 3, "three stage objects");
#define WAM_ATTN_BUF(st) ((st) == 0 ? lds0 : (st) == 1 ? lds1 : lds2)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, half = lane >> 5;
  constexpr int QT = 32 * W;
  constexpr int LPW = 2 * kAttnTile / 1024 / W;  // 1 KB direct-to-LDS loads per wave per stage
  static_assert(16 % W == 0, "waves must divide the 16 K blocks of a stage");

  const int nqt = (a.Mq + QT - 1) / QT;
  const int n_tail = nqt * a.H * a.B - n_full;  // split units
  int unit, split = 0, ns = 1;
  if ((int)blockIdx.x < n_full) {
    unit = xcd_remap(blockIdx.x, n_full);
  } else {
    // consecutive pieces: consecutive units of one key range (shared K/V in L2)
    const int piece = xcd_remap(blockIdx.x - n_full, gridDim.x - n_full);
    unit = n_full + piece % n_tail;
    split = piece / n_tail;
    ns = n_split;
  }
  unit = __builtin_amdgcn_readfirstlane(unit);
  split = __builtin_amdgcn_readfirstlane(split);
  ns = __builtin_amdgcn_readfirstlane(ns);
  const int qt = unit % nqt, bh = unit / nqt;
  const int b = bh % a.B, h = bh / a.B;  // head-major: the batch rows of one head are adjacent

  const int n_hist = a.n_hist_dev ? __builtin_amdgcn_readfirstlane(*a.n_hist_dev) : 0;
  const int n_tot = n_hist + a.Mk;
  const int prow = __builtin_amdgcn_readfirstlane(a.pool_rows ? clamp_row((int)a.pool_rows[b], a.pool_batch)
                                                              : (a.pool_batch > 0 ? clamp_row(b, a.pool_batch) : 0));
  const int krow = __builtin_amdgcn_readfirstlane(a.kv_rows ? clamp_row((int)a.kv_rows[b], a.kv_batch)
                                                            : clamp_row(b, a.kv_batch));
  const bf16* pool_k = a.pool_k ? static_cast<const bf16*>(a.pool_k) + (int64_t)prow * a.pool_bstride + h * kAttnHD : nullptr;
  const bf16* pool_v = a.pool_v ? static_cast<const bf16*>(a.pool_v) + (int64_t)prow * a.pool_bstride + h * kAttnHD : nullptr;
  const bf16* own_k = static_cast<const bf16*>(a.k) + (int64_t)krow * a.kv_bstride + h * kAttnHD;
  const bf16* own_v = static_cast<const bf16*>(a.v) + (int64_t)krow * a.kv_bstride + h * kAttnHD;

  // Q fragments (B operand of S^T = K Q^T): query qi, d = 16 ks + 8 half .. +8.
  const int qi = qt * QT + wave * 32 + l32;
  const bool q_ok = qi < a.Mq;
  const bool live = qt * QT + wave * 32 < a.Mq;  // wave-uniform

  // Direct-to-LDS staging.  Load g (0..31) of a stage fills 1 KB block g:
  // blocks 0-15 are the K tile, 16-31 the V tile, 4 rows (keys) each; lane L
  // lands in row 4 (g % 16) + L / 16, physical chunk L % 16, and fetches the
  // logical chunk the swizzle maps there.  Load i of wave w is g = w + i W.
  const int lrow = lane >> 4, pch = lane & 15;
  // The wave's loads cover 16 / W blocks of 4 keys (K and V of a block share
  // their rows).  Their pool slots are read with wave-uniform loads before
  // the wait and barrier that precede the issue, so that the loads' latency
  // overlaps that wait.
  constexpr int NB = 16 / W;
  struct TileSlots { int v[NB][4]; };
  auto tile_slots = [=](int t) {
    TileSlots ts;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int jj = t * kAttnKT + 4 * ((wave + b * W) & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = __builtin_amdgcn_readfirstlane(min(jj + r, n_tot - 1));
        ts.v[b][r] = j < n_hist ? slots[j] : 0;
      }
    }
    return ts;
  };
  auto issue = [=](int t, char* base, TileSlots ts) {
    const int j0 = t * kAttnKT;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int g = wave + i * W;
      const bool is_k = i < 16 / W;                 // compile-time per i
      const int gb = g & 15;
      const int row = 4 * gb + lrow;
      const int jj = j0 + 4 * gb;
      const int b = i % NB;                         // block (wave + b W) & 15 == gb
      const int slot = lrow == 0 ? ts.v[b][0] : (lrow == 1 ? ts.v[b][1] : (lrow == 2 ? ts.v[b][2] : ts.v[b][3]));
      const int j = min(jj + lrow, n_tot - 1);
      const int c = is_k ? (pch ^ (row & 15)) : (pch ^ ((row & 3) << 2));
      const bf16* src = j < n_hist ? (is_k ? pool_k : pool_v) + (int64_t)slot * a.pool_rstride
                                   : (is_k ? own_k : own_v) + (int64_t)(j - n_hist) * a.kv_rstride;
      asm_g_ld16_lds((uint64_t)(uintptr_t)(src + c * 8), base + (is_k ? 0 : kAttnTile) + gb * 1024);
    }
  };

  float sc = a.scale * kLog2e;
  if (a.q_ssq) sc *= q_rms_factor(a, b, qi);
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};

  // Transposed-read source addresses of this lane inside a V tile, per
  // (dt, ks, part): keys 16 ks + 4 half + 8 part + (lane % 16) / 4,
  // d = 32 dt + 16 ((lane / 16) % 2) + 4 (lane % 4).
  const int tr_i = lane & 15, tr_gh = (lane >> 4) & 1;

  // Key tiles [t_first, t_first + ntiles) of this workgroup's split; t below
  // counts from t_first.
  const int all_tiles = (n_tot + kAttnKT - 1) / kAttnKT;
  const int t_first = (int)((int64_t)split * all_tiles / ns);
  const int ntiles = (int)((int64_t)(split + 1) * all_tiles / ns) - t_first;
  // Q comes in through LDS too, ahead of the first stages: loads of the
  // wave's 32 rows, 4 rows (1 KB) per load, lane L fetching the logical chunk
  // that the K-tile swizzle puts at byte 16 L.  The stage waits below count
  // these loads, and the fragments are then read with ds_read, so no wait
  // for Q also waits for the stages behind it.
  char* const qbuf = ldsq + wave * (32 * kAttnHD * 2);
  {
    const bf16* qrow0 = static_cast<const bf16*>(a.q) + (int64_t)b * a.q_bstride + h * kAttnHD;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 4 * i + lrow;
      const int qr = min(qt * QT + wave * 32 + row, a.Mq - 1);
      const int c = pch ^ (row & 15);
      asm_g_ld16_lds((uint64_t)(uintptr_t)(qrow0 + (int64_t)qr * a.q_rstride + c * 8), qbuf + i * 1024);
    }
  }
#pragma unroll
  for (int st = 0; st < kAttnStages - 1; ++st)
    if (st < ntiles) issue(t_first + st, WAM_ATTN_BUF(st), tile_slots(t_first + st));
  // This wave's Q loads are done once at most the stage loads behind them
  // are outstanding.
  static_assert(kAttnStages == 3 && 2 * LPW < 64, "Q wait: vmcnt range");
  constexpr int kVm1 = (LPW & 15) | ((LPW >> 4) << 14) | (7 << 4) | (15 << 8);
  constexpr int kVm2 = ((2 * LPW) & 15) | (((2 * LPW) >> 4) << 14) | (7 << 4) | (15 << 8);
  if (ntiles >= 2) __builtin_amdgcn_s_waitcnt(kVm2);
  else if (ntiles == 1) __builtin_amdgcn_s_waitcnt(kVm1);
  else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
  // Q fragments (B operand of S^T = K Q^T): query qi, d = 16 ks + 8 half .. +8.
  bf16x8 qf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    qf[ks] = ld_bf16x8(qbuf + k_off(l32, 2 * ks + half));
    if (!q_ok) qf[ks] = bf16x8{};
  }

  // The tile loop is unrolled by the stage count so that every LDS reference
  // is to a fixed __shared__ object.
  for (int t0 = 0; t0 < ntiles; t0 += kAttnStages) {
#pragma unroll
    for (int st = 0; st < kAttnStages; ++st) {
      const int t = t0 + st;
      if (t >= ntiles) break;
      const bool refill = t + kAttnStages - 1 < ntiles;
      TileSlots ts{};
      if (refill) ts = tile_slots(t_first + t + kAttnStages - 1);
      if (t + kAttnStages - 2 < ntiles) {
        // stages t+1 .. t+STAGES-2 may still be in flight
        __builtin_amdgcn_s_waitcnt((((kAttnStages - 2) * LPW) & 15) | ((((kAttnStages - 2) * LPW) >> 4) << 14) |
                                   (7 << 4) | (15 << 8));
      } else {
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
      }
      __builtin_amdgcn_s_barrier();
      if (refill) issue(t_first + t + kAttnStages - 1, WAM_ATTN_BUF((st + kAttnStages - 1) % kAttnStages), ts);
      if (!live) continue;  // this wave's queries are all past Mq; it still loads and syncs
      const char* kb = WAM_ATTN_BUF(st);
      const char* vb = kb + kAttnTile;

      // The two 32-key halves alternate, so consecutive MFMAs never wait on
      // each other's accumulator.  K fragments are read two k-steps ahead of
      // their MFMAs, so an LDS read has two steps of MFMAs to land.
      f32x16 s[2];
      s[0] = f32x16{};
      s[1] = f32x16{};
      bf16x8 kf[3][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) kf[ks][kt] = ld_bf16x8(kb + k_off(kt * 32 + l32, 2 * ks + half));
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // the first two steps' reads
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        if (ks + 2 < 8) {
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
            kf[(ks + 2) % 3][kt] = ld_bf16x8(kb + k_off(kt * 32 + l32, 2 * (ks + 2) + half));
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
          s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks % 3][kt], qf[ks], s[kt], 0, 0, 0);
        if (ks + 2 < 8) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // the reads two steps ahead
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                  // then this step's MFMAs
      }
      if ((t_first + t + 1) * kAttnKT > n_tot) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int j = (t_first + t) * kAttnKT + kt * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
            if (j >= n_tot) s[kt][v] = -INFINITY;
          }
      }
      // Lazy rescaling: the running max m_run (log2 units, equal in both
      // lane halves of a query) only moves when a tile's max exceeds it by
      // more than 8, so exp2(s - m_run) <= 2^8.  A lane's own 32 keys decide
      // whether anything moved; only then are the halves' maxima exchanged,
      // the new running max set and O/l rescaled (the first tile, and rare
      // jumps after it).  sum(p v) / sum(p) does not depend on which max is
      // used.
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kt][v]);
      if (__builtin_amdgcn_ballot_w64(mx * sc > m_run + 8.0f)) {
        const float mt = fmaxf(mx, __shfl_xor(mx, 32, 64)) * sc;
        const bool grow = mt > m_run + 8.0f;
        const float m_new = grow ? mt : m_run;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
        m_run = m_new;
      }
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float pv = __builtin_amdgcn_exp2f(s[kt][v] * sc - m_run);
          s[kt][v] = pv;
          psum += pv;
        }
      l_run += psum;

      bf16x8 pb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int u = 0; u < 8; ++u) pb[ks][u] = static_cast<bf16>(s[ks >> 1][(ks & 1) * 8 + u]);
      // V^T fragments (two transposed reads each) are read two MFMAs ahead.
      auto vload = [&](int i) {
        const int ks = i >> 2, dt = i & 3;
        bf16x8 va;
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const int key = 16 * ks + 4 * half + 8 * part + (tr_i >> 2);
          const int d = 32 * dt + 16 * tr_gh + 4 * (tr_i & 3);
          const bf16x4 t4 = ld_tr16(vb + v_off(key, d >> 3) + (d & 7) * 2);
          va[4 * part + 0] = t4[0]; va[4 * part + 1] = t4[1];
          va[4 * part + 2] = t4[2]; va[4 * part + 3] = t4[3];
        }
        return va;
      };
      bf16x8 vf[3];
      vf[0] = vload(0);
      vf[1] = vload(1);
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i + 2 < 16) vf[(i + 2) % 3] = vload(i + 2);
        o[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[i % 3], pb[i >> 2], o[i & 3], 0, 0, 0);
        if (i + 2 < 16) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
    }
  }
#undef WAM_ATTN_BUF

  const float l = l_run + __shfl_xor(l_run, 32, 64);
  if (ns > 1) {
    // Partial result of this key range: O (unnormalised, relative to m_run),
    // and (m_run, l) of the query; an empty range leaves m = -inf, l = 0,
    // O = 0.  Row (split, split unit, query in tile).
    if (q_ok) {
      const int64_t row = ((int64_t)split * n_tail + (unit - n_full)) * QT + wave * 32 + l32;
      float* op = part + row * kAttnHD;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4*>(op + dt * 32 + 8 * g + 4 * half) =
              make_float4(o[dt][4 * g], o[dt][4 * g + 1], o[dt][4 * g + 2], o[dt][4 * g + 3]);
      if (half == 0) {
        float* ml = part + (int64_t)n_split * n_tail * QT * kAttnHD + row * 2;
        *reinterpret_cast<float2*>(ml) = make_float2(m_run, l);
      }
    }
    return;
  }
  const float inv = 1.f / l;
  if (q_ok) {
    bf16* op = static_cast<bf16*>(a.o) + (int64_t)b * a.o_bstride + (int64_t)qi * a.o_rstride + h * kAttnHD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 t4;
#pragma unroll
        for (int e = 0; e < 4; ++e) t4[e] = static_cast<bf16>(o[dt][4 * g + e] * inv);
        *reinterpret_cast<bf16x4*>(op + dt * 32 + 8 * g + 4 * half) = t4;
      }
  }
}

// ---------------------------------------------------------------------------
// Software-pipelined variant for calls whose keys are all this call's own
// (no KV pool): 8 waves x 32 queries, key tiles of 64 in 3 LDS stages (4
// with PP below).  Per tile t a wave issues
//   g1: S(t+1) = K_{t+1} Q^T (16 MFMAs)  interleaved with  softmax of S(t)
//   g2: O += V_t^T P(t)     (16 MFMAs)
// so the exponentials, row sums and bf16 packing of one tile run under the
// MFMAs of the next; in attention_kernel they ran between the wave's own MFMA
// phases, with both waves of a SIMD in the same phase (MFMA busy 34% on
// 4680 x 4680).  S(t) and S(t+1) live in two fixed register sets: tiles are
// processed in pairs, with a peeled last tile.  K/V come in through buffer
// loads straight to LDS (rows past Mk read zeros) and Q through buffer loads
// into registers.  Lane layouts of S^T, P and O^T are those of
// attention_kernel.
//
// PP (ping-pong, for long key ranges): the two waves of a SIMD run half a
// tile apart, so that one wave's softmax (VALU) runs beside the other's
// O += V^T P MFMAs instead of beside its own S MFMAs only.  A workgroup's
// waves land on the SIMDs in turn (wave w and w + 4 share one), so waves
// 0-3 form group A and the others group B.  Both run the same sequence per
// tile t, S(t+1) + softmax(t), then O += V_t P(t), with one barrier per tile:
// A's after its softmax, B's after its P V, and B one barrier behind A from
// the start.  Between two barriers A does P V(t) and S/softmax(t+1) while B
// does S/softmax(t) and P V(t).  Tile t+3 is issued right after barrier t
// into the stage of tile t-1 (four stages) and has landed by barrier t+1.
// Same arithmetic per wave as the one-phase schedule, so the results are
// identical; 4680 x 4680, 24 heads: 290-291 -> 273-275 us in the block.
// With 8 key tiles (cross attention over 512 keys) it measured 1-3% slower,
// so the host only picks it for long key ranges, and with pool keys (the
// 4 x 1560-query verify layer over 7800 keys) the layer took 15-30 us longer,
// so the pool path keeps one phase per tile.
template <bool HIST, int NW, bool PP>
__global__ __launch_bounds__(64 * NW, 1) void attention_sp_kernel(wam_attention_args a, const int* __restrict__ slots,
                                                                  int n_full, int n_split, float* __restrict__ part) {
  static_assert(NW == 8 || (NW == 7 && !HIST), "8 waves, or 7 without pool keys");
  static_assert(!(PP && HIST), "ping-pong without pool keys");
  // K/V stages (three, four with PP), then (pool keys only) the 64 slots of
  // each stage's tile, then each wave's query partial sums of squares (q_ssq)
  constexpr int NST = PP ? 4 : 3;
  constexpr int kQpSlots = kQssqMax / 2;  // direct-to-LDS dword loads per wave: 2 partials each
  constexpr int kQpOff = NST * kAttnStage + (HIST ? NST * kAttnKT * 4 : 0);
  __shared__ __attribute__((aligned(1024))) char lds[kQpOff + NW * kQpSlots * 256];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, half = lane >> 5;
  constexpr int QT = 32 * NW;
  const int nqt = (a.Mq + QT - 1) / QT;
  const int n_tail = nqt * a.H * a.B - n_full;
  int unit, split = 0, ns = 1;
  if ((int)blockIdx.x < n_full) {
    unit = xcd_remap(blockIdx.x, n_full);
  } else {
    const int piece = xcd_remap(blockIdx.x - n_full, gridDim.x - n_full);
    unit = n_full + piece % n_tail;
    split = piece / n_tail;
    ns = n_split;
  }
  unit = __builtin_amdgcn_readfirstlane(unit);
  split = __builtin_amdgcn_readfirstlane(split);
  ns = __builtin_amdgcn_readfirstlane(ns);
  const int qt = unit % nqt, bh = unit / nqt;
  const int b = bh % a.B, h = bh / a.B;
  const int krow = __builtin_amdgcn_readfirstlane(a.kv_rows ? clamp_row((int)a.kv_rows[b], a.kv_batch)
                                                            : clamp_row(b, a.kv_batch));
  // Keys: n_hist pool rows (through the slot list) and then the Mk own keys.
  const int n_hist = HIST ? __builtin_amdgcn_readfirstlane(*a.n_hist_dev) : 0;
  const int n_keys = n_hist + a.Mk;
  const int nkt = (n_keys + kAttnKT - 1) / kAttnKT;
  const int t_first = (int)((int64_t)split * nkt / ns);
  const int ntiles = (int)((int64_t)(split + 1) * nkt / ns) - t_first;

  const bf16* kbase = static_cast<const bf16*>(a.k) + (int64_t)krow * a.kv_bstride + h * kAttnHD;
  const bf16* vbase = static_cast<const bf16*>(a.v) + (int64_t)krow * a.kv_bstride + h * kAttnHD;
  const bf16 *pkbase = nullptr, *pvbase = nullptr;
  if (HIST) {
    const int prow = __builtin_amdgcn_readfirstlane(a.pool_rows ? clamp_row((int)a.pool_rows[b], a.pool_batch)
                                                                : clamp_row(b, a.pool_batch));
    pkbase = static_cast<const bf16*>(a.pool_k) + (int64_t)prow * a.pool_bstride + h * kAttnHD;
    pvbase = static_cast<const bf16*>(a.pool_v) + (int64_t)prow * a.pool_bstride + h * kAttnHD;
  }
  const uint32_t kv_bytes = (uint32_t)(((int64_t)(a.Mk - 1) * a.kv_rstride + kAttnHD) * 2);
  // bytes per pool row (the host only picks this kernel when it fits 32 bits)
  const uint32_t pool_row_bytes = (uint32_t)a.pool_rstride * 2u;
  const i32x4 rk = make_rsrc4(kbase, kv_bytes), rv = make_rsrc4(vbase, kv_bytes);
  // History in consecutive slots (kv_layout's info[2] = its first slot):
  // slot = base + key index, so no slot list is copied or read.
  const int hbase = HIST && a.hist_base_dev ? __builtin_amdgcn_readfirstlane(*a.hist_base_dev) : -1;
  const bf16* qbase = static_cast<const bf16*>(a.q) + (int64_t)b * a.q_bstride + h * kAttnHD;
  const __amdgpu_buffer_rsrc_t rq =
      make_rsrc(qbase, (uint32_t)(((int64_t)(a.Mq - 1) * a.q_rstride + kAttnHD) * 2));

  const int qi = qt * QT + wave * 32 + l32;
  const bool q_ok = qi < a.Mq;
  bf16x8 qf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks)
    qf[ks] = __builtin_bit_cast(
        bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, (qi * (int)a.q_rstride + 16 * ks + 8 * half) * 2, 0, 0));

  // Direct-to-LDS loads of a tile: 32 one-KB sub-blocks (K blocks 0-15, then
  // V blocks 0-15, 4 keys each); wave w takes sub-blocks w, w + NW, ... (4
  // per wave with 8 waves; 5 for waves 0-3 and 4 for waves 4-6 with 7).
  // Lane L takes key row 4 blk + L/16 of its block, physical chunk L % 16,
  // and fetches the logical chunk the swizzle puts there: (row & 15) =
  // 4 (blk & 3) + L/16 for K, (row & 3) = L/16 for V.  Keys past the end read
  // own key Mk - 1 (finite values; their probabilities are zero).  Own keys go
  // through buffer loads with 32-bit byte offsets (the host only picks this
  // kernel when they fit); a block of pool keys loads from the pool row base
  // in SGPRs plus slot * row bytes in 32 bits, with the slots of its rows
  // read from the stage's slot list in LDS (load_slots, one step ahead), or
  // formed as base + key index when the history is consecutive slots.  Per
  // tile and wave, against 64-bit per-lane addresses: 22 -> 14 spilled SGPRs
  // (to VGPR lanes); C4a 234.6 -> 232.9 us, verify layer 2647 -> 2641 us.
  constexpr int kSub = (32 + NW - 1) / NW;  // sub-block slots per wave
  const int nsub = (32 - wave + NW - 1) / NW;
  const int lr = lane >> 4, pch = lane & 15;
  // Slot list of the tile bound for stage st_bytes (64 ints).
  auto slot_list = [&](int st_bytes) { return lds + NST * kAttnStage + (st_bytes >> 15) * (kAttnKT * 4); };
  static_assert(kAttnStage == 1 << 15, "stage index is st_bytes >> 15");
  // The last wave (one of those with the fewest sub-blocks) copies the 64
  // slots of tile T into the list of its stage: lane L slot T*64 + L.
  auto load_slots = [&](int T, int st_bytes) {
    if (HIST && hbase < 0 && wave == NW - 1 && T * kAttnKT < n_hist) {
      const int* src = slots + min(T * kAttnKT + lane, n_hist - 1);
      asm_g_ld4_lds((uint64_t)(uintptr_t)src, slot_list(st_bytes));
    }
  };
  auto issue = [&](int T, int st_bytes) {
    char* sb = lds + st_bytes;
#pragma unroll
    for (int i = 0; i < kSub; ++i) {
      const int sbk = wave + NW * i;
      if (sbk >= 32) break;
      const bool isk = sbk < 16;
      const int blk = sbk & 15;
      const int j0 = T * kAttnKT + 4 * blk;
      const int lc = (isk ? (pch ^ (4 * (blk & 3) + lr)) : (pch ^ (lr << 2))) << 4;
      char* dst = sb + (isk ? 0 : kAttnTile) + blk * 1024;
      if (!HIST || j0 >= n_hist) {
        const int row = min(j0 + lr - n_hist, a.Mk - 1) * (int)a.kv_rstride * 2;
        asm_ld16_lds(isk ? rk : rv, dst, row + lc);
      } else if (j0 + 4 <= n_hist) {
        // four pool keys: pool row base (SGPRs) + slot * row bytes (32-bit;
        // the host only picks this kernel when a pool row block fits)
        const int j = j0 + lr;
        const int slot = hbase >= 0 ? hbase + j
                                    : *reinterpret_cast<const int*>(slot_list(st_bytes) + (4 * blk + lr) * 4);
        asm_gs_ld16_lds(isk ? pkbase : pvbase, (uint32_t)slot * pool_row_bytes + (uint32_t)lc, dst);
      } else {
        // the block that holds the last pool keys and the first own keys:
        // two loads under complementary lane masks (one more load in this
        // tile; the per-tile waits then wait for it too, never too little)
        const int j = j0 + lr;
        if (j < n_hist) {
          const int slot = hbase >= 0 ? hbase + j
                                      : *reinterpret_cast<const int*>(slot_list(st_bytes) + (4 * blk + lr) * 4);
          asm_gs_ld16_lds(isk ? pkbase : pvbase, (uint32_t)slot * pool_row_bytes + (uint32_t)lc, dst);
        } else {
          asm_ld16_lds(isk ? rk : rv, dst, min(j - n_hist, a.Mk - 1) * (int)a.kv_rstride * 2 + lc);
        }
      }
    }
  };
  // Wait until at most one tile's loads of this wave are in flight.
  auto wait_all_but_one_tile = [&]() {
    if (NW == 8 || nsub == 4) __builtin_amdgcn_s_waitcnt(4 | (7 << 4) | (15 << 8));
    else __builtin_amdgcn_s_waitcnt(5 | (7 << 4) | (15 << 8));
  };

  // Softmax scale in log2 units; with q_ssq, times the query's 1/rms (set in
  // the prologue).  The query's partial sums of squares go straight to LDS
  // ahead of the first tile (slot i of a wave: partial 2 i in lanes 0-31 and
  // 2 i + 1 in lanes 32-63), so the tile waits cover them and no register
  // load wait is placed by the compiler; read back after the first barrier.
  float sc = a.scale * kLog2e;
  char* const qp_lds = lds + kQpOff + wave * (kQpSlots * 256);
  auto q_lds_load = [&]() {
    const float* prow = a.q_ssq + ((int64_t)b * a.Mq + min(qi, a.Mq - 1)) * a.q_ssq_n;
    const int slots_used = (a.q_ssq_n + 1) >> 1;
    for (int i = 0; i < slots_used; ++i)
      asm_g_ld4_lds((uint64_t)(uintptr_t)(prow + min(2 * i + half, a.q_ssq_n - 1)), qp_lds + i * 256);
  };
  auto q_lds_factor = [&]() {
    float sum = 0.f;
    for (int t = 0; t < a.q_ssq_n; ++t)
      sum += *reinterpret_cast<const float*>(qp_lds + (t >> 1) * 256 + 4 * (l32 + 32 * (t & 1)));
    return rsqrtf(sum / (float)a.q_norm_dim + a.q_eps);
  };
  const int tr_i = lane & 15, tr_gh = (lane >> 4) & 1;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  f32x16 s0[2], s1[2];
  bf16x8 pb[4];

  // Per-lane LDS offsets inside a stage, computed once.  K fragment (kt, ks):
  // key kt*32 + l32, chunk 2 ks + half under the (key & 15) swizzle, i.e.
  // l32*256 + ((2 ks + half) ^ (l32 & 15)) * 16 + 8192 kt.  Bits 5-7 of that
  // offset are 32 (ks ^ ((l32 & 15) >> 1)) and no other term touches them, so
  // it is kofs0 ^ (32 ks) with kofs0 the ks = 0 offset (and a stage base,
  // a multiple of 32 KB, adds without touching them either).  Transposed V
  // fragment (dt, ks), part pt: key 16 ks + 4 half + 8 pt + (lane % 16) / 4,
  // d = 32 dt + 16 ((lane / 16) % 2) + 4 (lane % 4); with the V swizzle that
  // is vlane + 64 (dt ^ xs) + 4096 ks + 2048 pt, where 64 (dt ^ xs) alone sets
  // bits 6-7: vofs0 ^ (64 dt).  Two registers instead of twelve.
  const int kofs0 = l32 * 256 + ((half ^ (l32 & 15)) << 4);
  int vofs0;
  {
    const int xs = tr_i >> 2, low = 2 * tr_gh + ((tr_i & 3) >> 1);
    vofs0 = kAttnTile + (4 * half + xs) * 256 + (low << 4) + 8 * (tr_i & 1) + 64 * xs;
  }
  // S = K Q^T for one tile: K fragments are read two k-steps ahead of their
  // MFMAs (three rotating sets), so each read has two steps to land.
  // Stage byte offsets are wave-uniform values kept in scalar registers, so
  // that each fragment address is one xor of the stage's first fragment
  // address plus a constant in the instruction's offset field.
  // The fragment addresses of a stage are formed first, made opaque and
  // fenced off from what follows, so that the scheduling groups of the MFMA
  // block below only see the loads, the MFMAs and the softmax.
  auto s_mfma = [&](int st_bytes, f32x16 (&s)[2]) {
    const int sb = __builtin_amdgcn_readfirstlane(st_bytes);
    const int kb = sb + kofs0;
    int ka[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      ka[ks] = kb ^ (32 * ks);
      asm volatile("" : "+v"(ka[ks]));
    }
    __builtin_amdgcn_sched_barrier(0);
    s[0] = f32x16{};
    s[1] = f32x16{};
    bf16x8 kf[3][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) kf[ks][kt] = ld_bf16x8(lds + ka[ks] + 8192 * kt);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      if (ks + 2 < 8) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) kf[(ks + 2) % 3][kt] = ld_bf16x8(lds + ka[ks + 2] + 8192 * kt);
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks % 3][kt], qf[ks], s[kt], 0, 0, 0);
    }
  };
  // O += V^T P for one tile: transposed V fragments two MFMAs ahead.
  auto pv_mfma = [&](int st_bytes) {
    const int sb = __builtin_amdgcn_readfirstlane(st_bytes);
    const int vb = sb + vofs0;
    int va4[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      va4[dt] = vb ^ (64 * dt);
      asm volatile("" : "+v"(va4[dt]));
    }
    __builtin_amdgcn_sched_barrier(0);
    auto vload = [&](int i) {
      const int ks = i >> 2, dt = i & 3;
      bf16x8 va;
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) {
        const bf16x4 t4 = ld_tr16(lds + va4[dt] + 4096 * ks + 2048 * pt);
        va[4 * pt + 0] = t4[0]; va[4 * pt + 1] = t4[1];
        va[4 * pt + 2] = t4[2]; va[4 * pt + 3] = t4[3];
      }
      return va;
    };
    bf16x8 vf[3];
    vf[0] = vload(0);
    vf[1] = vload(1);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i + 2 < 16) vf[(i + 2) % 3] = vload(i + 2);
      o[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[i % 3], pb[i >> 2], o[i & 3], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + 2 < 16) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };
  // Softmax of tile T, without branches so that it can run between the
  // MFMAs of the next tile: maxima with the NaN-propagating maximum (MFMA
  // results need no quieting), a lazy running max (log2 units; it only moves
  // where a tile's max exceeds it by more than 8), probabilities packed to
  // bf16 and summed from the packed values (dot2 with ones), so the sum is
  // that of the weights O accumulates.  MASK: the tile may hold keys past Mk
  // (only the last tile of the key set).  Returns whether the max moved in
  // any lane; alpha is the factor O must then be scaled by (1 elsewhere).
  auto softmax = [&](f32x16 (&s)[2], int T, auto mask_tag, float& alpha) -> bool {
    if constexpr (decltype(mask_tag)::value) {
      const int valid = n_keys - T * kAttnKT;
      // key kt*32 + 8 (v / 4) + 4 half + v % 4 is past the end: compare the
      // compile-time part against one per-lane threshold
      const int thr = valid - 4 * half;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (kt * 32 + 8 * (v >> 2) + (v & 3) >= thr) s[kt][v] = -INFINITY;
    }
    // The tile max of a lane's 32 scores as a tree of three-input maxima
    // (16 v_maximum3: ten over triples, then the partial maxima), written
    // so; pairs of two-input maxima came out as v_maximum3 with a repeated
    // operand (27 per tile).
    auto mx3 = [](float a, float b, float c) {
      return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
    };
    float t[11];
#pragma unroll
    for (int i = 0; i < 10; ++i) {
      const int k0 = 3 * i, k1 = 3 * i + 1, k2 = 3 * i + 2;
      t[i] = mx3(s[k0 >> 4][k0 & 15], s[k1 >> 4][k1 & 15], s[k2 >> 4][k2 & 15]);
    }
    t[10] = __builtin_elementwise_maximum(s[1][14], s[1][15]);
    const float u0 = mx3(t[0], t[1], t[2]), u1 = mx3(t[3], t[4], t[5]), u2 = mx3(t[6], t[7], t[8]);
    const float mx = mx3(mx3(u0, u1, u2), t[9], t[10]);
    const float mt = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 32, 64)) * sc;
    const bool grow = mt > m_run + 8.0f;
    const float m_new = grow ? mt : m_run;
    alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kt][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][v], sc, -m_run));
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int u = 0; u < 8; ++u) pb[ks][u] = static_cast<bf16>(s[ks >> 1][(ks & 1) * 8 + u]);
    const bf16x2 ones = {static_cast<bf16>(1.0f), static_cast<bf16>(1.0f)};
    float ps[2] = {0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x2 w0 = __builtin_bit_cast(u32x2, __builtin_shufflevector(pb[ks], pb[ks], 0, 1, 2, 3)),
                  w1 = __builtin_bit_cast(u32x2, __builtin_shufflevector(pb[ks], pb[ks], 4, 5, 6, 7));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ps[j & 1] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, j < 2 ? w0[j] : w1[j - 2]), ones,
                                                    ps[j & 1], false);
    }
    l_run = __builtin_fmaf(l_run, alpha, ps[0] + ps[1]);
    return __builtin_amdgcn_ballot_w64(grow) != 0;
  };
  // The 16 MFMAs of S(t+1) with its K reads (one per MFMA, 12 after the
  // first 4 issued up front) and the softmax of S(t) between them: the max
  // reduction under the first four, then exponentials (transcendental group)
  // and the other VALU work under the rest.  Up to 8 VALU instructions per
  // MFMA (so the softmax ends earlier in the block; 6 per MFMA measured 1%
  // slower on 4680 x 4680, 7 to 12 the same as 8).
  auto interleave = [&]() {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      if (q < 12) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      if (q < 4) {
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // VALU
      } else {
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x400, 3, 0);  // transcendental
      }
    }
  };

  // A wave whose 32 queries all lie past Mq (in the partial last query tile
  // of a row: 1560 = 6 x 256 + 24 leaves seven of its eight waves without
  // queries) computes nothing: it issues its share of every tile's loads and
  // the slot lists, and joins every barrier of the schedule below (one after
  // the slot lists, one in the prologue, one per step; with PP those of a
  // group B wave), then exits.
  const bool live = qt * QT + wave * 32 < a.Mq;  // wave-uniform
  if constexpr (PP) {
    const bool grpA = wave < 4;
    // this wave's loads landed, then the barrier
    auto bar = [&]() {
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    // K/V of tiles 0-2, then one barrier with tiles 0 and 1 landed
    auto prologue = [&]() {
      if (live && a.q_ssq) q_lds_load();
      issue(t_first, 0);
      if (ntiles > 1) issue(t_first + 1, kAttnStage);
      if (ntiles > 2) issue(t_first + 2, 2 * kAttnStage);
      if (ntiles > 2) wait_all_but_one_tile();
      else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    // right after barrier t: tile t+3 into the stage of tile t-1 (st3),
    // landed by the issuing wave's next barrier
    auto issue_next = [&](int t, int st3) {
      if (t + 3 < ntiles) issue(t_first + t + 3, st3);
    };
    if (!live) {
      // the barriers of a group B wave: the prologue's, barrier 0, one per tile
      if (ntiles > 0) {
        prologue();
        bar();
        int st3 = 3 * kAttnStage;
        for (int t = 0; t < ntiles; ++t) {
          issue_next(t, st3);
          bar();
          st3 = st3 == 3 * kAttnStage ? 0 : st3 + kAttnStage;
        }
      }
      return;
    }
    if (ntiles > 0) {
      prologue();
      s_mfma(0, s0);
      if (a.q_ssq) {
        // the partials landed with tile 0 (issued before it); read after the barrier
        asm volatile("" ::: "memory");
        sc *= q_lds_factor();
      }
      if (!grpA) bar();  // B runs one barrier behind A
      // stages of tiles t, t+1, t+2 and t+3 (= t-1), rotated each tile
      int st0 = 0, st1 = kAttnStage, st2 = 2 * kAttnStage, st3 = 3 * kAttnStage;
      auto pstep = [&](int t, f32x16 (&scur)[2], f32x16 (&snxt)[2], auto mask_tag) {
        const bool has_next = t + 1 < ntiles;
        if (!grpA) issue_next(t, st3);
        float alpha;
        s_mfma(has_next ? st1 : st0, snxt);
        const bool moved = softmax(scur, t_first + t, mask_tag, alpha);
        interleave();
        asm volatile("" ::"v"(pb[0]), "v"(pb[1]), "v"(pb[2]), "v"(pb[3]));
        __builtin_amdgcn_sched_barrier(0);
        if (moved) {
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
        }
        __builtin_amdgcn_sched_barrier(0);
        if (grpA) {
          bar();
          issue_next(t, st3);
        }
        pv_mfma(st0);
        __builtin_amdgcn_sched_barrier(0);
        if (!grpA) bar();
        const int st_done = st0;
        st0 = st1;
        st1 = st2;
        st2 = st3;
        st3 = st_done;
      };
      const std::integral_constant<bool, false> full;
      const std::integral_constant<bool, true> last;
      const int nm = ntiles - 1;  // tiles before the last one hold no key past the end
      int t = 0;
      for (; t + 1 < nm; t += 2) {
        pstep(t, s0, s1, full);
        pstep(t + 1, s1, s0, full);
      }
      if (t < nm) {
        pstep(t, s0, s1, full);
        pstep(t + 1, s1, s0, last);
      } else {
        pstep(t, s0, s1, last);
      }
      if (grpA) __builtin_amdgcn_s_barrier();  // B's last barrier
    }
  } else {
    if (!live) {
      if (ntiles > 0) {
        if (HIST) {
          load_slots(t_first, 0);
          if (ntiles > 1) load_slots(t_first + 1, kAttnStage);
          if (ntiles > 2) load_slots(t_first + 2, 2 * kAttnStage);
          __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
          __builtin_amdgcn_s_barrier();
          asm volatile("" ::: "memory");
        }
        issue(t_first, 0);
        if (ntiles > 1) issue(t_first + 1, kAttnStage);
        if (ntiles > 1) wait_all_but_one_tile();
        else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
        __builtin_amdgcn_s_barrier();
        int st0 = 0, st1 = kAttnStage, st2 = 2 * kAttnStage;
        for (int t = 0; t < ntiles; ++t) {
          const int T = t_first + t;
          if (t + 1 < ntiles) __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
          __builtin_amdgcn_s_barrier();
          if (HIST) asm volatile("" ::: "memory");
          if (t + 2 < ntiles) issue(T + 2, st2);
          if (t + 3 < ntiles) load_slots(T + 3, st0);
          const int st_done = st0;
          st0 = st1;
          st1 = st2;
          st2 = st_done;
        }
      }
      return;
    }

    if (ntiles > 0) {
      // Three stages in rotation.  Prologue: tiles 0 and 1 in flight, S(0) once
      // tile 0 has landed.
      if (HIST) {
        // slot lists of the first three tiles, visible to every wave
        load_slots(t_first, 0);
        if (ntiles > 1) load_slots(t_first + 1, kAttnStage);
        if (ntiles > 2) load_slots(t_first + 2, 2 * kAttnStage);
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      if (a.q_ssq) q_lds_load();
      issue(t_first, 0);
      if (ntiles > 1) issue(t_first + 1, kAttnStage);
      if (ntiles > 1) wait_all_but_one_tile();
      else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
      __builtin_amdgcn_s_barrier();
      s_mfma(0, s0);
      if (a.q_ssq) {
        // the partials landed with tile 0 (issued before it); read after the barrier
        asm volatile("" ::: "memory");
        sc *= q_lds_factor();
      }
      // Stages of tiles t, t+1 and t+2, rotated each step (scalar values; an
      // expression in t would become per-lane induction variables).
      int st0 = 0, st1 = kAttnStage, st2 = 2 * kAttnStage;
      // One step: tile t's softmax under S(t+1) (the last tile's successor is
      // itself again, computed and discarded), O rescaled where the max moved,
      // then O += V_t P(t).  Only the last tile is masked.
      auto step = [&](int t, f32x16 (&scur)[2], f32x16 (&snxt)[2], auto mask_tag) {
        const int T = t_first + t;
        const bool has_next = t + 1 < ntiles;
        // tile t+1 (and the slot list of t+2) has landed and every wave is
        // done with the stage of t-1 (and with the slot list of t, read two
        // steps ago)
        if (has_next) __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
        __builtin_amdgcn_s_barrier();
        if (HIST) asm volatile("" ::: "memory");  // slot reads stay below the barrier
        if (t + 2 < ntiles) issue(T + 2, st2);
        if (t + 3 < ntiles) load_slots(T + 3, st0);
        float alpha;
        s_mfma(has_next ? st1 : st0, snxt);
        const bool moved = softmax(scur, T, mask_tag, alpha);
        interleave();
        // P(t) is complete here, before the branch below (keeps the
        // exponentials in this block, between the MFMAs of S(t+1)).
        asm volatile("" ::"v"(pb[0]), "v"(pb[1]), "v"(pb[2]), "v"(pb[3]));
        __builtin_amdgcn_sched_barrier(0);
        if (moved) {
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
        }
        pv_mfma(st0);
        __builtin_amdgcn_sched_barrier(0);
        const int st_done = st0;
        st0 = st1;
        st1 = st2;
        st2 = st_done;
      };
      const std::integral_constant<bool, false> full;
      const std::integral_constant<bool, true> last;
      const int nm = ntiles - 1;  // tiles before the last one hold no key past the end
      int t = 0;
      for (; t + 1 < nm; t += 2) {
        step(t, s0, s1, full);
        step(t + 1, s1, s0, full);
      }
      if (t < nm) {
        step(t, s0, s1, full);
        step(t + 1, s1, s0, last);
      } else {
        step(t, s0, s1, last);
      }
    }
  }

  const float l = l_run + __shfl_xor(l_run, 32, 64);
  if (ns > 1) {
    if (q_ok) {
      const int64_t row = ((int64_t)split * n_tail + (unit - n_full)) * QT + wave * 32 + l32;
      float* op = part + row * kAttnHD;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4*>(op + dt * 32 + 8 * g + 4 * half) =
              make_float4(o[dt][4 * g], o[dt][4 * g + 1], o[dt][4 * g + 2], o[dt][4 * g + 3]);
      if (half == 0) {
        float* ml = part + (int64_t)n_split * n_tail * QT * kAttnHD + row * 2;
        *reinterpret_cast<float2*>(ml) = make_float2(m_run, l);
      }
    }
    return;
  }
  const float inv = 1.f / l;
  if (q_ok) {
    bf16* op = static_cast<bf16*>(a.o) + (int64_t)b * a.o_bstride + (int64_t)qi * a.o_rstride + h * kAttnHD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 t4;
#pragma unroll
        for (int e = 0; e < 4; ++e) t4[e] = static_cast<bf16>(o[dt][4 * g + e] * inv);
        *reinterpret_cast<bf16x4*>(op + dt * 32 + 8 * g + 4 * half) = t4;
      }
  }
}

// Merge the n_split partial results of each query row of the split units:
// O = sum_i 2^(m_i - m) O_i / sum_i 2^(m_i - m) l_i with m = max_i m_i.  One
// wave per (split unit, query) row, two of the 128 outputs per lane; every
// range's loads are issued before any of them is used.
// QT: query rows per unit (256, or 224 for the 7-wave pipelined kernel).
constexpr int kAttnMaxSplit = 8;
__global__ __launch_bounds__(256) void attention_combine_kernel(wam_attention_args a, int n_full, int n_split,
                                                                int QT, const float* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int nqt = (a.Mq + QT - 1) / QT;
  const int n_tail = nqt * a.H * a.B - n_full;
  const int64_t rows = (int64_t)n_tail * QT;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int unit = n_full + (int)(row / QT), qq = (int)(row % QT);
  const int qt = unit % nqt, bh = unit / nqt;
  const int qi = qt * QT + qq;
  if (qi >= a.Mq) return;
  const int b = bh % a.B, h = bh / a.B;  // head-major: the batch rows of one head are adjacent
  const float* ml = part + (int64_t)n_split * rows * kAttnHD;
  float2 mlv[kAttnMaxSplit], ov[kAttnMaxSplit];
#pragma unroll
  for (int i = 0; i < kAttnMaxSplit; ++i) {
    mlv[i] = make_float2(-INFINITY, 0.f);
    ov[i] = make_float2(0.f, 0.f);
    if (i < n_split) {
      mlv[i] = *reinterpret_cast<const float2*>(ml + ((int64_t)i * rows + row) * 2);
      ov[i] = *reinterpret_cast<const float2*>(part + ((int64_t)i * rows + row) * kAttnHD + 2 * lane);
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kAttnMaxSplit; ++i) m = fmaxf(m, mlv[i].x);
  float den = 0.f, n0 = 0.f, n1 = 0.f;
#pragma unroll
  for (int i = 0; i < kAttnMaxSplit; ++i) {
    const float w = mlv[i].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mlv[i].x - m);
    den += w * mlv[i].y;
    n0 += w * ov[i].x;
    n1 += w * ov[i].y;
  }
  bf16* op = static_cast<bf16*>(a.o) + (int64_t)b * a.o_bstride + (int64_t)qi * a.o_rstride + h * kAttnHD;
  const float inv = 1.f / den;
  bf16x2 r;
  r[0] = static_cast<bf16>(n0 * inv);
  r[1] = static_cast<bf16>(n1 * inv);
  *reinterpret_cast<bf16x2*>(op + 2 * lane) = r;
}

// Launch plan of the split path: the first n_full units (of QT query rows)
// run whole, the other n_tail units are split into n_split key ranges each.
// Cost model, in units of one whole unit's run time on one CU (kt key tiles of
// 64 keys), for C CUs (256 on MI355X) taking workgroups in dispatch order:
//   n_full / C  +  ceil(pieces / C) * (1 / n_split + kFill / kt)
//                 +  pieces * kCombine / kt,         pieces = n_tail * n_split
// kFill: key tiles' worth of pipeline fill and partial-result store per
// piece; kCombine: the combine's time per piece (a 133 KB fp32 partial at
// about 4 TB/s, ~33 ns) in key-tile times (~2.5 us per tile and CU).  The plan
// with the lowest cost whose partials fit in max_bytes wins; no split when
// none beats the whole-unit grid.  E.g. 4 x 1560 queries over 7800 keys (672
// units, kt 122): 512 whole + 160 units in 3 ranges, 2.74 vs 3 rounds.
// Key tiles from which the pipelined kernel runs its ping-pong schedule (8
// tiles, cross attention over 512 keys, measured 1-3% slower with it).
constexpr int64_t kAttnPPMinTiles = 16;

struct AttnPlan {
  int n_full, n_split, n_tail, qt;
  double cost;  // in whole-unit times of this plan's units
};

static int64_t plan_bytes(const AttnPlan& p) {
  return p.n_split > 1 ? (int64_t)p.n_split * p.n_tail * p.qt * (kAttnHD + 2) * 4 : 0;
}

static AttnPlan attention_plan(int B, int Mq, int H, int64_t keys, int64_t max_bytes, int QT) {
  const int cus = device_cu_count();
  constexpr double kFill = 1.5, kCombine = 0.0133;
  const int64_t units = (int64_t)((Mq + QT - 1) / QT) * H * B;
  const int64_t piece_bytes = (int64_t)QT * (kAttnHD + 2) * 4;
  AttnPlan best{(int)units, 1, 0, QT, (double)((units + cus - 1) / cus)};
  if (units <= 0 || units >= (1 << 26)) return best;
  const double kt = (double)((keys > 0 ? keys : 1) + kAttnKT - 1) / kAttnKT;
  for (int64_t F = 0; F < units; F += cus) {
    const int64_t T = units - F;
    for (int ns = 2; ns <= kAttnMaxSplit; ++ns) {
      const int64_t pieces = T * ns;
      if (pieces * piece_bytes > max_bytes) break;
      const double cost = (double)F / cus +
                          (double)((pieces + cus - 1) / cus) * (1.0 / ns + kFill / kt) +
                          (double)pieces * kCombine / kt;
      if (cost < best.cost - 1e-9) best = AttnPlan{(int)F, ns, (int)T, QT, cost};
    }
  }
  return best;
}

// Selects the software-pipelined kernel (a switch for side-by-side
// measurement; always on in the library).
static bool g_attn_w4 = true;

// The pipelined kernel runs when every Q and own K/V row's byte offset fits in
// 31 bits, the pool rows of one batch row (slots < pool_bstride /
// pool_rstride) in 32 bits, and the query grid is at least 128 units of 256
// rows; smaller grids use attention_kernel<4>.
static bool sp_eligible(const wam_attention_args* a) {
  const int64_t grid8 = (int64_t)((a->Mq + 255) / 256) * a->H * a->B;
  return g_attn_w4 && grid8 >= 128 && ((int64_t)a->Mq + 256) * a->q_rstride * 2 < (int64_t)INT32_MAX &&
         ((int64_t)a->Mk + kAttnKT) * a->kv_rstride * 2 < (int64_t)INT32_MAX &&
         (!a->n_hist_dev || (a->pool_bstride >= a->pool_rstride && a->pool_bstride * 2 < (int64_t)UINT32_MAX));
}

// Query rows per unit of the pipelined kernel: 224 (7 waves) when its plan
// costs no more unit-times than the 256-row plan.  A 224-row unit takes about
// as long as a 256-row one (the SIMDs that hold two of its waves set the
// pace) but reads less from LDS per CU: at equal rounds it measured 1-2%
// faster (4680 x 4680, 24 heads: 504 units of 224 or 456 of 256, both two
// rounds of 256 CUs).  Both plans are priced with unlimited workspace so that
// the choice does not depend on the workspace a caller passes.
static int sp_query_tile(int B, int Mq, int H, int64_t keys) {
  const AttnPlan p256 = attention_plan(B, Mq, H, keys, INT64_MAX, 256);
  const AttnPlan p224 = attention_plan(B, Mq, H, keys, INT64_MAX, 224);
  return p224.cost <= p256.cost + 1e-9 ? 224 : 256;
}

// Calls with pool keys keep 256-query units: the pool path leaves the 7-wave
// kernel short of registers (with 32-bit pool offsets it still spills 14
// VGPRs to scratch), and a 224-query unit takes as long as a 256-query one on
// the SIMDs that hold two of its waves.
static int query_tile(const wam_attention_args* a, int64_t keys) {
  return sp_eligible(a) && a->n_hist_dev == nullptr ? sp_query_tile(a->B, a->Mq, a->H, keys) : 256;
}

int64_t attention_workspace_bytes(int B, int Mq, int H, int64_t max_keys) {
  // enough for either query tile (the call's strides, unknown here, decide)
  return std::max(plan_bytes(attention_plan(B, Mq, H, max_keys, INT64_MAX, 256)),
                  plan_bytes(attention_plan(B, Mq, H, max_keys, INT64_MAX, sp_query_tile(B, Mq, H, max_keys))));
}

int attention(const wam_attention_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr, "wam_attention: null args");
  WAM_REQUIRE(a->head_dim == kAttnHD, "wam_attention: head_dim must be 128 (got %d)", a->head_dim);
  WAM_REQUIRE(a->B >= 1 && a->H >= 1 && a->Mq >= 0 && a->Mk >= 1,
              "wam_attention: bad shape B=%d H=%d Mq=%d Mk=%d", a->B, a->H, a->Mq, a->Mk);
  WAM_REQUIRE(a->q && a->o && a->k && a->v, "wam_attention: null q/o/k/v");
  WAM_REQUIRE(a->q_rstride % 8 == 0 && a->o_rstride % 4 == 0 && a->kv_rstride % 8 == 0 &&
              a->q_bstride % 8 == 0 && a->kv_bstride % 8 == 0,
              "wam_attention: strides must keep 16-byte alignment");
  WAM_REQUIRE(a->kv_batch >= 1, "wam_attention: kv_batch must be >= 1");
  if (a->n_hist_dev) {
    WAM_REQUIRE(a->pool_k && a->pool_v && a->slots && a->pool_batch >= 1 &&
                a->pool_rstride % 8 == 0 && a->pool_bstride % 8 == 0,
                "wam_attention: history needs pool k/v, slots and pool_batch");
  }
  // Without a row map, batch row b reads pool/own row b, or row 0 when that
  // source has a single row (broadcast).
  if (!a->pool_rows && a->n_hist_dev)
    WAM_REQUIRE(a->B <= a->pool_batch || a->pool_batch == 1,
                "wam_attention: B=%d exceeds pool batch %d", a->B, a->pool_batch);
  if (!a->kv_rows)
    WAM_REQUIRE(a->B <= a->kv_batch || a->kv_batch == 1,
                "wam_attention: B=%d exceeds kv batch %d", a->B, a->kv_batch);
  WAM_REQUIRE(a->max_keys >= 0, "wam_attention: max_keys must be >= 0");
  WAM_REQUIRE(!a->q_ssq || (a->q_ssq_n >= 1 && a->q_ssq_n <= kQssqMax && a->q_norm_dim >= 1),
              "wam_attention: q_ssq needs 1..%d partials per row and q_norm_dim >= 1 (got %d, %d)", kQssqMax,
              a->q_ssq_n, a->q_norm_dim);
  if (a->Mq == 0) return WAM_OK;
  // 8 or 7 waves (256 or 224 queries) per workgroup, with the last dispatch
  // round split by key ranges when the plan says so and the caller gave a
  // workspace for the partial results; small grids use 4-wave workgroups.
  const int64_t grid8 = (int64_t)((a->Mq + 255) / 256) * a->H * a->B;
  WAM_REQUIRE(grid8 < (1 << 26), "wam_attention: grid too large");
  const int64_t keys = a->max_keys > 0 ? a->max_keys : a->Mk;
  const bool sp = sp_eligible(a);
  const int QT = query_tile(a, keys);
  const AttnPlan p = attention_plan(a->B, a->Mq, a->H, keys, a->workspace ? a->workspace_bytes : 0, QT);
  const bool hist = a->n_hist_dev != nullptr;
  // the ping-pong schedule for own keys only, in units of at least
  // kAttnPPMinTiles key tiles
  const bool pp = (keys + kAttnKT - 1) / kAttnKT >= kAttnPPMinTiles;
  auto sp_kernel = QT == 224 ? (pp ? attention_sp_kernel<false, 7, true>  // (never with pool keys)
                                   : attention_sp_kernel<false, 7, false>)
                   : hist    ? attention_sp_kernel<true, 8, false>
                             : (pp ? attention_sp_kernel<false, 8, true> : attention_sp_kernel<false, 8, false>);
  const dim3 sp_block(64 * (QT / 32));
  if (p.n_split > 1) {
    float* part = static_cast<float*>(a->workspace);
    const int64_t grid = (int64_t)p.n_full + (int64_t)p.n_tail * p.n_split;
    if (sp)
      hipLaunchKernelGGL(sp_kernel, dim3((unsigned)grid), sp_block, 0, s, *a, a->slots, p.n_full, p.n_split, part);
    else
      hipLaunchKernelGGL(attention_kernel<8>, dim3((unsigned)grid), dim3(512), 0, s, *a, a->slots, p.n_full,
                         p.n_split, part);
    WAM_LAUNCHED("attention_kernel");
    const int64_t rows = (int64_t)p.n_tail * QT;
    hipLaunchKernelGGL(attention_combine_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, *a,
                       p.n_full, p.n_split, QT, static_cast<const float*>(part));
    WAM_LAUNCHED("attention_combine_kernel");
    return WAM_OK;
  }
  if (sp) {
    const int64_t units = (int64_t)((a->Mq + QT - 1) / QT) * a->H * a->B;
    hipLaunchKernelGGL(sp_kernel, dim3((unsigned)units), sp_block, 0, s, *a, a->slots, (int)units, 1, nullptr);
  } else if (grid8 >= 256) {
    hipLaunchKernelGGL(attention_kernel<8>, dim3((unsigned)grid8), dim3(512), 0, s, *a, a->slots, (int)grid8, 1,
                       nullptr);
  } else {
    const int64_t grid4 = (int64_t)((a->Mq + 127) / 128) * a->H * a->B;
    hipLaunchKernelGGL(attention_kernel<4>, dim3((unsigned)grid4), dim3(256), 0, s, *a, a->slots, (int)grid4, 1,
                       nullptr);
  }
  WAM_LAUNCHED("attention_kernel");
  return WAM_OK;
}

// ------------------------------------------------------------ no allocation
// wam_attention for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops): the key-range split's partial
// results go to a file-scope device array instead of a caller workspace.
// Every GPU the library runs on holds its own copy of the array until the
// process ends; calls on one GPU share it, so calls that overlap on one GPU
// race.  Nothing in it needs clearing: every piece of a split writes its whole
// partial (an empty key range writes m = -inf, l = 0, O = 0) before the
// combine reads it.
constexpr int64_t kNoAllocScratchBytes = 64ll << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device with that device current.  The array's name is only a host-side
// stand-in: kernels get this address.
static int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  WAM_HIP(hipGetDevice(&dev));
  WAM_REQUIRE(dev >= 0 && dev < 64, "wam_attention_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    WAM_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    WAM_REQUIRE(p != nullptr, "wam_attention_noalloc: no address for the scratch array");
    addr[dev] = p;
  }
  *out = addr[dev];
  return WAM_OK;
}

int attention_noalloc(const wam_attention_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr, "wam_attention_noalloc: null args");
  WAM_REQUIRE(a->workspace == nullptr && a->workspace_bytes == 0,
              "wam_attention_noalloc: takes no workspace (the split uses the library's own scratch)");
  WAM_REQUIRE(a->B >= 1 && a->H >= 1 && a->Mq >= 0 && a->Mk >= 1 && a->max_keys >= 0,
              "wam_attention_noalloc: bad shape B=%d H=%d Mq=%d Mk=%d", a->B, a->H, a->Mq, a->Mk);
  // The split wam_attention would run with an unlimited workspace; shapes
  // whose partial results exceed the scratch are refused, not re-planned, so
  // that both entry points compute the same thing.
  const int64_t keys = a->max_keys > 0 ? a->max_keys : a->Mk;
  const int64_t need =
      a->Mq > 0 ? plan_bytes(attention_plan(a->B, a->Mq, a->H, keys, INT64_MAX, query_tile(a, keys))) : 0;
  WAM_REQUIRE(need <= kNoAllocScratchBytes,
              "wam_attention_noalloc: this shape's key-range split needs %lld bytes of scratch, more than "
              "the %lld-byte maximum; call wam_attention with a workspace instead",
              (long long)need, (long long)kNoAllocScratchBytes);
  wam_attention_args b = *a;
  if (need > 0) {
    void* p = nullptr;
    WAM_TRY(scratch_address(&p));
    b.workspace = p;
    b.workspace_bytes = need;
  }
  return attention(&b, s);
}

}  // namespace wam

extern "C" int wam_attention_noalloc(const wam_attention_args* args, void* stream) {
  return wam::attention_noalloc(args, static_cast<hipStream_t>(stream));
}

extern "C" int wam_attention(const wam_attention_args* args, void* stream) {
  return wam::attention(args, static_cast<hipStream_t>(stream));
}

extern "C" int64_t wam_attention_workspace_bytes(int B, int Mq, int H, int max_keys) {
  return wam::attention_workspace_bytes(B, Mq, H, max_keys);
}
