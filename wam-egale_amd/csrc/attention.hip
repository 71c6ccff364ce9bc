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
#include "wam_common.h"

namespace wam {

constexpr int kAttnHD = 128;
constexpr int kAttnWaves = 4;
constexpr int kAttnQTile = 32 * kAttnWaves;  // queries per workgroup
constexpr int kAttnKTile = 64;               // keys per LDS stage
constexpr int kAttnKBytes = kAttnKTile * kAttnHD * 2;
constexpr int kAttnStage = 2 * kAttnKBytes;  // K tile + V^T tile

// LDS bank layout: 64 banks x 4 bytes; ds_read_b128 serves 16 lanes per
// cycle, and an MFMA operand fetch reads 16 consecutive rows at one chunk.
// K tile: [64 keys][128 d], 256-byte rows (one bank line), chunk XOR key.
__device__ inline int k_off(int key, int c) { return key * 256 + ((c ^ (key & 15)) << 4); }
// V^T tile: [128 d][64 slots], 128-byte rows, two rows per bank line: chunk
// XOR (d / 2) so that 16 consecutive rows hit 16 distinct 16-byte slots.
__device__ inline int vt_off(int d, int c) { return d * 128 + ((c ^ ((d >> 1) & 7)) << 4); }

__global__ __launch_bounds__(256, 2) void attention_kernel(wam_attention_args a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kAttnStage];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, half = lane >> 5;

  const int nqt = (a.Mq + kAttnQTile - 1) / kAttnQTile;
  const int id = __builtin_amdgcn_readfirstlane(xcd_remap(blockIdx.x, gridDim.x));
  const int qt = id % nqt, bh = id / nqt;
  const int h = bh % a.H, b = bh / a.H;

  const int n_hist = a.n_hist_dev ? __builtin_amdgcn_readfirstlane(*a.n_hist_dev) : 0;
  const int n_tot = n_hist + a.Mk;
  int prow = a.pool_rows ? (int)a.pool_rows[b] : b;
  prow = prow < 0 ? 0 : (prow >= a.pool_batch ? a.pool_batch - 1 : prow);
  int krow = a.kv_rows ? (int)a.kv_rows[b] : b;
  krow = krow < 0 ? 0 : (krow >= a.kv_batch ? a.kv_batch - 1 : krow);
  prow = __builtin_amdgcn_readfirstlane(prow);
  krow = __builtin_amdgcn_readfirstlane(krow);

  const bf16* pool_k = a.pool_k ? static_cast<const bf16*>(a.pool_k) + (int64_t)prow * a.pool_bstride + h * kAttnHD : nullptr;
  const bf16* pool_v = a.pool_v ? static_cast<const bf16*>(a.pool_v) + (int64_t)prow * a.pool_bstride + h * kAttnHD : nullptr;
  const bf16* own_k = static_cast<const bf16*>(a.k) + (int64_t)krow * a.kv_bstride + h * kAttnHD;
  const bf16* own_v = static_cast<const bf16*>(a.v) + (int64_t)krow * a.kv_bstride + h * kAttnHD;

  // Q fragments (B operand of S^T): query qi, d = ks*16 + half*8 .. +8.
  const int qi = qt * kAttnQTile + wave * 32 + l32;
  const bool q_ok = qi < a.Mq;
  const bf16* qp = static_cast<const bf16*>(a.q) + (int64_t)b * a.q_bstride +
                   (int64_t)(q_ok ? qi : 0) * a.q_rstride + h * kAttnHD + half * 8;
  bf16x8 qf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    qf[ks] = ld_bf16x8(qp + ks * 16);
    if (!q_ok) qf[ks] = bf16x8{};
  }

  auto key_row = [&](const bf16* pool, const bf16* own, int j) -> const bf16* {
    j = j < n_tot ? j : n_tot - 1;
    return j < n_hist ? pool + (int64_t)a.slots[j] * a.pool_rstride
                      : own + (int64_t)(j - n_hist) * a.kv_rstride;
  };

  // Staging: K thread -> chunk (tid & 15) of keys (tid >> 4) + 16 i;
  //          V thread -> d-octet (tid >> 4) of keys 4 (tid & 15) + i.
  const int kc = tid & 15, kr = tid >> 4;
  const int vq = tid & 15, vd = tid >> 4;
  bf16x8 rk[4], rv[4];
  auto gload = [&](int t) {
    const int j0 = t * kAttnKTile;
#pragma unroll
    for (int i = 0; i < 4; ++i) rk[i] = ld_bf16x8(key_row(pool_k, own_k, j0 + kr + 16 * i) + kc * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) rv[i] = ld_bf16x8(key_row(pool_v, own_v, j0 + 4 * vq + i) + vd * 8);
  };
  // V^T slot of the key quad 4*vq..4*vq+3: 16-key group g = vq/4, and inside
  // the group quads 0,1,2,3 go to slots 0-3, 8-11, 4-7, 12-15.
  const int vgrp = vq >> 2, vqq = vq & 3;
  const int vchunk = 2 * vgrp + (vqq & 1), vbyte = (vqq >> 1) * 8;
  auto lstore = [&](int stage) {
    char* kb = smem + stage * kAttnStage;
    char* vb = kb + kAttnKBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) st_bf16x8(kb + k_off(kr + 16 * i, kc), rk[i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = vd * 8 + e;
      bf16x4 t;
      t[0] = rv[0][e]; t[1] = rv[1][e]; t[2] = rv[2][e]; t[3] = rv[3][e];
      *reinterpret_cast<bf16x4*>(vb + vt_off(d, vchunk) + vbyte) = t;
    }
  };

  const float c = a.scale * kLog2e;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};

  const int ntiles = (n_tot + kAttnKTile - 1) / kAttnKTile;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int cur = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    const char* kb = smem + cur * kAttnStage;
    const char* vb = kb + kAttnKBytes;

    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = f32x16{};
      const int key = kt * 32 + l32;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks)
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ld_bf16x8(kb + k_off(key, 2 * ks + half)),
                                                        qf[ks], s[kt], 0, 0, 0);
    }
    if ((t + 1) * kAttnKTile > n_tot) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int j = t * kAttnKTile + kt * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
          if (j >= n_tot) s[kt][v] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kt][v]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx * c);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float pv = __builtin_amdgcn_exp2f(s[kt][v] * c - m_new);
        s[kt][v] = pv;
        psum += pv;
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;

    bf16x8 pb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int u = 0; u < 8; ++u) pb[ks][u] = static_cast<bf16>(s[ks >> 1][(ks & 1) * 8 + u]);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int d = dt * 32 + l32;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ld_bf16x8(vb + vt_off(d, 2 * ks + half)),
                                                        pb[ks], o[dt], 0, 0, 0);
    }
    if (t + 1 < ntiles) lstore(cur ^ 1);
    __syncthreads();
  }

  const float l = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.f / l;
  if (q_ok) {
    bf16* op = static_cast<bf16*>(a.o) + (int64_t)b * a.o_bstride + (int64_t)qi * a.o_rstride + h * kAttnHD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 t;
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = static_cast<bf16>(o[dt][4 * g + e] * inv);
        *reinterpret_cast<bf16x4*>(op + dt * 32 + 8 * g + 4 * half) = t;
      }
  }
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
  if (a->Mq == 0) return WAM_OK;
  const int nqt = (a->Mq + kAttnQTile - 1) / kAttnQTile;
  const int64_t grid = (int64_t)nqt * a->H * a->B;
  WAM_REQUIRE(grid < (1 << 30), "wam_attention: grid too large");
  hipLaunchKernelGGL(attention_kernel, dim3((unsigned)grid), dim3(256), 0, s, *a);
  WAM_LAUNCHED("attention_kernel");
  return WAM_OK;
}

}  // namespace wam

extern "C" int wam_attention(const wam_attention_args* args, void* stream) {
  return wam::attention(args, static_cast<hipStream_t>(stream));
}
