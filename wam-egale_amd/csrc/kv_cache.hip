// Original-mode KV pool bookkeeping on the device (no host synchronisation).
//
// Pool state (model.py:417-434): k, v [B_cfg, P, H, hd] bf16, id [P] int64,
// mask [P] bool, is_pred [P] bool.  One call of the self-attention with a
// cache (model.py:662-686) does:
//   allocate_slots (model.py:547-566): if fewer than `tokens` slots are free,
//     evict the valid slots with the smallest ids (the reference sorts with
//     torch.argsort; ties are broken here by ascending slot, the order a
//     stable sort gives), then take the first `tokens` free slots;
//   update_cache (model.py:577-590): new id = max(valid id) + 1 (0 if none),
//     write K/V, mask = True, id = new id, is_pred = (update == 1);
//   attention over every valid slot in ascending slot order;
//   restore_cache for update == 0 (model.py:592-593, 683-685): mask = False.
// Candidate verification (model.py:624-660) is read only.
//
// This kernel does the index work of all of that; the K/V rows themselves are
// written by wam_kv_commit, and attention reads the history through
// hist_slots (the valid slots other than the new ones) plus the new rows
// straight from the projection output.  Softmax over a key set does not
// depend on key order, so [history || own] equals the reference's slot order
// up to fp32 summation order.  The native reference does the same work in
// layout_kernel / private_kernel / restore_kernel,
// 算子研究/wam_ops/baseline/csrc/block.cu:133-227.
#include "wam_common.h"

namespace wam {

constexpr int kLayoutThreads = 1024;
constexpr int kLayoutWaves = kLayoutThreads / 64;

__device__ inline int block_excl_scan(int v, int* sh, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh[w] = x;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kLayoutWaves; ++i) {
    const int t = sh[i];
    off += i < w ? t : 0;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return off + x - v;
}

__device__ inline int block_sum(int v, int* sh) {
  int tot;
  block_excl_scan(v, sh, &tot);
  return tot;
}

__device__ inline long long block_reduce_ll(long long v, bool take_max, long long* sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const long long y = __shfl_xor(v, o, 64);
    v = take_max ? (y > v ? y : v) : (y < v ? y : v);
  }
  if (lane == 0) sh[w] = v;
  __syncthreads();
  long long r = sh[0];
#pragma unroll
  for (int i = 1; i < kLayoutWaves; ++i) {
    const long long t = sh[i];
    r = take_max ? (t > r ? t : r) : (t < r ? t : r);
  }
  __syncthreads();
  return r;
}

// Thread t owns the contiguous slots [t * S, t * S + S) (S = ceil(P / 1024)),
// so every list below is built in ascending slot order by one block scan over
// per-thread counts.  With MAXS > 0 (S <= MAXS) the thread reads its slots'
// mask and ids once, all loads issued together, and keeps them in registers
// through the passes (eviction rounds, next id, history list); read from
// memory in every pass, each load sat in a branch of its own and cost one
// round trip.  MAXS == 0 reads memory in every pass (pools beyond 8192
// slots: 16 slots per thread in registers spilled).
template <int MAXS>
__global__ __launch_bounds__(kLayoutThreads) void kv_layout_kernel(wam_kv_layout_args a) {
  __shared__ int sh_i[kLayoutWaves];
  __shared__ long long sh_ll[kLayoutWaves];
  const int tid = threadIdx.x, P = a.pool;
  const int S = (P + kLayoutThreads - 1) / kLayoutThreads;
  const int lo = min(tid * S, P), hi = min(lo + S, P);
  static_assert(MAXS <= 32, "the valid flags are bits of one word");
  constexpr int NS = MAXS > 0 ? MAXS : 1;
  uint32_t mbits = 0;  // bit j: slot lo + j is valid
  long long idreg[NS];
  if constexpr (MAXS > 0) {
    uint8_t mreg[MAXS];
#pragma unroll
    for (int j = 0; j < MAXS; ++j) mreg[j] = a.mask[min(lo + j, P - 1)];
    if (!a.candidate) {
#pragma unroll
      for (int j = 0; j < MAXS; ++j) idreg[j] = (long long)a.ids[min(lo + j, P - 1)];
    }
#pragma unroll
    for (int j = 0; j < MAXS; ++j) mbits |= (lo + j < hi && mreg[j] != 0) ? 1u << j : 0u;
  }
  // slot lo + j of this thread (j < S): valid?  id?
  auto valid = [&](int j) -> bool {
    if constexpr (MAXS > 0) return (mbits >> j) & 1u;
    else return lo + j < hi && a.mask[lo + j] != 0;
  };
  auto id_of = [&](int j) -> long long {
    if constexpr (MAXS > 0) return idreg[j];
    else return (long long)a.ids[lo + j];
  };
  auto evict = [&](int j) {
    if constexpr (MAXS > 0) {
      mbits &= ~(1u << j);
      idreg[j] = -1;
    }
    a.mask[lo + j] = 0;
    a.ids[lo + j] = -1;
  };
  const int NJ = MAXS > 0 ? MAXS : S;  // slots visited per thread (MAXS: unrolled, masked)
  if (a.candidate) {
    // Read only (candidate verification): the history list and its summary
    // in one block pass: per wave a scan of the threads' valid counts and
    // the minimum / maximum valid slot and the row check, then one exchange
    // through LDS (the general path below runs five block scans and
    // reductions for the same results).
    __shared__ int sh_c[kLayoutWaves][4];
    const int lane = tid & 63, w = tid >> 6;
    int bad = 0;
    for (int b = tid; b < a.batch; b += kLayoutThreads)
      bad |= (a.rows[b] < 0 || a.rows[b] >= a.pool_batch);
    int nv = 0, first = 0x7fffffff, lastv = -1;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (valid(j)) {
        ++nv;
        first = min(first, lo + j);
        lastv = max(lastv, lo + j);
      }
    int x = nv;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      first = min(first, __shfl_xor(first, o, 64));
      lastv = max(lastv, __shfl_xor(lastv, o, 64));
      bad |= __shfl_xor(bad, o, 64);
    }
    const int wave_total = __shfl(x, 63, 64);
    if (lane == 0) {
      sh_c[w][0] = wave_total;
      sh_c[w][1] = first;
      sh_c[w][2] = lastv;
      sh_c[w][3] = bad;
    }
    __syncthreads();
    int off = 0, tv = 0, bf = 0x7fffffff, bl = -1, bb = 0;
#pragma unroll
    for (int i = 0; i < kLayoutWaves; ++i) {
      off += i < w ? sh_c[i][0] : 0;
      tv += sh_c[i][0];
      bf = min(bf, sh_c[i][1]);
      bl = max(bl, sh_c[i][2]);
      bb |= sh_c[i][3];
    }
    int pv = off + x - nv;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (valid(j)) a.hist_slots[pv++] = lo + j;
    if (tid == 0) {
      a.info[0] = tv;
      a.info[1] = bb ? 2 : 0;
      a.info[2] = (tv > 0 && bl - bf + 1 == tv) ? bf : -1;
    }
    return;
  }
  int error = 0;
  {
    // Eviction of the oldest ids (allocate_slots).
    int nfree = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) nfree += (lo + j < hi && !valid(j)) ? 1 : 0;
    int need = a.tokens - block_sum(nfree, sh_i);
    while (need > 0) {
      long long mn = 0x7fffffffffffffffLL;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (valid(j) && id_of(j) < mn) mn = id_of(j);
      mn = block_reduce_ll(mn, false, sh_ll);
      int f = 0;
#pragma unroll
      for (int j = 0; j < NJ; ++j) f += (valid(j) && id_of(j) == mn) ? 1 : 0;
      int tot;
      int pos = block_excl_scan(f, sh_i, &tot);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (valid(j) && id_of(j) == mn) {
          if (pos < need) evict(j);
          ++pos;
        }
      }
      need -= tot;
      __syncthreads();
      if (tot == 0) {  // no valid slot left to evict: the host checks make this unreachable
        error = 1;
        break;
      }
    }
  }
  // Next id over the (post-eviction) valid slots (_next_cache_id).
  long long next = -1;
  if (!a.candidate) {
    long long mx = -1;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (valid(j) && id_of(j) > mx) mx = id_of(j);
    next = block_reduce_ll(mx, true, sh_ll) + 1;
  }
  // History list and new slots, both in ascending slot order.
  int nv = 0, nf = 0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const bool in = lo + j < hi, v = valid(j);
    nv += v ? 1 : 0;
    nf += (!a.candidate && in && !v) ? 1 : 0;
  }
  int tv, tf;
  int pv = block_excl_scan(nv, sh_i, &tv);
  int pf = block_excl_scan(nf, sh_i, &tf);
  // Is the history one run of consecutive slots?  (Its first and last valid
  // slots, before this call's new slots are marked.)
  long long first = 0x7fffffffffffffffLL, lastv = -1;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    if (valid(j)) {
      first = min(first, (long long)(lo + j));
      lastv = max(lastv, (long long)(lo + j));
    }
  first = block_reduce_ll(first, false, sh_ll);
  lastv = block_reduce_ll(lastv, true, sh_ll);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int i = lo + j;
    if (i >= hi) continue;
    const bool v = valid(j);
    if (v) a.hist_slots[pv++] = i;
    if (!a.candidate && !v) {
      if (pf < a.tokens) {
        a.new_slots[pf] = i;
        a.mask[i] = a.update != 0 ? 1 : 0;
        a.ids[i] = next;
        a.is_pred[i] = a.update == 1 ? 1 : 0;
      }
      ++pf;
    }
  }
  if (tid == 0) {
    a.info[0] = tv;
    a.info[1] = error;
    a.info[2] = (tv > 0 && lastv - first + 1 == tv) ? (int)first : -1;
  }
}

int kv_layout(const wam_kv_layout_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr, "wam_kv_layout: null args");
  WAM_REQUIRE(a->mask && a->ids && a->is_pred && a->hist_slots && a->info,
              "wam_kv_layout: null pool state");
  WAM_REQUIRE(a->pool > 0, "wam_kv_layout: empty pool");
  if (a->candidate) {
    WAM_REQUIRE(a->rows != nullptr && a->batch > 0 && a->pool_batch > 0,
                "wam_kv_layout: candidate mode needs rows");
    WAM_REQUIRE(a->update == 0, "candidate verification requires existing read-only KV (update 0)");
  } else {
    WAM_REQUIRE(a->new_slots != nullptr, "wam_kv_layout: null new_slots");
    WAM_REQUIRE(a->update >= 0 && a->update <= 2, "wam_kv_layout: update must be 0, 1 or 2");
    WAM_REQUIRE(a->tokens >= 1 && a->tokens <= a->pool,
                "wam_kv_layout: %d new tokens do not fit a pool of %d slots", a->tokens, a->pool);
  }
  const int S = (a->pool + kLayoutThreads - 1) / kLayoutThreads;
  if (S <= 8) hipLaunchKernelGGL(kv_layout_kernel<8>, dim3(1), dim3(kLayoutThreads), 0, s, *a);
  else hipLaunchKernelGGL(kv_layout_kernel<0>, dim3(1), dim3(kLayoutThreads), 0, s, *a);
  WAM_LAUNCHED("kv_layout_kernel");
  return WAM_OK;
}

__global__ __launch_bounds__(256) void kv_commit_kernel(wam_kv_commit_args a) {
  const int chunks = a.D >> 3;
  const int64_t n = (int64_t)a.B * a.tokens * chunks;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    int64_t row, cc;
    split_row(i, chunks, row, cc);  // i < 2^31: B * tokens * D / 8 elements
    const int c = (int)cc;
    int64_t b, t;
    split_row(row, a.tokens, b, t);
    const int64_t src = row * a.ld + c * 8;
    const int64_t dst = b * a.pool_bstride + (int64_t)a.new_slots[t] * a.pool_rstride + c * 8;
    st_bf16x8(static_cast<bf16*>(a.pool_k) + dst, ld_bf16x8(static_cast<const bf16*>(a.k) + src));
    st_bf16x8(static_cast<bf16*>(a.pool_v) + dst, ld_bf16x8(static_cast<const bf16*>(a.v) + src));
  }
}

int kv_commit(const wam_kv_commit_args* a, hipStream_t s) {
  WAM_REQUIRE(a != nullptr && a->k && a->v && a->pool_k && a->pool_v && a->new_slots,
              "wam_kv_commit: null pointer");
  WAM_REQUIRE(a->D % 8 == 0 && a->ld % 8 == 0 && a->pool_rstride % 8 == 0 && a->pool_bstride % 8 == 0,
              "wam_kv_commit: 16-byte alignment contract");
  const int64_t n = (int64_t)a->B * a->tokens * (a->D / 8);
  WAM_REQUIRE(a->B >= 0 && a->tokens >= 0 && n < (1ll << 31), "wam_kv_commit: B * tokens * D / 8 must be < 2^31");
  if (n == 0) return WAM_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(kv_commit_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, *a);
  WAM_LAUNCHED("kv_commit_kernel");
  return WAM_OK;
}

}  // namespace wam

extern "C" int wam_kv_layout(const wam_kv_layout_args* args, void* stream) {
  return wam::kv_layout(args, static_cast<hipStream_t>(stream));
}
extern "C" int wam_kv_commit(const wam_kv_commit_args* args, void* stream) {
  return wam::kv_commit(args, static_cast<hipStream_t>(stream));
}
