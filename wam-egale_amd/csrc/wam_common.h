// Shared device/host helpers of libwam_block.so (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <atomic>
#include "../../include/wam_block.h"

namespace wam {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- host side
void set_error(const char* fmt, ...);

#define WAM_REQUIRE(cond, ...)              \
  do {                                      \
    if (!(cond)) {                          \
      ::wam::set_error(__VA_ARGS__);        \
      return WAM_ERR_ARG;                   \
    }                                       \
  } while (0)

#define WAM_HIP(call)                                                        \
  do {                                                                       \
    hipError_t e_ = (call);                                                  \
    if (e_ != hipSuccess) {                                                  \
      ::wam::set_error("%s failed: %s", #call, hipGetErrorString(e_));       \
      return WAM_ERR_HIP;                                                    \
    }                                                                        \
  } while (0)

#define WAM_LAUNCHED(name)                                                   \
  do {                                                                       \
    hipError_t e_ = hipGetLastError();                                       \
    if (e_ != hipSuccess) {                                                  \
      ::wam::set_error("launch of %s failed: %s", name, hipGetErrorString(e_)); \
      return WAM_ERR_HIP;                                                    \
    }                                                                        \
  } while (0)

#define WAM_TRY(expr)            \
  do {                           \
    int rc_ = (expr);            \
    if (rc_ != WAM_OK) return rc_; \
  } while (0)

// Host-side contract of a modulation source read over `rows` token rows.
inline int check_modulation(const wam_modulation& m, int64_t rows, const char* who) {
  WAM_REQUIRE(m.table && m.temb && m.tokens > 0 && rows % m.tokens == 0,
              "%s: modulation needs table, temb and rows (%lld) divisible by tokens (%d)", who,
              (long long)rows, m.tokens);
  WAM_REQUIRE(m.temb_len >= 1 && m.temb_len <= m.tokens && m.tokens % m.temb_len == 0,
              "%s: temb length %d must be 1, the token count %d or a divisor of it", who, m.temb_len,
              m.tokens);
  WAM_REQUIRE(m.temb_mods == 0 || m.temb_mods == 6 || m.temb_mods == 1, "%s: temb mods %d must be 6 or 1",
              who, m.temb_mods);
  WAM_REQUIRE((m.table_dtype == WAM_F32 || m.table_dtype == WAM_BF16) &&
              (m.temb_dtype == WAM_F32 || m.temb_dtype == WAM_BF16), "%s: modulation dtypes", who);
  return WAM_OK;
}

// Workgroup i is dispatched to XCD i % 8 on MI355X.  Remap so that each XCD
// receives one contiguous range of logical ids (bijective for any n).
__host__ __device__ inline int xcd_remap(int i, int n) {
  const int q = n >> 3, r = n & 7;
  const int x = i & 7, k = i >> 3;
  return x * q + (x < r ? x : r) + k;
}

// Compute units of the current device (cached per device; 256 when the
// query fails, e.g. without a GPU).  Launch plans size their dispatch rounds
// with it.
inline int device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// --------------------------------------------------------------- device side
__device__ inline float ld_scalar(const void* p, int dtype, int64_t i) {
  return dtype == WAM_F32 ? static_cast<const float*>(p)[i]
                          : static_cast<float>(static_cast<const bf16*>(p)[i]);
}

// Force a wave-uniform pointer into SGPRs (the compiler cannot always prove
// uniformity of pointers selected from kernel arguments).
template <class T>
__device__ inline T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// Raw buffer resource over `bytes` bytes at p: loads past the end return 0.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform_ptr(p)), (short)0,
                                           (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
__device__ inline bf16x8 buf_ld16(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Eight OCP fp8 e4m3 values (bytes 0..7 of q) widened to bf16 (exact: every
// e4m3 value is a bf16 value).  v_cvt_scalef32_pk_bf16_fp8 with scale 1.0
// converts the two bytes of one 16-bit half.
__device__ inline bf16x8 fp8x8_to_bf16x8(u32x2 q) {
  const bf16x2 c0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, false);
  const bf16x2 c1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, true);
  const bf16x2 c2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, false);
  const bf16x2 c3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, true);
  return bf16x8{c0[0], c0[1], c1[0], c1[1], c2[0], c2[1], c3[0], c3[1]};
}

// Buffer resource as four dwords (gfx9 layout: base, base[47:32] with stride
// 0, num_records in bytes, format dword), for use in inline assembly.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ inline i32x4 make_rsrc4(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  i32x4 r;
  r[0] = (int)__builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = (int)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);
  r[2] = (int)__builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000;
  // The dwords may have been written by v_readfirstlane: a VMEM instruction
  // that reads an SGPR written by a VALU needs 5 wait states in between, and
  // the compiler does not see the loads inside inline assembly.
  asm volatile("s_nop 4" : "+s"(r));
  return r;
}

// Direct-to-LDS load through inline assembly: the compiler does not see an
// LDS write here, so it inserts no waits of its own; the caller orders the
// load with explicit s_waitcnt vmcnt and barriers.  Lane L writes bytes
// [16 L, 16 L + 16) of the 1 KB block at `lds` (wave-uniform).
__device__ inline void asm_ld16_lds(i32x4 rsrc, void* lds, int voff) {
  // The low 32 bits of a generic pointer into LDS are the LDS byte offset;
  // it goes to M0 as an operand of the statement, so the compiler writes M0
  // itself and knows its value.  One wait state between that write and the
  // LDS DMA that reads it.
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "{m0}"(m0) : "memory");
}

// Same for a per-lane 64-bit global address (global_load_lds_dwordx4).
__device__ inline void asm_g_ld16_lds(uint64_t gaddr, void* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(gaddr), "{m0}"(m0) : "memory");
}

// Same from a wave-uniform 64-bit base (in SGPRs) plus a per-lane 32-bit byte
// offset: one VGPR of address per lane instead of two.  Four wait states
// cover an SGPR of the base written by a VALU instruction just before.
__device__ inline void asm_gs_ld16_lds(const void* base, uint32_t voff, void* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  const uint64_t b = reinterpret_cast<uint64_t>(uniform_ptr(base));
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" :: "v"(voff), "s"(b), "{m0}"(m0) : "memory");
}

// 4 bytes per lane from a per-lane 64-bit global address into LDS
// (global_load_lds_dword): lane L writes bytes [4 L, 4 L + 4) at `lds`.
__device__ inline void asm_g_ld4_lds(uint64_t gaddr, void* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" :: "v"(gaddr), "{m0}"(m0) : "memory");
}

// 16 bytes per lane from a buffer resource straight into LDS: lane L writes
// bytes [16 L, 16 L + 16) of the 1 KB block at `lds` (wave-uniform).
__device__ inline void buf_ld16_lds(__amdgpu_buffer_rsrc_t r, void* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// 16 bytes per lane from a global address straight into LDS: lane L writes
// bytes [16 L, 16 L + 16) of the 1 KB block at `lds` (wave-uniform).
__device__ inline void g_ld16_lds(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// ds_read_b64_tr_b16: within each 16-lane group, source lane j addresses 4
// consecutive 16-bit elements; lane i receives element (i % 4) of source
// lanes i / 4, i / 4 + 4, i / 4 + 8, i / 4 + 12 (a 4 x 16 transpose).
__device__ inline bf16x4 ld_tr16(const void* lds) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)lds);
  return __builtin_bit_cast(bf16x4, v);
}

__device__ inline bf16x8 ld_bf16x8(const void* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
__device__ inline void st_bf16x8(void* p, bf16x8 v) {
  *reinterpret_cast<bf16x8*>(p) = v;
}

// (b, t) = (row / tokens, row % tokens) in 32-bit arithmetic (token rows are
// below 2^31 everywhere in this library; a 64-bit division is a long
// software sequence on the GPU).
__device__ inline void split_row(int64_t row, int tokens, int64_t& b, int64_t& t) {
  const uint32_t r = (uint32_t)row, n = (uint32_t)tokens;
  const uint32_t q = r / n;
  b = q;
  t = r - q * n;
}

// fp32 values of 8 consecutive elements held as raw words: a and c are the
// 8 fp32 values (f32), or a holds the 8 bf16 values (c unused).
__device__ inline void widen8(bool f32, u32x4 a, u32x4 c, float out[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const unsigned lo = a[e >> 1], hi = a[2 + (e >> 1)];
    out[e] = __uint_as_float(f32 ? a[e] : ((e & 1) ? (lo & 0xffff0000u) : (lo << 16)));
    out[4 + e] = __uint_as_float(f32 ? c[e] : ((e & 1) ? (hi & 0xffff0000u) : (hi << 16)));
  }
}
// 8 consecutive values p[off .. off+8) of a bf16 or fp32 vector, widened to
// fp32.  Both 16-byte loads are issued whatever the dtype (for bf16 the
// second repeats the first), so neither sits in a branch of its own: the
// compiler waits for a load inside a branch before the branch ends, which
// turns a run of such calls into one memory round trip each.
__device__ inline void ld8_f32(const void* p, int dtype, int64_t off, float out[8]) {
  const bool f32 = dtype == WAM_F32;
  const char* base = static_cast<const char*>(p) + off * (f32 ? 4 : 2);
  const u32x4 a = *reinterpret_cast<const u32x4*>(base);
  const u32x4 c = *reinterpret_cast<const u32x4*>(base + (f32 ? 16 : 0));
  widen8(f32, a, c, out);
}
// Row of temb that serves token row `row`: per sample, per token, or per
// group of tokens / temb_len consecutive tokens (one latent frame).
__device__ inline int64_t temb_row(const wam_modulation& m, int64_t row) {
  int64_t b, t;
  split_row(row, m.tokens, b, t);
  if (m.temb_len == 1) return b;
  if (m.temb_len == m.tokens) return b * m.tokens + t;
  const uint32_t group = (uint32_t)m.tokens / (uint32_t)m.temb_len;
  return b * m.temb_len + (uint32_t)t / group;
}
// First token row served by temb row `trow` (temb_row does not decrease
// along the token rows, so row r is served by trow or a later row iff r >=
// this).
__device__ inline int64_t temb_first_row(const wam_modulation& m, int64_t trow) {
  if (m.temb_len == 1) return trow * m.tokens;
  if (m.temb_len == m.tokens) return trow;
  const int64_t b = trow / m.temb_len, k = trow - b * m.temb_len;
  return b * m.tokens + k * (m.tokens / m.temb_len);
}
// Element offset of temb[trow, idx, d]: [.., 6, D] rows, or one vector per row.
__device__ inline int64_t temb_off(const wam_modulation& m, int64_t trow, int idx, int D, int d) {
  return m.temb_mods == 1 ? trow * D + d : (trow * 6 + idx) * (int64_t)D + d;
}
// 8 consecutive modulation values mod[b, t, idx, d .. d+8) = table + temb,
// for token row `row` (b = row / tokens, t = row % tokens).
__device__ inline void ld_mod8(const wam_modulation m, int D, int64_t row, int idx, int d, float out[8]) {
  float tb[8];
  ld8_f32(m.table, m.table_dtype, (int64_t)idx * D + d, out);
  ld8_f32(m.temb, m.temb_dtype, temb_off(m, temb_row(m, row), idx, D, d), tb);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] += tb[e];
}

// Sum over the 64 lanes of a wave: DPP adds within each 16-lane row
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror),
// then the four row sums through readlane.  The result is wave-uniform.
template <int CTRL>
__device__ inline float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ inline float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  const int i = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 16)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 32)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 48));
}

// The same butterfly with max (wave-uniform result).
__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  const int i = __builtin_bit_cast(int, v);
  return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 0)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 16))),
               fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 32)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 48))));
}

// Max over each aligned group of 8 lanes (quad exchanges, then the mirror
// of the 8-lane half row); every lane of a group gets the group's max.
__device__ inline float max8_lanes(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  return fmaxf(v, dpp<0x141>(v));
}

// e8m0 exponent of an MX block of e4m3 values (OCP MX: one power-of-two
// scale per 32 values): the smallest X with amax <= 448 * 2^X, so that no
// scaled value exceeds the e4m3 maximum.  With amax = m * 2^E, m in [1, 2):
// X = E - 8 when m <= 1.75 (448 = 1.75 * 2^8), else E - 7.  Floored at -127
// (amax 0 or subnormal); amax must be finite and >= 0.
__device__ inline int mx_exponent(float amax) {
  const uint32_t b = __float_as_uint(amax);
  const int X = (int)(b >> 23) - 135 + ((b & 0x7fffffu) > 0x600000u ? 1 : 0);
  return X < -127 ? -127 : X;
}

// Eight sums over the 64 lanes of a wave at once: v[k] summed over all lanes
// lands in out[j] for k = j + 2 (r & 1) + 4 (r >> 1), r = lane / 16, on all
// 16 lanes of row r.  Two halving exchanges (v_permlane32_swap trades the
// upper 32 lanes of its first operand for the lower 32 of its second, so the
// sum of the two results holds v[j] in lanes 0-31 and v[j + 4] in 32-63;
// v_permlane16_swap does the same with odd and even 16-lane rows), then
// rotations within the rows of 16: 20 instructions for 8 sums.
__device__ inline void wave_sum8(const float v[8], float out[2]) {
  float t[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[j + 4]), false, false);
    t[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(t[j]), __float_as_uint(t[j + 2]), false, false);
    float s = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    s += dpp<0x128>(s);  // row_ror:8
    s += dpp<0x124>(s);  // row_ror:4
    s += dpp<0x4E>(s);   // quad_perm [2, 3, 0, 1]
    s += dpp<0xB1>(s);   // quad_perm [1, 0, 3, 2]
    out[j] = s;
  }
}

// GELU, tanh approximation: 0.5 x (1 + tanh(u)) = x * sigmoid(2u),
// u = sqrt(2/pi) (x + 0.044715 x^3).  sigmoid via v_exp_f32 and v_rcp_f32,
// with the constants folded: -2 log2(e) u = x (A + B x^2), so an output is
// x^2, one FMA, one multiply, the exponential, an add, the reciprocal and a
// multiply.
__device__ inline float gelu_tanh(float x) {
  constexpr float A = -2.0f * 1.4426950408889634f * 0.7978845608028654f;
  constexpr float B = A * 0.044715f;
  const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(x * x, B, A));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

}  // namespace wam
