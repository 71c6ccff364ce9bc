// On-device MFMA throughput probe: the measured denominators of the roofline
// next to the vendor peaks.  Every wave keeps four independent accumulator
// chains of one MFMA shape busy for `iters` rounds; two workgroups of four
// waves per CU (two waves per SIMD) hide the dependent-issue latency.  The
// operands come from the thread index so nothing folds, and the sums are
// written out so nothing is dead.
#include "wam_common.h"

namespace wam {

typedef int i32x8 __attribute__((ext_vector_type(8)));

template <int KIND>
__global__ __launch_bounds__(256, 2) void mfma_peak_kernel(float* __restrict__ sink, int iters) {
  const int t = threadIdx.x;
  float s = 0.f;
  if constexpr (KIND == WAM_PEAK_BF16_32 || KIND == WAM_PEAK_BF16_16) {
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = static_cast<bf16>((float)((t + e) & 7) * 0.125f);
      b[e] = static_cast<bf16>((float)((t * 3 + e) & 7) * 0.125f);
    }
    if constexpr (KIND == WAM_PEAK_BF16_32) {
      f32x16 c[4] = {};
      for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j], 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s += c[j][0] + c[j][15];
    } else {
      f32x4 c[8] = {};
      for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c[j], 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s += c[j][0] + c[j][3];
    }
  } else {
    i32x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = 0x38303830 + ((t + e) & 3);   // small e4m3 values
      b[e] = 0x30383038 + ((t * 5 + e) & 3);
    }
    // Unit block scales (E8M0 exponent 127 = 1.0); cbsz = blgp = 0: e4m3 operands.
    if constexpr (KIND == WAM_PEAK_FP8_32) {
      f32x16 c[4] = {};
      for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          c[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c[j], 0, 0, 0, 127, 0, 127);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s += c[j][0] + c[j][15];
    } else {
      f32x4 c[8] = {};
      for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          c[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c[j], 0, 0, 0, 127, 0, 127);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s += c[j][0] + c[j][3];
    }
  }
  sink[(int64_t)blockIdx.x * 256 + t] = s;
}

// FLOP of one MFMA instruction of each probe kind.
static double mfma_flop(int kind) {
  switch (kind) {
    case WAM_PEAK_BF16_32: return 2.0 * 32 * 32 * 16;
    case WAM_PEAK_BF16_16: return 2.0 * 16 * 16 * 32;
    case WAM_PEAK_FP8_32: return 2.0 * 32 * 32 * 64;
    default: return 2.0 * 16 * 16 * 128;
  }
}

int mfma_peak(int kind, int iters, void* sink, int64_t sink_bytes, double* flop, hipStream_t s) {
  WAM_REQUIRE(kind >= WAM_PEAK_BF16_32 && kind <= WAM_PEAK_FP8_16, "wam_mfma_peak: kind %d", kind);
  WAM_REQUIRE(iters >= 1 && sink && flop, "wam_mfma_peak: iters >= 1, sink and flop required");
  const int blocks = 2 * device_cu_count();
  WAM_REQUIRE(sink_bytes >= (int64_t)blocks * 256 * 4, "wam_mfma_peak: sink needs %lld bytes",
              (long long)blocks * 256 * 4);
  float* out = static_cast<float*>(sink);
  switch (kind) {
    case WAM_PEAK_BF16_32: hipLaunchKernelGGL(mfma_peak_kernel<WAM_PEAK_BF16_32>, dim3(blocks), dim3(256), 0, s, out, iters); break;
    case WAM_PEAK_BF16_16: hipLaunchKernelGGL(mfma_peak_kernel<WAM_PEAK_BF16_16>, dim3(blocks), dim3(256), 0, s, out, iters); break;
    case WAM_PEAK_FP8_32: hipLaunchKernelGGL(mfma_peak_kernel<WAM_PEAK_FP8_32>, dim3(blocks), dim3(256), 0, s, out, iters); break;
    default: hipLaunchKernelGGL(mfma_peak_kernel<WAM_PEAK_FP8_16>, dim3(blocks), dim3(256), 0, s, out, iters); break;
  }
  WAM_LAUNCHED("mfma_peak_kernel");
  const int chains = (kind == WAM_PEAK_BF16_32 || kind == WAM_PEAK_FP8_32) ? 4 : 8;
  *flop = (double)blocks * 4 /* waves */ * iters * chains * mfma_flop(kind);
  return WAM_OK;
}

}  // namespace wam

extern "C" int wam_mfma_peak(int kind, int iters, void* sink, int64_t sink_bytes, double* flop, void* stream) {
  return wam::mfma_peak(kind, iters, sink, sink_bytes, flop, static_cast<hipStream_t>(stream));
}
