// Diagnostic kernels (not part of the attention path): a clock calibration
// whose matrix-core cycle count is known by construction.
//
// fl_diag_mfma_clock launches `groups` work-groups of 64 * waves lanes,
// each holding `lds_bytes` of (unused) dynamic LDS so that the caller can
// force one work-group per CU (> 80 KiB) and hence one wave per SIMD.
// Every wave issues `rounds` x 16 independent v_mfma_f32_32x32x16_f16 (four
// accumulators, so no MFMA waits on the previous one): with one wave per
// SIMD the matrix core is busy for exactly rounds * 16 * 32 shader cycles.
// Each wave records s_memtime (shader-clock counter) and s_memrealtime
// (the constant-rate counter, hipDeviceAttributeWallClockRate) before and
// after its loop, so the host can check that s_memtime advances by the
// known cycle count and derive the shader clock under a sustained MFMA
// load.  `random` selects random-bit operands (the power-hungry case)
// instead of a constant.  The same launch under rocprofv3 --pmc shows
// which hardware counters (SQ_CYCLES, GRBM_GUI_ACTIVE, ...) tick at that
// clock.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(1024) mfma_clock_kernel(int rounds, int random,
                                                          unsigned long long* out, float* sink) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  half8_t a, b;
  uint32_t x = 0x9E3779B9u * (uint32_t)(wave * 64 + lane + 1);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    // Random: a finite fp16 in (-2, 2) with random mantissa bits.
    const uint16_t bits = (uint16_t)((x & 0x83FFu) | 0x3800u);
    const _Float16 r = __builtin_bit_cast(_Float16, bits);
    a[e] = random ? r : (_Float16)0.5f;
    b[e] = random ? (_Float16)(-r) : (_Float16)0.25f;
  }
  float16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < rounds; ++i) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
    }
  }
  // The asm keeps the loop's results live until the second timestamps.
  asm volatile("" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3));
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) s += c0[e] + c1[e] + c2[e] + c3[e];
  sink[wave * 64 + lane] = s;
  if (lane == 0) {
    out[2 * wave] = t1 - t0;
    out[2 * wave + 1] = r1 - r0;
  }
}

}  // namespace

extern "C" {

// out: 2 * groups * waves uint64 (s_memtime delta, s_memrealtime delta per
// wave); sink: groups * waves * 64 floats.  Returns a hipError_t.
int fl_diag_mfma_clock(int groups, int waves, int rounds, int random, int lds_bytes, void* out,
                       void* sink, void* stream) {
  if (groups < 1 || waves < 1 || waves > 16 || rounds < 1 || lds_bytes < 0 ||
      lds_bytes > 160 * 1024 || out == nullptr || sink == nullptr)
    return (int)hipErrorInvalidValue;
  if (lds_bytes > 64 * 1024 &&
      hipFuncSetAttribute((const void*)mfma_clock_kernel,
                          hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes) != hipSuccess)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_clock_kernel, dim3((unsigned)groups), dim3((unsigned)(64 * waves)),
                     (unsigned)lds_bytes, (hipStream_t)stream, rounds, random,
                     (unsigned long long*)out, (float*)sink);
  return (int)hipGetLastError();
}

// Rate of s_memrealtime in kHz.
int fl_diag_wall_clock_khz(int device) {
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device) != hipSuccess) return -1;
  return khz;
}

}  // extern "C"
