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

// Issue-rate probe: 16 independent v_mfma_f32_32x32x16_f16 per round (four
// accumulators), each followed by the same short sequence of independent
// VALU instructions, all in one inline-assembly block so the compiler
// neither reorders nor removes them.  MODE selects the sequence per MFMA:
//   0: none                       4: 4 x v_add_f32
//   1: 2 x v_exp_f32              5: 8 x v_add_f32
//   2: 4 x v_exp_f32              6: 2 x v_exp_f32 + 1 x v_cvt_pk_f16_f32
//   3: 2 x v_exp_f32 + 2 x v_add_f32   7: 2 x v_cvt_pk_f16_f32
//   8: 2 x v_exp_f32 + v_cvt_pk_f16_f32 + v_pk_add_f16
//   9: 1 x ds_read_b128          10: 2 x ds_read_b64_tr_b16
//  11: 1 x ds_read_b128 + 2 x v_exp_f32 + v_cvt_pk_f16_f32
//  12: 2 x ds_read_b64_tr_b16 + 2 x v_exp_f32 + v_cvt_pk_f16_f32
//  (the LDS modes wait for their reads once per four MFMAs, lgkmcnt(4))
// No instruction reads a result of the sequence, so only issue limits show.
// Per wave: s_memtime and s_memrealtime deltas over the rounds.
// Operands: %0-%3 accumulators, %4-%7 VALU results, %8 / %9 LDS results,
// %10 / %11 fp32 inputs, %12 a packed-fp16 input, %13 / %14 the MFMA
// operands, %15 the LDS address.
#define FL_MIX1 "v_exp_f32 %4, %10\n\tv_exp_f32 %5, %11\n\t"
#define FL_MIX2 "v_exp_f32 %4, %10\n\tv_exp_f32 %5, %11\n\tv_exp_f32 %6, %10\n\tv_exp_f32 %7, %11\n\t"
#define FL_MIX3 "v_exp_f32 %4, %10\n\tv_exp_f32 %5, %11\n\tv_add_f32 %6, %10, %11\n\tv_add_f32 %7, %11, %10\n\t"
#define FL_MIX4 "v_add_f32 %4, %10, %11\n\tv_add_f32 %5, %11, %10\n\tv_add_f32 %6, %10, %10\n\tv_add_f32 %7, %11, %11\n\t"
#define FL_MIX5 FL_MIX4 FL_MIX4
#define FL_MIX6 "v_exp_f32 %4, %10\n\tv_exp_f32 %5, %11\n\tv_cvt_pk_f16_f32 %6, %10, %11\n\t"
#define FL_MIX7 "v_cvt_pk_f16_f32 %6, %10, %11\n\tv_cvt_pk_f16_f32 %7, %11, %10\n\t"
#define FL_MIX8 "v_exp_f32 %4, %10\n\tv_exp_f32 %5, %11\n\tv_cvt_pk_f16_f32 %6, %10, %11\n\tv_pk_add_f16 %7, %12, %12\n\t"
#define FL_MIX9 "ds_read_b128 %8, %15\n\t"
#define FL_MIX10 "ds_read_b64_tr_b16 %9, %15\n\tds_read_b64_tr_b16 %9, %15 offset:512\n\t"
#define FL_MIX11 FL_MIX9 FL_MIX6
#define FL_MIX12 FL_MIX10 FL_MIX6
#define FL_MFMA(ACC, X) "v_mfma_f32_32x32x16_f16 " ACC ", %13, %14, " ACC "\n\t" X
#define FL_MIX_QUAD(X) FL_MFMA("%0", X) FL_MFMA("%1", X) FL_MFMA("%2", X) FL_MFMA("%3", X)
#define FL_MIX_ROUND(X) FL_MIX_QUAD(X) FL_MIX_QUAD(X) FL_MIX_QUAD(X) FL_MIX_QUAD(X)
#define FL_MIX_ROUND_LDS(X)                                                                 \
  FL_MIX_QUAD(X) "s_waitcnt lgkmcnt(4)\n\t" FL_MIX_QUAD(X) "s_waitcnt lgkmcnt(4)\n\t"     \
  FL_MIX_QUAD(X) "s_waitcnt lgkmcnt(4)\n\t" FL_MIX_QUAD(X) "s_waitcnt lgkmcnt(0)\n\t"

template <int MODE>
__global__ void __launch_bounds__(1024) mfma_mix_kernel(int rounds, unsigned long long* out,
                                                        float* sink) {
  extern __shared__ __attribute__((aligned(16))) uint8_t mix_lds[];
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  half8_t a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (_Float16)(0.001f * (float)(lane + e));
    b[e] = (_Float16)(0.002f * (float)(lane - e));
  }
  float16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  float t0 = 0.0f, t1 = 0.0f, t2 = 0.0f, t3 = 0.0f;
  const float x0 = -0.25f * (float)(lane & 7), x1 = -0.5f * (float)(lane & 3);
  const uint32_t hx = 0x3c003c00u + (uint32_t)lane;
  // LDS operand reads (modes 9-12): conflict-free lane addresses in the
  // dynamic LDS, results into registers nothing reads.
  const uint32_t lds_addr = (uint32_t)(uintptr_t)mix_lds + 16u * (uint32_t)lane;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  u32x4 ld4 = {0, 0, 0, 0};
  u32x2 ld2 = {0, 0};
  const unsigned long long ts0 = __builtin_amdgcn_s_memtime();
  const unsigned long long rs0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < rounds; ++i) {
#define FL_MIX_ASM_R(R, X)                                                               \
  asm volatile(R(X)                                                                      \
               : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3), "+v"(t0), "+v"(t1), "+v"(t2),  \
                 "+v"(t3), "+v"(ld4), "+v"(ld2)                                          \
               : "v"(x0), "v"(x1), "v"(hx), "v"(a), "v"(b), "v"(lds_addr)               \
               : "memory")
#define FL_MIX_ASM(X) FL_MIX_ASM_R(FL_MIX_ROUND, X)
#define FL_MIX_ASM_LDS(X) FL_MIX_ASM_R(FL_MIX_ROUND_LDS, X)
    if constexpr (MODE == 0) FL_MIX_ASM("");
    if constexpr (MODE == 1) FL_MIX_ASM(FL_MIX1);
    if constexpr (MODE == 2) FL_MIX_ASM(FL_MIX2);
    if constexpr (MODE == 3) FL_MIX_ASM(FL_MIX3);
    if constexpr (MODE == 4) FL_MIX_ASM(FL_MIX4);
    if constexpr (MODE == 5) FL_MIX_ASM(FL_MIX5);
    if constexpr (MODE == 6) FL_MIX_ASM(FL_MIX6);
    if constexpr (MODE == 7) FL_MIX_ASM(FL_MIX7);
    if constexpr (MODE == 8) FL_MIX_ASM(FL_MIX8);
    if constexpr (MODE == 9) FL_MIX_ASM_LDS(FL_MIX9);
    if constexpr (MODE == 10) FL_MIX_ASM_LDS(FL_MIX10);
    if constexpr (MODE == 11) FL_MIX_ASM_LDS(FL_MIX11);
    if constexpr (MODE == 12) FL_MIX_ASM_LDS(FL_MIX12);
#undef FL_MIX_ASM
#undef FL_MIX_ASM_LDS
#undef FL_MIX_ASM_R
  }
  // Wait out the last MFMAs (no hazard information crosses the asm).
  asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");
  const unsigned long long ts1 = __builtin_amdgcn_s_memtime();
  const unsigned long long rs1 = __builtin_amdgcn_s_memrealtime();
  float s = t0 + t1 + t2 + t3 + (float)(ld4[0] ^ ld4[3] ^ ld2[1]) * 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) s += c0[e] + c1[e] + c2[e] + c3[e];
  sink[wave * 64 + lane] = s;
  if (lane == 0) {
    out[2 * wave] = ts1 - ts0;
    out[2 * wave + 1] = rs1 - rs0;
  }
}

// The launch floor: a kernel that does nothing, launched with a given grid.
__global__ void empty_kernel() {}

}  // namespace

extern "C" {

// One launch of empty_kernel (groups x 64*waves lanes) on `stream`.
int fl_diag_empty(int groups, int waves, void* stream) {
  if (groups < 1 || waves < 1 || waves > 16) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(empty_kernel, dim3((unsigned)groups), dim3((unsigned)(64 * waves)), 0,
                     (hipStream_t)stream);
  return (int)hipGetLastError();
}

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

// Issue-rate probe (mfma_mix_kernel): same arguments as fl_diag_mfma_clock
// plus the sequence `mode` (0-12; the LDS modes need lds_bytes >= 2 KiB).
int fl_diag_mfma_mix(int groups, int waves, int rounds, int mode, int lds_bytes, void* out,
                     void* sink, void* stream) {
  if (groups < 1 || waves < 1 || waves > 16 || rounds < 1 || mode < 0 || mode > 12 ||
      lds_bytes < 0 || lds_bytes > 160 * 1024 || out == nullptr || sink == nullptr)
    return (int)hipErrorInvalidValue;
  // Modes 9-12 read lane*16 + offset:512 bytes of dynamic LDS (up to
  // 1.5 KiB): refuse a smaller allocation.
  if (mode >= 9 && lds_bytes < 2048) return (int)hipErrorInvalidValue;
  const void* fns[13] = {
      (const void*)mfma_mix_kernel<0>,  (const void*)mfma_mix_kernel<1>,
      (const void*)mfma_mix_kernel<2>,  (const void*)mfma_mix_kernel<3>,
      (const void*)mfma_mix_kernel<4>,  (const void*)mfma_mix_kernel<5>,
      (const void*)mfma_mix_kernel<6>,  (const void*)mfma_mix_kernel<7>,
      (const void*)mfma_mix_kernel<8>,  (const void*)mfma_mix_kernel<9>,
      (const void*)mfma_mix_kernel<10>, (const void*)mfma_mix_kernel<11>,
      (const void*)mfma_mix_kernel<12>};
  if (lds_bytes > 64 * 1024 &&
      hipFuncSetAttribute(fns[mode], hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes) !=
          hipSuccess)
    return (int)hipErrorInvalidValue;
  const dim3 grid((unsigned)groups), block((unsigned)(64 * waves));
  auto* o = (unsigned long long*)out;
  auto* sk = (float*)sink;
  auto st = (hipStream_t)stream;
  const unsigned lds = (unsigned)lds_bytes;
  switch (mode) {
    case 0: hipLaunchKernelGGL(mfma_mix_kernel<0>, grid, block, lds, st, rounds, o, sk); break;
    case 1: hipLaunchKernelGGL(mfma_mix_kernel<1>, grid, block, lds, st, rounds, o, sk); break;
    case 2: hipLaunchKernelGGL(mfma_mix_kernel<2>, grid, block, lds, st, rounds, o, sk); break;
    case 3: hipLaunchKernelGGL(mfma_mix_kernel<3>, grid, block, lds, st, rounds, o, sk); break;
    case 4: hipLaunchKernelGGL(mfma_mix_kernel<4>, grid, block, lds, st, rounds, o, sk); break;
    case 5: hipLaunchKernelGGL(mfma_mix_kernel<5>, grid, block, lds, st, rounds, o, sk); break;
    case 6: hipLaunchKernelGGL(mfma_mix_kernel<6>, grid, block, lds, st, rounds, o, sk); break;
    case 7: hipLaunchKernelGGL(mfma_mix_kernel<7>, grid, block, lds, st, rounds, o, sk); break;
    case 8: hipLaunchKernelGGL(mfma_mix_kernel<8>, grid, block, lds, st, rounds, o, sk); break;
    case 9: hipLaunchKernelGGL(mfma_mix_kernel<9>, grid, block, lds, st, rounds, o, sk); break;
    case 10: hipLaunchKernelGGL(mfma_mix_kernel<10>, grid, block, lds, st, rounds, o, sk); break;
    case 11: hipLaunchKernelGGL(mfma_mix_kernel<11>, grid, block, lds, st, rounds, o, sk); break;
    default: hipLaunchKernelGGL(mfma_mix_kernel<12>, grid, block, lds, st, rounds, o, sk); break;
  }
  return (int)hipGetLastError();
}

// Rate of s_memrealtime in kHz.
int fl_diag_wall_clock_khz(int device) {
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device) != hipSuccess) return -1;
  return khz;
}

}  // extern "C"
