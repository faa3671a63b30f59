// Un-fused attention baseline for gfx950: one work-group per query row.
//
// Reference: csrc/kernel_naive.cu of thebigblender/FlashLite
// (naive_attention_kernel :125-237, host :242-323).  Same algorithm and
// launch shape -- grid (N, B*H), the row's scores staged in LDS, a block max,
// exp, a block sum, then P.V -- written for 64-lane waves:
//   * reductions are wave-level butterflies (ds_swizzle/DPP via __shfl_xor)
//     plus one LDS slot per wave, with a separate slot set for the max and
//     the sum and a barrier between them (the reference reuses one slot and
//     races: kernel_naive.cu:66 vs :81-83);
//   * scores are kept in the log2 domain (s * sm_scale * log2 e) and
//     exponentiated with v_exp_f32;
//   * the P.V product splits keys over the 4 waves and head-dim over lanes,
//     and the four partial rows are added through LDS.
// Any head_dim >= 1 is accepted (the reference has no restriction either).
// N_k may differ from N_q (the reference indexes K and V with N_q's head
// stride, kernel_naive.cu:148, :270); the causal diagonal is then aligned bottom-right
// (key j visible to query i iff j <= i + N_k - N_q) and a row with no
// visible key returns 0.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "fl_internal.h"

namespace fl {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsLimit = 160 * 1024;

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

// LDS layout (floats): scores[N_k] | part[kWaves][D] | qrow[D] | red[2*kWaves]
__global__ void __launch_bounds__(kThreads)
naive_fwd_kernel(const _Float16* __restrict__ Q, const _Float16* __restrict__ K,
                 const _Float16* __restrict__ V, _Float16* __restrict__ O, int seq_q,
                 int seq_k, int dim, float c, int causal) {
  extern __shared__ float smem[];
  float* scores = smem;
  float* part = scores + seq_k;
  float* qrow = part + kWaves * dim;
  float* red = qrow + dim;

  const int qi = blockIdx.x;
  const int bh = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const size_t q_off = (size_t)bh * (size_t)seq_q * (size_t)dim;
  const size_t kv_off = (size_t)bh * (size_t)seq_k * (size_t)dim;
  const _Float16* qp = Q + q_off + (size_t)qi * dim;
  const _Float16* Kh = K + kv_off;
  const _Float16* Vh = V + kv_off;
  _Float16* op = O + q_off + (size_t)qi * dim;

  for (int d = tid; d < dim; d += kThreads) qrow[d] = (float)qp[d];
  __syncthreads();

  // 1. scores in log2 units; keys past the causal limit are never scored
  const int nvis = causal ? min(max(qi + 1 + seq_k - seq_q, 0), seq_k) : seq_k;
  float tmax = -__builtin_huge_valf();
  for (int j = tid; j < nvis; j += kThreads) {
    const _Float16* kr = Kh + (size_t)j * dim;
    float dot = 0.0f;
    for (int d = 0; d < dim; ++d) dot = __builtin_fmaf(qrow[d], (float)kr[d], dot);
    const float s = dot * c;
    scores[j] = s;
    tmax = fmaxf(tmax, s);
  }
  tmax = wave_max(tmax);
  if (lane == 0) red[wave] = tmax;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) m = fmaxf(m, red[w]);

  // 2. exponentiate in place and sum (slots red[kWaves..] -- distinct from
  //    the max slots, so no thread can still be reading what is overwritten)
  float tsum = 0.0f;
  for (int j = tid; j < nvis; j += kThreads) {
    const float p = __builtin_amdgcn_exp2f(scores[j] - m);
    scores[j] = p;
    tsum += p;
  }
  tsum = wave_sum(tsum);
  if (lane == 0) red[kWaves + wave] = tsum;
  __syncthreads();  // also publishes every scores[j]
  float l = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) l += red[kWaves + w];
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;

  // 3. O = P.V: wave w takes keys j = w (mod 4), lane takes head dims
  for (int d0 = 0; d0 < dim; d0 += 64) {
    const int d = d0 + lane;
    float acc = 0.0f;
    if (d < dim) {
      for (int j = wave; j < nvis; j += kWaves)
        acc = __builtin_fmaf(scores[j], (float)Vh[(size_t)j * dim + d], acc);
      part[wave * dim + d] = acc;
    }
  }
  __syncthreads();
  for (int d = tid; d < dim; d += kThreads) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) acc += part[w * dim + d];
    op[d] = (_Float16)(acc * inv);
  }
}

size_t naive_lds_bytes(int64_t seq, int64_t dim) {
  return sizeof(float) * (size_t)(seq + kWaves * dim + dim + 2 * kWaves);
}

}  // namespace

int64_t naive_max_seq(int64_t head_dim) {
  const int64_t fixed = (int64_t)naive_lds_bytes(0, head_dim);
  if (fixed >= kLdsLimit) return 0;
  return (kLdsLimit - fixed) / (int64_t)sizeof(float);
}

hipError_t launch_naive(const FwdArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)a.seq, (unsigned)a.batch_heads);
  const size_t lds = naive_lds_bytes(a.seq_k, a.head_dim);
  // Dynamic LDS above 64 KiB needs the per-function limit raised once.
  static std::once_flag raised;
  static hipError_t raise_err = hipSuccess;
  std::call_once(raised, [] {
    raise_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&naive_fwd_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
  });
  if (raise_err != hipSuccess) return raise_err;
  hipLaunchKernelGGL(naive_fwd_kernel, grid, dim3(kThreads), lds, stream,
                     static_cast<const _Float16*>(a.q), static_cast<const _Float16*>(a.k),
                     static_cast<const _Float16*>(a.v), static_cast<_Float16*>(a.o), a.seq,
                     a.seq_k, a.head_dim, a.negate ? -a.scale_log2 : a.scale_log2, a.causal);
  return hipGetLastError();
}

}  // namespace fl
