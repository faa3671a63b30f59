// FlashAttention-2 forward for gfx950 (MI355X, CDNA4), fp16 in / fp32 accumulate.
//
// Reference: csrc/kernel_flash2.cu of thebigblender/FlashLite -- the two
// kernels flash_attn2_wmma_br64_kernel (:54-387) and
// flash_attn2_wmma_br128_kernel (:393-727).  This is a fresh design for
// 64-lane wavefronts and MFMA, not a translation; the math and the mask
// semantics are the same:
//   O = softmax(Q K^T * sm_scale [+ causal mask]) V,
//   causal: key j visible to query i iff j <= i (top-left, N_q == N_k),
//   keys >= N masked, query rows >= N never written (:373, :380),
//   P rounded to fp16 before the PV product (:278-285), fp32 row sums.
//
// Work decomposition.  A work-group of W waves owns 32*W consecutive query
// rows of one (batch, head); wave w owns 32 of them.  The KV sequence is
// walked in tiles of 64 keys staged in LDS (double-buffered, one barrier per
// tile) and shared by the W waves.
//
// MFMA formulation (v_mfma_f32_32x32x16_f16, 64 lanes, lane l: column l%32,
// k-group g = l/32):
//   GEMM1  S^T[key][query] = K . Q^T   A = K rows from LDS (ds_read_b128),
//                                      B = the wave's Q rows, held in VGPRs.
//     Each lane then owns ONE query (column l%32) and 16 of a 32-key block
//     (rows 8*(r/4) + 4*g + r%4 of accumulator r); the other 16 sit in lane
//     l^32.  A row max/sum is 16 in-lane ops plus one v_permlane32_swap.
//   GEMM2  O^T[d][query] += V^T . P^T  B = P^T straight from the GEMM1
//                                      accumulators (packed to fp16),
//                                      A = V^T read with ds_read_b64_tr_b16,
//     whose 4-keys-per-lane transposed layout is exactly the k-order of the
//     GEMM1 accumulators, so P never leaves registers.
// The A-operand rows of GEMM2 are permuted (bits 2 and 3 of the row index
// swapped via the tr-read addresses) so each lane ends with 8 contiguous
// head-dim values per accumulator half: the epilogue stores 16-byte vectors.
//
// Softmax.  Scores stay raw (unscaled) in fp32; the running max m is kept in
// raw units and p = exp2(s*c - m*c) is one FMA plus v_exp_f32, with
// c = |sm_scale| * log2(e) (the reference's prescale, kernel_flash2.cu:772).
// The max is only moved when some lane's new tile max exceeds it by more
// than 8 in the log2 domain, so p <= 2^8 (exact in fp16 range); this skips
// the O rescale on almost every tile and is exact math (softmax is shift
// invariant).  Each lane accumulates the row sum of its own 32 keys; the two
// halves of a row are added once, in the epilogue.
//
// Causal.  Key blocks entirely above a wave's diagonal are skipped (never
// multiplied); blocks on the diagonal and the ragged tail are masked to -inf;
// every other block runs unmasked.  Work-groups are issued heaviest-first.
//
// LDS.  Rows of 128 B (64 halfs).  16-byte chunks are XOR-swizzled per row:
// K with (row&7)^((row>>3)&1), V with 2*(row&3), which makes the GEMM1
// ds_read_b128 pattern, the GEMM2 ds_read_b64_tr_b16 pattern and the
// row-contiguous tile stores conflict-free for 32- or 64-bank LDS.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fl_internal.h"

namespace fl {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kD = 64;                 // head dim
constexpr int kBc = 64;                // keys per KV tile
constexpr int kRowBytes = kD * 2;      // 128
constexpr int kTileBytes = kBc * kRowBytes;  // 8 KiB
constexpr float kTau = 8.0f;           // max lag of the running max, log2 units

__device__ __forceinline__ int k_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int v_swz(int row) { return (row & 3) << 1; }

__device__ __forceinline__ float ninf() { return -__builtin_huge_valf(); }

// Value of x in lane l^32, combined with the own value: returns
// {x[l], x[l^32]} in some order for every lane.
__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ half4_t lds_read_tr(const uint8_t* p) {
  short4_t s = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (short4_t __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(half4_t, s);
}

template <int W, bool CAUSAL>
__global__ void __launch_bounds__(64 * W)
fa2_fwd_kernel(const _Float16* Q, const _Float16* __restrict__ K,
               const _Float16* __restrict__ V, _Float16* O, int seq, int nqb,
               float c, int negate) {
  constexpr int kThreads = 64 * W;
  constexpr int kBr = 32 * W;
  constexpr int kChunksPerThread = (kTileBytes / 16) / kThreads;  // per tensor
  static_assert(kChunksPerThread * kThreads * 16 == kTileBytes, "tile split");

  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][kTileBytes];  // [buf][K,V]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int col = lane & 31;

  // Work-group -> (batch*head, query block).  Work-groups are dealt to the
  // 8 XCDs round-robin; remap so that consecutive query blocks of one head
  // land on the same XCD (shared K/V in its L2).  Causal: heaviest first.
  const int total = gridDim.x;
  int lin = blockIdx.x;
  if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
  const int bh = lin / nqb;
  int qb = lin - bh * nqb;
  if (CAUSAL) qb = nqb - 1 - qb;

  const size_t head_off = (size_t)bh * (size_t)seq * kD;
  const _Float16* Qh = Q + head_off;
  const _Float16* Kh = K + head_off;
  const _Float16* Vh = V + head_off;
  _Float16* Oh = O + head_off;

  const int q0 = qb * kBr;
  const int qw = q0 + 32 * wave;   // first query of this wave (32-aligned)
  const int my_q = qw + col;

  // Q^T B-operand: lane holds Q[my_q][16s + 8g .. +7] for s = 0..3.
  half8_t qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (my_q < seq) {
      u32x4_t raw = *reinterpret_cast<const u32x4_t*>(Qh + (size_t)my_q * kD + 16 * s + 8 * g);
      if (negate) raw ^= (u32x4_t){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
      qf[s] = __builtin_bit_cast(half8_t, raw);
    } else {
      qf[s] = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  int ntiles = (seq + kBc - 1) / kBc;
  if (CAUSAL) {
    const int q_last = min(q0 + kBr, seq) - 1;
    ntiles = min(ntiles, q_last / kBc + 1);
  }

  // Tile staging: thread t moves 16-byte chunks t + i*kThreads of each of
  // the K and V tiles (chunk id -> row id/8, chunk id%8).
  u32x4_t kreg[kChunksPerThread], vreg[kChunksPerThread];
  auto load_tile = [&](int j) {
    const int k0 = j * kBc;
#pragma unroll
    for (int i = 0; i < kChunksPerThread; ++i) {
      const int id = tid + i * kThreads;
      const int row = id >> 3, ch = id & 7;
      const int key = k0 + row;
      if (key < seq) {
        kreg[i] = *reinterpret_cast<const u32x4_t*>(Kh + (size_t)key * kD + 8 * ch);
        vreg[i] = *reinterpret_cast<const u32x4_t*>(Vh + (size_t)key * kD + 8 * ch);
      } else {
        kreg[i] = (u32x4_t){0, 0, 0, 0};
        vreg[i] = (u32x4_t){0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kChunksPerThread; ++i) {
      const int id = tid + i * kThreads;
      const int row = id >> 3, ch = id & 7;
      *reinterpret_cast<u32x4_t*>(&lds[buf][0][row * kRowBytes + 16 * (ch ^ k_swz(row))]) = kreg[i];
      *reinterpret_cast<u32x4_t*>(&lds[buf][1][row * kRowBytes + 16 * (ch ^ v_swz(row))]) = vreg[i];
    }
  };

  // Per-lane GEMM2 tr-read address pieces (see header comment): lane l is
  // lane j = l%16 of 16-lane group G = l/16; it points at key row
  // 4*(G/2) + j/4 (+16t, +8 for the second read) and head-dim column
  // 16*(G%2) + 4*swap2(j%4) (+32 per d-block).
  const int trG = lane >> 4, trj = lane & 15;
  const int tr_row = 4 * (trG >> 1) + (trj >> 2);
  const int tr_x = trj & 3;
  const int tr_col = 16 * (trG & 1) + 4 * (((tr_x & 1) << 1) | (tr_x >> 1));

  float16_t o_acc[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[db][r] = 0.0f;
  float m_used = ninf();   // running max, raw score units
  float mc = ninf();       // m_used * c
  float l_part = 0.0f;     // this lane's share of the row sum

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int j = 0; j < ntiles; ++j) {
    const int buf = j & 1;
    if (j + 1 < ntiles) load_tile(j + 1);

    const int k0 = j * kBc;
    // Key blocks (32 keys) this wave needs: block kb starts at k0 + 32kb.
    int nkb = (k0 + 32 < seq) ? 2 : 1;
    if (CAUSAL) {
      if (k0 > qw) nkb = 0;
      else if (k0 + 32 > qw) nkb = min(nkb, 1);
    }
    if (nkb > 0) {
      const uint8_t* Ks = lds[buf][0];
      const uint8_t* Vs = lds[buf][1];

      // ---- GEMM1: S^T = K . Q^T
      float16_t s_acc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        if (kb < nkb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) s_acc[kb][r] = 0.0f;
          const int row = 32 * kb + col;
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int ch = 2 * s + g;
            half8_t a = *reinterpret_cast<const half8_t*>(Ks + row * kRowBytes + 16 * (ch ^ k_swz(row)));
            s_acc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[s], s_acc[kb], 0, 0, 0);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) s_acc[kb][r] = ninf();
        }
      }

      // ---- mask: ragged tail (keys >= seq) and the causal diagonal block
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int kstart = k0 + 32 * kb;
        const bool tail = kstart + 32 > seq;
        const bool diag = CAUSAL && (kstart == qw);
        if (kb < nkb && (tail || diag)) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kstart + 8 * (r >> 2) + 4 * g + (r & 3);
            const bool ok = key < seq && (!CAUSAL || key <= my_q);
            s_acc[kb][r] = ok ? s_acc[kb][r] : ninf();
          }
        }
      }

      // ---- running max (lazy: moved only when it lags by > kTau)
      float mx = ninf();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_acc[kb][r]);
      mx = pair_max(mx);
      const bool need = (mx - m_used) * c > kTau;
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
        const float m_new = fmaxf(m_used, mx);
        const float alpha = __builtin_amdgcn_exp2f((m_used - m_new) * c);
        l_part *= alpha;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o_acc[db][r] *= alpha;
        m_used = m_new;
        mc = m_used * c;
      }

      // ---- P = exp2(s*c - m*c), row-sum share, pack to fp16 B-operands
      half8_t pf[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        if (kb >= nkb) continue;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s_acc[kb][8 * h + e], c, -mc));
            l_part += p;
            pf[kb][h][e] = (_Float16)p;
          }
        }
      }

      // ---- GEMM2: O^T += V^T . P^T
#pragma unroll
      for (int db = 0; db < 2; ++db) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          if (kb < nkb) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int t = 2 * kb + h;
              const int r1 = 16 * t + tr_row;
              const int r2 = r1 + 8;
              const int dcol = 32 * db + tr_col;
              const int ch = dcol >> 3, hb = ((dcol >> 2) & 1) * 8;
              half4_t lo = lds_read_tr(Vs + r1 * kRowBytes + 16 * (ch ^ v_swz(r1)) + hb);
              half4_t hi = lds_read_tr(Vs + r2 * kRowBytes + 16 * (ch ^ v_swz(r2)) + hb);
              half8_t a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
              o_acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[kb][h], o_acc[db], 0, 0, 0);
            }
          }
        }
      }
    }

    if (j + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O = O^T / l, 16-byte stores of 8 contiguous head dims
  const float l_tot = pair_sum(l_part);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (my_q < seq) {
    _Float16* orow = Oh + (size_t)my_q * kD;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        half8_t out;
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = (_Float16)(o_acc[db][8 * hh + e] * inv);
        *reinterpret_cast<half8_t*>(orow + 32 * db + 16 * hh + 8 * g) = out;
      }
    }
  }
}

template <int W>
hipError_t launch_w(const FwdArgs& a, hipStream_t stream) {
  const int br = 32 * W;
  const int nqb = (a.seq + br - 1) / br;
  const dim3 grid((unsigned)(nqb * a.batch_heads));
  const dim3 block(64 * W);
  const auto* q = static_cast<const _Float16*>(a.q);
  const auto* k = static_cast<const _Float16*>(a.k);
  const auto* v = static_cast<const _Float16*>(a.v);
  auto* o = static_cast<_Float16*>(a.o);
  if (a.causal)
    hipLaunchKernelGGL((fa2_fwd_kernel<W, true>), grid, block, 0, stream, q, k, v, o, a.seq, nqb,
                       a.scale_log2, a.negate);
  else
    hipLaunchKernelGGL((fa2_fwd_kernel<W, false>), grid, block, 0, stream, q, k, v, o, a.seq, nqb,
                       a.scale_log2, a.negate);
  return hipGetLastError();
}

}  // namespace

const Fa2Config kFa2Configs[kNumFa2Configs] = {
    {1, "br32_bc64_w1"},
    {2, "br64_bc64_w2"},
    {4, "br128_bc64_w4"},
    {8, "br256_bc64_w8"},
};

hipError_t launch_fa2(const FwdArgs& a, int cfg, hipStream_t stream) {
  switch (kFa2Configs[cfg].waves) {
    case 1: return launch_w<1>(a, stream);
    case 2: return launch_w<2>(a, stream);
    case 4: return launch_w<4>(a, stream);
    case 8: return launch_w<8>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fl
