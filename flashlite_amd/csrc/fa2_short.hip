// Key-quarter schedule for key ranges of at most 512 keys (configuration
// br32_kv512_w4_quarters).  Shared building blocks: fa2_common.h.

#include "fa2_common.h"

// Per-wave timeline marks (entry, loads issued, loads landed, tiles done,
// merged, exit), compiled only into the diagnostic library
// (diag_timeline.hip); empty in the product.
#ifndef FL_ST_MARK
#define FL_ST_DECL()
#define FL_ST_MARK(index)
#define FL_ST_FLUSH(wave, lane, count)
#endif

namespace fl {

namespace {

// ---------------------------------------------------------------------------
// Short key ranges (e.g. C1, B2 H8 N512): the one-pass configurations give
// each wave 32 query rows and the whole key range, 8 tiles walked one after
// another by a single wave per SIMD, on 64 work-groups for C1 (a quarter of
// the CUs).  Here a work-group of 4 waves owns one 32-row query block and
// wave w the key tiles [2w, 2w+2): a quarter of at most 512 keys.  Each wave
// fetches its own two K and two V tiles into its own 32 KiB of LDS by DMA
// and reads nothing another wave wrote, so no barrier precedes the compute;
// Q goes straight to registers, its loads issued first so their latency
// overlaps the fetches.  Each wave runs its tiles through the checked
// softmax (the stabiliser follows the row max tile by tile, so no second
// pass; the second tile's GEMM1 goes out before the first tile's softmax),
// then the quarters' O, m and l merge through LDS in 16-byte chunks at
// their larger m: 1, 2 and 3 into 0, which stores.  C1 then runs 1024
// waves of 2 tiles instead of 256 waves of 8.  LDS: 4 x 32 KiB, one
// work-group per CU.  (Eight waves of one tile each, two per SIMD, measured
// 7% slower on C1.)
constexpr int kQuarterWaves = 4;

template <int NW, bool CAUSAL, bool SCALED>
__global__ void __launch_bounds__(64 * NW, 1)
fa2_fwd_quarter_kernel(const _Float16* Q, const _Float16* __restrict__ K,
                       const _Float16* __restrict__ V, _Float16* O, const Geom geom, int nqb,
                       float cq, float cr) {
  using RowsT = Rows<CAUSAL, SCALED, _Float16>;
  using V8 = typename RowsT::V8;
  constexpr int kQuarterTiles = kQuarterMaxKeys / kBc / NW;  // key tiles per wave
  constexpr int kQuarterWaveBytes = 2 * kQuarterTiles * kTileBytes;
  static_assert(NW * kQuarterTiles * kBc == kQuarterMaxKeys, "key range");
  __shared__ __attribute__((aligned(16))) uint8_t buf[NW][kQuarterWaveBytes];

  FL_ST_DECL();
  FL_ST_MARK(0);
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // key quarter
  const int bh = blockIdx.x / nqb, qb = blockIdx.x - bh * nqb;
  const HeadPtrs<_Float16> hp = head_ptrs(geom, bh, Q, K, V, O);
  const int seq = geom.seq_q;
  const int q0 = 32 * qb;
  int ntiles = (geom.seq_k + kBc - 1) / kBc;
  if (CAUSAL) ntiles = min(ntiles, causal_tiles(min(q0 + 32, seq), geom.coff));
  const int t0 = kQuarterTiles * w;
  const int t1 = min(t0 + kQuarterTiles, ntiles);
  uint8_t* const kb = buf[w];
  uint8_t* const vb = buf[w] + kQuarterTiles * kTileBytes;

  // Q rows first, straight to registers: their latency then overlaps the
  // issue of the tile fetches below (which waits while the memory pipeline
  // is backed up).
  const int my_q = q0 + (lane & 31), g = lane >> 5;
  u32x4_t qraw[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qraw[s] = my_q < seq ? *reinterpret_cast<const u32x4_t*>(hp.q + (long long)my_q * geom.q_sr +
                                                            16 * s + 8 * g)
                         : (u32x4_t){0u, 0u, 0u, 0u};
  // This wave's K and V tiles, whole (8 segments each); rows >= N_k read
  // as zeros through the buffer bound.
  if (t0 < t1) {
    const FetchOff<8> fk = fetch_offsets<8, false>(0, lane, 2 * geom.k_sr);
    const FetchOff<8> fv = fetch_offsets<8, true>(0, lane, 2 * geom.v_sr);
#pragma unroll
    for (int i = 0; i < kQuarterTiles; ++i) {
      fetch_tile<8>(hp.rk, kb + i * kTileBytes, t0 + i, t1 - 1, 0, fk);
      fetch_tile<8>(hp.rv, vb + i * kTileBytes, t0 + i, t1 - 1, 0, fv);
    }
  }
  RowsT rows;
  rows.place(lane, q0, seq, geom.seq_k, geom.coff, cr);
  rows.set_q(qraw, cq);
  rows.reset();
  FL_ST_MARK(1);
  if (t0 < t1) {
    // This wave's own fetches have landed in LDS.
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    FL_ST_MARK(2);
    // Tile t0 sets the stabiliser to its exact row max, so its p are at most
    // 1 and its checked softmax never moves m: tile t0+1's GEMM1 can go out
    // before that softmax, against the same m.
    static_assert(kQuarterTiles == 2, "two tiles per wave");
    float16_t S0[2], S1[2];
    V8 P[2][2];
    {
      V8 ka[2][4];
      rows.read_k(kb, ka);
      rows.gemm1(ka, S0);
    }
    rows.mask(t0, S0);
    rows.first_tile(S0);
    const bool two = t0 + 1 < t1;
    if (two) {
      V8 ka[2][4];
      rows.read_k(kb + kTileBytes, ka);
      rows.gemm1(ka, S1);
    }
    rows.softmax_checked(S0, P);
    {
      V8 va[2][4];
      rows.read_v(vb, va);
      rows.gemm2(va, P);
    }
    if (two) {
      rows.mask(t0 + 1, S1);
      rows.softmax_checked(S1, P);
      V8 va[2][4];
      rows.read_v(vb + kTileBytes, va);
      rows.gemm2(va, P);
    }
  }
  FL_ST_MARK(3);
  // Merge through each sender's own (now idle) LDS: waves 1..NW-1 store
  // their partials at once and, after one barrier, wave 0 merges them in
  // order (measured 5% faster on C1 than a two-step tree, which took a
  // second barrier).  A range with no visible key holds l = 0 and is
  // skipped by the merge.
  float4* const part = reinterpret_cast<float4*>(buf[w]);
  asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");  // own LDS reads done
  if (w != 0) rows.save_partial4(part, lane);
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int s = 1; s < NW; ++s)
      rows.merge_partial4(reinterpret_cast<const float4*>(buf[s]), lane);
  }
  FL_ST_MARK(4);
  if (w != 0) {
    FL_ST_FLUSH(w, lane, 5);
    return;
  }
  rows.launder();
  rows.store(hp.o, geom.o_sr, hp.lse);
  FL_ST_FLUSH(w, lane, 5);
}

struct QuarterLaunch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      hipLaunchKernelGGL((fa2_fwd_quarter_kernel<kQuarterWaves, C, S>), grid,
                         dim3(64 * kQuarterWaves), 0, st,
                         static_cast<const _Float16*>(a.q), static_cast<const _Float16*>(a.k),
                         static_cast<const _Float16*>(a.v), static_cast<_Float16*>(a.o), g, nqb,
                         cq, cr);
      return hipSuccess;
    }
  };
};

}  // namespace

// One 4-wave work-group per 32-row query block (grid B*H*ceil(N_q/32)).
hipError_t launch_quarter(const FwdArgs& a, hipStream_t stream) {
  if (!quarter_config_fits(a)) return hipErrorInvalidValue;
  return dispatch<QuarterLaunch::L>(a, stream, 32);
}

}  // namespace fl
