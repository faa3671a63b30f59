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
// and reads no K or V another wave wrote; the block's Q comes through one
// shared 4 KiB of LDS by the same DMA, issued first, a quarter by each
// wave, and one barrier publishes it.  Each wave
// computes both tiles' scores, takes their exact row max as the one
// stabiliser (every p <= 1, so no range check and no second pass), then
// exponentiates and multiplies tile by tile; the quarters' O, m and l
// merge through LDS in 16-byte chunks at their largest m, each wave merging
// and storing a quarter of the head dims of every row.  C1 then runs 1024
// waves of 2 tiles instead of 256 waves of 8.  LDS: 4 x 32 KiB, one
// work-group per CU, plus 4 KiB of Q.  (Eight waves of one tile each, two
// per SIMD, measured 7% slower on C1.)
//
// RB = 2 (more than 256 blocks of 32 rows, up to 512): a work-group of 8
// waves owns two 32-row blocks, wave 4 rb + q taking row block rb and key
// quarter q.  The two waves of a quarter fetch half of its tiles each into
// the quarter's 32 KiB and read all of it, so a barrier publishes the tiles;
// two more order the merge (every quarter's K/V read before any partial
// overwrites it; partials written before the row block's waves fold them
// in).  Up to 512 blocks then still run in one round, two waves per
// SIMD.
//
// KVSPLIT (split-KV chunks of at most 8 tiles, RB = 1): work-group i takes
// key chunk i % nsplit of its query block, the waves a quarter of the
// chunk each, and the merged partial (O unnormalised, m, l) that
// splitkv_combine_kernel folds together is written as the one-wave chunks
// of the pipelined kernel write theirs, a quarter of the head dims by each
// wave.  A decode step's chunk is then a 2-tile chain
// per wave instead of an up-to-8-tile one.
constexpr int kQuarterWaves = 4;

template <int NW, int RB, bool CAUSAL, bool SCALED, class T, bool KVSPLIT = false>
__global__ void __launch_bounds__(64 * NW * RB, 1)
fa2_fwd_quarter_kernel(const T* Q, const T* __restrict__ K, const T* __restrict__ V, T* O,
                       const Geom geom, int nqb, float cq, float cr) {
  using RowsT = Rows<CAUSAL, SCALED, T>;
  using V8 = typename RowsT::V8;
  constexpr int kQuarterTiles = kQuarterMaxKeys / kBc / NW;  // key tiles per wave
  constexpr int kQuarterWaveBytes = 2 * kQuarterTiles * kTileBytes;
  static_assert(NW * kQuarterTiles * kBc == kQuarterMaxKeys, "key range");
  static_assert(RB == 1 || RB == 2, "row blocks per group");
  static_assert(!KVSPLIT || RB == 1, "split-KV chunks hold one row block");
  static_assert(RB * (9 * 64) * 16 <= kQuarterWaveBytes, "partials fit a quarter's LDS");
  constexpr int kSegs = 8 / RB;  // 1 KiB segments of a tile each wave of a quarter fetches
  __shared__ __attribute__((aligned(16))) uint8_t buf[NW][kQuarterWaveBytes];
  // each row block's 32 query rows (4 KiB), fetched a quarter by each of
  // its NW waves
  __shared__ __attribute__((aligned(16))) uint8_t qbuf[RB][32 * kRowBytes];
  static_assert(NW == 4, "one 1 KiB Q segment per wave of a row block");

  FL_ST_DECL();
  FL_ST_MARK(0);
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = RB == 1 ? w : w % NW;  // key quarter
  const int rb = RB == 1 ? 0 : w / NW;  // 32-row block within the group
  int bh, qb, chunk = 0;
  if constexpr (KVSPLIT) {
    const int r = blockIdx.x / geom.nsplit;
    chunk = blockIdx.x - r * geom.nsplit;
    bh = r / nqb;
    qb = r - bh * nqb;
  } else {
    bh = blockIdx.x / nqb;
    qb = blockIdx.x - bh * nqb;
  }
  const HeadPtrs<T> hp = head_ptrs<T>(geom, bh, Q, K, V, O);
  const int seq = geom.seq_q;
  const int q0 = 32 * RB * qb;  // the group's first row
  const int all_tiles = (geom.seq_k + kBc - 1) / kBc;
  int ntiles = all_tiles;
  if (CAUSAL) ntiles = min(ntiles, causal_tiles(min(q0 + 32 * RB, seq), geom.coff));
  // The group's key tiles [cbeg, cend): all of them, or its split-KV chunk
  // (the same cut as the pipelined kernel's chunks).
  int cbeg = 0, cend = ntiles;
  if constexpr (KVSPLIT) {
    const int per = (max(all_tiles, 1) + geom.nsplit - 1) / geom.nsplit;
    cbeg = chunk * per;
    cend = min(ntiles, cbeg + per);
  }
  const int t0 = cbeg + kQuarterTiles * kq;
  const int t1 = min(t0 + kQuarterTiles, cend);
  uint8_t* const kb = buf[kq];
  uint8_t* const vb = buf[kq] + kQuarterTiles * kTileBytes;
  uint8_t* const qblk = qbuf[rb];

  // The row block's 32 query rows come by DMA like a K half-tile (rows >=
  // N_q read as zeros through the resource's bound), 8 rows by each of its
  // four waves, then each wave's quarter's tiles in the order they are used:
  // K, K, V, V.  Each wave waits for one piece at a time (the DMA is
  // invisible to the compiler's own counting, so the waits are explicit);
  // one barrier publishes the Q rows, and a wave starts computing as soon as
  // K of its first tile has landed.  Tiles past the quarter land as zeros
  // with no traffic.
  const int qr = q0 + 32 * rb;  // this wave's rows
  {
    const int qrows = min(32, seq - qr);
    const i32x4_t rq = buffer_rsrc(hp.q + (long long)(qrows > 0 ? qr : 0) * geom.q_sr,
                                   qrows > 0 ? (qrows - 1) * (2 * geom.q_sr) + kRowBytes : 0);
    const FetchOff<1> fq = fetch_offsets<1, false>(kq, lane, 2 * geom.q_sr);
    fetch_tile_z<1>(rq, qblk, 0, 1, kq, fq);
  }
  i32x4_t rk, rv;
  kv_rsrc_rows(geom, bh, K, V, t1 * kBc, rk, rv);
  const bool any = t0 < t1;
  const FetchOff<kSegs> fk = fetch_offsets<kSegs, false>(rb, lane, 2 * geom.k_sr);
  const FetchOff<kSegs> fv = fetch_offsets<kSegs, true>(rb, lane, 2 * geom.v_sr);
  auto fetch_k = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kQuarterTiles; ++i)
      fetch_tile_z<kSegs>(rk, kb + i * kTileBytes, t0 + i, t1, rb, fk);
  };
  auto fetch_v = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kQuarterTiles; ++i)
      fetch_tile_z<kSegs>(rv, vb + i * kTileBytes, t0 + i, t1, rb, fv);
  };
  // RB = 1: Q and K go out first and V after the first tile's scores: a
  // DMA instruction waits at issue while the CU's memory pipeline is backed
  // up, so issuing V before any compute would hold every wave behind all
  // of its CU's loads.  Outstanding fetches of the wave, oldest first:
  // its Q segment (1), K(t0), K(t0+1), then V(t0), V(t0+1) (kSegs each).
  // RB = 2 issues everything at once: a barrier publishes the tiles either
  // way.
  static_assert(kQuarterTiles == 2, "two tiles per wave");
  constexpr int kT = kSegs;
  if (any) fetch_k();
  if (RB > 1 && any) fetch_v();
  RowsT rows;
  rows.place(lane, qr, seq, geom.seq_k, geom.coff, cr);
  rows.reset();
  if constexpr (RB == 1) {
    // this wave's Q segment; one barrier publishes the block's four
    if (any)
      asm volatile("s_waitcnt vmcnt(%0)" : : "n"(2 * kT) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    __syncthreads();
  } else {
    // the other wave of each quarter fetched half of every tile, and the
    // row block's other waves the rest of its Q: one barrier publishes
    // them all (taken by every wave)
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    __syncthreads();
  }
  rows.set_q_lds(qblk, cq);
  FL_ST_MARK(1);
  if (any) {
    FL_ST_MARK(2);
    // Both tiles' scores against one stabiliser, the exact row max over
    // them: every p is then at most 1 and the row sum at most 128, so the
    // softmax needs no range check.  A row with no visible key gets m = 0
    // and p = 0.
    const bool two = t0 + 1 < t1;
    float16_t S0[2], S1[2];
    V8 P[2][2];
    if constexpr (RB == 1) asm volatile("s_waitcnt vmcnt(%0)" : : "n"(kT) : "memory");
    {
      V8 ka[2][4];
      rows.read_k(kb, ka);
      rows.gemm1(ka, S0);
    }
    if constexpr (RB == 1) {
      fetch_v();
      asm volatile("s_waitcnt vmcnt(%0)" : : "n"(2 * kT) : "memory");
    }
    {
      V8 ka[2][4];
      rows.read_k(kb + kTileBytes, ka);
      rows.gemm1(ka, S1);
    }
    rows.mask(t0, S0);
    if (two) rows.mask(t0 + 1, S1);
    {
      float mx = ninf();
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, S0[h][r]);
      if (two) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, S1[h][r]);
      }
      mx = pair_max(mx);
      mx = mx == ninf() ? 0.0f : mx;
      RowsT::sub(S0, mx);
      if (two) RowsT::sub(S1, mx);
      rows.set_m(mx);
    }
    rows.l = rows.exponentiate(S0, P);
    if constexpr (RB == 1) asm volatile("s_waitcnt vmcnt(%0)" : : "n"(kT) : "memory");
    {
      V8 va[2][4];
      rows.read_v(vb, va);
      rows.gemm2(va, P);
    }
    if (two) {
      rows.l += rows.exponentiate(S1, P);
      if constexpr (RB == 1) asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
      V8 va[2][4];
      rows.read_v(vb + kTileBytes, va);
      rows.gemm2(va, P);
    }
  }
  FL_ST_MARK(3);
  // Merge through each quarter's (now idle) LDS.  Row block rb's partials
  // start rb x 9 KiB into the quarter's buffer; a range with no visible key
  // holds l = 0 and is skipped by the merge.  Every quarter stores its
  // partial and, after one barrier, wave kq of the row block merges and
  // stores the kq-th 8-column chunk of every row (Rows::merge_store_chunk,
  // or for a split-KV chunk the fp32 partial, merge_store_partial_chunk):
  // 12 of the partials' 36 float4s per lane and a quarter of the stores
  // each.
  float4* const part = reinterpret_cast<float4*>(buf[kq]) + rb * (9 * 64);
  // own LDS reads done, and every fetch landed (a one-tile quarter's zero
  // tiles too: nothing may still write this LDS once the group ends)
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" : : : "memory");
  if constexpr (RB > 1) __syncthreads();  // and the other row block's
  rows.save_partial4(part, lane);
  __syncthreads();
  const float4* parts[NW];
#pragma unroll
  for (int j = 0; j < NW; ++j) parts[j] = reinterpret_cast<const float4*>(buf[j]) + rb * (9 * 64);
  if constexpr (KVSPLIT)
    rows.template merge_store_partial_chunk<NW>(
        parts, kq, lane, geom.part + (long long)(chunk * geom.batch_heads + bh) * seq * kPartStride);
  else
    rows.template merge_store_chunk<NW>(parts, kq, lane, hp.o, geom.o_sr, hp.lse);
  FL_ST_MARK(4);
  FL_ST_FLUSH(w, lane, 5);
}

template <int RB, class T>
struct QuarterLaunch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      hipLaunchKernelGGL((fa2_fwd_quarter_kernel<kQuarterWaves, RB, C, S, T>), grid,
                         dim3(64 * kQuarterWaves * RB), 0, st, static_cast<const T*>(a.q),
                         static_cast<const T*>(a.k), static_cast<const T*>(a.v),
                         static_cast<T*>(a.o), g, nqb, cq, cr);
      return hipSuccess;
    }
  };
};

template <class T>
hipError_t launch_quarter_t(const FwdArgs& a, hipStream_t stream) {
  const int64_t blocks32 = (a.seq + 31) / 32 * (int64_t)a.batch_heads;
  if (blocks32 > device_cus())
    return dispatch<QuarterLaunch<2, T>::template L>(a, stream, 64);
  return dispatch<QuarterLaunch<1, T>::template L>(a, stream, 32);
}

}  // namespace

// fp16 or bf16 by a.dtype: one 4-wave work-group per 32-row query block
// (grid B*H*ceil(N_q/32)) up to one per CU; beyond that one 8-wave
// work-group per 64 rows.
hipError_t launch_quarter(const FwdArgs& a, hipStream_t stream) {
  if (!quarter_config_fits(a)) return hipErrorInvalidValue;
  return a.dtype == kDtypeBF16 ? launch_quarter_t<__bf16>(a, stream)
                               : launch_quarter_t<_Float16>(a, stream);
}

#ifndef FL_QUARTER_NO_SPLITKV
// Split-KV with key-quarter chunks (fp16): grid B*H*ceil(N_q/32)*nsplit
// 4-wave work-groups, every chunk at most kQuarterMaxKeys keys, then the
// combine kernel on the same stream.
hipError_t launch_kvsplit_quarter(const FwdArgs& a, float* part, int nsplit, hipStream_t st) {
  const int all_tiles = a.seq_k > 0 ? (a.seq_k + kBc - 1) / kBc : 1;
  if (a.dtype != kDtypeF16 || nsplit < 1 ||
      (all_tiles + nsplit - 1) / nsplit * kBc > kQuarterMaxKeys)
    return hipErrorInvalidValue;
  const int nqb = (a.seq + 31) / 32;
  const Scales sc(a);
  Geom g = make_geom(a);
  g.part = part;
  g.nsplit = nsplit;
  const dim3 grid((unsigned)(nqb * a.batch_heads * nsplit));
  const dim3 block(64 * kQuarterWaves);
  const _Float16 *q = static_cast<const _Float16*>(a.q), *k = static_cast<const _Float16*>(a.k),
                 *v = static_cast<const _Float16*>(a.v);
  _Float16* o = static_cast<_Float16*>(a.o);
  constexpr int NW = kQuarterWaves;
  if (a.causal) {
    if (sc.scaled)
      hipLaunchKernelGGL((fa2_fwd_quarter_kernel<NW, 1, true, true, _Float16, true>), grid, block,
                         0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_quarter_kernel<NW, 1, true, false, _Float16, true>), grid,
                         block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
  } else {
    if (sc.scaled)
      hipLaunchKernelGGL((fa2_fwd_quarter_kernel<NW, 1, false, true, _Float16, true>), grid,
                         block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_quarter_kernel<NW, 1, false, false, _Float16, true>), grid,
                         block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_splitkv_combine(a, part, nsplit, st);
}
#endif

}  // namespace fl
