// Slot-scheduled schedule (configurations br256_bc64_w8_slot and
// br128_bc64_w4_slot), fp16 and bf16 at head_dim 64.  Shared building
// blocks: fa2_common.h.

#include "fa2_common.h"

#ifndef SLOT_SPLIT_FV
#define SLOT_SPLIT_FV 3
#endif

// Per-wave timeline stamps (entry, first pass, loop start and end, store,
// exit), compiled only into the diagnostic library (diag_timeline.hip);
// empty in the product.
#ifndef FL_TL_STAMP
#define FL_TL_STAMP(name)
#define FL_TL_RECORD(...)
#endif

namespace fl {

namespace {

// ---------------------------------------------------------------------------
// Causal pair schedule (PAIR, configuration br128_bc64_w4_pair; causal,
// N_q = N_k = 128 nqb, nqb even).  Block qb of a head sees n(qb) = 2qb + 2
// key tiles, so blocks hi = nqb-1-p and lo = p (p < nqb/2) carry
// T = n(hi) + n(lo) = 2 nqb + 2 tiles together.  Two work-groups share
// each pair: member 0 walks the first h of the pair's T tiles (block hi's,
// then block lo's), member 1 the rest, so at most one block is cut between
// them.  With two co-resident work-groups per CU neither ever runs alone
// at one wave per SIMD for long, which is
// where the one-block-per-work-group causal launch loses its time (its
// heaviest block's CU finishes last).  h is above T/2 (kPairNum / 128 of
// T): the older of two work-groups on a CU issues first, so member 0 (the
// older) progresses faster while both run.
// The two members meet over the cut block in the caller's workspace, each
// at the end of its walk: member 0 (whose walk ends with the lower range)
// stores its O, m and l there (Rows::save_partial_coherent) and raises the
// pair's flag; member 1 (whose walk ends with the upper range) waits for
// the flag, merges and writes the block.  Member 0 never waits, and it is
// dispatched first (pair_coords: the same XCD, an earlier position), so
// member 1's wait always ends; it is also bounded in time (kPairWaitTicks
// of the 100 MHz s_memrealtime clock), after which member 1 writes NaN to
// the block instead of a wrong result.  Member 0 usually finishes first:
// it is the older of the two work-groups on a CU and issues first.
#ifndef FL_PAIR_NUM
#define FL_PAIR_NUM 74
#endif
constexpr int kPairNum = FL_PAIR_NUM;
constexpr int kPairPartFloats = 34 * 64;  // one wave: O (32 x 64), m, l
constexpr unsigned long long kPairWaitTicks = 10000000;  // 100 ms

// One segment of a pair member's walk: block qb, key tiles [tbeg, tend);
// role 0 = the whole block, 1 / 2 = the lower / upper key range of the cut
// block (always the walk's last segment).
struct PairSeg {
  int qb, tbeg, tend, role;
};

__device__ __forceinline__ int pair_cut(int nqb) {
  const int t = 2 * nqb + 2;
  return min(max(t * kPairNum / 128, 1), t - 1);
}

__device__ __forceinline__ int pair_nseg(int nqb, int p, int member) {
  const int n_hi = 2 * (nqb - p), h = pair_cut(nqb);
  return 1 + (member == 0 ? (h > n_hi) : (h < n_hi));
}

__device__ __forceinline__ PairSeg pair_seg(int nqb, int p, int member, int seg) {
  const int hi = nqb - 1 - p, n_hi = 2 * hi + 2, n_lo = 2 * p + 2;
  const int h = pair_cut(nqb);
  if (member == 0)
    return seg == 0 ? PairSeg{hi, 0, min(h, n_hi), h < n_hi ? 1 : 0} : PairSeg{p, 0, h - n_hi, 1};
  if (h < n_hi) return seg == 0 ? PairSeg{p, 0, n_lo, 0} : PairSeg{hi, h, n_hi, 2};
  return PairSeg{p, h - n_hi, n_lo, h > n_hi ? 2 : 0};
}

// Work-group -> (batch*head, pair p, member).  Whole heads per XCD (the
// shapes the pair schedule takes): an XCD's first half of work-groups are
// the members 0 of its pairs and the second half the members 1 in the same
// order, so each member 0 is dispatched before its member 1 on the same
// XCD, and a CU's two slots (filled in the same CU order, see wg_coords)
// hold the two members of one pair.
__device__ __forceinline__ void pair_coords(int nqb, int& bh, int& p, int& member) {
  const int per = gridDim.x >> 3;
  const int hx = per / nqb;  // whole heads per XCD
  const int half = per >> 1;
  const int i = blockIdx.x;
  const int k = i >> 3;      // dispatch position within the XCD
  member = k >= half ? 1 : 0;
  const int r = k - member * half;
  bh = (i & 7) * hx + r % hx;
  p = r / hx;
}

// Member 0, at the end of its walk: the partials of the cut block, then the
// flag.  Every access to the workspace is a relaxed device-scope atomic
// (coherent by itself across XCDs, with no cache-wide write-back); the
// partial stores are ordered before the flag by waiting for them.
template <class R>
__device__ __forceinline__ void pair_publish(unsigned* flag, float* part, int lane, const R& rows) {
  rows.save_partial_coherent(part, lane);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores acknowledged ...
  __syncthreads();                // ... and every wave's, before the flag
  if (threadIdx.x == 0) __hip_atomic_store(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Member 1, at the end of its walk: wait for the flag, clear it for the
// next call, merge.  `seen` is an LDS word no wave reads or fetches into at
// this point.
template <class R>
__device__ __forceinline__ void pair_merge(unsigned* flag, const float* part, int lane, R& rows,
                                           int* seen) {
  if (threadIdx.x == 0) {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    int ok = 0;
    for (;;) {
      if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
        ok = 1;
        break;
      }
      if (__builtin_amdgcn_s_memrealtime() - t0 > kPairWaitTicks) break;
      __builtin_amdgcn_s_sleep(2);
    }
    __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *seen = ok;
  }
  __syncthreads();  // the flag seen before any wave loads the partials
  rows.merge_partial_coherent(part, lane, /*self_lower=*/false);
  if (*seen == 0) rows.poison();
}

// ---------------------------------------------------------------------------
// Slot-scheduled pipeline: W waves of 32 query rows, one key stream.
//
// Same work per iteration j as fa2_fwd_kernel (GEMM1, GEMM2 of tile j-1
// with P(j-1), softmax of tile j), laid out as 16 MFMA slots separated by
// scheduling fences (slot map: Rows::read_slot / mfma_slot).  Each slot
// carries two exponentials of the softmax with their fp16 pack and row-sum
// share, and the LDS read of the A operand of slot +kAhead.  Measured on
// gfx950: two exponentials and two simple VALU ops issue free under one
// 32x32x16 MFMA, while longer runs of exponentials between MFMAs stall the
// matrix core, so the even spread is what keeps it busy.  GEMM1 is skewed
// by half a tile (key block 1 of tile j in slots 0-6, block 0 of tile j+1
// in slots 8-14) so that one S buffer serves both the scores being
// exponentiated and the ones being computed.
//
// The operands of the next iteration's first kAhead slots are read at the
// end of this one (K(j+1) block 1 and V(j)), so no iteration starts by
// waiting for LDS.  Iteration j reads K(j), K(j+1), V(j-1) and V(j); the
// barrier ending it publishes K(j+2) and V(j+1).  K is fetched FV+1 tiles
// ahead and V FV, into rings of FV+2 slots each, with FV-1 fetch groups in
// flight at a barrier.  Slot reuse: K(X) lands in the slot of K(X-FV-2),
// last read in iteration X-FV-2 and fetched in iteration X-FV-1; V(X) in
// that of V(X-FV-2), last read in iteration X-FV-1 and fetched in X-FV.
//
// Row sums: a packed-fp16 tree (Rows::sum_slot) on tiles that need no mask,
// fp32 adds on the masked ones (diagonal / tail), where a short causal row
// sums a few p.  Blocks whose first pass saw a tile sum out of the
// fp16-safe range are recomputed by a plain one-tile-per-step checked pass.
//
// SPLIT = 2 (configuration br128_bc64_w4x2_slot): 2W waves, two per SIMD,
// hold the same 32W query rows; waves 0..W-1 (stream 0) walk the first
// ceil(n/2) of the block's n key tiles and waves W..2W-1 (stream 1) the rest,
// each stream through its own rings, and the halves merge through LDS at
// the end (Rows::save_partial / merge_partial).  Both streams run the same
// iterations (the shorter one ends on a fully masked tile), so every wave
// meets the same barriers.  This halves the longest key walk: a causal
// work-group's time follows half its tiles, and heaviest-first dispatch of
// one work-group per CU then balances the CUs.
//
// PAIR (4 waves, causal): the pair schedule above; a work-group runs one or
// two segments (block, key-tile range) through the same pipeline, and
// geom.part holds the pairs' flags (pair_flag_words) then the partials.
template <int W, int FV, bool CAUSAL, bool SCALED, class T = _Float16, int SPLIT = 1,
          bool PAIR = false>
__global__ void __launch_bounds__(64 * W * SPLIT, 2)  // <= 256 VGPRs: 2 waves per SIMD
fa2_fwd_slot_kernel(const T* Q, const T* __restrict__ K, const T* __restrict__ V, T* O,
                    const Geom geom, int nqb, float cq, float cr) {
  using RowsT = Rows<CAUSAL, SCALED, T>;
  using V8 = typename RowsT::V8;
  // fp16: unmasked tiles sum P with the packed-fp16 tree; bf16 P keeps
  // fp32 sums throughout (an 8-bit mantissa tree would cost accuracy).
  constexpr bool kFp16 = __is_same(T, _Float16);
  // The packed-fp16 row-sum tree on unmasked tiles (fp16).
  constexpr bool kTree = kFp16;
  // bf16: row sums on the matrix core (Rows::init_msum), four 16x16x32 MFMAs
  // per tile in place of 32 fp32 adds, measured 4-7% faster on B2 H8 N4096.
  // For fp16 the packed tree's 15 adds cost less than the MFMAs (3% the
  // other way), so it keeps the tree.
  constexpr bool kMfmaSum = !kFp16;
  constexpr int FK = FV + 1;
  constexpr int kSlots = FV + 2;  // per ring
  constexpr int kUnroll = (kSlots % 2 == 0) ? kSlots : 2 * kSlots;
  constexpr int kBr = 32 * W;
  constexpr int kSegs = 8 / W;
  constexpr int kDmaPerIter = 2 * kSegs;
  constexpr int kAhead = 6;  // slots between an operand's LDS read and its MFMA
  // LDS reads of the first kAhead slots (K slots: 1, V slots: 2).
  constexpr int kTailReads = kAhead + kAhead / 2;
  constexpr int kRingBytes = kSlots * kTileBytes;
  // Two work-groups share a CU when both rings fit its 160 KiB and the
  // waves fit two per SIMD (<= 4 waves each).
  constexpr int kWgPerCu =
      (W * SPLIT <= 4 && 2 * 2 * SPLIT * kRingBytes <= 160 * 1024) ? 2 : 1;
  static_assert(kSegs * W == 8, "tile split");
  static_assert(FV >= 2 && FV <= 6, "fetch distance");
  static_assert(kAhead % 2 == 0 && kAhead < 16, "read-ahead");
  static_assert(SPLIT == 1 || SPLIT == 2, "key-range split");
  static_assert(SPLIT == 1 || SPLIT * kRingBytes >= W * 34 * 64 * 4, "merge buffer");
  static_assert(!PAIR || (CAUSAL && SPLIT == 1 && W == 4), "pair schedule: causal, 4 waves");
  __shared__ __attribute__((aligned(16))) uint8_t kring[SPLIT * kRingBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vring[SPLIT * kRingBytes];

  FL_TL_STAMP(tl_entry);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int stream = wave / W;       // key-range half (0 unless SPLIT)
  const int rw = wave - stream * W;  // 32-row block within the work-group
  int bh, qb;
  int pair = 0, member = 0;
  if constexpr (PAIR)
    pair_coords(nqb, bh, pair, member);
  else
    wg_coords<CAUSAL, kWgPerCu>(nqb, bh, qb);
  const HeadPtrs<T> hp = head_ptrs(geom, bh, Q, K, V, O);
  const i32x4_t rk = hp.rk, rv = hp.rv;
  const FetchOff<kSegs> fk = fetch_offsets<kSegs, false>(rw, lane, 2 * geom.k_sr);
  const FetchOff<kSegs> fv = fetch_offsets<kSegs, true>(rw, lane, 2 * geom.v_sr);
  const int seq = geom.seq_q;
  const StreamRings<kSlots> rings = {kring + stream * kRingBytes, vring + stream * kRingBytes};

  const int nseg = PAIR ? pair_nseg(nqb, pair, member) : 1;
  for (int seg = 0; seg < nseg; ++seg) {
  int role = 0;  // PAIR: see PairSeg
  int tbeg, tend, t0;
  if constexpr (PAIR) {
    const PairSeg sg = pair_seg(nqb, pair, member, seg);
    qb = sg.qb;
    role = sg.role;
    tbeg = sg.tbeg;
    tend = sg.tend;
    t0 = tend - tbeg;
  }
  const int q0 = qb * kBr;

  int ntiles = max(1, (geom.seq_k + kBc - 1) / kBc);
  if (CAUSAL) ntiles = min(ntiles, causal_tiles(min(q0 + kBr, seq), geom.coff));
  // This stream's key tiles [tbeg, tend); iterations 0 .. t0 on tile tbeg + j
  // (the last one only drains GEMM2; with SPLIT the shorter stream's last
  // tile lies past the range and is masked).
  if constexpr (!PAIR) {
    t0 = SPLIT == 2 ? (ntiles + 1) / 2 : ntiles;
    tbeg = stream == 0 ? 0 : t0;
    tend = stream == 0 ? t0 : ntiles;
  }
  const int last = max(tend - 1, tbeg);  // fetch clamp

  // Prologue fetch groups -FK .. -1 (V tiles < 0 read as zeros through the
  // buffer bound, which also zeroes the slot GEMM2(-1) reads under P = 0),
  // issued before the Q loads so the two latencies overlap.
  static_for(std::make_integer_sequence<int, FK>{}, [&](auto i) __attribute__((always_inline)) {
    constexpr int G = decltype(i)::value - FK;
    // (tile tbeg - 1 of stream 1 is a real tile: the zeroed P of
    // iteration 0 keeps it out of O)
    fetch_tile<kSegs>(rk, rings.kslot(Ic<G + FK>{}), tbeg + G + FK, last, rw, fk);
    fetch_tile<kSegs>(rv, rings.vslot(Ic<G + FV>{}), tbeg + G + FV, last, rw, fv);
  });
  RowsT rows;
  rows.init(hp.q, geom.q_sr, lane, q0 + 32 * rw, seq, geom.seq_k, geom.coff, cq, cr);
  if constexpr (kMfmaSum) rows.init_msum(lane);
  if ((SPLIT == 2 && stream == 0) || role == 1) rows.kv_lim = min(rows.kv_lim, tend * kBc);

  // Iterations j < jm need no mask on tiles tbeg + j and tbeg + j + 1.
  int tm = rows.kv_lim >> 6;
  if (CAUSAL) tm = min(tm, (rows.qd + 1) >> 6);
  const int jm = max(0, tm - tbeg - 1);

  // ---- first pass ----
  FL_TL_STAMP(tl_first);
  sync_ring_ahead<(FK - 1) * kDmaPerIter, 0>();  // K(0)
  float16_t S[2];
  V8 P0[2][2], P1[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) P1[a][b] = (V8){0, 0, 0, 0, 0, 0, 0, 0};
  {
    // S(tbeg) with the exact row max; iteration 0 recomputes block 1
    // against it.
    V8 ka[2][4];
    rows.read_k(rings.kslot(Ic<0>{}), ka);
    rows.gemm1(ka, S);
  }
  rows.mask(tbeg, S);
  rows.first_tile(S);
  sync_ring_ahead<(FV - 1) * kDmaPerIter, 0>();  // K(1), V(0)
  V8 ahead[kAhead];
  static_for(std::make_integer_sequence<int, kAhead>{}, [&](auto a) __attribute__((always_inline)) {
    constexpr int L = decltype(a)::value;
    ahead[L] = rows.template read_slot<L>(rings.kslot(Ic<0>{}), rings.kslot(Ic<1>{}),
                                          rings.vslot(Ic<-1>{}));
  });

  uint64_t out_of_range = 0;
  // Iteration j at unrolled position I (ring slots static): fetch K(j+FK)
  // and V(j+FV); 16 slots; the range check of tile j's sum; on MASKED
  // iterations, mask block 1 of tile j (after slot 7, before its
  // exponentials) and block 0 of tile j+1; publish K(j+2), V(j+1).
  auto iteration = [&](auto i, int j, V8 (&P)[2][2], const V8 (&Pp)[2][2],
                       auto masked) __attribute__((always_inline)) {
    constexpr int I = decltype(i)::value;
    constexpr bool kMasked = decltype(masked)::value;
    fetch_tile<kSegs>(rk, rings.kslot(Ic<I + FK>{}), tbeg + j + FK, last, rw, fk);
    fetch_tile<kSegs>(rv, rings.vslot(Ic<I + FV>{}), tbeg + j + FV, last, rw, fv);
    V8 op[16];
#pragma unroll
    for (int a = 0; a < kAhead; ++a) op[a] = ahead[a];
    half2_t tree[14];
    float sum[4];
    // SCALED: each slot scales the next slot's pair, so a slot's
    // exponentials never wait on its own multiplies.
    float xs[2][2];
    static_for(std::make_integer_sequence<int, 16>{}, [&](auto sl) __attribute__((always_inline)) {
      constexpr int L = decltype(sl)::value;
      // The MFMA goes first (fenced): its operand's wait then never covers
      // the read issued in the same slot.
      rows.template mfma_slot<L, kMfmaSum>(op[L], S, Pp);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (L + kAhead < 16)
        op[L + kAhead] = rows.template read_slot<L + kAhead>(
            rings.kslot(Ic<I>{}), rings.kslot(Ic<I + 1>{}), rings.vslot(Ic<I - 1>{}));
      else
        ahead[L + kAhead - 16] = rows.template read_slot<L + kAhead - 16>(
            rings.kslot(Ic<I + 1>{}), rings.kslot(Ic<I + 2>{}), rings.vslot(Ic<I>{}));
      if constexpr (L == 0) rows.template scale_pair<0>(S, xs[0]);
      const float epair = rows.template exp_pair<L>(xs[L & 1], P);
      if constexpr (kMfmaSum)
        ;
      else if constexpr (kTree && !kMasked)
        RowsT::template sum_slot<L>(P, tree);
      else
        RowsT::template sum_pair_f32<L>(epair, sum);
      if constexpr (kMasked && L == 7) rows.template mask_block<1>(tbeg + j, S[1]);
      if constexpr (L < 15) rows.template scale_pair<L + 1>(S, xs[(L + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (!kMfmaSum) {
      float tot;
      if constexpr (kTree && !kMasked)
        tot = RowsT::sum_root(tree);
      else
        tot = (sum[0] + sum[1]) + (sum[2] + sum[3]);
      rows.l += tot;
      out_of_range |= __builtin_amdgcn_ballot_w64(!(tot <= kSumLimit));
    }
    if constexpr (kMasked) rows.template mask_block<0>(tbeg + j + 1, S[0]);
    sync_ring_ahead<(FV - 1) * kDmaPerIter, kTailReads>();
  };
  auto group = [&](int j0, auto masked) __attribute__((always_inline)) {
    static_for(std::make_integer_sequence<int, kUnroll>{}, [&](auto i) __attribute__((always_inline)) {
      constexpr int I = decltype(i)::value;
      const int j = j0 + I;
      if (!decltype(masked)::value || j <= t0) {
        if constexpr (I % 2 == 0)
          iteration(i, j, P0, P1, masked);
        else
          iteration(i, j, P1, P0, masked);
      }
    });
  };
  FL_TL_STAMP(tl_loop);
  {
    int j0 = 0;
    for (; j0 + kUnroll <= jm; j0 += kUnroll) group(j0, Ic<false>{});
    for (; j0 <= t0; j0 += kUnroll) group(j0, Ic<true>{});
  }
  FL_TL_STAMP(tl_loop_end);
  if constexpr (kMfmaSum) {
    // Every p of the first pass is in its row's sum, so a sum within 2^40
    // bounds every p by 2^40 (finite O terms for any |V| below 2^88); a
    // larger sum, inf or NaN (a row max far above the first tile's) sends
    // the block to the checked pass.
    rows.l = rows.msum_share();
    out_of_range = __builtin_amdgcn_ballot_w64(!(rows.l <= kMsumLimit));
  }

  // ---- checked pass, when any wave saw a tile sum out of range ----
  // The work-group's flag lives in stream 0's K ring slot 1, which the
  // checked pass never refills (the rings are idle here: every wave has
  // drained its fetches and reads before the first barrier).  No extra
  // LDS, so two 80 KiB work-groups still fit one CU.  Both streams read the
  // one flag, so every wave takes the same barriers.
  __builtin_amdgcn_s_waitcnt(0);
  int* redo = reinterpret_cast<int*>(kring + kTileBytes);
  __syncthreads();
  if (threadIdx.x == 0) *redo = 0;
  __syncthreads();
  if (out_of_range != 0 && lane == 0) *redo = 1;
  __syncthreads();
  if (*redo) {
    rows.launder();
    rows.reset();
    // Both streams take t0 steps (tile tbeg + t; past tend: masked).
    for (int t = 0; t < t0; ++t) {
      fetch_tile<kSegs>(rk, rings.kslot(Ic<0>{}), tbeg + t, last, rw, fk);
      fetch_tile<kSegs>(rv, rings.vslot(Ic<0>{}), tbeg + t, last, rw, fv);
      sync_ring_ahead<0, 0>();
      float16_t Sc[2];
      V8 Pc[2][2];
      {
        V8 ka[2][4];
        rows.read_k(rings.kslot(Ic<0>{}), ka);
        rows.gemm1(ka, Sc);
      }
      rows.mask(tbeg + t, Sc);
      if (t == 0) rows.first_tile(Sc);
      rows.softmax_checked(Sc, Pc);
      {
        V8 va[2][4];
        rows.read_v(rings.vslot(Ic<0>{}), va);
        rows.gemm2(va, Pc);
      }
      sync_ring_ahead<0, 0>();  // every wave's reads done before the next fetch
    }
  }
  if constexpr (SPLIT == 2) {
    // Stream 1 hands its O, m, l to stream 0 through the (idle) rings.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    float* xchg = reinterpret_cast<float*>(kring) + rw * (34 * 64);
    if (stream == 1) rows.save_partial(xchg, lane);
    __syncthreads();
    if (stream == 1) {
      FL_TL_STAMP(tl_store);
      FL_TL_RECORD(W * SPLIT, wave, lane, t0 + 1, tl_entry, tl_first, tl_loop, tl_loop_end,
                   tl_store);
      return;
    }
    rows.merge_partial(xchg, lane);
  }
  bool owner = true;  // this work-group writes the block's output
  if constexpr (PAIR) {
    if (role != 0) {
      const long long sb = (long long)bh * (nqb >> 1) + pair;
      unsigned* flag = reinterpret_cast<unsigned*>(geom.part) + sb;
      float* part = geom.part + pair_flag_words(geom.batch_heads, nqb) +
                    (sb * W + rw) * kPairPartFloats;
      if (role == 1) {
        pair_publish(flag, part, lane, rows);
        owner = false;
      } else {
        // a word of the idle K ring past the checked pass's flag
        pair_merge(flag, part, lane, rows, reinterpret_cast<int*>(kring + kTileBytes) + 4);
      }
    }
  }
  FL_TL_STAMP(tl_store);
  if (owner) {
    rows.launder();
    rows.store(hp.o, geom.o_sr, hp.lse);
  }
  FL_TL_RECORD(W * SPLIT, wave, lane, t0 + 1, tl_entry, tl_first, tl_loop, tl_loop_end, tl_store);
  // PAIR: every wave is past its reads of the rings and their words before
  // the next segment's prologue fetches into them.
  if (PAIR && seg + 1 < nseg) __syncthreads();
  }  // segments
}

template <int W, int FV, class T = _Float16, int SPLIT = 1, bool PAIR = false>
struct SlotLaunch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      hipLaunchKernelGGL((fa2_fwd_slot_kernel<W, FV, C, S, T, SPLIT, PAIR>), grid,
                         dim3(64 * W * SPLIT), 0, st,
                         static_cast<const T*>(a.q), static_cast<const T*>(a.k),
                         static_cast<const T*>(a.v), static_cast<T*>(a.o), g, nqb, cq, cr);
      return hipSuccess;
    }
  };
};

}  // namespace

// fp16 or bf16 by a.dtype; W = 8 (256-row groups, one per CU, V fetched 4
// tiles ahead) or 4 (128-row groups, two per CU, 3 tiles ahead).
hipError_t launch_slot(const FwdArgs& a, int waves, hipStream_t stream) {
  const bool bf = a.dtype == kDtypeBF16;
  if (waves == 8)
    return bf ? dispatch<SlotLaunch<8, 4, __bf16>::L>(a, stream, 256)
              : dispatch<SlotLaunch<8, 4>::L>(a, stream, 256);
  if (waves == 4)
    return bf ? dispatch<SlotLaunch<4, 3, __bf16>::L>(a, stream, 128)
              : dispatch<SlotLaunch<4, 3>::L>(a, stream, 128);
  return hipErrorInvalidValue;
}

// Causal pair schedule (pair_fits): 128-row groups of 4 waves, two per
// CU, each half of a block pair; `workspace` as described at
// pair_workspace_bytes.
hipError_t launch_slot_pair(const FwdArgs& a, void* workspace, hipStream_t stream) {
  if (!pair_fits(a) || workspace == nullptr) return hipErrorInvalidValue;
  const int nqb = a.seq / 128;
  Geom g = make_geom(a);
  g.part = static_cast<float*>(workspace);
  const dim3 grid((unsigned)(a.batch_heads * nqb));
  const Scales sc(a);
  using Pair = SlotLaunch<4, 3, _Float16, 1, true>;
  const hipError_t e =
      sc.scaled ? Pair::template L<true, true>::run(a, g, grid, nqb, sc.cq, sc.cr, stream)
                : Pair::template L<true, false>::run(a, g, grid, nqb, sc.cq, sc.cr, stream);
  return e != hipSuccess ? e : hipGetLastError();
}

// fp16: 128-row groups of 2 x 4 waves, the key range halved between them.
hipError_t launch_slot_split(const FwdArgs& a, hipStream_t stream) {
  if (a.dtype != kDtypeF16) return hipErrorInvalidValue;
  return dispatch<SlotLaunch<4, SLOT_SPLIT_FV, _Float16, 2>::L>(a, stream, 128);
}

}  // namespace fl
