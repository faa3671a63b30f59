// Slot-scheduled schedule (configurations br256_bc64_w8_slot,
// br128_bc64_w4_slot, the key-range splits br128_bc64_w4x2_slot and
// br64_bc64_w2x2_slot, and the block pairs br128_bc64_w4x2_pair), fp16 and
// bf16 at head_dim 64.  Shared building blocks: fa2_common.h.

#include "fa2_common.h"


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
// Slot-scheduled pipeline: W waves of 32 query rows, one key stream.
//
// Same work per iteration j as fa2_fwd_kernel (GEMM1, GEMM2 of tile j-1
// with P(j-1), softmax of tile j), laid out as 16 MFMA slots separated by
// scheduling fences where two waves share a SIMD (kFence; slot map:
// Rows::read_slot / mfma_slot).  Each slot
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
// Row sums on the matrix core (Rows::init_msum): each key step's GEMM2 slot
// carries a 16x16x32 MFMA that sums the fp16- (bf16-) rounded p of that
// step, the weights GEMM2 multiplies, in fp32, four per tile in place of
// a VALU sum.  A packed-fp16 tree of the same p (15 adds per tile) ran as
// fast but rounded its partial sums to fp16: up to about 1e-3 of l, which
// moved moderately peaked rows (sm_scale -0.3) past the 2e-3 bound.  Blocks
// whose row sums leave the safe range (above 2^40, inf or NaN) are
// recomputed by a plain one-tile-per-step checked pass.
//
// SPLIT = 2 (configurations br128_bc64_w4x2_slot, W = 4, and
// br64_bc64_w2x2_slot, W = 2): 2W waves hold the same 32W query rows (W = 4:
// two waves per SIMD; W = 2: one per SIMD, and twice as many groups for the
// same problem, so up to 256 CUs get one each in a single round); waves
// 0..W-1 (stream 0) walk the first ceil(n/2) of the block's n key tiles and
// waves W..2W-1 (stream 1) the rest, each stream through its own rings,
// and the halves merge through LDS at the end (Rows::save_partial4 /
// merge_partial4).  Both streams run the same iterations (the shorter one
// ends on a fully masked tile), so every wave meets the same barriers.
// This halves the longest key walk: a causal work-group's time follows half
// its tiles, and heaviest-first dispatch of one work-group per CU then
// balances the CUs.
//
// PAIR (SPLIT = 2, configurations br128_bc64_w4x2_pair, W = 4, and
// br64_bc64_w2x2_pair, W = 2): a work-group walks two blocks of 32W rows of
// a head one after the other, p and nqb-1-p (the heavier first), each with
// its key range split between the streams.  Under the causal mask the two
// need about the same tiles as any other pair (2 nqb + 2 at N_q = N_k), so
// one round of work-groups, one per CU, carries equal work: no lone heavy
// block at the end (the 4-wave groups' tail) and no second round of
// start-ups (the one-block split's).
template <int W, int FV, bool CAUSAL, bool SCALED, class T = _Float16, int SPLIT = 1,
          bool PAIR = false>
// Register budget for 2 waves per SIMD (<= 256 VGPRs).  W = 2 with SPLIT
// holds 128 KiB of LDS, so one work-group (one wave per SIMD) per CU: the
// compiler reports that target as missed; that code is the measured one.
__global__ void __launch_bounds__(64 * W * SPLIT, 2)
fa2_fwd_slot_kernel(const T* Q, const T* __restrict__ K, const T* __restrict__ V, T* O,
                    const Geom geom, int nqb, float cq, float cr) {
  using RowsT = Rows<CAUSAL, SCALED, T>;
  using V8 = typename RowsT::V8;
  constexpr bool kFp16 = __is_same(T, _Float16);
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
  // Each row block's 32 query rows; with SPLIT the two streams' waves of a
  // row block share them, each fetching half.
  constexpr int kQBytes = W * 32 * kRowBytes;
  // Two work-groups share a CU when both rings and Q blocks fit its 160 KiB
  // and the waves fit two per SIMD (<= 4 waves each).
  constexpr int kWgPerCu =
      (W * SPLIT <= 4 && 2 * (2 * SPLIT * kRingBytes + kQBytes) <= 160 * 1024) ? 2 : 1;
  // Slot fences: with two waves per SIMD the even spread of each slot's
  // work keeps the matrix cores busy; a lone wave per SIMD (2 x 2 waves, one
  // group per CU) runs 2-3% faster left to the compiler's own order, and so
  // do causal fp16 4-wave groups (0.5-4%), whose heavy blocks end their walks
  // alone on their CU (bf16 ones lost 2.5% at B1 H16 N16384 without them).
  constexpr bool kFence = W * SPLIT * kWgPerCu > 4 && !(CAUSAL && kWgPerCu == 2 && kFp16);
  static_assert(kSegs * W == 8, "tile split");
  static_assert(FV >= 2 && FV <= 6, "fetch distance");
  static_assert(kAhead % 2 == 0 && kAhead < 16, "read-ahead");
  static_assert(SPLIT == 1 || SPLIT == 2, "key-range split");
  // The streams' exchange: stream 1's wave rw leaves its O, m, l (9 KiB)
  // in V ring slots 1 .. kSlots-1 of stream rw / ceil(W/2), clear of slot 0
  // (a block pair's next V(0) lands there meanwhile) and of the flag in the
  // last 16 bytes.
  constexpr int kXchgBytes = 9 * 64 * 16;
  constexpr int kXchgPerRing = (W + 1) / 2;
  static_assert(SPLIT == 1 || (kSlots - 1) * kTileBytes - 16 >= kXchgPerRing * kXchgBytes,
                "merge buffer");
  static_assert(!PAIR || SPLIT == 2, "block pairs: key-range split groups");
  __shared__ __attribute__((aligned(16))) uint8_t kring[SPLIT * kRingBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vring[SPLIT * kRingBytes];
  __shared__ __attribute__((aligned(16))) uint8_t qbuf[kQBytes];

  FL_TL_STAMP(tl_entry);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int stream = wave / W;       // key-range half (0 unless SPLIT)
  const int rw = wave - stream * W;  // 32-row block within the work-group
  int bh, qb, qb2 = 0, nblk = 1;
  if constexpr (PAIR) {
    int pr;
    pair_coords(nqb, geom.xcds, bh, pr);
    qb = nqb - 1 - pr;
    qb2 = pr;
    nblk = qb2 < qb ? 2 : 1;  // the middle block of an odd count walks alone
  } else {
    wg_coords<CAUSAL, kWgPerCu>(nqb, geom.xcds, geom.cus_per_xcd, bh, qb);
  }
  const HeadPtrs<T> hp = head_ptrs(geom, bh, Q, K, V, O);
  const FetchOff<kSegs> fk = fetch_offsets<kSegs, false>(rw, lane, 2 * geom.k_sr);
  const FetchOff<kSegs> fv = fetch_offsets<kSegs, true>(rw, lane, 2 * geom.v_sr);
  const int seq = geom.seq_q;
  const StreamRings<kSlots> rings = {kring + stream * kRingBytes, vring + stream * kRingBytes};
  // The walk of block bi: its first query row, and this stream's key tiles
  // [tbeg, tend); iterations 0 .. t0 - 1 on tile tbeg + j (with SPLIT the
  // shorter stream's last tile lies past the range and is masked).  K and V end with the stream's range: fetches
  // past it (the pipeline's look-ahead near the end of the walk) land as
  // zeros with no traffic.
  struct Walk {
    int q0, t0, tbeg, tend;
    i32x4_t rk, rv;
  };
  auto walk_of = [&](int bi) __attribute__((always_inline)) {
    Walk w;
    w.q0 = (bi == 0 ? qb : qb2) * kBr;
    int ntiles = max(1, (geom.seq_k + kBc - 1) / kBc);
    if (CAUSAL) ntiles = min(ntiles, causal_tiles(min(w.q0 + kBr, seq), geom.coff));
    w.t0 = SPLIT == 2 ? (ntiles + 1) / 2 : ntiles;
    w.tbeg = stream == 0 ? 0 : w.t0;
    w.tend = stream == 0 ? w.t0 : ntiles;
    kv_rsrc_rows(geom, bh, K, V, w.tend * kBc, w.rk, w.rv);
    return w;
  };
  uint8_t* const qblk = qbuf + rw * 32 * kRowBytes;
  // PAIR: the next block's Q and first two K tiles, fetched during this
  // block's merge and store.
  bool prefetched = false;
  // One block's walk (inlined once, or twice for a pair: a loop around the
  // body pushes the register allocator into spills).
  auto run_block = [&](const int bi) __attribute__((always_inline)) {
  FL_TL_STAMP(tl_block);
  const Walk wk = walk_of(bi);
  const int q0 = wk.q0, t0 = wk.t0, tbeg = wk.tbeg, tend = wk.tend;
  const i32x4_t rk = wk.rk, rv = wk.rv;
  const int last = max(tend - 1, tbeg);  // fetch clamp of the checked pass
  const int tzero = tend;
  // Tiles of the range this wave's rows need (through their causal
  // diagonal; none for a wave wholly past the last query row), at least
  // one: iteration nw - 1 ends the wave's GEMM2, later ones only fetch and
  // meet the barrier.
  int nw = tend - tbeg;
  if (CAUSAL) nw = min(nw, causal_tiles(min(q0 + 32 * rw + 32, seq), geom.coff) - tbeg);
  if (q0 + 32 * rw >= seq) nw = 1;
  nw = max(nw, 1);

  // This wave's 32 query rows by DMA into its Q block (first, so they
  // land first), then the prologue fetch groups -FK .. -1: K tiles
  // 0 .. FK-1 and V tiles 0 .. FV-1 of the range (iteration 0 has no
  // GEMM2, so no tile -1).  Q goes through LDS rather than straight to
  // registers: the compiler cannot see these DMA operations, so a plain
  // load of Q would wait for every one of them, one Q chunk at a time.
  // Groups -FK and -FK+1 go out before the first pass, the rest after its
  // GEMM1: a DMA instruction waits at issue while the CU's memory pipeline
  // is backed up, so the first pass would otherwise wait behind all of
  // them.  (The loop's waits count only the newest FV - 1 groups.)
  auto prologue_group = [&](auto i) __attribute__((always_inline)) {
    constexpr int G = decltype(i)::value - FK;
    fetch_tile_z<kSegs>(rk, rings.kslot(Ic<G + FK>{}), tbeg + G + FK, tzero, rw, fk);
    if constexpr (G + FV >= 0)
      fetch_tile_z<kSegs>(rv, rings.vslot(Ic<G + FV>{}), tbeg + G + FV, tzero, rw, fv);
  };
  // (A block pair's second block had Q and groups -FK, -FK+1 (K(0), K(1),
  // V(0)) fetched during the first block's merge, in the same order, so
  // the waits below count the same fetches.)
  if (!PAIR || !prefetched) {
    fetch_q_block<SPLIT>(hp.q, geom.q_sr, q0 + 32 * rw, seq, qblk, lane, stream);
    prologue_group(Ic<0>{});
    prologue_group(Ic<1>{});
  }
  RowsT rows;

  // ---- first pass ----
  FL_TL_STAMP(tl_first);
  sync_ring_ahead<kDmaPerIter, 0>();  // Q, K(0)
  rows.init_lds(qblk, lane, q0 + 32 * rw, seq, geom.seq_k, geom.coff, cq, cr);
  rows.init_msum(lane);
  if (SPLIT == 2 && stream == 0) rows.kv_lim = min(rows.kv_lim, tend * kBc);
  // Iterations j < jm need no mask on tiles tbeg + j and tbeg + j + 1.
  int tm = rows.kv_lim >> 6;
  if (CAUSAL) tm = min(tm, (rows.qd + 1) >> 6);
  const int jm = max(0, tm - tbeg - 1);
  float16_t S[2];
  V8 P0[2][2], P1[2][2];
  // Operands of the next iteration's first kAhead slots.
  V8 ahead[kAhead];
  // Key block 0 of S(tbeg), with its exact row max as the stabiliser;
  // iteration 0 computes block 1 in its even slots 0-6 and exponentiates
  // both.
  rows.gemm1_block0(rings.kslot(Ic<0>{}), S);
  static_for(std::make_integer_sequence<int, FK - 2>{}, [&](auto i) __attribute__((always_inline)) {
    prologue_group(Ic<decltype(i)::value + 2>{});
  });
  rows.template mask_block<0>(tbeg, S[0]);
  rows.first_block(S[0]);
  // iteration 0's slots 0, 2 and 4: K(tbeg) block 1, steps 0-2
  static_for(std::make_integer_sequence<int, kAhead / 2>{}, [&](auto i) __attribute__((always_inline)) {
    constexpr int a = 2 * decltype(i)::value;
    ahead[a] = rows.template read_slot<a>(rings.kslot(Ic<0>{}), rings.kslot(Ic<1>{}),
                                          rings.vslot(Ic<-1>{}));
  });
  sync_ring_ahead<(FV - 1) * kDmaPerIter, kAhead / 2>();  // K(1), V(0)

  // Iteration kinds (bits): a full iteration j runs GEMM1 of tile j block 1
  // (even slots 0-6) and of tile j+1 block 0 (even slots 8-14), GEMM2 of
  // tile j-1 (odd slots) and the softmax of tile j.  kFirst (j = 0): block
  // 0 of tile 0 comes from the first pass and there is no tile -1, so no
  // GEMM2.  kLast (the wave's last tile, j = nw - 1):
  // there is no tile after it, so even slots 8-14 run GEMM2 of tile j's
  // first 32 keys (their P is done by slot 7), and the last 32 keys'
  // GEMM2 follows slot 15 (kLastTail MFMAs): the pipeline drains inside
  // the iteration, with no iteration of its own.  Skipped MFMAs skip their
  // operand reads too.
  constexpr int kFull = 0, kFirst = 1, kLast = 2;
  constexpr int kLastTail = 4;
  constexpr auto runs = [](int kind, int L) { return (L & 1) == 0 || (kind & kFirst) == 0; };
  // kLast: the GEMM2 step (head-dim block, key step) of even slot L >= 8,
  // and of tail MFMA i.
  constexpr auto fold_db = [](int L) { return ((L - 8) >> 1) & 1; };
  constexpr auto fold_t = [](int L) { return (L - 8) >> 2; };
  // Iteration j at unrolled position I (ring slots static): fetch K(j+FK)
  // and V(j+FV); 16 slots; the range check of tile j's sum; on MASKED
  // iterations, mask block 1 of tile j (after slot 7, before its
  // exponentials) and block 0 of tile j+1; publish K(j+2), V(j+1).
  auto iteration = [&](auto i, int j, V8 (&P)[2][2], const V8 (&Pp)[2][2], auto masked,
                       auto kind) __attribute__((always_inline)) {
    constexpr int I = decltype(i)::value;
    constexpr bool kMasked = decltype(masked)::value;
    constexpr int Kd = decltype(kind)::value;
    constexpr bool kFold = (Kd & kLast) != 0;
    fetch_tile_z<kSegs>(rk, rings.kslot(Ic<I + FK>{}), tbeg + j + FK, tzero, rw, fk);
    fetch_tile_z<kSegs>(rv, rings.vslot(Ic<I + FV>{}), tbeg + j + FV, tzero, rw, fv);
    V8 op[16];
    V8 top[kLastTail];  // kLast: the tail MFMAs' operands
#pragma unroll
    for (int a = 0; a < kAhead; ++a)
      if (runs(Kd, a)) op[a] = ahead[a];
    // SCALED: each slot scales the next slot's pair, so a slot's
    // exponentials never wait on its own multiplies.
    float xs[2][2];
    static_for(std::make_integer_sequence<int, 16>{}, [&](auto sl) __attribute__((always_inline)) {
      constexpr int L = decltype(sl)::value;
      // The MFMA goes first (fenced): its operand's wait then never covers
      // the read issued in the same slot.
      if constexpr (runs(Kd, L)) {
        if constexpr (kFold && L % 2 == 0 && L >= 8)
          rows.template gemm2_step<fold_db(L), fold_t(L), true>(op[L], P);
        else
          rows.template mfma_slot<L, true>(op[L], S, Pp);
      }
      if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
      if constexpr (L + kAhead < 16) {
        constexpr int La = L + kAhead;
        if constexpr (runs(Kd, La)) {
          if constexpr (kFold && La % 2 == 0 && La >= 8)
            op[La] = rows.read_v_op(rings.vslot(Ic<I>{}), fold_db(La), fold_t(La));
          else
            op[La] = rows.template read_slot<La>(rings.kslot(Ic<I>{}), rings.kslot(Ic<I + 1>{}),
                                                 rings.vslot(Ic<I - 1>{}));
        }
      } else if constexpr (!kFold) {
        ahead[L + kAhead - 16] = rows.template read_slot<L + kAhead - 16>(
            rings.kslot(Ic<I + 1>{}), rings.kslot(Ic<I + 2>{}), rings.vslot(Ic<I>{}));
      } else if constexpr (L + kAhead - 16 < kLastTail) {
        // V(j) key steps 2 and 3 for the tail MFMAs
        constexpr int ti = L + kAhead - 16;
        top[ti] = rows.read_v_op(rings.vslot(Ic<I>{}), ti & 1, 2 + (ti >> 1));
      }
      if constexpr (L == 0) rows.template scale_pair<0>(S, xs[0]);
      rows.template exp_pair<L>(xs[L & 1], P);
      if constexpr (kMasked && L == 7) rows.template mask_block<1>(tbeg + j, S[1]);
      if constexpr (L < 15) rows.template scale_pair<L + 1>(S, xs[(L + 1) & 1]);
      if constexpr (kFence) __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (kFold) {
      // GEMM2 of tile j's last 32 keys (P complete since slot 15)
      static_for(std::make_integer_sequence<int, kLastTail>{}, [&](auto t) __attribute__((always_inline)) {
        constexpr int ti = decltype(t)::value;
        rows.template gemm2_step<ti & 1, 2 + (ti >> 1), true>(top[ti], P);
      });
    }
    if constexpr (kMasked && !kFold) rows.template mask_block<0>(tbeg + j + 1, S[0]);
    sync_ring_ahead<(FV - 1) * kDmaPerIter, kFold ? 0 : kTailReads>();
  };
  auto group = [&](int j0, auto masked, auto first) __attribute__((always_inline)) {
    static_for(std::make_integer_sequence<int, kUnroll>{}, [&](auto i) __attribute__((always_inline)) {
      constexpr int I = decltype(i)::value;
      const int j = j0 + I;
      auto& P = I % 2 == 0 ? P0 : P1;
      auto& Pp = I % 2 == 0 ? P1 : P0;
      if constexpr (decltype(first)::value && I == 0)
        iteration(i, j, P, Pp, masked, Ic<kFirst>{});
      else if (!decltype(masked)::value || j < nw - 1)
        iteration(i, j, P, Pp, masked, Ic<kFull>{});
    });
  };
  // The wave's last tile (j = nw - 1, at unrolled position I).
  auto tail = [&](auto i) __attribute__((always_inline)) {
    constexpr int I = decltype(i)::value;
    auto& P = I % 2 == 0 ? P0 : P1;
    auto& Pp = I % 2 == 0 ? P1 : P0;
    if constexpr (I == 0) {
      if (nw == 1)
        iteration(i, 0, P, Pp, Ic<true>{}, Ic<kFirst | kLast>{});
      else
        iteration(i, nw - 1, P, Pp, Ic<true>{}, Ic<kLast>{});
    } else {
      iteration(i, nw - 1, P, Pp, Ic<true>{}, Ic<kLast>{});
    }
  };
  FL_TL_STAMP(tl_loop);
  {
    // iterations 0 .. nw - 2 in unrolled groups: unmasked while every tile
    // is below the diagonal and the range end (j < jm <= nw - 1), then
    // masked; then the wave's last tile, whose iteration drains GEMM2
    if (nw >= 2) {
      int j0 = kUnroll;
      if (kUnroll <= jm) {
        group(0, Ic<false>{}, Ic<true>{});
        for (; j0 + kUnroll <= jm; j0 += kUnroll) group(j0, Ic<false>{}, Ic<false>{});
      } else {
        group(0, Ic<true>{}, Ic<true>{});
      }
      for (; j0 < nw - 1; j0 += kUnroll) group(j0, Ic<true>{}, Ic<false>{});
    }
    static_for(std::make_integer_sequence<int, kUnroll>{}, [&](auto i) __attribute__((always_inline)) {
      if ((nw - 1) % kUnroll == decltype(i)::value) tail(i);
    });
    // Past its last tile (iterations nw .. t0 - 1, when other waves of the
    // work-group need more tiles) a wave only fetches its share of the
    // tiles and meets the barrier.
    for (int j = nw; j < t0; ++j) {
      fetch_tile_z<kSegs>(rk, rings.k + kTileBytes * ((j + FK) % kSlots), tbeg + j + FK, tzero, rw,
                          fk);
      fetch_tile_z<kSegs>(rv, rings.v + kTileBytes * ((j + FV) % kSlots), tbeg + j + FV, tzero, rw,
                          fv);
      sync_ring_ahead<(FV - 1) * kDmaPerIter, 0>();
    }
  }
  FL_TL_STAMP(tl_loop_end);
  // Every p of the first pass is in its row's sum, so a sum within 2^40
  // bounds every p by 2^40 (finite O terms for any |V| below 2^88); a
  // larger sum, inf or NaN (a row max far above the first tile's, or an
  // fp16 p past 65504) sends the block to the checked pass.
  rows.l = rows.msum_share();
  const uint64_t out_of_range = __builtin_amdgcn_ballot_w64(!(rows.l <= kMsumLimit));

  // ---- checked pass, when any wave saw a row sum out of range ----
  // The work-group's flag lives in the last 16 bytes of the V rings, which
  // neither the checked pass (slot 0) nor the streams' exchange touches
  // (the rings are idle here: every wave has drained its fetches and reads
  // before the first barrier).  No extra LDS, so two 4-wave work-groups
  // still fit one CU.  Both streams read the one flag,
  // so every wave takes the same barriers.
  __builtin_amdgcn_s_waitcnt(0);
  int* redo = reinterpret_cast<int*>(vring + SPLIT * kRingBytes - 16);
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
  if (PAIR && bi + 1 < nblk) {
    // Every wave is past its reads of the rings and of its Q block (the
    // flag's barriers, or the checked pass's last one): the next block's Q,
    // K(0), K(1) and V(0) go out now, to land during the merge and store.
    const Walk nx = walk_of(bi + 1);
    fetch_q_block<SPLIT>(hp.q, geom.q_sr, nx.q0 + 32 * rw, seq, qblk, lane, stream);
    fetch_tile_z<kSegs>(nx.rk, rings.kslot(Ic<0>{}), nx.tbeg, nx.tend, rw, fk);
    fetch_tile_z<kSegs>(nx.rk, rings.kslot(Ic<1>{}), nx.tbeg + 1, nx.tend, rw, fk);
    fetch_tile_z<kSegs>(nx.rv, rings.vslot(Ic<0>{}), nx.tbeg, nx.tend, rw, fv);
    prefetched = true;
  }
  if constexpr (SPLIT == 2) {
    // Stream 1 hands its O, m, l to stream 0 through the (idle) V rings.
    // (Only LDS needs to settle: the fetches still in flight, the next
    // block's, write the K rings, V slot 0 and the Q blocks.)
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    __syncthreads();
    float4* const xchg = reinterpret_cast<float4*>(
        vring + (rw / kXchgPerRing) * kRingBytes + kTileBytes + (rw % kXchgPerRing) * kXchgBytes);
    if (stream == 1) rows.save_partial4(xchg, lane);
    __syncthreads();
    if (stream == 0) rows.merge_partial4(xchg, lane);
  }
  FL_TL_STAMP(tl_store);
  if (SPLIT == 1 || stream == 0) {
    rows.launder();
    rows.store(hp.o, geom.o_sr, hp.lse);
  }
  // (a pair records each block: wave + 8 bi of 16 records per work-group)
  FL_TL_RECORD(PAIR ? 2 * W * SPLIT : W * SPLIT, wave + bi * W * SPLIT, lane, t0,
               (bi == 0 ? tl_entry : tl_block), tl_first, tl_loop, tl_loop_end, tl_store);
  // PAIR: every wave past its reads of the rings (the merge's included)
  // before the next block's prologue fetches into them.
  if (PAIR && bi + 1 < nblk) __syncthreads();
  };  // run_block
  run_block(0);
  if constexpr (PAIR) {
    if (nblk > 1) run_block(1);
  }
}

template <int W, int FV, class T = _Float16, int SPLIT = 1, bool PAIR = false>
struct SlotLaunch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      if constexpr (PAIR) grid = dim3((unsigned)(a.batch_heads * ((nqb + 1) / 2)));
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
// tiles ahead) or 4 (128-row groups, two per CU, 2 tiles ahead: 64 KiB of
// rings, measured 0.3-4% faster than 3 from N 1024 to 8192, causal C2
// included).
hipError_t launch_slot(const FwdArgs& a, int waves, hipStream_t stream) {
  const bool bf = a.dtype == kDtypeBF16;
  if (waves == 8)
    return bf ? dispatch<SlotLaunch<8, 4, __bf16>::L>(a, stream, 256)
              : dispatch<SlotLaunch<8, 4>::L>(a, stream, 256);
  if (waves == 4)
    return bf ? dispatch<SlotLaunch<4, 2, __bf16>::L>(a, stream, 128)
              : dispatch<SlotLaunch<4, 2>::L>(a, stream, 128);
  return hipErrorInvalidValue;
}

// V fetch distance of the key-range splits: rings of 4 tiles (128 KiB per
// group), measured 1-6% faster than 3 (160 KiB) on the shapes the
// dispatcher sends to them; their walks are short, so the shorter prologue
// matters more than the deeper pipeline.
constexpr int kSplitFv = 2;

// fp16 or bf16 by a.dtype: groups of 2 x `waves` waves (4: 128-row blocks,
// 2: 64-row blocks) walking a pair of blocks of a head, p and nqb-1-p, each
// with its key range halved between the streams (grid B*H*ceil(nqb/2)).
hipError_t launch_slot_pair(const FwdArgs& a, int waves, hipStream_t stream) {
  const bool bf = a.dtype == kDtypeBF16;
  if (waves == 4)
    return bf ? dispatch<SlotLaunch<4, kSplitFv, __bf16, 2, true>::L>(a, stream, 128)
              : dispatch<SlotLaunch<4, kSplitFv, _Float16, 2, true>::L>(a, stream, 128);
  if (waves == 2)
    return bf ? dispatch<SlotLaunch<2, kSplitFv, __bf16, 2, true>::L>(a, stream, 64)
              : dispatch<SlotLaunch<2, kSplitFv, _Float16, 2, true>::L>(a, stream, 64);
  return hipErrorInvalidValue;
}

// fp16 or bf16 by a.dtype: groups of 2 x `waves` waves (4: 128 rows, 2: 64
// rows), the key range halved between them.
hipError_t launch_slot_split(const FwdArgs& a, int waves, hipStream_t stream) {
  const bool bf = a.dtype == kDtypeBF16;
  if (waves == 4)
    return bf ? dispatch<SlotLaunch<4, kSplitFv, __bf16, 2>::L>(a, stream, 128)
              : dispatch<SlotLaunch<4, kSplitFv, _Float16, 2>::L>(a, stream, 128);
  if (waves == 2)
    return bf ? dispatch<SlotLaunch<2, kSplitFv, __bf16, 2>::L>(a, stream, 64)
              : dispatch<SlotLaunch<2, kSplitFv, _Float16, 2>::L>(a, stream, 64);
  return hipErrorInvalidValue;
}

}  // namespace fl
