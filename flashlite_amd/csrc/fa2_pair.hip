// Paired-block slot schedule (configuration br256_bc64_w4_pair): each wave
// owns 64 query rows -- two 32-row blocks A and B (struct Rows each) -- so
// every K and V^T operand read from LDS feeds two MFMAs, one per block.  A
// work-group is 4 waves (256 rows) with one wave per SIMD, which leaves the
// SIMD's whole register file to one wave.
// Shared building blocks: fa2_common.h.
//
// Why.  In the 32-row slot schedule (fa2_slot.hip) at two waves per SIMD,
// the C2 counters show the matrix core busy about half of the kernel's
// cycles, with roughly a third of SIMD cycles issuing nothing (both waves
// waiting).  Per MFMA this layout halves the LDS reads, the waits on them,
// the fetch instructions and the barriers, and a single wave per SIMD
// issues in the order the slots fix, with no second wave competing for the
// matrix core or the VALU.
//
// Iteration j: 32 MFMA slots; slot L = 2u + q.
//   q = 0 (GEMM1), block X = u & 1, K operand k = u >> 1 serving both blocks:
//     u < 8:  S_X[1] (+)= K(j) rows 32-63 . Q'_X (st = u >> 1)
//     u >= 8: S_X[0] (+)= K(j+1) rows 0-31 . Q'_X (st = (u - 8) >> 1)
//   Exponentials, two per slot: slot group g = L >> 2 exponentiates key
//   step t = g >> 1 of block g & 1 (scores 4t .. 4t+3 of the block's 16
//   per-lane pairs), i.e. A t0, B t0, A t1, B t1, A t2, ... B t3, packing
//   P_X(t) as it goes.
//   q = 1 (GEMM2), O_X[db] += V^T(j)(db, t) . P_X(t), two slots after the
//   exponentials that finish P_X(t) (table kGemm2 below); block B's last
//   key step runs in slots 1 and 3 of the next iteration.  So GEMM2 trails
//   the softmax by a few slots instead of a whole tile, and one P buffer
//   per block suffices: P_X(t) of tile j+1 is written only after GEMM2 of
//   tile j has read it.
// Each S block is rewritten only after its exponentials have read it:
// S_X[1](j) is computed in slots 0-14 and exponentiated in 16-31; S_X[0](j+1)
// is computed in slots 16-30 after S_X[0](j) was exponentiated in 0-15.
// Operands are read 8 slots before their first MFMA; those of the next
// iteration's first slots are read at the end of this one, from tiles the
// previous barrier published (K(j+1), V(j+1)).
//
// Registers.  The scores must sit in VGPRs, where the exponentials read
// them; left to itself the compiler gives every MFMA of a one-wave-per-SIMD
// kernel an AGPR destination, which would cost a v_accvgpr_read per score.
// GEMM1 is therefore issued from inline assembly with VGPR operands
// (mfma_s below) while GEMM2 keeps the builtin, whose O accumulators then
// live in AGPRs.  The assembly carries no hazard information, so every
// reader of an S block is placed by construction at least two MFMA slots
// (64 cycles) after the MFMA that writes it, beyond the 32x32x16
// XDL-write-to-VALU-read wait of gfx950, and an explicit wait guards the
// one place where that does not hold (the mask of S_X[0](j+1) right after
// the last slot).
//
// K/V rings, fetch distances, the branch-free first pass with its range
// check, and the work-group-wide checked recompute are those of the 32-row
// slot schedule; the first pass has no drain iteration (GEMM2 of the last
// tile finishes two MFMAs after the loop).

#include "fa2_common.h"

#ifndef PAIR_AHEAD
#define PAIR_AHEAD 8
#endif

namespace fl {

namespace {

// S (+)= A . B in VGPRs.  First step: C from a separate register set (the
// -m bias); the early clobber keeps the destination off every source.
__device__ __forceinline__ void mfma_s_first(float16_t& d, const half8_t& a, const half8_t& b,
                                             const float16_t& c) {
  asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, %3" : "=&v"(d) : "v"(a), "v"(b), "v"(c));
}
__device__ __forceinline__ void mfma_s_acc(float16_t& d, const half8_t& a, const half8_t& b) {
  asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}

// GEMM2 slot table: odd slot 2u+1 -> (block, key step t, head-dim block db).
// u 0-1 finish block B's key step 3 of the previous tile.
struct G2 {
  int blk, t, db;
};
constexpr G2 kGemm2[16] = {{1, 3, 0}, {1, 3, 1}, {0, 0, 0}, {0, 0, 1}, {1, 0, 0}, {1, 0, 1},
                           {0, 1, 0}, {0, 1, 1}, {1, 1, 0}, {1, 1, 1}, {0, 2, 0}, {0, 2, 1},
                           {1, 2, 0}, {1, 2, 1}, {0, 3, 0}, {0, 3, 1}};
// V^T operand v = 2t + db: first use (block A) at slot kVFirst[v]; block B
// reuses it four slots later (t = 3: slots 1 and 3 of the next iteration).
constexpr int kVFirst[8] = {5, 7, 13, 15, 21, 23, 29, 31};
// V^T operands whose first use lies less than `ahead` slots into the
// iteration.
constexpr int kVAhead(int ahead) {
  int n = 0;
  for (int v = 0; v < 8; ++v) n += kVFirst[v] < ahead ? 1 : 0;
  return n;
}

template <int FV, int AHEAD, bool CAUSAL, bool SCALED>
__global__ void __launch_bounds__(256, 1)  // one wave per SIMD
fa2_fwd_pair_kernel(const _Float16* Q, const _Float16* __restrict__ K,
                    const _Float16* __restrict__ V, _Float16* O, const Geom geom, int nqb,
                    float cq, float cr) {
  using RowsT = Rows<CAUSAL, SCALED, _Float16>;
  using V8 = half8_t;
  constexpr int W = 4;
  constexpr int FK = FV + 1;
  constexpr int kSlots = FV + 2;  // per ring
  constexpr int kUnroll = (kSlots % 2 == 0) ? kSlots : 2 * kSlots;
  constexpr int kBr = 64 * W;
  constexpr int kSegs = 8 / W;
  constexpr int kDmaPerIter = 2 * kSegs;
  // Slots between an operand's LDS read and its first MFMA; operands whose
  // read slot falls before slot 0 are read at the end of the previous
  // iteration (kAheadK K operands, kAheadV V^T operands).
  constexpr int kAhead = AHEAD;
  constexpr int kAheadK = (kAhead + 3) / 4;
  constexpr int kAheadV = kVAhead(kAhead);
  // LDS read instructions of the next iteration's first operands (one per
  // K operand, two per V^T operand) that may be in flight at the barrier.
  constexpr int kTailReads = kAheadK + 2 * kAheadV;
  static_assert(kAhead >= 4 && kAhead <= 16 && kTailReads < 16, "read-ahead");
  constexpr int kRingBytes = kSlots * kTileBytes;
  static_assert(FV >= 2 && FV <= 8, "fetch distance");
  static_assert(2 * kRingBytes <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) uint8_t kring[kRingBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vring[kRingBytes];

  const int lane = threadIdx.x & 63;
  const int rw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int bh, qb;
  wg_coords<CAUSAL, 1>(nqb, bh, qb);
  const HeadPtrs<_Float16> hp = head_ptrs(geom, bh, Q, K, V, O);
  const i32x4_t rk = hp.rk, rv = hp.rv;
  const FetchOff<kSegs> fk = fetch_offsets<kSegs, false>(rw, lane, 2 * geom.k_sr);
  const FetchOff<kSegs> fv = fetch_offsets<kSegs, true>(rw, lane, 2 * geom.v_sr);
  const int seq = geom.seq_q;
  const int q0 = qb * kBr;
  const StreamRings<kSlots> rings = {kring, vring};

  int ntiles = max(1, (geom.seq_k + kBc - 1) / kBc);
  if (CAUSAL) ntiles = min(ntiles, causal_tiles(min(q0 + kBr, seq), geom.coff));
  const int last = ntiles - 1;

  // Prologue fetch groups: K(0..FV) and V(0..FV); V(t) is consumed in
  // iteration t like K(t), so both rings run FK tiles ahead.
  static_for(std::make_integer_sequence<int, FK>{}, [&](auto i) __attribute__((always_inline)) {
    constexpr int G = decltype(i)::value;
    fetch_tile<kSegs>(rk, rings.kslot(Ic<G>{}), G, last, rw, fk);
    fetch_tile<kSegs>(rv, rings.vslot(Ic<G>{}), G, last, rw, fv);
  });
  RowsT ra, rb;
  ra.init(hp.q, geom.q_sr, lane, q0 + 64 * rw, seq, geom.seq_k, geom.coff, cq, cr);
  rb.init(hp.q, geom.q_sr, lane, q0 + 64 * rw + 32, seq, geom.seq_k, geom.coff, cq, cr);

  // Iterations j < jm need no mask on tiles j and j + 1 (block A has the
  // earlier diagonal).
  int tm = ra.kv_lim >> 6;
  if (CAUSAL) tm = min(tm, (ra.qd + 1) >> 6);
  const int jm = max(0, tm - 1);

  // ---- first pass ----
  sync_ring_ahead<(FK - 1) * kDmaPerIter, 0>();  // K(0)
  float16_t SA[2], SB[2];
  // P^T operands, block X, key step t = 2kb + h: dwords PX[kb][h][0..3]
  // (fp16 pairs), as MFMA operands bit_cast to half8_t.
  u32x4_t PA[2][2], PB[2][2];
  V8 carry[2];  // V^T(j) operands of key step 3, for block B's GEMM2 in slots 1, 3 of j+1
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    carry[a] = (V8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < 2; ++b) PB[a][b] = (u32x4_t){0, 0, 0, 0};
  }
  {
    // S(0) with the exact row maxima; iteration 0 recomputes key block 1.
    V8 ka[2][4];
    ra.read_k(rings.kslot(Ic<0>{}), ka);
    ra.gemm1(ka, SA);
    rb.gemm1(ka, SB);
  }
  ra.mask(0, SA);
  rb.mask(0, SB);
  ra.first_tile(SA);
  rb.first_tile(SB);
  // K(1) and V(0) landed (V(j) is read in iteration j).
  sync_ring_ahead<(FV - 1) * kDmaPerIter, 0>();

  // K operand k of iteration j: K(j) key block 1 (k < 4) or K(j+1) key
  // block 0; V^T operand v = 2t + db of V(j).
  auto read_kop = [&](int k, const uint8_t* k_cur, const uint8_t* k_next)
                      __attribute__((always_inline)) {
    return k < 4 ? ra.read_k_op(k_cur, 1, k) : ra.read_k_op(k_next, 0, k - 4);
  };
  auto read_vop = [&](int v, const uint8_t* vt) __attribute__((always_inline)) {
    return ra.read_v_op(vt, v & 1, v >> 1);
  };
  V8 aheadK[kAheadK], aheadV[kAheadV];
#pragma unroll
  for (int a = 0; a < kAheadK; ++a) aheadK[a] = read_kop(a, rings.kslot(Ic<0>{}), rings.kslot(Ic<1>{}));
#pragma unroll
  for (int a = 0; a < kAheadV; ++a) aheadV[a] = read_vop(a, rings.vslot(Ic<0>{}));

  // Exponentials of slot L (block X, pair E) land in ex[L & 1]; one slot
  // later they are packed to fp16 and added to the row sum, so no
  // instruction of a slot waits on another of the same slot (one wave per
  // SIMD issues in order: a stalled VALU instruction would hold back the
  // next MFMA).  Row sums are fp32 sums of the unrounded p, as the
  // reference takes them (kernel_flash2.cu:268-276, :339): per block, the
  // pair sums of a tile go round four chains (partial[X][c]); the tile sum
  // (their total) is range-checked and added to l after the tile.
  float ex[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
  float partial[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  auto exps = [&](auto L_, float (&e)[2]) __attribute__((always_inline)) {
    constexpr int L = decltype(L_)::value;
    constexpr int grp = L >> 2;
    constexpr int E = 4 * (grp >> 1) + (L & 3);
    constexpr int kb = E >> 3, r = 2 * (E & 7);
    const float16_t(&S)[2] = (grp & 1) ? SB : SA;
    float x0 = S[kb][r], x1 = S[kb][r + 1];
    if (SCALED) {
      x0 *= cr;
      x1 *= cr;
    }
    e[0] = __builtin_amdgcn_exp2f(x0);
    e[1] = __builtin_amdgcn_exp2f(x1);
  };
  // The empty asm pins the v_cvt_pk_f16_f32 to its slot (otherwise it is
  // emitted next to the MFMA that reads the operand).
  auto pack = [&](auto L_, const float (&e)[2]) __attribute__((always_inline)) {
    constexpr int L = decltype(L_)::value;
    constexpr int grp = L >> 2;
    constexpr int E = 4 * (grp >> 1) + (L & 3);
    constexpr int kb = E >> 3, h = (E >> 2) & 1, d = E & 3;
    u32x4_t(&P)[2][2] = (grp & 1) ? PB : PA;
    const half2_t pk = {(_Float16)e[0], (_Float16)e[1]};
    uint32_t w = __builtin_bit_cast(uint32_t, pk);
    asm volatile("" : "+v"(w));
    P[kb][h][d] = w;
  };
  auto pop = [](const u32x4_t& w) __attribute__((always_inline)) {
    return __builtin_bit_cast(half8_t, w);
  };
  // Row-sum share of slot L's pair (block X, pair E): chain E % 4 of the
  // block, started fresh by the tile's first four pairs.
  auto add_sum = [&](auto L_, const float (&e)[2]) __attribute__((always_inline)) {
    constexpr int L = decltype(L_)::value;
    constexpr int grp = L >> 2;
    constexpr int E = 4 * (grp >> 1) + (L & 3);
    float(&c)[4] = partial[grp & 1];
    const float t = e[0] + e[1];
    if constexpr (E < 4)
      c[E & 3] = t;
    else
      c[E & 3] += t;
  };
  // The tile's sums for block X (after its last pair was added).
  auto tile_sum = [&](int X) __attribute__((always_inline)) {
    const float(&c)[4] = partial[X];
    return (c[0] + c[1]) + (c[2] + c[3]);
  };
  uint64_t out_of_range = 0;

  // Iteration j at unrolled position I: K(j), V(j) in slot I of their
  // rings, K(j+1), V(j+1) in slot I+1; fetch K(j+FK) and V(j+FK).  Slot
  // reuse: tile X lands in the slot of tile X - FV - 2, whose last reads
  // (iteration X - FV - 2 and the tail reads before it) completed before the
  // barrier that ends iteration X - FV - 2, and the fetch is issued after
  // it, in iteration X - FK.
  auto iteration = [&](auto i, int j, auto masked) __attribute__((always_inline)) {
    constexpr int I = decltype(i)::value;
    constexpr bool kMasked = decltype(masked)::value;
    fetch_tile<kSegs>(rk, rings.kslot(Ic<I + FK>{}), j + FK, last, rw, fk);
    fetch_tile<kSegs>(rv, rings.vslot(Ic<I + FK>{}), j + FK, last, rw, fv);
    V8 kop[8], vop[8];
#pragma unroll
    for (int a = 0; a < kAheadK; ++a) kop[a] = aheadK[a];
#pragma unroll
    for (int a = 0; a < kAheadV; ++a) vop[a] = aheadV[a];
    static_for(std::make_integer_sequence<int, 32>{}, [&](auto sl) __attribute__((always_inline)) {
      constexpr int L = decltype(sl)::value;
      constexpr int u = L >> 1;
      // The MFMA goes first (fenced): its operand's wait then never covers
      // the read issued in the same slot.
      if constexpr ((L & 1) == 0) {
        constexpr bool kB = (u & 1) != 0;
        constexpr int k = u >> 1;
        constexpr int kb = u < 8 ? 1 : 0, st = k & 3;
        RowsT& r = kB ? rb : ra;
        float16_t& s = kB ? SB[kb] : SA[kb];
        if constexpr (st == 0)
          mfma_s_first(s, kop[k], r.qf[st], r.bias);
        else
          mfma_s_acc(s, kop[k], r.qf[st]);
      } else {
        constexpr G2 g = kGemm2[u];
        constexpr int v = 2 * g.t + g.db;
        RowsT& r = g.blk ? rb : ra;
        const u32x4_t(&pp)[2][2] = g.blk ? PB : PA;
        const V8& a = (u < 2) ? carry[g.db] : vop[v];
        r.o[g.db] = RowsT::E::mfma(a, pop(pp[g.t >> 1][g.t & 1]), r.o[g.db]);
      }
      __builtin_amdgcn_sched_barrier(0);
      // Operand reads, kAhead slots before the first use: K op k at slot
      // 4k - kAhead, V^T op v at kVFirst[v] - kAhead (the previous
      // iteration's slot + 32 when negative).
      static_for(std::make_integer_sequence<int, 8>{}, [&](auto kk) __attribute__((always_inline)) {
        constexpr int k = decltype(kk)::value;
        constexpr int at = 4 * k - kAhead;
        if constexpr (at == L) kop[k] = read_kop(k, rings.kslot(Ic<I>{}), rings.kslot(Ic<I + 1>{}));
        if constexpr (at + 32 == L)
          aheadK[k] = read_kop(k, rings.kslot(Ic<I + 1>{}), rings.kslot(Ic<I + 2>{}));
      });
      static_for(std::make_integer_sequence<int, 8>{}, [&](auto vv) __attribute__((always_inline)) {
        constexpr int v = decltype(vv)::value;
        constexpr int at = kVFirst[v] - kAhead;
        if constexpr (at == L) vop[v] = read_vop(v, rings.vslot(Ic<I>{}));
        if constexpr (at + 32 == L) aheadV[v] = read_vop(v, rings.vslot(Ic<I + 1>{}));
      });
      // Two exponentials of this slot's pair; the pack and row-sum share of
      // the previous slot's (slot 31's pair, block B's last, is packed in
      // slot 0 of the next iteration; block A's tile sum is complete after
      // slot 28, block B's after slot 0 of the next iteration and is taken
      // before B's next tile restarts the chains in slot 5).
      exps(Ic<L>{}, ex[L & 1]);
      pack(Ic<(L + 31) & 31>{}, ex[(L + 1) & 1]);
      add_sum(Ic<(L + 31) & 31>{}, ex[(L + 1) & 1]);
      if constexpr (L == 2) {
        // Block B of the previous tile (0 before iteration 0).
        const float tb = tile_sum(1);
        rb.l += tb;
        out_of_range |= __builtin_amdgcn_ballot_w64(!(tb <= kSumLimit));
      }
      if constexpr (L == 29) {
        const float ta = tile_sum(0);
        ra.l += ta;
        out_of_range |= __builtin_amdgcn_ballot_w64(!(ta <= kSumLimit));
      }
      // Masked iterations: key block 1 of tile j, after its last GEMM1
      // MFMA (slot 12 for A, 14 for B) and before its exponentials (slots
      // 16 and 20).
      if constexpr (kMasked && L == 15) ra.template mask_block<1>(j, SA[1]);
      if constexpr (kMasked && L == 19) rb.template mask_block<1>(j, SB[1]);
      __builtin_amdgcn_sched_barrier(0);
    });
    carry[0] = vop[6];
    carry[1] = vop[7];
    if constexpr (kMasked) {
      // S_B[0](j+1) was written by slot 30's MFMA: wait it out before the
      // VALU reads it.
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      ra.template mask_block<0>(j + 1, SA[0]);
      rb.template mask_block<0>(j + 1, SB[0]);
    }
    sync_ring_ahead<(FV - 1) * kDmaPerIter, kTailReads>();
  };
  auto group = [&](int j0, auto masked) __attribute__((always_inline)) {
    static_for(std::make_integer_sequence<int, kUnroll>{}, [&](auto i) __attribute__((always_inline)) {
      const int j = j0 + decltype(i)::value;
      if (!decltype(masked)::value || j < ntiles) iteration(i, j, masked);
    });
  };
  {
    int j0 = 0;
    for (; j0 + kUnroll <= jm; j0 += kUnroll) group(j0, Ic<false>{});
    for (; j0 < ntiles; j0 += kUnroll) group(j0, Ic<true>{});
  }
  // The last tile: block B's last pack and row-sum share, its tile sum and
  // its key step 3.
  pack(Ic<31>{}, ex[1]);
  add_sum(Ic<31>{}, ex[1]);
  {
    const float tb = tile_sum(1);
    rb.l += tb;
    out_of_range |= __builtin_amdgcn_ballot_w64(!(tb <= kSumLimit));
  }
  rb.o[0] = RowsT::E::mfma(carry[0], pop(PB[1][1]), rb.o[0]);
  rb.o[1] = RowsT::E::mfma(carry[1], pop(PB[1][1]), rb.o[1]);

  // ---- checked pass, when any wave saw a tile sum out of range ----
  // (flag in K ring slot 1, as in the 32-row slot schedule)
  __builtin_amdgcn_s_waitcnt(0);
  int* redo = reinterpret_cast<int*>(rings.kslot(Ic<1>{}));
  __syncthreads();
  if (threadIdx.x == 0) *redo = 0;
  __syncthreads();
  if (out_of_range != 0 && lane == 0) *redo = 1;
  __syncthreads();
  if (*redo) {
    ra.launder();
    rb.launder();
    ra.reset();
    rb.reset();
    for (int t = 0; t < ntiles; ++t) {
      fetch_tile<kSegs>(rk, rings.kslot(Ic<0>{}), t, last, rw, fk);
      fetch_tile<kSegs>(rv, rings.vslot(Ic<0>{}), t, last, rw, fv);
      sync_ring_ahead<0, 0>();
      float16_t Sa[2], Sb[2];
      V8 Pa[2][2], Pb[2][2];
      {
        V8 ka[2][4];
        ra.read_k(rings.kslot(Ic<0>{}), ka);
        ra.gemm1(ka, Sa);
        rb.gemm1(ka, Sb);
      }
      ra.mask(t, Sa);
      rb.mask(t, Sb);
      if (t == 0) {
        ra.first_tile(Sa);
        rb.first_tile(Sb);
      }
      ra.softmax_checked(Sa, Pa);
      rb.softmax_checked(Sb, Pb);
      {
        V8 va[2][4];
        ra.read_v(rings.vslot(Ic<0>{}), va);
        ra.gemm2(va, Pa);
        rb.gemm2(va, Pb);
      }
      sync_ring_ahead<0, 0>();  // every wave's reads done before the next fetch
    }
  }
  ra.launder();
  rb.launder();
  ra.store(hp.o, geom.o_sr, hp.lse);
  rb.store(hp.o, geom.o_sr, hp.lse);
}

template <int FV>
struct PairLaunch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      hipLaunchKernelGGL((fa2_fwd_pair_kernel<FV, PAIR_AHEAD, C, S>), grid, dim3(256), 0, st,
                         static_cast<const _Float16*>(a.q), static_cast<const _Float16*>(a.k),
                         static_cast<const _Float16*>(a.v), static_cast<_Float16*>(a.o), g, nqb,
                         cq, cr);
      return hipSuccess;
    }
  };
};

}  // namespace

// fp16 at head_dim 64: 256-row groups of 4 waves, one per CU.
hipError_t launch_pair(const FwdArgs& a, hipStream_t stream) {
  if (a.dtype != kDtypeF16) return hipErrorInvalidValue;
  return dispatch<PairLaunch<4>::L>(a, stream, 256);
}

}  // namespace fl
