// Head dim 128 (fp16 and bf16): the slot schedule over 32-key tiles.
// Shared building blocks: fa2_common.h.

#include "fa2_common.h"

namespace fl {

namespace {

// ---------------------------------------------------------------------------
// Head dim 128 (beyond the reference, whose kernels take D = 64 only,
// kernel_flash2.cu:756-757).  Key tiles of 32 rows x 256 bytes keep the
// 8 KiB tile of D = 64, so an iteration is again 16 MFMA slots: GEMM1 is one
// 32-key block over 8 head-dim steps (one chain), GEMM2 four head-dim
// blocks over 2 key steps.  With 16 scores per lane per tile there is one
// exponential per MFMA, so the softmax VALU work fits under the matrix
// core with room to spare and the row sums stay fp32.
constexpr int kBc2 = 32;
constexpr int kRowBytes2 = 2 * kD2;  // 256

// LDS swizzles of 256-byte rows.  A row is one whole sweep of the 64 banks,
// so unlike the 128-byte rows of D = 64 the row index does not move a read
// to other banks: the swizzles must use all 4 bits of the 16-byte chunk
// index.  K (ds_read_b128, 16 lanes = 16 rows per pass): chunk ^ (row % 16)
// puts the 16 rows of a pass on 16 different chunks.  V (ds_read_b64_tr_b16:
// 2 key-rows x 2 lane groups x 4 chunks x 2 halves per 32-lane pass): the
// D = 64 pattern (row bits 0-1 on chunk bits 1-2) plus row bit 0 on chunk
// bit 3.  Both are conflict-free for every lane pattern of read_k_op and
// read_v_op (the D = 64 swizzles left 2-way conflicts on both).
__device__ __forceinline__ int k_swz128(int row) { return row & 15; }
__device__ __forceinline__ int v_swz128(int row) { return ((row & 3) << 1) | ((row & 1) << 3); }

// DMA lane offsets for 256-byte rows: segment i of wave w is rows
// 4(w kSegs + i) .. +3; lane l lands at byte 16 l of it, i.e. row l/16,
// physical chunk l%16, which holds logical chunk (l%16) ^ swz(row).
template <int kSegs, bool IS_V>
__device__ __forceinline__ FetchOff<kSegs> fetch_offsets128(int wave, int lane, int row_bytes) {
  FetchOff<kSegs> f;
#pragma unroll
  for (int i = 0; i < kSegs; ++i) {
    const int seg = wave * kSegs + i;
    const int row = 4 * seg + (lane >> 4);
    const int phys = lane & 15;
    const int logical = phys ^ (IS_V ? v_swz128(row) : k_swz128(row));
    f.lane[i] = row * row_bytes + 16 * logical;
    asm volatile("" : "+v"(f.lane[i]));
  }
  f.tile_bytes = kBc2 * row_bytes;
  return f;
}

// The 32 query rows one wave owns at head dim 128 (same lane roles as Rows:
// one query per lane, 16 of a 32-key block's scores per lane).
template <bool CAUSAL, bool SCALED, class T>
struct Rows128 {
  using E = Elem<T>;
  using V8 = typename E::v8;
  using V4 = typename E::v4;
  int g, col, qw, my_q, seq, qd, my_d, kv_lim, tr_row, tr_col;
  float cr;
  V8 qf[8];          // Q'^T B-operand, head-dim steps 0-7
  float16_t o[4];    // O^T accumulator, head-dim blocks 0-3
  float16_t bias;    // -m broadcast
  float m, l;

  __device__ __forceinline__ void init(const T* Qh, int q_sr, int lane, int qw_, int seq_,
                                       int seq_k, int coff, float cq, float cr_) {
    g = lane >> 5;
    col = lane & 31;
    qw = qw_;
    my_q = qw + col;
    qd = qw + coff;
    my_d = my_q + coff;
    seq = seq_;
    kv_lim = seq_k;
    cr = cr_;
    const int trG = lane >> 4, trj = lane & 15;
    tr_row = 4 * (trG >> 1) + (trj >> 2);
    const int tr_x = trj & 3;
    tr_col = 16 * (trG & 1) + 4 * (((tr_x & 1) << 1) | (tr_x >> 1));
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (my_q < seq) {
        const V8 raw = *reinterpret_cast<const V8*>(Qh + (long long)my_q * q_sr + 16 * s + 8 * g);
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[s][e] = (T)((float)raw[e] * cq);
      } else {
        qf[s] = (V8){0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
    reset();
  }
  __device__ __forceinline__ void launder() {
    asm volatile("" : "+v"(col), "+v"(g), "+v"(my_q), "+v"(tr_row), "+v"(tr_col));
  }
  __device__ __forceinline__ void set_m(float mm) {
    m = mm;
#pragma unroll
    for (int r = 0; r < 16; ++r) bias[r] = -mm;
  }
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    set_m(0.0f);
    l = 0.0f;
  }
  __device__ __forceinline__ V8 read_k_op(const uint8_t* kt, int st) const {
    const int ch = 2 * st + g;
    return *reinterpret_cast<const V8*>(kt + col * kRowBytes2 + 16 * (ch ^ k_swz128(col)));
  }
  __device__ __forceinline__ V8 read_v_op(const uint8_t* vt, int db, int t) const {
    const int r1 = 16 * t + tr_row;
    const int r2 = r1 + 8;
    const int dcol = 32 * db + tr_col;
    const int ch = dcol >> 3, hb = ((dcol >> 2) & 1) * 8;
    const V4 lo = lds_read_tr<V4>(vt + r1 * kRowBytes2 + 16 * (ch ^ v_swz128(r1)) + hb);
    const V4 hi = lds_read_tr<V4>(vt + r2 * kRowBytes2 + 16 * (ch ^ v_swz128(r2)) + hb);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  // Slot map: L even, GEMM1 head-dim step L/2 of the next tile (one chain,
  // steps two slots apart); L odd, u = L/2: GEMM2 head-dim block u % 4 at
  // key step u / 4.
  template <int L>
  __device__ __forceinline__ V8 read_slot(const uint8_t* kt, const uint8_t* vt) const {
    constexpr int u = L >> 1;
    if constexpr ((L & 1) == 0)
      return read_k_op(kt, u);
    else
      return read_v_op(vt, u & 3, u >> 2);
  }
  template <int L>
  __device__ __forceinline__ void mfma_slot(const V8& a, float16_t& sn, const V8 (&pp)[2]) {
    constexpr int u = L >> 1;
    if constexpr ((L & 1) == 0)
      sn = E::mfma(a, qf[u], u == 0 ? bias : sn);
    else
      o[u & 3] = E::mfma(a, pp[u >> 2], o[u & 3]);
  }
  // Softmax share of slot L: score L -> one exponential, its element of
  // the P operand (P[t] holds keys 16t + 4g + {0..3, 8..11}) and the fp32
  // row sum in four chains.
  template <int L>
  __device__ __forceinline__ void exp_slot(const float16_t& s, V8 (&pn)[2], float (&sum)[4]) const {
    float x = s[L];
    if (SCALED) x *= cr;
    const float e = __builtin_amdgcn_exp2f(x);
    pn[L >> 3][L & 7] = (T)e;
    if constexpr (L < 4)
      sum[L] = e;
    else
      sum[L & 3] += e;
  }
  // Keys >= kv_lim and, causal, past the lane's diagonal, of tile t.
  __device__ __forceinline__ void mask(int t, float16_t& s) const {
    const int k0 = t * kBc2;
    if (k0 + kBc2 > kv_lim || (CAUSAL && k0 + kBc2 - 1 > qd)) {
      const int base = k0 + 4 * g;
      int lim = kv_lim - base;
      if (CAUSAL) lim = min(lim, my_d + 1 - base);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 8 * (r >> 2) + (r & 3);
        s[r] = c < lim ? s[r] : ninf();
      }
    }
  }
  __device__ __forceinline__ float tile_max(const float16_t& s) const {
    float mx = ninf();
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
    return pair_max(mx);
  }
  __device__ __forceinline__ static void sub(float16_t& s, float d) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] -= d;
  }
  __device__ __forceinline__ void first_tile(float16_t& s) {
    float m0 = tile_max(s);
    m0 = m0 == ninf() ? 0.0f : m0;
    sub(s, m0);
    set_m(m0);
  }
  __device__ __forceinline__ float exponentiate(const float16_t& s, V8 (&pn)[2]) const {
    float sum[2] = {0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = s[r];
      if (SCALED) x *= cr;
      const float e = __builtin_amdgcn_exp2f(x);
      pn[r >> 3][r & 7] = (T)e;
      sum[r & 1] += e;
    }
    return sum[0] + sum[1];
  }
  // As Rows::softmax_checked, for one 32-key tile.
  __device__ __forceinline__ void softmax_checked(float16_t& s, V8 (&pn)[2]) {
    float sum = exponentiate(s, pn);
    if (__builtin_amdgcn_ballot_w64(!(sum <= kSumLimit)) != 0) {
      const float d = fmaxf(tile_max(s), 0.0f);
      const float alpha = __builtin_amdgcn_exp2f(-(SCALED ? cr : 1.0f) * d);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      sub(s, d);
      set_m(m + d);
      sum = exponentiate(s, pn);
    }
    l += sum;
  }
  // O = O^T / l, 16-byte stores of 8 contiguous head dims; the log-sum-exp
  // as in Rows::store.
  __device__ __forceinline__ void store(T* Oh, int o_sr, float* lse) const {
    const float l_tot = pair_sum(l);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (lse != nullptr && g == 0 && my_q < seq) {
      const float lg = m * (SCALED ? cr : 1.0f) + __builtin_amdgcn_logf(l_tot);
      lse[my_q] = l_tot > 0.0f ? 0.693147180559945309f * lg : ninf();
    }
    if (my_q < seq) {
      T* orow = Oh + (long long)my_q * o_sr;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          V8 out;
#pragma unroll
          for (int e = 0; e < 8; ++e) out[e] = (T)(o[db][8 * hh + e] * inv);
          *reinterpret_cast<V8*>(orow + 32 * db + 16 * hh + 8 * g) = out;
        }
    }
  }
};

// Causal key tiles of 32 keys a block of query rows [q0, q_end) needs.
__device__ __forceinline__ int causal_tiles32(int q_end, int coff) {
  const int last_key = q_end - 1 + coff;
  return last_key < 0 ? 1 : last_key / kBc2 + 1;
}

// Slot-scheduled head-dim-128 pipeline: W waves of 32 query rows.  Iteration
// j: GEMM1 of tile j+1 (even slots), GEMM2 of tile j-1 with P(j-1) (odd
// slots), the softmax of tile j (one exponential per slot), the LDS read of
// the operand of slot +kAhead.  S and P are double-buffered.  The operands
// of the next iteration's first kAhead slots come from K(j+2) and V(j), so
// the barrier ending iteration j publishes K(j+3) and V(j+1); K is fetched
// FK tiles ahead and V FK-2 into rings of FK slots, FK-3 fetch groups in
// flight at a barrier.  Slot reuse: K(X) lands in the slot of K(X-FK), last
// read in iteration X-FK-1; V(X) in that of V(X-FK), last read in iteration
// X-FK+1 (fetched in iteration X-FK+2).  Masked tiles, the range check and
// the checked recompute pass follow fa2_fwd_slot_kernel.
template <int W, int FK, int AHEAD, bool CAUSAL, bool SCALED, class T>
__global__ void __launch_bounds__(64 * W, 2)
fa2_fwd_d128_kernel(const T* Q, const T* __restrict__ K, const T* __restrict__ V, T* O,
                    const Geom geom, int nqb, float cq, float cr) {
  using RowsT = Rows128<CAUSAL, SCALED, T>;
  using V8 = typename RowsT::V8;
  constexpr int FV = FK - 2;
  constexpr int kSlots = FK;
  constexpr int kUnroll = (kSlots % 2 == 0) ? kSlots : 2 * kSlots;
  constexpr int kBr = 32 * W;
  constexpr int kSegs = 8 / W;
  constexpr int kDmaPerIter = 2 * kSegs;
  constexpr int kAhead = AHEAD;  // slots between an operand's LDS read and its MFMA
  constexpr int kTailReads = kAhead + kAhead / 2;  // K slots: 1 read, V slots: 2
  constexpr int kRingBytes = kSlots * kTileBytes;
  // Two work-groups share a CU when both rings fit its 160 KiB and the
  // waves fit two per SIMD (<= 4 waves each).
  constexpr int kWgPerCu = (W <= 4 && 2 * 2 * kRingBytes <= 160 * 1024) ? 2 : 1;
  static_assert(kSegs * W == 8, "tile split");
  static_assert(FK >= 4 && FK <= 8, "fetch distance");
  static_assert(kAhead % 2 == 0 && kAhead < 16, "read-ahead");
  static_assert(kTileBytes == kBc2 * kRowBytes2, "tile size");
  __shared__ __attribute__((aligned(16))) uint8_t kring[kRingBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vring[kRingBytes];

  const int lane = threadIdx.x & 63;
  const int rw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int bh, qb;
  wg_coords<CAUSAL, kWgPerCu>(nqb, geom.xcds, geom.cus_per_xcd, bh, qb);
  const HeadPtrs<T> hp = head_ptrs<T, kRowBytes2>(geom, bh, Q, K, V, O);
  const i32x4_t rk = hp.rk, rv = hp.rv;
  const FetchOff<kSegs> fk = fetch_offsets128<kSegs, false>(rw, lane, 2 * geom.k_sr);
  const FetchOff<kSegs> fv = fetch_offsets128<kSegs, true>(rw, lane, 2 * geom.v_sr);
  const int seq = geom.seq_q;
  const int q0 = qb * kBr;
  const StreamRings<kSlots> rings = {kring, vring};

  int ntiles = max(1, (geom.seq_k + kBc2 - 1) / kBc2);
  if (CAUSAL) ntiles = min(ntiles, causal_tiles32(min(q0 + kBr, seq), geom.coff));
  const int t0 = ntiles;
  const int last = ntiles - 1;

  static_for(std::make_integer_sequence<int, FK>{}, [&](auto i) __attribute__((always_inline)) {
    constexpr int G = decltype(i)::value - FK;
    fetch_tile<kSegs>(rk, rings.kslot(Ic<G + FK>{}), G + FK, last, rw, fk);
    fetch_tile<kSegs>(rv, rings.vslot(Ic<G + FV>{}), G + FV, last, rw, fv);
  });
  RowsT rows;
  rows.init(hp.q, geom.q_sr, lane, q0 + 32 * rw, seq, geom.seq_k, geom.coff, cq, cr);

  // Iterations j < jm need no mask on tile j + 1.
  int tm = rows.kv_lim / kBc2;
  if (CAUSAL) tm = min(tm, (rows.qd + 1) / kBc2);
  const int jm = max(0, tm - 1);

  sync_ring_ahead<(FK - 1) * kDmaPerIter, 0>();  // K(0)
  float16_t S0, S1;
  V8 P0[2], P1[2];
  P1[0] = P1[1] = (V8){0, 0, 0, 0, 0, 0, 0, 0};
  {
    V8 ka[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) ka[st] = rows.read_k_op(rings.kslot(Ic<0>{}), st);
#pragma unroll
    for (int st = 0; st < 8; ++st) S0 = RowsT::E::mfma(ka[st], rows.qf[st], st == 0 ? rows.bias : S0);
  }
  // Iteration 0 refills K(0)'s slot: every wave's reads of it are done.
  sync_ring_ahead<(FK - 3) * kDmaPerIter, 0>();  // K(2), V(0)
  rows.mask(0, S0);
  rows.first_tile(S0);
  V8 ahead[kAhead];
  static_for(std::make_integer_sequence<int, kAhead>{}, [&](auto a) __attribute__((always_inline)) {
    constexpr int L = decltype(a)::value;
    ahead[L] = rows.template read_slot<L>(rings.kslot(Ic<1>{}), rings.vslot(Ic<-1>{}));
  });

  uint64_t out_of_range = 0;
  auto iteration = [&](auto i, int j, float16_t& S, float16_t& Sn, V8 (&P)[2], const V8 (&Pp)[2],
                       auto masked) __attribute__((always_inline)) {
    constexpr int I = decltype(i)::value;
    fetch_tile<kSegs>(rk, rings.kslot(Ic<I + FK>{}), j + FK, last, rw, fk);
    fetch_tile<kSegs>(rv, rings.vslot(Ic<I + FV>{}), j + FV, last, rw, fv);
    V8 op[16];
#pragma unroll
    for (int a = 0; a < kAhead; ++a) op[a] = ahead[a];
    float sum[4];
    static_for(std::make_integer_sequence<int, 16>{}, [&](auto sl) __attribute__((always_inline)) {
      constexpr int L = decltype(sl)::value;
      rows.template mfma_slot<L>(op[L], Sn, Pp);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (L + kAhead < 16)
        op[L + kAhead] = rows.template read_slot<L + kAhead>(rings.kslot(Ic<I + 1>{}),
                                                             rings.vslot(Ic<I - 1>{}));
      else
        ahead[L + kAhead - 16] = rows.template read_slot<L + kAhead - 16>(
            rings.kslot(Ic<I + 2>{}), rings.vslot(Ic<I>{}));
      rows.template exp_slot<L>(S, P, sum);
      __builtin_amdgcn_sched_barrier(0);
    });
    const float tot = (sum[0] + sum[1]) + (sum[2] + sum[3]);
    rows.l += tot;
    out_of_range |= __builtin_amdgcn_ballot_w64(!(tot <= kSumLimit));
    if constexpr (decltype(masked)::value) rows.mask(j + 1, Sn);
    sync_ring_ahead<(FK - 3) * kDmaPerIter, kTailReads>();
  };
  auto group = [&](int j0, auto masked) __attribute__((always_inline)) {
    static_for(std::make_integer_sequence<int, kUnroll>{}, [&](auto i) __attribute__((always_inline)) {
      constexpr int I = decltype(i)::value;
      const int j = j0 + I;
      if (!decltype(masked)::value || j <= t0) {
        if constexpr (I % 2 == 0)
          iteration(i, j, S0, S1, P0, P1, masked);
        else
          iteration(i, j, S1, S0, P1, P0, masked);
      }
    });
  };
  {
    int j0 = 0;
    for (; j0 + kUnroll <= jm; j0 += kUnroll) group(j0, Ic<false>{});
    for (; j0 <= t0; j0 += kUnroll) group(j0, Ic<true>{});
  }

  // Checked pass (as in fa2_fwd_slot_kernel); the flag lives in K ring slot 1.
  __builtin_amdgcn_s_waitcnt(0);
  int* redo = reinterpret_cast<int*>(rings.kslot(Ic<1>{}));
  __syncthreads();
  if (threadIdx.x == 0) *redo = 0;
  __syncthreads();
  if (out_of_range != 0 && lane == 0) *redo = 1;
  __syncthreads();
  if (*redo) {
    rows.launder();
    rows.reset();
    for (int t = 0; t < ntiles; ++t) {
      fetch_tile<kSegs>(rk, rings.kslot(Ic<0>{}), t, last, rw, fk);
      fetch_tile<kSegs>(rv, rings.vslot(Ic<0>{}), t, last, rw, fv);
      sync_ring_ahead<0, 0>();
      float16_t Sc;
      V8 Pc[2];
      {
        V8 ka[8];
#pragma unroll
        for (int st = 0; st < 8; ++st) ka[st] = rows.read_k_op(rings.kslot(Ic<0>{}), st);
#pragma unroll
        for (int st = 0; st < 8; ++st)
          Sc = RowsT::E::mfma(ka[st], rows.qf[st], st == 0 ? rows.bias : Sc);
      }
      rows.mask(t, Sc);
      if (t == 0) rows.first_tile(Sc);
      rows.softmax_checked(Sc, Pc);
      {
        V8 va[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) va[u] = rows.read_v_op(rings.vslot(Ic<0>{}), u & 3, u >> 2);
#pragma unroll
        for (int u = 0; u < 8; ++u) rows.o[u & 3] = RowsT::E::mfma(va[u], Pc[u >> 2], rows.o[u & 3]);
      }
      sync_ring_ahead<0, 0>();
    }
  }
  rows.launder();
  rows.store(hp.o, geom.o_sr, hp.lse);
}

template <int W, int FK, int AHEAD, class T>
struct D128Launch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      hipLaunchKernelGGL((fa2_fwd_d128_kernel<W, FK, AHEAD, C, S, T>), grid, dim3(64 * W), 0, st,
                         static_cast<const T*>(a.q), static_cast<const T*>(a.k),
                         static_cast<const T*>(a.v), static_cast<T*>(a.o), g, nqb, cq, cr);
      return hipSuccess;
    }
  };
};

}  // namespace

// W = 8 (256-row groups) or 4 (128-row groups); fp16 or bf16 by a.dtype.
hipError_t launch_d128(const FwdArgs& a, int waves, hipStream_t stream) {
  const bool bf = a.dtype == kDtypeBF16;
  if (waves == 8)
    return bf ? dispatch<D128Launch<8, 5, 4, __bf16>::L>(a, stream, 256)
              : dispatch<D128Launch<8, 5, 4, _Float16>::L>(a, stream, 256);
  if (waves == 4)
    return bf ? dispatch<D128Launch<4, 5, 4, __bf16>::L>(a, stream, 128)
              : dispatch<D128Launch<4, 5, 4, _Float16>::L>(a, stream, 128);
  return hipErrorInvalidValue;
}

}  // namespace fl
