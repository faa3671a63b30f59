// Streaming persistent schedule for key ranges of at most 256 keys
// (configuration br256_kv256_w8_stream).  Shared building blocks:
// fa2_common.h.

#include "fa2_common.h"

// Per-wave timeline marks (kernel entry; per unit: past its barrier, loads of
// the next unit issued, stores issued), compiled only into the diagnostic
// library (diag_timeline.hip); empty in the product.
#ifndef FL_ST_MARK
#define FL_ST_DECL()
#define FL_ST_MARK(index)
#define FL_ST_FLUSH(wave, lane, count)
#endif

namespace fl {

namespace {

// ---------------------------------------------------------------------------
// Short key ranges (N_k <= 256, e.g. many heads of 256 tokens): a unit is
// one head's block of up to 256 query rows, whose whole K and V (4 tiles
// each, 64 KiB) fit one LDS buffer.  A persistent work-group of 8 waves (32
// rows each) walks units u = blockIdx.x, + gridDim.x, ... through two such
// buffers: after the barrier that publishes unit i, each wave reads its Q
// rows, then issues unit i+1's K/V fetches (into the buffer unit i-1 used)
// and its own next Q rows (into the 4 KiB it just read), then computes unit
// i and stores it.  Causal units with all 256 rows: waves 0-3 (1-2 key tiles
// each) issue the fetches of their SIMD-mates w+4 (3-4 tiles) as well, after
// a barrier that has every wave's Q rows read; a DMA instruction waits at
// issue while the memory pipeline is backed up (2-7 us for a unit's loads),
// and the mates' longer walks then start at once.  Per-wave memory
// operations per unit are fixed (8 K/V and 4 Q fetches, or 16 + 8 and none
// when sharing; 5 stores last; out-of-range rows are dropped by the buffer
// bounds, never branched around), so "unit i's loads have landed" is
// exactly vmcnt <= 5: only unit i-1's stores may still be in flight.  With
// one short unit per work-group, the start-up latency of every unit (Q and
// K/V from HBM) would idle the CU; here it overlaps the previous unit's
// compute.  LDS: 2 x 64 KiB of K/V + 32 KiB of Q = all 160 KiB of the CU.
// Within a unit no barrier is needed: every key tile is resident, so each
// wave pipelines its own tiles (GEMM1 of tile t+1 and GEMM2 of tile t-1
// beside the softmax of tile t) and, in the rare case its stabiliser check
// fails, recomputes them one at a time (Rows::softmax_checked).
constexpr int kStreamBr = 256;                           // query rows per unit
constexpr int kStreamTiles = 4;                          // key tiles per unit (N_k <= 256)
constexpr int kStreamHalf = kStreamTiles * kTileBytes;   // K (or V) of a unit: 32 KiB

// vmcnt wait then the work-group barrier (a compiler memory barrier too).
template <int kPending>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(kPending >= 0 && kPending < 64, "vmcnt range");
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(kPending) : "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// SPREAD (at least 4 units per work-group over 4 key tiles): the next
// unit's K/V fetches go out one tile pair per tile step of the current
// unit's compute (the rest after it) instead of all before it, so a wave's
// compute starts without waiting for their issue.  Measured 4-6% faster on
// B32 H32 N256 and slower where a work-group has one or two short units,
// where the extra code in the steps costs more than it hides.
template <bool CAUSAL, bool SCALED, class T = _Float16, bool SPREAD = false>
__global__ void __launch_bounds__(512, 2)  // <= 256 VGPRs: 8 waves, two per SIMD
fa2_fwd_stream_kernel(const T* Q, const T* __restrict__ K, const T* __restrict__ V, T* O,
                      const Geom geom, int nqb, int units, float cq, float cr) {
  using RowsT = Rows<CAUSAL, SCALED, T>;
  using V8 = typename RowsT::V8;
  constexpr int kStores = 5;  // Rows::store_rsrc
  __shared__ __attribute__((aligned(16))) uint8_t buf[2][2 * kStreamHalf];  // [unit parity][K | V]
  __shared__ __attribute__((aligned(16))) uint8_t qbuf[8 * 4096];            // 32 Q rows per wave

  FL_ST_DECL();
  const int lane = threadIdx.x & 63;
  const int rw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5, col = lane & 31;
  const FetchOff<1> fk = fetch_offsets<1, false>(rw, lane, 2 * geom.k_sr);
  const FetchOff<1> fv = fetch_offsets<1, true>(rw, lane, 2 * geom.v_sr);
  const int seq = geom.seq_q;
  const int qrow_bytes = 2 * geom.q_sr;
  int ntiles = (geom.seq_k + kBc - 1) / kBc;  // 1..4 (the host checks N_k <= 256)
  // The wave's 32-row block of a unit.  Waves w and w+4 share a SIMD; under
  // the causal mask block j needs j/2 + 1 tiles, so pairing blocks j and
  // 7-j gives every SIMD five tiles per unit instead of four to six.
  const int blk = CAUSAL && rw >= 4 ? 11 - rw : rw;

  // Unit u's K/V tiles 0..3 into buffer b (rows >= N_k read as zeros) and
  // 32 Q rows into a wave's 4 KiB of qbuf (rows >= N_q read as zeros), all
  // by LDS DMA; chunks swizzled as K tiles are.  Wave w fetches segment w
  // (rows 8w..8w+7) of every tile and its own Q rows; with `mate`, also
  // those of wave w+4.
  auto q_offsets = [&](int b_blk, int (&off)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int lrow = 8 * i + (lane >> 3);
      off[i] = (32 * b_blk + lrow) * qrow_bytes + 16 * ((lane & 7) ^ k_swz(lrow));
      asm volatile("" : "+v"(off[i]));
    }
  };
  int qoff[4];
  q_offsets(blk, qoff);
  // Causal units whose mates' blocks (rows 128-255) all hold rows.
  constexpr bool kShare = CAUSAL;
  const bool share = kShare && seq > kStreamBr - 32;
  int qoff2[4];  // wave w+4's Q rows and tile segments (waves 0-3)
  FetchOff<1> fk2 = fk, fv2 = fv;
  if constexpr (kShare) {
    q_offsets(11 - (rw + 4), qoff2);
    fk2 = fetch_offsets<1, false>(rw + 4, lane, 2 * geom.k_sr);
    fv2 = fetch_offsets<1, true>(rw + 4, lane, 2 * geom.v_sr);
  }
  uint8_t* const qdst = qbuf + 4096 * rw;
  auto issue_kv = [&](const HeadPtrs<T>& hp, int b, int t, bool mate) __attribute__((always_inline)) {
    fetch_tile<1>(hp.rk, buf[b] + t * kTileBytes, t, kStreamTiles - 1, rw, fk);
    fetch_tile<1>(hp.rv, buf[b] + kStreamHalf + t * kTileBytes, t, kStreamTiles - 1, rw, fv);
    if (kShare && mate) {
      fetch_tile<1>(hp.rk, buf[b] + t * kTileBytes, t, kStreamTiles - 1, rw + 4, fk2);
      fetch_tile<1>(hp.rv, buf[b] + kStreamHalf + t * kTileBytes, t, kStreamTiles - 1, rw + 4,
                    fv2);
    }
  };
  auto issue_q = [&](const HeadPtrs<T>& hp, int u, bool mate) __attribute__((always_inline)) {
    const int q0 = (u - (u / nqb) * nqb) * kStreamBr;
    const int valid = min(kStreamBr, seq - q0);
    const i32x4_t rq =
        buffer_rsrc(hp.q + (long long)q0 * geom.q_sr, (valid - 1) * qrow_bytes + kRowBytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lds_base = (uint32_t)(uintptr_t)(qdst + 1024 * i);
      asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(qoff[i]), "s"(rq),
                   "{m0}"(lds_base));
    }
    if (kShare && mate) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lds_base = (uint32_t)(uintptr_t)(qdst + 4 * 4096 + 1024 * i);
        asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(qoff2[i]), "s"(rq),
                     "{m0}"(lds_base));
      }
    }
  };
  auto issue_loads = [&](int u, int b, bool mate) __attribute__((always_inline)) {
    const HeadPtrs<T> hp = head_ptrs<T>(geom, u / nqb, Q, K, V, O);
#pragma unroll
    for (int t = 0; t < kStreamTiles; ++t) issue_kv(hp, b, t, mate);
    issue_q(hp, u, mate);
  };

  const int G = gridDim.x;
  // Unit u in buffer b; its loads have landed and every wave is done with
  // the other buffer.
  auto unit = [&](int u, int b, int ui) __attribute__((always_inline)) {
    (void)ui;  // the unit's index within this work-group (timeline marks)
    const int bh = u / nqb, qb = u - bh * nqb;
    const int q0 = qb * kStreamBr;
    const int qw = q0 + 32 * blk;
    RowsT rows;
    rows.place(lane, qw, seq, geom.seq_k, geom.coff, cr);
    // Opaque per unit: with N_q <= 256 every unit has the same rows, and the
    // masks and addresses derived from them would otherwise be hoisted out
    // of the unit loop and kept live (spilled) across it.
    rows.launder();
    asm volatile("" : "+v"(rows.my_d), "+v"(rows.qd), "+v"(rows.kv_lim), "+v"(rows.qw));
    {
      u32x4_t raw[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        raw[s] = *reinterpret_cast<const u32x4_t*>(qdst + 128 * col +
                                                    16 * ((2 * s + g) ^ k_swz(col)));
      rows.set_q(raw, cq);
    }
    rows.reset();
    // This wave's Q reads are done before its DMA refills the same rows
    // (when sharing: every wave's, before waves 0-3 refill their mates').
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    const bool more = u + G < units;
    if (share && more) __syncthreads();
    const bool fetcher = more && (!share || rw < 4);
    // SPREAD: the next unit's Q rows now, its K/V tile pairs one per tile
    // step below and the rest after the steps.
    const HeadPtrs<T> hn = head_ptrs<T>(geom, SPREAD && more ? (u + G) / nqb : 0, Q, K, V, O);
    int kv_sent = SPREAD && fetcher ? 0 : kStreamTiles;
    auto kv_next = [&]() __attribute__((always_inline)) {
      if (SPREAD && kv_sent < kStreamTiles) {
        issue_kv(hn, b ^ 1, kv_sent, share);
        ++kv_sent;
      }
    };
    if (fetcher) {
      if constexpr (SPREAD)
        issue_q(hn, u + G, share);
      else
        issue_loads(u + G, b ^ 1, share);
    }
    FL_ST_MARK(2 + 3 * ui);

    int nt = ntiles;
    if (CAUSAL) nt = min(nt, causal_tiles(min(qw + 32, seq), geom.coff));
    if (qw < seq) {
      const uint8_t* kb = buf[b];
      const uint8_t* vb = buf[b] + kStreamHalf;
      // Units with at least 3 tiles for this wave: a software-pipelined
      // first pass.  Step t issues GEMM2 of tile t-1 (with P(t-1), whose
      // registers the softmax of S(t) then refills) and GEMM1 of tile t+1,
      // both MFMA chains independent of that softmax, with the stabiliser m
      // fixed at tile 0's exact row max; out_of_range records, branch-free,
      // any tile sum that left the fp16-safe range.  The last step's GEMM1
      // (tile nt, never used) reads other finite LDS data and is masked;
      // below 3 tiles that waste outweighs the overlap and the tiles go
      // straight to the one-at-a-time checked loop.
      bool checked = nt < 3;
      if (!checked) {
        uint64_t out_of_range = 0;
        float16_t S0[2], S1[2];
        V8 P[2][2];
        {
          V8 ka[2][4];
          rows.read_k(kb, ka);
          rows.gemm1(ka, S0);
        }
        rows.mask(0, S0);
        rows.first_tile(S0);
        auto step = [&](int t, float16_t (&S)[2], float16_t (&Sn)[2]) __attribute__((always_inline)) {
          if constexpr (SPREAD) kv_next();
          V8 ka[2][4];
          rows.read_k(kb + (t + 1) * kTileBytes, ka);
          if (t > 0) {
            V8 va[2][4];
            rows.read_v(vb + (t - 1) * kTileBytes, va);
            rows.gemm2(va, P);
          }
          rows.gemm1(ka, Sn);
          out_of_range |= rows.softmax_fast(S, P);
          rows.mask(t + 1, Sn);
        };
        // At most kStreamTiles steps: unrolled, so S0 / S1 keep fixed roles.
        step(0, S0, S1);
        static_for(std::make_integer_sequence<int, kStreamTiles - 1>{}, [&](auto i)
                   __attribute__((always_inline)) {
          constexpr int t = decltype(i)::value + 1;
          if (t < nt) {
            if constexpr (t & 1)
              step(t, S1, S0);
            else
              step(t, S0, S1);
          }
        });
        {
          V8 va[2][4];
          rows.read_v(vb + (nt - 1) * kTileBytes, va);
          rows.gemm2(va, P);
        }
        checked = out_of_range != 0;
      }
      // The checked loop: one tile at a time, rescaling when a row max rises
      // (also the recompute for a wave whose first pass left the range).
      if (checked) {
        rows.reset();
        for (int t = 0; t < nt; ++t) {
          if constexpr (SPREAD) kv_next();
          float16_t S[2];
          V8 P[2][2];
          {
            V8 ka[2][4];
            rows.read_k(kb + t * kTileBytes, ka);
            rows.gemm1(ka, S);
          }
          rows.mask(t, S);
          if (t == 0) rows.first_tile(S);
          rows.softmax_checked(S, P);
          {
            V8 va[2][4];
            rows.read_v(vb + t * kTileBytes, va);
            rows.gemm2(va, P);
          }
        }
      }
    }
    if constexpr (SPREAD)
      while (kv_sent < kStreamTiles) kv_next();
    const int valid = min(kStreamBr, seq - q0);
    const int b_ = bh / geom.heads, h_ = bh - b_ * geom.heads;
    T* oh = O + (b_ * geom.o_sb + h_ * geom.o_sh) + (long long)q0 * geom.o_sr;
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        (void*)oh, 0, (valid - 1) * 2 * geom.o_sr + kRowBytes, 0x00020000);
    float* lh = geom.lse ? geom.lse + (long long)bh * seq + q0 : geom.lse;
    const __amdgpu_buffer_rsrc_t rl =
        __builtin_amdgcn_make_buffer_rsrc((void*)lh, 0, geom.lse ? 4 * valid : 0, 0x00020000);
    FL_ST_MARK(3 + 3 * ui);
    rows.store_rsrc(ro, q0, 2 * geom.o_sr, rl);
  };
  // The first unit is peeled off: its wait also covers the launch's first
  // loads, and every later one has exactly one unit's stores behind it.
  FL_ST_MARK(0);
  int u = blockIdx.x;
  issue_loads(u, 0, false);
  wait_vm_barrier<0>();
  FL_ST_MARK(1);
  unit(u, 0, 0);
  u += G;
  int i = 1;
  for (; u < units; ++i, u += G) {
    wait_vm_barrier<kStores>();  // only unit i-1's stores may be in flight
    FL_ST_MARK(1 + 3 * i);
    unit(u, i & 1, i);
  }
  FL_ST_FLUSH(rw, lane, 1 + 3 * i);
}

// Streaming short-key kernel: one persistent work-group per CU (its two
// 64 KiB buffers take 128 KiB of the CU's 160 KiB), at most one per unit.
template <class T, bool SPREAD>
hipError_t launch_stream_v(const FwdArgs& a, hipStream_t st, dim3 grid, int nqb, int units) {
  const Scales sc(a);
  const Geom g = make_geom(a);
  const T *q = static_cast<const T*>(a.q), *k = static_cast<const T*>(a.k),
          *v = static_cast<const T*>(a.v);
  T* o = static_cast<T*>(a.o);
  if (a.causal) {
    if (sc.scaled)
      hipLaunchKernelGGL((fa2_fwd_stream_kernel<true, true, T, SPREAD>), grid, dim3(512), 0, st, q, k, v, o, g, nqb, units, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_stream_kernel<true, false, T, SPREAD>), grid, dim3(512), 0, st, q, k, v, o, g, nqb, units, sc.cq, sc.cr);
  } else {
    if (sc.scaled)
      hipLaunchKernelGGL((fa2_fwd_stream_kernel<false, true, T, SPREAD>), grid, dim3(512), 0, st, q, k, v, o, g, nqb, units, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_stream_kernel<false, false, T, SPREAD>), grid, dim3(512), 0, st, q, k, v, o, g, nqb, units, sc.cq, sc.cr);
  }
  return hipGetLastError();
}

template <class T>
hipError_t launch_stream_t(const FwdArgs& a, hipStream_t st) {
  const int cus = device_cus();
  const int nqb = (a.seq + kStreamBr - 1) / kStreamBr;
  const int units = nqb * a.batch_heads;
  const dim3 grid((unsigned)min(units, cus));
  // at least 4 units per work-group, every one over 4 key tiles
  const bool spread = units >= 4 * cus && a.seq_k > 3 * kBc;
  return spread ? launch_stream_v<T, true>(a, st, grid, nqb, units)
                : launch_stream_v<T, false>(a, st, grid, nqb, units);
}

}  // namespace

// fp16 or bf16 by a.dtype.
hipError_t launch_stream(const FwdArgs& a, hipStream_t stream) {
  if (!stream_config_fits(a)) return hipErrorInvalidValue;
  return a.dtype == kDtypeBF16 ? launch_stream_t<__bf16>(a, stream)
                               : launch_stream_t<_Float16>(a, stream);
}

}  // namespace fl
