// Pipelined schedule (configurations br32_bc64_w1 and br64_bc64_w2) and
// split-KV ("flash-decoding") with its combine kernel.  Shared building
// blocks: fa2_common.h.

#include "fa2_common.h"

namespace fl {

namespace {

// ---------------------------------------------------------------------------
// Pipelined schedule: W waves of 32 query rows, D = fetch distance in tiles.
// KVSPLIT ("split-KV", for few query rows over many keys): work-group i
// takes key chunk i % nsplit of its query block and writes a partial result
// (Rows::store_partial) that splitkv_combine_kernel merges.
template <int W, int D, bool CAUSAL, bool SCALED, bool KVSPLIT = false>
__global__ void __launch_bounds__(64 * W, 2)  // 2 waves per SIMD: <= 256 VGPRs
fa2_fwd_kernel(const _Float16* Q, const _Float16* __restrict__ K,
               const _Float16* __restrict__ V, _Float16* O, const Geom geom, int nqb,
               float cq, float cr) {
  constexpr int kSlots = D + 1;
  constexpr int kUnroll = (kSlots % 2 == 0) ? kSlots : 2 * kSlots;
  constexpr int kBr = 32 * W;
  constexpr int kSegs = 8 / W;            // 1 KiB DMA segments per wave per tile
  constexpr int kDmaPerIter = 2 * kSegs;  // K + V loads a wave issues per iteration
  constexpr int kRingBytes = kSlots * kTileBytes;
  static_assert(kSegs * W == 8, "tile split");
  __shared__ __attribute__((aligned(16))) uint8_t kring[kRingBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vring[kRingBytes];

  const int lane = threadIdx.x & 63;
  const int rw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // 32-row block
  int bh, qb, chunk = 0;
  if constexpr (KVSPLIT) {
    const int r = blockIdx.x / geom.nsplit;
    chunk = blockIdx.x - r * geom.nsplit;
    bh = r / nqb;
    qb = r - bh * nqb;
  } else {
    wg_coords<CAUSAL, W == 4 ? 2 : 1>(nqb, geom.xcds, geom.cus_per_xcd, bh, qb);
  }
  const HeadPtrs hp = head_ptrs(geom, bh, Q, K, V, O);
  const i32x4_t rk = hp.rk, rv = hp.rv;
  const FetchOff<kSegs> fk = fetch_offsets<kSegs, false>(rw, lane, 2 * geom.k_sr);
  const FetchOff<kSegs> fv = fetch_offsets<kSegs, true>(rw, lane, 2 * geom.v_sr);
  const int seq = geom.seq_q;
  const int q0 = qb * kBr;
  const StreamRings<kSlots> rings = {kring, vring};

  Rows<CAUSAL, SCALED> rows;
  rows.init(hp.q, geom.q_sr, lane, q0 + 32 * rw, seq, geom.seq_k, geom.coff, cq, cr);

  const int all_tiles = max(1, (geom.seq_k + kBc - 1) / kBc);
  int ntiles = all_tiles;
  if (CAUSAL) ntiles = min(ntiles, causal_tiles(min(q0 + kBr, seq), geom.coff));
  // This work-group's key tiles start at cbeg: 0, or its split-KV chunk.
  int cbeg = 0;
  float* part = nullptr;
  if constexpr (KVSPLIT) {
    const int per = (all_tiles + geom.nsplit - 1) / geom.nsplit;
    cbeg = chunk * per;
    const int cend = min(ntiles, cbeg + per);
    rows.kv_lim = min(geom.seq_k, cend * kBc);
    ntiles = cend - cbeg;
    part = geom.part + (long long)(chunk * geom.batch_heads + bh) * seq * kPartStride;
    if (ntiles <= 0) {  // the whole chunk lies past the causal limit
      rows.store_partial(part);
      return;
    }
  }
  // Key tiles [tbeg, tend): t0 + 1 iterations.
  const int t0 = ntiles;
  const int tbeg = cbeg;
  const int tend = cbeg + ntiles;
  const int last = max(tend - 1, tbeg);  // fetch clamp

  // Iteration j (position I of the unrolled loop), for j = 0 .. t0, on key
  // tile t = tbeg + j: fetch K(t+D+1) and V(t+D-1) into the slots of K(t)
  // and V(t-2), vacated before the previous barrier; read the K(t+1) and
  // V(t-1) operands; then three independent pieces of work the compiler
  // interleaves: GEMM1(t+1), GEMM2(t-1) with P(t-1), and the softmax of S(t)
  // into P(t).  Finally mask S(t+1) (MASKED iterations only), wait for this
  // wave's part of K(t+2) and V(t), barrier.  Iteration 0 multiplies a
  // zeroed V slot by P = 0, and iteration t0 exponentiates a fully masked S
  // (p = 0); both only fill the pipeline.
  //
  // Two passes.  The first never moves the stabiliser m (the exact row max
  // of the first tile): it only records, branch-free, whether any tile's p
  // left the fp16-safe range (Rows::softmax_fast).  If one did anywhere in
  // the work-group (rare: a later key scores far above the first tile's
  // best), the whole query block is recomputed by the CHECKED pass, which
  // rescales when needed (Rows::softmax_trailing).  Without per-tile
  // branches the first pass's iterations are single basic blocks.
  uint64_t out_of_range = 0;
  auto iteration = [&](auto i, int j, float16_t (&S)[2], float16_t (&Sn)[2], half8_t (&P)[2][2],
                       const half8_t (&Pp)[2][2], auto masked, auto checked)
                       __attribute__((always_inline)) {
    constexpr int I = decltype(i)::value;
    const int t = tbeg + j;
    fetch_tile<kSegs>(rk, rings.kslot(Ic<I + D + 1>{}), t + D + 1, last, rw, fk);
    fetch_tile<kSegs>(rv, rings.vslot(Ic<I + D - 1>{}), t + D - 1, last, rw, fv);
    half8_t ka[2][4], va[2][4];
    rows.read_k(rings.kslot(Ic<I + 1>{}), ka);
    rows.read_v(rings.vslot(Ic<I - 1>{}), va);
    // GEMM1 of a tile past the range reads a stale slot; its result is masked.
    rows.gemm12(ka, Sn, va, Pp);
    if constexpr (decltype(checked)::value) {
      rows.softmax_trailing(S, P, [&](float d) __attribute__((always_inline)) {
        Rows<CAUSAL, SCALED>::sub(Sn, d);
      });
    } else {
      out_of_range |= rows.softmax_fast(S, P);
    }
    if constexpr (decltype(masked)::value) rows.mask(t + 1, Sn);
    sync_ring<(D - 1) * kDmaPerIter>();
  };

  // Iterations j < jm need no mask (tile tbeg + j + 1 lies below both the
  // key limit and, causal, this wave's first query row).  The split point
  // may differ between waves: every iteration has exactly one barrier.
  int tm = rows.kv_lim >> 6;
  if (CAUSAL) tm = min(tm, (rows.qd + 1) >> 6);
  const int jm = max(0, tm - tbeg - 1);

  auto run_pass = [&](auto checked) __attribute__((always_inline)) {
    // ---- prologue: K(tbeg), K(tbeg+1) landed; fetch groups of iterations
    // 1-D .. -1 in flight; S(tbeg) with the exact row max.
    {
      const u32x4_t z = {0, 0, 0, 0};
      for (int off = 16 * (int)threadIdx.x; off < kRingBytes; off += 16 * 64 * W)
        *reinterpret_cast<u32x4_t*>(vring + off) = z;
      __syncthreads();
    }
    fetch_tile<kSegs>(rk, rings.kslot(Ic<0>{}), tbeg, last, rw, fk);
    fetch_tile<kSegs>(rk, rings.kslot(Ic<1>{}), tbeg + 1, last, rw, fk);
    sync_ring<0>();
    static_for(std::make_integer_sequence<int, D - 1>{}, [&](auto i) __attribute__((always_inline)) {
      constexpr int G = decltype(i)::value + 1 - D;  // iteration 1-D+i
      fetch_tile<kSegs>(rk, rings.kslot(Ic<G + D + 1>{}), tbeg + G + D + 1, last, rw, fk);
      fetch_tile<kSegs>(rv, rings.vslot(Ic<G + D - 1>{}), tbeg + G + D - 1, last, rw, fv);
    });
    float16_t S0[2], S1[2];
    half8_t P0[2][2], P1[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) P1[a][b] = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
    {
      half8_t ka[2][4];
      rows.read_k(rings.kslot(Ic<0>{}), ka);
      rows.gemm1(ka, S0);
    }
    // Iteration 0 refills K(tbeg)'s slot: every wave's reads of it must be done.
    sync_ring<(D - 1) * kDmaPerIter>();
    rows.mask(tbeg, S0);
    rows.first_tile(S0);

    // ---- loops, unrolled so ring slots and S / P roles are static ----
    auto group = [&](int j0, auto masked) __attribute__((always_inline)) {
      static_for(std::make_integer_sequence<int, kUnroll>{}, [&](auto i) __attribute__((always_inline)) {
        constexpr int I = decltype(i)::value;
        const int j = j0 + I;
        if (!decltype(masked)::value || j <= t0) {
          if constexpr (I % 2 == 0)
            iteration(i, j, S0, S1, P0, P1, masked, checked);
          else
            iteration(i, j, S1, S0, P1, P0, masked, checked);
        }
      });
    };
    int j0 = 0;
    if constexpr (!decltype(checked)::value)
      for (; j0 + kUnroll <= jm; j0 += kUnroll) group(j0, Ic<false>{});
    for (; j0 <= t0; j0 += kUnroll) group(j0, Ic<true>{});
  };

  run_pass(Ic<false>{});
  {
    // Work-group-wide decision: redo the block if any wave saw a tile out
    // of range.  Drain this pass's fetches before the rings are refilled.
    // The flag lives in the first K ring slot: once every wave has drained
    // its fetches (first barrier) the rings are idle, and the checked pass
    // refills that slot only after the barrier that ends its V-ring
    // clearing, when every wave has read the flag.  No LDS beyond the
    // rings, so five single-wave work-groups (32 KiB each) fit one CU.
    __builtin_amdgcn_s_waitcnt(0);
    int* redo = reinterpret_cast<int*>(kring);
    __syncthreads();
    if (threadIdx.x == 0) *redo = 0;
    __syncthreads();
    if (out_of_range != 0 && lane == 0) *redo = 1;
    __syncthreads();
    if (*redo) {
      rows.reset();
      run_pass(Ic<true>{});
    }
  }

  // No fetch may still be writing LDS when the work-group retires.
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (KVSPLIT)
    rows.store_partial(part);
  else
    rows.store(hp.o, geom.o_sr, hp.lse);
}

// ---------------------------------------------------------------------------
// Split-KV combine: one wave per query row merges the nsplit partials of the
// row (O unnormalised at stabiliser m_s, row sum l_s) at their largest m:
//   O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s,
// and writes O (fp16, lane = head dim) and, when asked, the log-sum-exp.
// Lane j holds m and l of chunks j, j + 64, ...; its weight w_j goes to the
// whole wave by readlane, and each batch of 8 chunks issues its 8 O loads
// before the first multiply, so the row costs a few memory round trips
// rather than one per chunk.  A chunk with no visible key stored m = -inf
// and l = 0: weight 0, skipped by a select, not a branch.
__device__ __forceinline__ float wave_max64(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
  return x;
}

__device__ __forceinline__ float wave_sum64(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

__global__ void __launch_bounds__(256)
splitkv_combine_kernel(_Float16* O, const Geom geom) {
  const int lane = threadIdx.x & 63;
  const int row_id = blockIdx.x * 4 + (threadIdx.x >> 6);  // bh * N_q + row
  if (row_id >= geom.batch_heads * geom.seq_q) return;
  const int bh = row_id / geom.seq_q, row = row_id - bh * geom.seq_q;
  const long long split_stride = (long long)geom.batch_heads * geom.seq_q * kPartStride;
  const float* p0 = geom.part + (long long)row_id * kPartStride;
  const int ns = geom.nsplit;
  float mx = ninf();
  for (int s = lane; s < ns; s += 64) mx = fmaxf(mx, p0[s * split_stride + 64]);
  mx = wave_max64(mx);
  float acc = 0.0f, lpart = 0.0f;
  for (int s0 = 0; s0 < ns; s0 += 64) {
    float w = 0.0f;
    if (s0 + lane < ns) {
      const float* ps = p0 + (s0 + lane) * split_stride;
      const float m = ps[64];
      w = m == ninf() ? 0.0f : __builtin_amdgcn_exp2f(m - mx);
      lpart += w * ps[65];
    }
    // Chunk s0 + j's weight, from lane j; a weight of 0 skips the chunk.
    auto fold = [&](int j, float oj) __attribute__((always_inline)) {
      const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
      acc += wj == 0.0f ? 0.0f : wj * oj;
    };
    const int cnt = min(64, ns - s0);
    const float* pb = p0 + (long long)s0 * split_stride + lane;
    int j = 0;
    for (; j + 8 <= cnt; j += 8) {
      float o[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) o[u] = pb[(j + u) * split_stride];
#pragma unroll
      for (int u = 0; u < 8; ++u) fold(j + u, o[u]);
    }
    for (; j < cnt; ++j) fold(j, pb[j * split_stride]);
  }
  const float lsum = wave_sum64(lpart);
  const int b = bh / geom.heads, h = bh - b * geom.heads;
  _Float16* orow = O + (b * geom.o_sb + h * geom.o_sh) + (long long)row * geom.o_sr;
  orow[lane] = (_Float16)(lsum > 0.0f ? acc / lsum : 0.0f);
  if (geom.lse != nullptr && lane == 0)
    geom.lse[row_id] =
        lsum > 0.0f ? 0.693147180559945309f * (mx + __builtin_amdgcn_logf(lsum)) : ninf();
}

template <int W, int D>
struct PipelinedLaunch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, C, S>), grid, dim3(64 * W), 0, st,
                         static_cast<const _Float16*>(a.q), static_cast<const _Float16*>(a.k),
                         static_cast<const _Float16*>(a.v), static_cast<_Float16*>(a.o), g, nqb,
                         cq, cr);
      return hipSuccess;
    }
  };
};

// Split-KV: the chunk kernel (grid = query blocks x chunks) and the
// combine kernel, back to back on the stream.
template <int W, int D>
hipError_t launch_kvsplit_w(const FwdArgs& a, float* part, int nsplit, hipStream_t st) {
  constexpr int br = 32 * W;
  const int nqb = (a.seq + br - 1) / br;
  const Scales sc(a);
  Geom g = make_geom(a);
  g.part = part;
  g.nsplit = nsplit;
  const dim3 grid((unsigned)(nqb * a.batch_heads * nsplit));
  const dim3 block(64 * W);
  const _Float16 *q = static_cast<const _Float16*>(a.q), *k = static_cast<const _Float16*>(a.k),
                 *v = static_cast<const _Float16*>(a.v);
  _Float16* o = static_cast<_Float16*>(a.o);
  if (a.causal) {
    if (sc.scaled)
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, true, true, true>), grid, block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, true, false, true>), grid, block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
  } else {
    if (sc.scaled)
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, false, true, true>), grid, block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, false, false, true>), grid, block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_splitkv_combine(a, part, nsplit, st);
}

}  // namespace

// The combine kernel over `nsplit` chunk partials in `part`: one wave per
// query row, 4 rows per work-group.
hipError_t launch_splitkv_combine(const FwdArgs& a, float* part, int nsplit, hipStream_t st) {
  Geom g = make_geom(a);
  g.part = part;
  g.nsplit = nsplit;
  const int rows = a.batch_heads * a.seq;
  hipLaunchKernelGGL(splitkv_combine_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st,
                     static_cast<_Float16*>(a.o), g);
  return hipGetLastError();
}

hipError_t launch_pipe(const FwdArgs& a, int cfg, hipStream_t stream) {
  switch (cfg) {
    case kCfgW1: return dispatch<PipelinedLaunch<1, 1>::L>(a, stream, 32);
    case kCfgW2: return dispatch<PipelinedLaunch<2, 3>::L>(a, stream, 64);
    default: return hipErrorInvalidValue;
  }
}

// Two-wave chunks fetch two tiles ahead (48 KiB of rings): three work-groups
// per CU instead of two, measured 3-7% faster on 64-row decode.  The
// one-pass two-wave configuration keeps three tiles: with room for three
// groups per CU its typical 2-groups-per-CU grids pack unevenly (14-21%
// slower measured on B1 H8 N4096 and B4 H8 N1024).
hipError_t launch_kvsplit(const FwdArgs& a, int waves, float* part, int nsplit,
                          hipStream_t stream) {
  switch (waves) {
    case 1: return launch_kvsplit_w<1, 1>(a, part, nsplit, stream);
    case 2: return launch_kvsplit_w<2, 2>(a, part, nsplit, stream);
    case 4: return launch_kvsplit_w<4, 3>(a, part, nsplit, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fl
