// FlashAttention-2 forward for gfx950 (MI355X, CDNA4), fp16 (and bf16) in /
// fp32 accumulate, head_dim 64 (and 128).
//
// Reference: csrc/kernel_flash2.cu of thebigblender/FlashLite -- the two
// kernels flash_attn2_wmma_br64_kernel (:54-387) and
// flash_attn2_wmma_br128_kernel (:393-727).  This is a fresh design for
// 64-lane wavefronts and MFMA, not a translation; the math and the mask
// semantics are the same:
//   O = softmax(Q K^T * sm_scale [+ causal mask]) V,
//   causal: key j visible to query i iff j <= i (top-left when N_q == N_k;
//   with N_k != N_q the diagonal is aligned bottom-right, j <= i + N_k - N_q,
//   and a query row with no visible key returns 0, as :364-365 do),
//   keys >= N_k masked, query rows >= N_q never written (:373, :380),
//   P rounded to fp16 before the PV product (:278-285), fp32 row sums.
//
// Work decomposition.  A work-group owns 32*W consecutive query rows of one
// (batch, head); each of its W waves owns 32 of them (struct Rows below).
// The KV sequence is walked in tiles of 64 keys staged in LDS and shared by
// the W waves.
//
// MFMA formulation (v_mfma_f32_32x32x16_f16, 64 lanes, lane l: column l%32,
// k-group g = l/32):
//   GEMM1  S^T[key][query] = K . Q'^T - m   A = K rows from LDS
//                                           (ds_read_b128), B = the wave's
//                                           prescaled Q rows in VGPRs, C = -m.
//     Each lane then owns ONE query (column l%32) and 16 of a 32-key block
//     (rows 8*(r/4) + 4*g + r%4 of accumulator r); the other 16 sit in lane
//     l^32.  A row max is 16 in-lane ops plus one v_permlane32_swap.
//   GEMM2  O^T[d][query] += V^T . P^T  B = P^T straight from the GEMM1
//                                      accumulators (packed to fp16),
//                                      A = V^T read with ds_read_b64_tr_b16,
//     whose 4-keys-per-lane transposed layout is exactly the k-order of the
//     GEMM1 accumulators, so P never leaves registers.
// The A-operand rows of GEMM2 are permuted (bits 2 and 3 of the row index
// swapped via the tr-read addresses) so each lane ends with 8 contiguous
// head-dim values per accumulator half: the epilogue stores 16-byte vectors.
//
// Softmax, at one exp per score.  For fp16 at head_dim 64, Q is prescaled
// by c = |sm_scale| * log2 e (the reference's prescale,
// kernel_flash2.cu:772) when c <= 1, so GEMM1
// returns base-2 logits; the running stabiliser m enters as the MFMA
// accumulator's initial value, so GEMM1 returns logit - m and p = v_exp_f32
// of the accumulator.  m is the exact row max of the first tile and later
// only moves when a tile would push p out of range (a stale m is exact math
// since softmax is shift invariant; m never exceeds the running max, so the
// row sum stays >= 1).  p is packed to fp16 for GEMM2.  Row sums: fp32 adds
// of the fp32 p (the reference also sums fp32 p, :339) in the older
// schedules; the slot schedule sums fp16 tiles with a packed-fp16 tree of
// the rounded p and bf16 tiles on the matrix core (Rows::init_msum) --
// v_dot2_f32_f16 would stall the matrix core.  Each lane sums its own keys
// and the two halves of a row meet once, in the epilogue.  When c > 1
// (SCALED) Q keeps its scale and the logits are multiplied by c instead, so
// |Q'| never exceeds |Q|.
//
// K/V staging.  Tiles are fetched straight into LDS with buffer_load ... lds
// (no VGPRs, no LDS-store instructions; rows past N read as zeros through
// the buffer resource's bound) D tiles ahead, into rings of D+1 slots per
// tensor.  Loops are unrolled by the ring length, so every slot address is
// a constant offset.  One explicit "s_waitcnt vmcnt(n); s_barrier" per step
// makes a tile visible.
//
// Schedules:
//   fa2_fwd_slot_kernel (W = 8 or 4; the dispatcher's choice for N_k > 256):
//     16 fenced MFMA slots per tile, each carrying two exponentials and the
//     LDS read of a later slot's operand; GEMM1 skewed by half a tile so one
//     score buffer serves both the tile being exponentiated and the next.
//   fa2_fwd_stream_kernel (N_k <= 256): one persistent 8-wave work-group per
//     CU walks whole units (a head's 256-row block with all its keys) through
//     two LDS buffers, loading the next unit while it computes the current.
//   fa2_fwd_d128_kernel (head_dim 128): the slot schedule over 32-key tiles.
//   fa2_fwd_kernel (any W; SPLIT = 1 or 2): iteration j runs GEMM1 of tile
//     j+1, GEMM2 of tile j-1 and the softmax of tile j -- three independent
//     pieces of work the compiler interleaves -- and checks the stabiliser
//     after the exponentials (Rows::softmax_trailing); one barrier per tile.
//     SPLIT = 2 doubles the waves: the second set walks the second half of
//     the key range with its own rings, and the halves merge through LDS.
//   fa2_fwd_pp_kernel (W = 8, "ping-pong"): waves w and w+4 of a 512-lane
//     work-group share a SIMD, so group A = waves 0-3 and group B = waves
//     4-7 alternate an MFMA phase (GEMM2 of tile j-1 + GEMM1 of tile j) and
//     a softmax phase, with a barrier per phase.
//   The ping-pong kernel decides the stabiliser before the exponentials
//   (Rows::restabilise).  fa2_fwd_kernel serves small problems and split-KV;
//   the ping-pong kernel is kept as a selectable, tested alternative.
//
// Causal.  Keys after a lane's query and keys >= N are masked to -inf on the
// diagonal and tail tiles only; work-groups are fed to each XCD heaviest
// first, with heavy and light blocks paired on a CU (wg_coords).
//
// LDS.  Rows of 128 B (64 halfs).  16-byte chunks are XOR-swizzled per row:
// K with (row&7)^((row>>3)&1), V with 2*(row&3), which makes the GEMM1
// ds_read_b128 pattern, the GEMM2 ds_read_b64_tr_b16 pattern and the
// row-contiguous tile writes conflict-free for 32- or 64-bank LDS.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "fl_internal.h"

namespace fl {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));

// Operand vectors and the 32x32x16 MFMA of one 16-bit element type (fp16:
// the reference's type; bf16: beyond it).  Both accumulate in fp32.
template <class T>
struct Elem;
template <>
struct Elem<_Float16> {
  using v8 = half8_t;
  using v4 = half4_t;
  __device__ __forceinline__ static float16_t mfma(const v8& a, const v8& b, const float16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static float4_t mfma16(const v8& a, const v8& b, const float4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Elem<__bf16> {
  using v8 = bf16x8_t;
  using v4 = bf16x4_t;
  __device__ __forceinline__ static float16_t mfma(const v8& a, const v8& b, const float16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static float4_t mfma16(const v8& a, const v8& b, const float4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

constexpr int kD = 64;                       // head dim
constexpr int kBc = 64;                      // keys per KV tile
constexpr int kRowBytes = kD * 2;            // 128
constexpr int kTileBytes = kBc * kRowBytes;  // 8 KiB
constexpr float kLag = 8.0f;                 // max lag of m behind a row max, log2 units
constexpr float kSumLimit = 32768.0f;        // lane tile-sum bound that keeps p in fp16 range
constexpr float kMsumLimit = 1099511627776.0f;  // 2^40: row-sum bound of the matrix-core sums

__device__ __forceinline__ int k_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int v_swz(int row) { return (row & 3) << 1; }

__device__ __forceinline__ float ninf() { return -__builtin_huge_valf(); }

// v_permlane32_swap of x with itself yields {x[l], x[l^32]} in some order
// in every lane l, so max/sum of the pair combine the two halves of a row.
__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Raw buffer resource (gfx9 layout): 48-bit base, stride 0, num_records
// bytes, dword 3 = 0x00020000 (32-bit data format, no swizzle).  Loads at
// offsets >= num_records return zeros.
__device__ __forceinline__ i32x4_t buffer_rsrc(const void* base, int bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xFFFF);
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000;
  return r;
}

// Addressing of one launch: element strides of q, k, v, o over
// [batch][head][row] (head_dim is unit stride), the sizes, the causal
// diagonal offset N_k - N_q, and the optional log-sum-exp output.
struct Geom {
  long long q_sb, q_sh, k_sb, k_sh, v_sb, v_sh, o_sb, o_sh;
  int q_sr, k_sr, v_sr, o_sr;
  int heads, seq_q, seq_k, coff;
  float* lse;  // [B*H][N_q] or null
  // split-KV launches: partial results [nsplit][B*H][N_q][kPartStride]
  float* part;
  int nsplit, batch_heads;
};

// Floats per row of a split-KV partial result: O[64] unnormalised, the
// stabiliser in base-2 logit units, the row sum, 2 pad (16-byte rows).
constexpr int kPartStride = 68;

// Per-head base pointers and buffer resources of a work-group.
template <class T = _Float16>
struct HeadPtrs {
  const T* q;
  T* o;
  float* lse;
  i32x4_t rk, rv;
};

template <class T, int kRowB = kRowBytes>
__device__ __forceinline__ HeadPtrs<T> head_ptrs(const Geom& g, int bh, const T* Q, const T* K,
                                                 const T* V, T* O) {
  const int b = bh / g.heads, h = bh - b * g.heads;
  HeadPtrs<T> p;
  p.q = Q + (b * g.q_sb + h * g.q_sh);
  p.o = O + (b * g.o_sb + h * g.o_sh);
  p.lse = g.lse ? g.lse + (long long)bh * g.seq_q : nullptr;
  // num_records covers the last row's kRowB bytes; later rows read as zeros.
  const int kb = g.seq_k > 0 ? (g.seq_k - 1) * (2 * g.k_sr) + kRowB : 0;
  const int vb = g.seq_k > 0 ? (g.seq_k - 1) * (2 * g.v_sr) + kRowB : 0;
  p.rk = buffer_rsrc(K + (b * g.k_sb + h * g.k_sh), kb);
  p.rv = buffer_rsrc(V + (b * g.v_sb + h * g.v_sh), vb);
  return p;
}

// Key tiles a causal block of query rows [q0, q_end) needs: through the
// diagonal of its last row (at least one, fully masked when no row of the
// block sees a key).
__device__ __forceinline__ int causal_tiles(int q_end, int coff) {
  const int last_key = q_end - 1 + coff;
  return last_key < 0 ? 1 : last_key / kBc + 1;
}

template <class V4 = half4_t>
__device__ __forceinline__ V4 lds_read_tr(const uint8_t* p) {
  short4_t s = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (short4_t __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(V4, s);
}

// End of a step: this wave's LDS fetches older than its newest `pending`
// ones have landed, its own LDS reads have completed, then the work-group
// barrier.  The asm is a compiler memory barrier, and the sched_barriers
// keep the scheduler from moving any instruction (MFMAs included) across
// it, so each step's work stays in its step.
template <int kPending>
__device__ __forceinline__ void sync_ring() {
  static_assert(kPending >= 0 && kPending < 64, "vmcnt range");
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(kPending) : "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <int N>
struct Ic {
  static constexpr int value = N;
};

template <int... I, class F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f) {
  (f(Ic<I>{}), ...);
}

// Work-group -> (batch*head, query block).  Work-groups are dealt to the 8
// XCDs round-robin; remap so that the query blocks of a head land on the
// same XCD (shared K/V in its L2).  Causal work-groups differ in length, so
// each XCD is fed heaviest first (heads interleaved).  Measured dispatch on
// gfx950: an XCD fills its 32 CUs in a fixed order with its first 32
// work-groups; with two co-resident work-groups per CU its next 32 fill the
// second slots of the same CUs in the same order; after that each goes to
// whichever CU frees first.  So with kSlotsPerCu == 2 the second 32 are
// taken in reverse (CU j pairs the j-th heaviest block with the j-th
// lightest of the first 64), and every later position keeps the
// longest-processing-time order.
template <bool CAUSAL, int kSlotsPerCu>
__device__ __forceinline__ void wg_coords(int nqb, int& bh, int& qb) {
  constexpr int kCusPerXcd = 32;
  const int total = gridDim.x;
  const int i = blockIdx.x;
  const int per = total >> 3;
  if ((total & 7) != 0) {
    bh = i / nqb;
    qb = i - bh * nqb;
  } else if (!CAUSAL || per % nqb != 0) {
    const int lin = (i & 7) * per + (i >> 3);
    bh = lin / nqb;
    qb = lin - bh * nqb;
  } else {
    const int hx = per / nqb;  // whole heads per XCD
    const int k = i >> 3;      // dispatch position within the XCD
    constexpr int first = kCusPerXcd * kSlotsPerCu;
    int r = k;                 // work rank, 0 = heaviest
    if (kSlotsPerCu == 2 && per >= first && k >= kCusPerXcd && k < first)
      r = first - 1 - (k - kCusPerXcd);
    bh = (i & 7) * hx + r % hx;
    qb = r / hx;
  }
  if (CAUSAL) qb = nqb - 1 - qb;
}

// K/V rings: kSlots LDS objects per tensor, selected by a static index
// (negative indices wrap).
template <int kSlots>
struct Rings {
  static_assert(kSlots >= 2 && kSlots <= 8, "ring depth");
  uint8_t* k[8];
  uint8_t* v[8];
  template <int I>
  __device__ __forceinline__ uint8_t* kslot(Ic<I>) const {
    return k[((I % kSlots) + kSlots) % kSlots];
  }
  template <int I>
  __device__ __forceinline__ uint8_t* vslot(Ic<I>) const {
    return v[((I % kSlots) + kSlots) % kSlots];
  }
};

// Asynchronous fetch of tile t (clamped to the last tile the work-group
// needs) straight into LDS with buffer_load_dwordx4 ... lds: each wave moves
// `kSegs` 1 KiB segments (8 rows); lane i of a segment lands at byte 16*i,
// i.e. row i/8, physical chunk i%8, which holds logical chunk
// (i%8) ^ swz(row).  Issued from inline assembly so the compiler does not
// guard LDS reads of other slots with waits on it; sync_ring<> tracks it.
template <int kSegs>
struct FetchOff {
  int lane[kSegs];  // this lane's byte offset of segment i within a tile
  int tile_bytes;   // kBc rows
};

template <int kSegs, bool IS_V>
__device__ __forceinline__ FetchOff<kSegs> fetch_offsets(int wave, int lane, int row_bytes) {
  FetchOff<kSegs> f;
#pragma unroll
  for (int i = 0; i < kSegs; ++i) {
    const int seg = wave * kSegs + i;
    const int row = 8 * seg + (lane >> 3);
    const int phys = lane & 7;
    const int logical = phys ^ (IS_V ? v_swz(row) : k_swz(row));
    f.lane[i] = row * row_bytes + 16 * logical;
    // Opaque to the optimiser: keeps the per-tile address an SALU product
    // plus one add instead of a re-derived 64-bit multiply-add.
    asm volatile("" : "+v"(f.lane[i]));
  }
  f.tile_bytes = kBc * row_bytes;
  return f;
}

template <int kSegs>
__device__ __forceinline__ void fetch_tile(const i32x4_t& rs, const uint8_t* slot, int t,
                                           int last_tile, int wave, const FetchOff<kSegs>& f) {
  t = min(t, last_tile);
  const int tb = t * f.tile_bytes;
#pragma unroll
  for (int i = 0; i < kSegs; ++i) {
    const int seg = wave * kSegs + i;
    const int voff = tb + f.lane[i];
    const uint32_t lds_base = (uint32_t)(uintptr_t)(slot + 1024 * seg);
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(rs), "{m0}"(lds_base));
  }
}

// The 32 query rows one wave owns: prescaled Q, running max, row sums and
// O accumulator, plus the tile-level building blocks.
template <bool CAUSAL, bool SCALED, class T = _Float16>
struct Rows {
  using E = Elem<T>;
  using V8 = typename E::v8;
  using V4 = typename E::v4;
  int g, col, qw, my_q, seq;
  int qd, my_d;     // causal diagonals: the last key visible to row qw / my_q
  int kv_lim;       // keys >= kv_lim are masked (N_k, or the end of a split range)
  int tr_row, tr_col;
  float cr;
  V8 qf[4];    // Q'^T B-operand
  float16_t o[2];   // O^T accumulator, d-blocks 0 / 1
  float16_t bias;   // -m broadcast, GEMM1's accumulator input
  float m;          // running stabiliser, units of t = q'.k
  float l;          // this lane's share of the row sum
  V8 p[2][2];  // fp16 P^T B-operands of the last softmaxed tile
  float4_t lacc;    // row sums on the matrix core (init_msum / msum_share)
  V8 sel;           // their A operand

  // Lane placement: rows qw_ .. qw_+31 of a head with seq_ query rows and
  // seq_k keys (causal diagonal offset coff).
  __device__ __forceinline__ void place(int lane, int qw_, int seq_, int seq_k, int coff,
                                        float cr_) {
    g = lane >> 5;
    col = lane & 31;
    qw = qw_;
    my_q = qw + col;
    qd = qw + coff;
    my_d = my_q + coff;
    seq = seq_;
    kv_lim = seq_k;
    cr = cr_;
    // GEMM2 tr-read address pieces: lane l is lane j = l%16 of 16-lane group
    // G = l/16; it points at key row 4*(G/2) + j/4 (+16t, +8 for the second
    // read) and head-dim column 16*(G%2) + 4*swap2(j%4) (+32 per d-block).
    const int trG = lane >> 4, trj = lane & 15;
    tr_row = 4 * (trG >> 1) + (trj >> 2);
    const int tr_x = trj & 3;
    tr_col = 16 * (trG & 1) + 4 * (((tr_x & 1) << 1) | (tr_x >> 1));
  }
  // Q'^T from the raw 16-byte chunks Q[my_q][16s + 8g .. +7] (s = 0..3).
  __device__ __forceinline__ void set_q(const u32x4_t (&raw)[4], float cq) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const V8 x = __builtin_bit_cast(V8, raw[s]);
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[s][e] = (T)((float)x[e] * cq);
    }
  }
  __device__ __forceinline__ void init(const T* Qh, int q_sr, int lane, int qw_, int seq_,
                                       int seq_k, int coff, float cq, float cr_) {
    place(lane, qw_, seq_, seq_k, coff, cr_);
    // Q'^T: lane holds cq * Q[my_q][16s + 8g .. +7] for s = 0..3, in fp16.
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (my_q < seq) {
        const V8 raw =
            *reinterpret_cast<const V8*>(Qh + (long long)my_q * q_sr + 16 * s + 8 * g);
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[s][e] = (T)((float)raw[e] * cq);
      } else {
        qf[s] = (V8){0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      o[0][r] = 0.0f;
      o[1][r] = 0.0f;
      bias[r] = 0.0f;
    }
    m = 0.0f;
    l = 0.0f;
  }

  // Makes the per-lane index fields opaque, so addresses derived from them
  // are recomputed after this point instead of being kept live (and, under
  // register pressure, spilled) from an earlier use.
  __device__ __forceinline__ void launder() {
    asm volatile("" : "+v"(col), "+v"(g), "+v"(my_q), "+v"(tr_row), "+v"(tr_col));
  }
  // K operands of GEMM1 (both 32-key blocks, 4 head-dim steps each).
  __device__ __forceinline__ void read_k(const uint8_t* kt, V8 (&ka)[2][4]) const {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int row = 32 * kb + col;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int ch = 2 * st + g;
        ka[kb][st] =
            *reinterpret_cast<const V8*>(kt + row * kRowBytes + 16 * (ch ^ k_swz(row)));
      }
    }
  }
  // V^T operands of GEMM2 (2 d-blocks x 4 16-key steps).
  __device__ __forceinline__ void read_v(const uint8_t* vt, V8 (&va)[2][4]) const {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int r1 = 16 * t + tr_row;
        const int r2 = r1 + 8;
        const int dcol = 32 * db + tr_col;
        const int ch = dcol >> 3, hb = ((dcol >> 2) & 1) * 8;
        const V4 lo = lds_read_tr<V4>(vt + r1 * kRowBytes + 16 * (ch ^ v_swz(r1)) + hb);
        const V4 hi = lds_read_tr<V4>(vt + r2 * kRowBytes + 16 * (ch ^ v_swz(r2)) + hb);
        va[db][t] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
  }
  // GEMM1: s[kb] = K[32kb + row] . Q'^T - m.
  __device__ __forceinline__ void gemm1(const V8 (&ka)[2][4], float16_t (&s)[2]) const {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int st = 0; st < 4; ++st)
        s[kb] = E::mfma(ka[kb][st], qf[st], st == 0 ? bias : s[kb]);
  }
  // GEMM2: O^T += V^T . P^T
  __device__ __forceinline__ void gemm2(const V8 (&va)[2][4], const V8 (&pp)[2][2]) {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        o[db] = E::mfma(va[db][t], pp[t >> 1][t & 1], o[db]);
  }
  __device__ __forceinline__ void gemm2(const V8 (&va)[2][4]) { gemm2(va, p); }
  // GEMM1 of one tile and GEMM2 of another, issued as four interleaved
  // accumulation chains (s[0], o[0], s[1], o[1]) so consecutive MFMAs never
  // depend on each other.
  __device__ __forceinline__ void gemm12(const V8 (&ka)[2][4], float16_t (&s)[2],
                                         const V8 (&va)[2][4], const V8 (&pp)[2][2]) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        s[h] = E::mfma(ka[h][st], qf[st], st == 0 ? bias : s[h]);
        o[h] = E::mfma(va[h][st], pp[st >> 1][st & 1], o[h]);
      }
    }
  }
  // A operands of single MFMAs: 32 K rows of key block kb at head-dim step
  // st (one ds_read_b128), or V^T of head-dim block db at key step t (two
  // ds_read_b64_tr_b16); the same reads as read_k / read_v.
  __device__ __forceinline__ V8 read_k_op(const uint8_t* kt, int kb, int st) const {
    const int row = 32 * kb + col;
    const int ch = 2 * st + g;
    return *reinterpret_cast<const V8*>(kt + row * kRowBytes + 16 * (ch ^ k_swz(row)));
  }
  __device__ __forceinline__ V8 read_v_op(const uint8_t* vt, int db, int t) const {
    const int r1 = 16 * t + tr_row;
    const int r2 = r1 + 8;
    const int dcol = 32 * db + tr_col;
    const int ch = dcol >> 3, hb = ((dcol >> 2) & 1) * 8;
    const V4 lo = lds_read_tr<V4>(vt + r1 * kRowBytes + 16 * (ch ^ v_swz(r1)) + hb);
    const V4 hi = lds_read_tr<V4>(vt + r2 * kRowBytes + 16 * (ch ^ v_swz(r2)) + hb);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  // Slot map of the skewed slot schedule (fa2_fwd_slot_kernel).  Iteration
  // j has 16 MFMA slots; slot L = 2u + q:
  //   q = 0, u < 4:  S[1] (+)= K(j) rows 32-63 . Q'(st = u)    GEMM1, tile j
  //   q = 0, u >= 4: S[0] (+)= K(j+1) rows 0-31 . Q'(st = u-4)  GEMM1, tile j+1
  //   q = 1:         O[u & 1] += V^T(j-1)(key step u/2) . P(j-1) GEMM2
  // The exponentials of slots 0-7 read S[0] (tile j) and those of slots
  // 8-15 read S[1] (tile j), so each block is rewritten only after its
  // scores are consumed: one S buffer instead of two.
  template <int L>
  __device__ __forceinline__ V8 read_slot(const uint8_t* k_cur, const uint8_t* k_next,
                                               const uint8_t* vt) const {
    constexpr int u = L >> 1;
    if constexpr ((L & 1) == 0)
      return u < 4 ? read_k_op(k_cur, 1, u) : read_k_op(k_next, 0, u - 4);
    else
      return read_v_op(vt, u & 1, u >> 1);
  }
  template <int L, bool MS = false>
  __device__ __forceinline__ void mfma_slot(const V8& a, float16_t (&s)[2],
                                            const V8 (&pp)[2][2]) {
    constexpr int u = L >> 1;
    if constexpr ((L & 1) == 0) {
      constexpr int kb = u < 4 ? 1 : 0, st = u & 3;
      s[kb] = E::mfma(a, qf[st], st == 0 ? bias : s[kb]);
    } else {
      constexpr int db = u & 1, t = u >> 1;
      o[db] = E::mfma(a, pp[t >> 1][t & 1], o[db]);
      // With MS, the row sums of key step t ride in the slot's second MFMA.
      if constexpr (MS && db == 1) lacc = E::mfma16(sel, pp[t >> 1][t & 1], lacc);
    }
  }
  // Row sums on the matrix core.  The 16x16x32 MFMA takes a 32x32x16 P^T
  // B operand (lane l: query l%32, keys 8(l/32) .. +7 of a 16-key step) as
  // B16[k = 8(l/16) + e][n = l%16], i.e. query n + 16h (h = bit 4 of l) at
  // keys 8g + e (g = l/32).  With A16[0][k] = 1 where h = 0 and A16[1][k] =
  // 1 where h = 1 (zero elsewhere), D16 row 0 accumulates query n's sum of
  // p and row 1 query n+16's: the fp16-rounded p that GEMM2 multiplies,
  // summed in fp32.
  __device__ __forceinline__ void init_msum(int lane) {
    const int m = lane & 15, h = (lane >> 4) & 1;
    const T one = (T)(((m == 0 && h == 0) || (m == 1 && h == 1)) ? 1.0f : 0.0f);
#pragma unroll
    for (int e = 0; e < 8; ++e) sel[e] = one;
    lacc = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
  }
  // This lane's share of its query's row sum (D16 rows 0 and 1 sit in
  // lanes 0-15, elements 0 and 1): the total in lanes 0-31, 0 in 32-63.
  __device__ __forceinline__ float msum_share() const {
    const int src = col & 15;
    const float a0 = __shfl(lacc[0], src), a1 = __shfl(lacc[1], src);
    return g == 0 ? (col < 16 ? a0 : a1) : 0.0f;
  }
  // Softmax share of slot I: scores 2(I%8), 2(I%8)+1 of key block I/8 ->
  // two exponentials and one fp16 pack into dword I of the tile's P operand
  // (exponentiate() spread over 16 slots).
  template <int I>
  __device__ __forceinline__ void exp_slot(const float16_t (&s)[2], V8 (&pn)[2][2]) const {
    constexpr int kb = I >> 3, r = 2 * (I & 7), h = r >> 3, e = r & 7;
    float x0 = s[kb][r], x1 = s[kb][r + 1];
    if (SCALED) {
      x0 *= cr;
      x1 *= cr;
    }
    const float e0 = __builtin_amdgcn_exp2f(x0), e1 = __builtin_amdgcn_exp2f(x1);
    pn[kb][h][e] = (T)e0;
    pn[kb][h][e + 1] = (T)e1;
  }
  // Dword i (0-15) of a tile's P operand: the fp16 pair of slot i.
  __device__ __forceinline__ static half2_t p_pair(const half8_t (&pn)[2][2], int i) {
    const half8_t& v = pn[i >> 3][(i >> 2) & 1];
    const int e = 2 * (i & 3);
    return (half2_t){v[e], v[e + 1]};
  }
  // Row-sum share of slot I: a pairwise tree of packed fp16 additions over
  // the tile's P, i.e. the fp16-rounded p that GEMM2 multiplies (level 1
  // at odd slots, level 2 every 4th, level 3 every 8th; sum_root finishes
  // it).  One v_pk_add_f16 per slot instead of two fp32 adds keeps a slot's
  // VALU work within what issues under one MFMA.  t[0..7] level 1, t[8..11]
  // level 2, t[12..13] level 3.
  template <int I>
  __device__ __forceinline__ static void sum_slot(const half8_t (&pn)[2][2], half2_t (&t)[14]) {
    if constexpr (I & 1) t[I >> 1] = p_pair(pn, I - 1) + p_pair(pn, I);
    if constexpr ((I & 3) == 3) t[8 + (I >> 2)] = t[(I >> 1) - 1] + t[I >> 1];
    if constexpr ((I & 7) == 7) t[12 + (I >> 3)] = t[8 + (I >> 2) - 1] + t[8 + (I >> 2)];
  }
  // fp32 row-sum share of slot I: the slot's two p, recomputed from the
  // scores (the exponentials of exp_slot, which the compiler shares), in
  // four partial chains.
  template <int I>
  __device__ __forceinline__ static void sum_slot_f32(const float16_t (&s)[2], float (&sum)[4],
                                                      float crr) {
    constexpr int kb = I >> 3, r = 2 * (I & 7);
    float x0 = s[kb][r], x1 = s[kb][r + 1];
    if (SCALED) {
      x0 *= crr;
      x1 *= crr;
    }
    const float e = __builtin_amdgcn_exp2f(x0) + __builtin_amdgcn_exp2f(x1);
    if constexpr (I < 4)
      sum[I] = e;
    else
      sum[I & 3] += e;
  }
  // This lane's tile sum in fp32 from the two level-3 nodes (each half of
  // the root sums 16 of the lane's 32 values).  A tile whose sum leaves the
  // fp16-safe range overflows to inf here or exceeds kSumLimit; either way
  // the caller's range check sends the block to the checked pass.
  __device__ __forceinline__ static float sum_root(const half2_t (&t)[14]) {
    const half2_t r = t[12] + t[13];
    return (float)r[0] + (float)r[1];
  }
  // Masks keys >= kv_lim and, when causal, keys past the lane's diagonal
  // (tile t).  Score r of block kb is key k0 + 4g + c with the constant
  // c = 32kb + 8(r/4) + r%4, so one per-lane bound on c decides every score
  // (no per-score key indices to keep live).
  __device__ __forceinline__ void mask(int t, float16_t (&s)[2]) const {
    const int k0 = t * kBc;
    if (k0 + kBc > kv_lim || (CAUSAL && k0 + kBc - 1 > qd)) {
      const int base = k0 + 4 * g;
      int lim = kv_lim - base;                    // visible iff c < lim
      if (CAUSAL) lim = min(lim, my_d + 1 - base);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = 32 * kb + 8 * (r >> 2) + (r & 3);
          s[kb][r] = c < lim ? s[kb][r] : ninf();
        }
    }
  }
  // The same for key block KB of tile t alone.
  template <int KB>
  __device__ __forceinline__ void mask_block(int t, float16_t& s) const {
    const int k0 = t * kBc + 32 * KB;
    if (k0 + 32 > kv_lim || (CAUSAL && k0 + 31 > qd)) {
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
  // One key tile, unpipelined, with the stabiliser checked: the recompute
  // pass for blocks whose first pass saw a tile sum out of range.  S = the
  // tile's scores (GEMM1 done, masked); P and the sums follow, and when a
  // lane's tile sum leaves the fp16-safe range m moves up to the tile's row
  // max, with O and l rescaled, before the tile is exponentiated again.
  __device__ __forceinline__ void softmax_checked(float16_t (&s)[2], V8 (&pn)[2][2]) {
    float sum = exponentiate(s, pn);
    if (__builtin_amdgcn_ballot_w64(!(sum <= kSumLimit)) != 0) {
      const float d = fmaxf(tile_max(s), 0.0f);
      const float alpha = __builtin_amdgcn_exp2f(-(SCALED ? cr : 1.0f) * d);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      sub(s, d);
      set_m(m + d);
      sum = exponentiate(s, pn);
    }
    l += sum;
  }
  // Row max of a tile (both halves of the row).
  __device__ __forceinline__ float tile_max(const float16_t (&s)[2]) const {
    float mx = ninf();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    return pair_max(mx);
  }
  __device__ __forceinline__ static void sub(float16_t (&s)[2], float d) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] -= d;
  }
  __device__ __forceinline__ void set_m(float mm) {
    m = mm;
#pragma unroll
    for (int r = 0; r < 16; ++r) bias[r] = -mm;
  }
  // First tile: m = the exact row max.  A row with no key in the tile (the
  // second range of a split, or a row above a bottom-right causal diagonal
  // when N_q > N_k; such a row then has no key in its whole range) gets
  // m = 0 and p = 0 throughout.
  __device__ __forceinline__ void first_tile(float16_t (&s)[2]) {
    float m0 = tile_max(s);
    m0 = m0 == ninf() ? 0.0f : m0;
    sub(s, m0);
    set_m(m0);
  }
  // p = 2^(t - m) (times cr when SCALED) packed to fp16 B-operands; returns
  // this lane's sum of p, taken in fp32 over four chains.  (The row sum uses
  // v_add_f32 rather than v_dot2_f32_f16 on the packed p: on gfx950 the dot2
  // instructions do not issue alongside MFMA work, adds and conversions do.)
  __device__ __forceinline__ float exponentiate(const float16_t (&s)[2], V8 (&pn)[2][2]) const {
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float x0 = s[kb][8 * h + e], x1 = s[kb][8 * h + e + 1];
          if (SCALED) {
            x0 *= cr;
            x1 *= cr;
          }
          const float e0 = __builtin_amdgcn_exp2f(x0), e1 = __builtin_amdgcn_exp2f(x1);
          pn[kb][h][e] = (T)e0;
          pn[kb][h][e + 1] = (T)e1;
          sum[2 * kb + h] += e0 + e1;
        }
    return (sum[0] + sum[1]) + (sum[2] + sum[3]);
  }
  __device__ __forceinline__ float exponentiate(const float16_t (&s)[2]) { return exponentiate(s, p); }
  // Softmax of tile j into pn at the current m, no rescaling: returns the
  // lanes whose tile sum left the range where every p is a finite fp16
  // (also catches inf / NaN); the caller then recomputes with rescaling.
  __device__ __forceinline__ uint64_t softmax_fast(const float16_t (&s)[2], V8 (&pn)[2][2]) {
    const float sum = exponentiate(s, pn);
    l += sum;
    return __builtin_amdgcn_ballot_w64(!(sum <= kSumLimit));
  }
  // Back to the state after init (Q stays loaded).
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      o[0][r] = 0.0f;
      o[1][r] = 0.0f;
    }
    set_m(0.0f);
    l = 0.0f;
  }
  // Softmax of tile j into pn with the stabiliser checked after the fact,
  // for schedules where GEMM2 trails by one tile: at this point O holds tiles
  // < j and S_next (tile j+1) was computed against the current m.  When a
  // lane's partial row sum exceeds 2^15 (rare: a row max rose well above m;
  // also catches inf/NaN), m moves up to the tile's row max, O, l and
  // S_next are rescaled / shifted and the tile is exponentiated again.
  // Nothing in the common path depends on a comparison, so the exponentials
  // are free to interleave with both GEMMs.
  template <class F>
  __device__ __forceinline__ void softmax_trailing(float16_t (&s)[2], V8 (&pn)[2][2],
                                                   F&& on_shift) {
    float sum = exponentiate(s, pn);
    // Keep the fp16 packing ahead of the branch (it would otherwise be sunk
    // past it, out of reach of the MFMAs it can overlap).
    asm volatile("" : : "v"(pn[0][0]), "v"(pn[0][1]), "v"(pn[1][0]), "v"(pn[1][1]));
    if (__builtin_amdgcn_ballot_w64(!(sum <= kSumLimit)) != 0) {
      const float d = fmaxf(tile_max(s), 0.0f);
      const float alpha = __builtin_amdgcn_exp2f(-(SCALED ? cr : 1.0f) * d);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      sub(s, d);
      on_shift(d);
      set_m(m + d);
      sum = exponentiate(s, pn);
    }
    l += sum;
  }
  // Lazy stabiliser, decided before any exponential: scores are t - m and
  // while every row's tile max stays within kLag (log2 units) of m, p stays
  // <= 2^kLag (exact in fp16) and nothing is rescaled.  Otherwise (rare) m
  // moves up to the new row max and what was accumulated is rescaled;
  // `on_shift(d)` lets the caller shift scores computed against the old m.
  // Deciding first keeps the exponentials free of any later dependency, so
  // they interleave with the MFMAs of the same iteration.
  template <class F>
  __device__ __forceinline__ void restabilise(float16_t (&s)[2], F&& on_shift) {
    const float mx = tile_max(s);
    const float lag = SCALED ? mx * cr : mx;
    if (__builtin_amdgcn_ballot_w64(lag > kLag) != 0) {
      const float d = fmaxf(mx, 0.0f);
      const float alpha = __builtin_amdgcn_exp2f(-(SCALED ? cr : 1.0f) * d);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      sub(s, d);
      on_shift(d);
      set_m(m + d);
    }
  }
  // Softmax of one tile into p (restabilise, then exponentiate) and the row
  // sum update.
  template <class F>
  __device__ __forceinline__ void softmax(float16_t (&s)[2], F&& on_shift) {
    restabilise(s, on_shift);
    l += exponentiate(s);
  }
  // Split key range: the partner wave holds the same rows over a disjoint
  // key range.  Its O, m and l go through LDS as part[k * 64 + lane]
  // (k < 32: O, 32: m, 33: l) and are combined at the larger m.
  __device__ __forceinline__ void save_partial(float* part, int lane) const {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) part[(16 * db + r) * 64 + lane] = o[db][r];
    part[32 * 64 + lane] = m;
    part[33 * 64 + lane] = l;
  }
  // Symmetric in the two ranges: a row with no key in one range (l == 0
  // across the lane pair) takes the other's values.
  __device__ __forceinline__ void merge_partial(const float* part, int lane) {
    const float m1 = part[32 * 64 + lane], l1 = part[33 * 64 + lane];
    const bool has0 = pair_sum(l) > 0.0f;
    const bool has1 = pair_sum(l1) > 0.0f;
    const float mm = has0 ? (has1 ? fmaxf(m, m1) : m) : m1;
    const float k = SCALED ? cr : 1.0f;
    const float a0 = has0 ? __builtin_amdgcn_exp2f(k * (m - mm)) : 0.0f;
    const float a1 = has1 ? __builtin_amdgcn_exp2f(k * (m1 - mm)) : 0.0f;
    l = a0 * l + a1 * l1;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] = a0 * o[db][r] + a1 * part[(16 * db + r) * 64 + lane];
    m = mm;
  }
  // Split-KV partial of the rows over one key chunk: O unnormalised
  // (relative to the stabiliser), the stabiliser in base-2 logit units
  // (m * cr) and the row sum, kPartStride floats per row.  A row with no key
  // in the chunk stores m = -inf and l = 0.
  __device__ __forceinline__ void store_partial(float* part) const {
    const float l_tot = pair_sum(l);
    if (my_q < seq) {
      float* r = part + (long long)my_q * kPartStride;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float* dst = r + 32 * db + 16 * hh + 8 * g;
          const float4 lo = {o[db][8 * hh], o[db][8 * hh + 1], o[db][8 * hh + 2], o[db][8 * hh + 3]};
          const float4 hi = {o[db][8 * hh + 4], o[db][8 * hh + 5], o[db][8 * hh + 6],
                             o[db][8 * hh + 7]};
          *reinterpret_cast<float4*>(dst) = lo;
          *reinterpret_cast<float4*>(dst + 4) = hi;
        }
      if (g == 0) {
        r[64] = l_tot > 0.0f ? m * (SCALED ? cr : 1.0f) : ninf();
        r[65] = l_tot;
      }
    }
  }
  // O = O^T / l, 16-byte stores of 8 contiguous head dims; rows >= N skipped.
  // With `lse`, also the row's log-sum-exp in natural-log units,
  // ln(sum_j exp(sm_scale q.k_j)) = ln 2 * (m * cr + log2 l) (-inf for a row
  // with no visible key).
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
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          V8 out;
#pragma unroll
          for (int e = 0; e < 8; ++e) out[e] = (T)(o[db][8 * hh + e] * inv);
          *reinterpret_cast<V8*>(orow + 32 * db + 16 * hh + 8 * g) = out;
        }
    }
  }
  // As store(), through buffer resources whose ranges end at the last valid
  // row: O (rows r0.. of the resource, row_bytes apart) and the log-sum-exp
  // (one float per row; an empty range when not requested).  Every lane
  // issues the same five stores and the hardware drops the out-of-range
  // ones, so a wave's count of outstanding memory operations is fixed.
  __device__ __forceinline__ void store_rsrc(__amdgpu_buffer_rsrc_t ro, int r0, int row_bytes,
                                             __amdgpu_buffer_rsrc_t rl) const {
    const float l_tot = pair_sum(l);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const int row = my_q - r0;
    const float lg = m * (SCALED ? cr : 1.0f) + __builtin_amdgcn_logf(l_tot);
    const float lse = l_tot > 0.0f ? 0.693147180559945309f * lg : ninf();
    // Lanes of the second half repeat their row's value: point them past
    // the range (a row past the end never fits a range of whole rows).
    const int lse_off = g == 0 ? 4 * row : 0x7ffffff0;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lse), rl, lse_off, 0, 0);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        V8 out;
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = (T)(o[db][8 * hh + e] * inv);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, out), ro,
                                               row * row_bytes + 2 * (32 * db + 16 * hh + 8 * g),
                                               0, 0);
      }
  }
};

// Zeroes every V slot once: a tail tile's rows past N then hold zeros (or
// earlier finite data), never uninitialised bits, under p == 0.
template <int kSlots, int kThreads>
__device__ __forceinline__ void zero_v_slots(const Rings<kSlots>& rings) {
  const u32x4_t z = {0, 0, 0, 0};
  static_for(std::make_integer_sequence<int, kSlots>{}, [&](auto i) __attribute__((always_inline)) {
    for (int off = 16 * (int)threadIdx.x; off < kTileBytes; off += 16 * kThreads)
      *reinterpret_cast<u32x4_t*>(rings.vslot(i) + off) = z;
  });
  __syncthreads();
}

#define FL_DECLARE_RINGS(R)                                                          \
  __shared__ __attribute__((aligned(16))) uint8_t kr0[kTileBytes], kr1[kTileBytes], \
      kr2[kTileBytes], kr3[kTileBytes], kr4[kTileBytes], kr5[kTileBytes],           \
      kr6[kTileBytes], kr7[kTileBytes];                                              \
  __shared__ __attribute__((aligned(16))) uint8_t vr0[kTileBytes], vr1[kTileBytes], \
      vr2[kTileBytes], vr3[kTileBytes], vr4[kTileBytes], vr5[kTileBytes],           \
      vr6[kTileBytes], vr7[kTileBytes];                                              \
  const Rings<R> rings = {{kr0, kr1, kr2, kr3, kr4, kr5, kr6, kr7},                \
                          {vr0, vr1, vr2, vr3, vr4, vr5, vr6, vr7}}

// K/V rings of one key-range stream: kSlots consecutive tiles per tensor,
// slot I selected by a static index (negative indices wrap), so every slot
// address is the stream base plus a constant.
template <int kSlots>
struct StreamRings {
  uint8_t* k;
  uint8_t* v;
  template <int I>
  __device__ __forceinline__ uint8_t* kslot(Ic<I>) const {
    return k + kTileBytes * (((I % kSlots) + kSlots) % kSlots);
  }
  template <int I>
  __device__ __forceinline__ uint8_t* vslot(Ic<I>) const {
    return v + kTileBytes * (((I % kSlots) + kSlots) % kSlots);
  }
};

// ---------------------------------------------------------------------------
// Pipelined schedule: W waves of 32 query rows, D = fetch distance in tiles.
// SPLIT = 2 adds a second set of W waves for the same rows that walks the
// second half of the key range with its own rings (waves w and w + W share
// a SIMD); the halves are merged through LDS at the end.  That halves the
// longest key walk, the critical path of causal attention's last q-blocks.
// KVSPLIT ("split-KV", for few query rows over many keys): work-group i
// takes key chunk i % nsplit of its query block and writes a partial result
// (Rows::store_partial) that splitkv_combine_kernel merges.
template <int W, int D, int SPLIT, bool CAUSAL, bool SCALED, bool KVSPLIT = false>
__global__ void __launch_bounds__(64 * W * SPLIT, 2)  // 2 waves per SIMD: <= 256 VGPRs
fa2_fwd_kernel(const _Float16* Q, const _Float16* __restrict__ K,
               const _Float16* __restrict__ V, _Float16* O, const Geom geom, int nqb,
               float cq, float cr) {
  constexpr int kSlots = D + 1;
  constexpr int kUnroll = (kSlots % 2 == 0) ? kSlots : 2 * kSlots;
  constexpr int kBr = 32 * W;
  constexpr int kSegs = 8 / W;            // 1 KiB DMA segments per wave per tile
  constexpr int kDmaPerIter = 2 * kSegs;  // K + V loads a wave issues per iteration
  constexpr int kRingBytes = SPLIT * kSlots * kTileBytes;
  static_assert(kSegs * W == 8, "tile split");
  static_assert(SPLIT == 1 || SPLIT == 2, "key-range split");
  static_assert(SPLIT == 1 || kRingBytes >= W * 34 * 64 * 4, "merge buffer");
  __shared__ __attribute__((aligned(16))) uint8_t kring[kRingBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vring[kRingBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int stream = wave / W;       // key-range half
  const int rw = wave - stream * W;  // 32-row block within the work-group
  static_assert(!KVSPLIT || SPLIT == 1, "one split kind at a time");
  int bh, qb, chunk = 0;
  if constexpr (KVSPLIT) {
    const int r = blockIdx.x / geom.nsplit;
    chunk = blockIdx.x - r * geom.nsplit;
    bh = r / nqb;
    qb = r - bh * nqb;
  } else {
    wg_coords<CAUSAL, (W == 4 && SPLIT == 1) ? 2 : 1>(nqb, bh, qb);
  }
  const HeadPtrs hp = head_ptrs(geom, bh, Q, K, V, O);
  const i32x4_t rk = hp.rk, rv = hp.rv;
  const FetchOff<kSegs> fk = fetch_offsets<kSegs, false>(rw, lane, 2 * geom.k_sr);
  const FetchOff<kSegs> fv = fetch_offsets<kSegs, true>(rw, lane, 2 * geom.v_sr);
  const int seq = geom.seq_q;
  const int q0 = qb * kBr;
  const StreamRings<kSlots> rings = {kring + stream * (kSlots * kTileBytes),
                                     vring + stream * (kSlots * kTileBytes)};

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
  // Key tiles [tbeg, tend) of this stream; both streams run t0 + 1
  // iterations (the same barriers), the shorter one on masked tiles.
  constexpr bool kSplit = SPLIT == 2;
  const int t0 = kSplit ? (ntiles + 1) / 2 : ntiles;
  const int tbeg = cbeg + (stream == 0 ? 0 : t0);
  const int tend = cbeg + (stream == 0 ? t0 : ntiles);
  const int last = max(tend - 1, tbeg);  // fetch clamp
  if (kSplit && stream == 0) rows.kv_lim = min(rows.kv_lim, tend * kBc);

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
      for (int off = 16 * (int)threadIdx.x; off < kRingBytes; off += 16 * 64 * W * SPLIT)
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

  // No fetch may still be writing LDS when the work-group retires or the
  // rings are reused for the merge.
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (SPLIT == 2) {
    __syncthreads();
    float* xchg = reinterpret_cast<float*>(kring) + rw * (34 * 64);
    if (stream == 1) rows.save_partial(xchg, lane);
    __syncthreads();
    if (stream == 1) return;
    rows.merge_partial(xchg, lane);
  }
  if constexpr (KVSPLIT)
    rows.store_partial(part);
  else
    rows.store(hp.o, geom.o_sr, hp.lse);
}

// ---------------------------------------------------------------------------
// Ping-pong schedule, 8 waves: group A (waves 0-3) and group B (waves 4-7)
// alternate MFMA and softmax phases on shared SIMDs.  Step s ends with a
// barrier; the MFMA phase M(j) is GEMM2(j-1) + GEMM1(j), the softmax phase
// V(j) turns S(j) into P(j):
//     step   0     1     2     3    ...  2j     2j+1  ...  2n     2n+1
//     A     M(0)  V(0)  M(1)  V(1)  ...  M(j)   V(j)  ...  M(n)    -
//     B      -    M(0)  V(0)  M(1)  ...  V(j-1) M(j)  ...  V(n-1) M(n)
// K(t) is read in steps 2t, 2t+1 and V(t) in 2t+2, 2t+3; step 2u (even)
// fetches K(u+D) and V(u+D-1) into rings of D+1 slots, and every odd step
// ends by waiting for the fetch group issued D-1 groups earlier.
template <int D, bool CAUSAL, bool SCALED>
__global__ void __launch_bounds__(512, 1)
fa2_fwd_pp_kernel(const _Float16* Q, const _Float16* __restrict__ K,
                  const _Float16* __restrict__ V, _Float16* O, const Geom geom, int nqb,
                  float cq, float cr) {
  constexpr int kSlots = D + 1;
  constexpr int kBr = 256;
  constexpr int kPending = (D - 1) * 2;  // one K and one V segment per wave per group
  FL_DECLARE_RINGS(kSlots);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool group_b = wave >= 4;
  int bh, qb;
  wg_coords<CAUSAL, 1>(nqb, bh, qb);
  const HeadPtrs hp = head_ptrs(geom, bh, Q, K, V, O);
  const i32x4_t rk = hp.rk, rv = hp.rv;
  const FetchOff<1> fk = fetch_offsets<1, false>(wave, lane, 2 * geom.k_sr);
  const FetchOff<1> fv = fetch_offsets<1, true>(wave, lane, 2 * geom.v_sr);
  const int seq = geom.seq_q;
  const int q0 = qb * kBr;

  Rows<CAUSAL, SCALED> rows;
  rows.init(hp.q, geom.q_sr, lane, q0 + 32 * wave, seq, geom.seq_k, geom.coff, cq, cr);

  int ntiles = max(1, (geom.seq_k + kBc - 1) / kBc);
  if (CAUSAL) ntiles = min(ntiles, causal_tiles(min(q0 + kBr, seq), geom.coff));
  const int n = ntiles;
  const int last = n - 1;

  // Fetch group u (ring position U = u mod kSlots, static): K(u+D), V(u+D-1).
  auto fetch_group = [&](auto upos, int u) __attribute__((always_inline)) {
    constexpr int U = decltype(upos)::value;
    fetch_tile<1>(rk, rings.kslot(Ic<U + D>{}), u + D, last, wave, fk);
    fetch_tile<1>(rv, rings.vslot(Ic<U + D - 1>{}), max(u + D - 1, 0), last, wave, fv);
  };
  float16_t S[2];
  // MFMA phase M(j) at ring position J = j mod kSlots: GEMM2(j-1), GEMM1(j).
  auto mfma_phase = [&](auto jpos, auto has_v, auto has_k) __attribute__((always_inline)) {
    constexpr int J = decltype(jpos)::value;
    half8_t ka[2][4], va[2][4];
    if constexpr (decltype(has_v)::value) rows.read_v(rings.vslot(Ic<J - 1>{}), va);
    if constexpr (decltype(has_k)::value) rows.read_k(rings.kslot(Ic<J>{}), ka);
    if constexpr (decltype(has_v)::value) rows.gemm2(va);
    if constexpr (decltype(has_k)::value) rows.gemm1(ka, S);
  };
  // Softmax phase V(j).
  auto softmax_phase = [&](int j) __attribute__((always_inline)) {
    rows.mask(j, S);
    if (j == 0) rows.first_tile(S);
    rows.softmax(S, [](float) {});
  };

  // ---- prologue: zero V slots, fetch groups -D .. -1, wait for group -D.
  zero_v_slots<kSlots, 512>(rings);
  static_for(std::make_integer_sequence<int, D>{}, [&](auto i) __attribute__((always_inline)) {
    constexpr int u = decltype(i)::value - D;
    fetch_group(Ic<u>{}, u);
  });
  sync_ring<kPending>();

  if (!group_b) {
    // step 0: M(0) (GEMM1 only); step 1: V(0)
    fetch_group(Ic<0>{}, 0);
    mfma_phase(Ic<0>{}, Ic<0>{}, Ic<1>{});
    sync_ring<63>();
    softmax_phase(0);
    sync_ring<kPending>();
    // steps 2j, 2j+1 for j = 1 .. n-1
    for (int j0 = 1; j0 < n; j0 += kSlots) {
      static_for(std::make_integer_sequence<int, kSlots>{}, [&](auto i) __attribute__((always_inline)) {
        constexpr int J = 1 + decltype(i)::value;  // position of j0 + i (j0 = 1 mod kSlots)
        const int j = j0 + decltype(i)::value;
        if (j < n) {
          fetch_group(Ic<J>{}, j);
          mfma_phase(Ic<J>{}, Ic<1>{}, Ic<1>{});
          sync_ring<63>();
          softmax_phase(j);
          sync_ring<kPending>();
        }
      });
    }
    // step 2n: M(n) (GEMM2 only) at position n mod kSlots
    static_for(std::make_integer_sequence<int, kSlots>{}, [&](auto i) __attribute__((always_inline)) {
      constexpr int J = decltype(i)::value;
      if (n % kSlots == J) {
        fetch_group(Ic<J>{}, n);
        mfma_phase(Ic<J>{}, Ic<1>{}, Ic<0>{});
      }
    });
    sync_ring<63>();
    // step 2n+1: idle
    sync_ring<kPending>();
  } else {
    // step 0: idle; step 1: M(0); step 2: V(0)
    fetch_group(Ic<0>{}, 0);
    sync_ring<63>();
    mfma_phase(Ic<0>{}, Ic<0>{}, Ic<1>{});
    sync_ring<kPending>();
    fetch_group(Ic<1>{}, 1);
    softmax_phase(0);
    sync_ring<63>();
    // steps 2j+1, 2j+2 for j = 1 .. n-1
    for (int j0 = 1; j0 < n; j0 += kSlots) {
      static_for(std::make_integer_sequence<int, kSlots>{}, [&](auto i) __attribute__((always_inline)) {
        constexpr int J = 1 + decltype(i)::value;
        const int j = j0 + decltype(i)::value;
        if (j < n) {
          mfma_phase(Ic<J>{}, Ic<1>{}, Ic<1>{});
          sync_ring<kPending>();
          fetch_group(Ic<J + 1>{}, j + 1);
          softmax_phase(j);
          sync_ring<63>();
        }
      });
    }
    // step 2n+1: M(n) (GEMM2 only)
    static_for(std::make_integer_sequence<int, kSlots>{}, [&](auto i) __attribute__((always_inline)) {
      constexpr int J = decltype(i)::value;
      if (n % kSlots == J) mfma_phase(Ic<J>{}, Ic<1>{}, Ic<0>{});
    });
    sync_ring<kPending>();
  }

  __builtin_amdgcn_s_waitcnt(0);
  rows.store(hp.o, geom.o_sr, hp.lse);
}

// End of a slot-scheduled iteration: this wave's LDS fetches older than its
// newest kVm have landed and all but its newest kLgkm LDS reads (the
// operands read ahead for the next iteration) have completed; barrier.
template <int kVm, int kLgkm>
__device__ __forceinline__ void sync_ring_ahead() {
  static_assert(kVm >= 0 && kVm < 64 && kLgkm >= 0 && kLgkm < 16, "waitcnt range");
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(%1)\n\ts_barrier" : : "n"(kVm), "n"(kLgkm) : "memory");
  __builtin_amdgcn_sched_barrier(0);
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
template <int W, int FV, bool CAUSAL, bool SCALED, class T = _Float16>
__global__ void __launch_bounds__(64 * W, 2)  // <= 256 VGPRs: 2 waves per SIMD at W = 8
fa2_fwd_slot_kernel(const T* Q, const T* __restrict__ K, const T* __restrict__ V, T* O,
                    const Geom geom, int nqb, float cq, float cr) {
  using RowsT = Rows<CAUSAL, SCALED, T>;
  using V8 = typename RowsT::V8;
  // fp16: unmasked tiles sum P with the packed-fp16 tree; bf16 P keeps
  // fp32 sums throughout (an 8-bit mantissa tree would cost accuracy).
  constexpr bool kFp16 = __is_same(T, _Float16);
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
  constexpr int kWgPerCu = (W <= 4 && 2 * 2 * kRingBytes <= 160 * 1024) ? 2 : 1;
  static_assert(kSegs * W == 8, "tile split");
  static_assert(FV >= 2 && FV <= 6, "fetch distance");
  static_assert(kAhead % 2 == 0 && kAhead < 16, "read-ahead");
  __shared__ __attribute__((aligned(16))) uint8_t kring[kRingBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vring[kRingBytes];

  const int lane = threadIdx.x & 63;
  const int rw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int bh, qb;
  wg_coords<CAUSAL, kWgPerCu>(nqb, bh, qb);
  const HeadPtrs<T> hp = head_ptrs(geom, bh, Q, K, V, O);
  const i32x4_t rk = hp.rk, rv = hp.rv;
  const FetchOff<kSegs> fk = fetch_offsets<kSegs, false>(rw, lane, 2 * geom.k_sr);
  const FetchOff<kSegs> fv = fetch_offsets<kSegs, true>(rw, lane, 2 * geom.v_sr);
  const int seq = geom.seq_q;
  const int q0 = qb * kBr;
  const StreamRings<kSlots> rings = {kring, vring};

  int ntiles = max(1, (geom.seq_k + kBc - 1) / kBc);
  if (CAUSAL) ntiles = min(ntiles, causal_tiles(min(q0 + kBr, seq), geom.coff));
  const int t0 = ntiles;  // iterations 0 .. t0; the last one only drains GEMM2
  const int last = ntiles - 1;

  // Prologue fetch groups -FK .. -1 (V tiles < 0 read as zeros through the
  // buffer bound, which also zeroes the slot GEMM2(-1) reads under P = 0),
  // issued before the Q loads so the two latencies overlap.
  static_for(std::make_integer_sequence<int, FK>{}, [&](auto i) __attribute__((always_inline)) {
    constexpr int G = decltype(i)::value - FK;
    fetch_tile<kSegs>(rk, rings.kslot(Ic<G + FK>{}), G + FK, last, rw, fk);
    fetch_tile<kSegs>(rv, rings.vslot(Ic<G + FV>{}), G + FV, last, rw, fv);
  });
  RowsT rows;
  rows.init(hp.q, geom.q_sr, lane, q0 + 32 * rw, seq, geom.seq_k, geom.coff, cq, cr);
  if constexpr (kMfmaSum) rows.init_msum(lane);

  // Iterations j < jm need no mask on tiles j and j + 1.
  int tm = rows.kv_lim >> 6;
  if (CAUSAL) tm = min(tm, (rows.qd + 1) >> 6);
  const int jm = max(0, tm - 1);

  // ---- first pass ----
  sync_ring_ahead<(FK - 1) * kDmaPerIter, 0>();  // K(0)
  float16_t S[2];
  V8 P0[2][2], P1[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) P1[a][b] = (V8){0, 0, 0, 0, 0, 0, 0, 0};
  {
    // S(0) with the exact row max; iteration 0 recomputes block 1 against it.
    V8 ka[2][4];
    rows.read_k(rings.kslot(Ic<0>{}), ka);
    rows.gemm1(ka, S);
  }
  rows.mask(0, S);
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
    fetch_tile<kSegs>(rk, rings.kslot(Ic<I + FK>{}), j + FK, last, rw, fk);
    fetch_tile<kSegs>(rv, rings.vslot(Ic<I + FV>{}), j + FV, last, rw, fv);
    V8 op[16];
#pragma unroll
    for (int a = 0; a < kAhead; ++a) op[a] = ahead[a];
    half2_t tree[14];
    float sum[4];
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
      rows.template exp_slot<L>(S, P);
      if constexpr (kMfmaSum)
        ;
      else if constexpr (kFp16 && !kMasked)
        RowsT::template sum_slot<L>(P, tree);
      else
        RowsT::template sum_slot_f32<L>(S, sum, rows.cr);
      if constexpr (kMasked && L == 7) rows.template mask_block<1>(j, S[1]);
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (!kMfmaSum) {
      float tot;
      if constexpr (kFp16 && !kMasked)
        tot = RowsT::sum_root(tree);
      else
        tot = (sum[0] + sum[1]) + (sum[2] + sum[3]);
      rows.l += tot;
      out_of_range |= __builtin_amdgcn_ballot_w64(!(tot <= kSumLimit));
    }
    if constexpr (kMasked) rows.template mask_block<0>(j + 1, S[0]);
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
  {
    int j0 = 0;
    for (; j0 + kUnroll <= jm; j0 += kUnroll) group(j0, Ic<false>{});
    for (; j0 <= t0; j0 += kUnroll) group(j0, Ic<true>{});
  }
  if constexpr (kMfmaSum) {
    // Every p of the first pass is in its row's sum, so a sum within 2^40
    // bounds every p by 2^40 (finite O terms for any |V| below 2^88); a
    // larger sum, inf or NaN (a row max far above the first tile's) sends
    // the block to the checked pass.
    rows.l = rows.msum_share();
    out_of_range = __builtin_amdgcn_ballot_w64(!(rows.l <= kMsumLimit));
  }

  // ---- checked pass, when any wave saw a tile sum out of range ----
  // The work-group's flag lives in K ring slot 1, which the checked pass
  // never refills (the rings are idle here: every wave has drained its
  // fetches and reads before the first barrier).  No extra LDS, so two
  // 80 KiB work-groups still fit one CU.
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
      float16_t Sc[2];
      V8 Pc[2][2];
      {
        V8 ka[2][4];
        rows.read_k(rings.kslot(Ic<0>{}), ka);
        rows.gemm1(ka, Sc);
      }
      rows.mask(t, Sc);
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
  rows.launder();
  rows.store(hp.o, geom.o_sr, hp.lse);
}

// ---------------------------------------------------------------------------
// Short key ranges (N_k <= 256, e.g. many heads of 256 tokens): a unit is
// one head's block of up to 256 query rows, whose whole K and V (4 tiles
// each, 64 KiB) fit one LDS buffer.  A persistent work-group of 8 waves (32
// rows each) walks units u = blockIdx.x, + gridDim.x, ... through two such
// buffers: after the barrier that publishes unit i, each wave reads its Q
// rows, then issues unit i+1's K/V fetches (into the buffer unit i-1 used)
// and its own next Q rows (into the 4 KiB it just read), then computes unit
// i and stores it.  Per-wave memory operations per unit are fixed (8 K/V
// and 4 Q fetches, 5 stores; out-of-range rows are dropped by the buffer
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

template <bool CAUSAL, bool SCALED, class T = _Float16>
__global__ void __launch_bounds__(512, 2)  // <= 256 VGPRs: 8 waves, two per SIMD
fa2_fwd_stream_kernel(const T* Q, const T* __restrict__ K, const T* __restrict__ V, T* O,
                      const Geom geom, int nqb, int units, float cq, float cr) {
  using RowsT = Rows<CAUSAL, SCALED, T>;
  using V8 = typename RowsT::V8;
  constexpr int kStores = 5;  // Rows::store_rsrc
  __shared__ __attribute__((aligned(16))) uint8_t buf[2][2 * kStreamHalf];  // [unit parity][K | V]
  __shared__ __attribute__((aligned(16))) uint8_t qbuf[8 * 4096];            // 32 Q rows per wave

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
  // this wave's 32 Q rows into its 4 KiB of qbuf (rows >= N_q read as
  // zeros), all by LDS DMA; chunks swizzled as K tiles are.
  int qoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int lrow = 8 * i + (lane >> 3);
    qoff[i] = (32 * blk + lrow) * qrow_bytes + 16 * ((lane & 7) ^ k_swz(lrow));
    asm volatile("" : "+v"(qoff[i]));
  }
  uint8_t* const qdst = qbuf + 4096 * rw;
  auto issue_loads = [&](int u, int b) __attribute__((always_inline)) {
    const int bh = u / nqb, qb = u - bh * nqb;
    const HeadPtrs<T> hp = head_ptrs<T>(geom, bh, Q, K, V, O);
#pragma unroll
    for (int t = 0; t < kStreamTiles; ++t) {
      fetch_tile<1>(hp.rk, buf[b] + t * kTileBytes, t, kStreamTiles - 1, rw, fk);
      fetch_tile<1>(hp.rv, buf[b] + kStreamHalf + t * kTileBytes, t, kStreamTiles - 1, rw, fv);
    }
    const int q0 = qb * kStreamBr;
    const int valid = min(kStreamBr, seq - q0);
    const i32x4_t rq =
        buffer_rsrc(hp.q + (long long)q0 * geom.q_sr, (valid - 1) * qrow_bytes + kRowBytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lds_base = (uint32_t)(uintptr_t)(qdst + 1024 * i);
      asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(qoff[i]), "s"(rq),
                   "{m0}"(lds_base));
    }
  };

  const int G = gridDim.x;
  // Unit u in buffer b; its loads have landed and every wave is done with
  // the other buffer.
  auto unit = [&](int u, int b) __attribute__((always_inline)) {
    const int bh = u / nqb, qb = u - bh * nqb;
    const int q0 = qb * kStreamBr;
    const int qw = q0 + 32 * blk;
    RowsT rows;
    rows.place(lane, qw, seq, geom.seq_k, geom.coff, cr);
    {
      u32x4_t raw[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        raw[s] = *reinterpret_cast<const u32x4_t*>(qdst + 128 * col +
                                                    16 * ((2 * s + g) ^ k_swz(col)));
      rows.set_q(raw, cq);
    }
    rows.reset();
    // This wave's Q reads are done before its DMA refills the same rows.
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    if (u + G < units) issue_loads(u + G, b ^ 1);

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
    const int valid = min(kStreamBr, seq - q0);
    const int b_ = bh / geom.heads, h_ = bh - b_ * geom.heads;
    T* oh = O + (b_ * geom.o_sb + h_ * geom.o_sh) + (long long)q0 * geom.o_sr;
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        (void*)oh, 0, (valid - 1) * 2 * geom.o_sr + kRowBytes, 0x00020000);
    float* lh = geom.lse ? geom.lse + (long long)bh * seq + q0 : geom.lse;
    const __amdgpu_buffer_rsrc_t rl =
        __builtin_amdgcn_make_buffer_rsrc((void*)lh, 0, geom.lse ? 4 * valid : 0, 0x00020000);
    rows.store_rsrc(ro, q0, 2 * geom.o_sr, rl);
  };
  // The first unit is peeled off: its wait also covers the launch's first
  // loads, and every later one has exactly one unit's stores behind it.
  int u = blockIdx.x;
  issue_loads(u, 0);
  wait_vm_barrier<0>();
  unit(u, 0);
  u += G;
  for (int i = 1; u < units; ++i, u += G) {
    wait_vm_barrier<kStores>();  // only unit i-1's stores may be in flight
    unit(u, i & 1);
  }
}

// ---------------------------------------------------------------------------
// Head dim 128 (beyond the reference, whose kernels take D = 64 only,
// kernel_flash2.cu:756-757).  Key tiles of 32 rows x 256 bytes keep the
// 8 KiB tile of D = 64, so an iteration is again 16 MFMA slots: GEMM1 is one
// 32-key block over 8 head-dim steps (one chain), GEMM2 four head-dim
// blocks over 2 key steps.  With 16 scores per lane per tile there is one
// exponential per MFMA, so the softmax VALU work fits under the matrix
// core with room to spare and the row sums stay fp32.
constexpr int kD2 = 128;
constexpr int kBc2 = 32;
constexpr int kRowBytes2 = 2 * kD2;  // 256

// DMA lane offsets for 256-byte rows: segment i of wave w is rows
// 4(w kSegs + i) .. +3; lane l lands at byte 16 l of it, i.e. row l/16,
// physical chunk l%16, which holds logical chunk (l%16) ^ swz(row) (the
// swizzles flip the low 3 chunk bits only).
template <int kSegs, bool IS_V>
__device__ __forceinline__ FetchOff<kSegs> fetch_offsets128(int wave, int lane, int row_bytes) {
  FetchOff<kSegs> f;
#pragma unroll
  for (int i = 0; i < kSegs; ++i) {
    const int seg = wave * kSegs + i;
    const int row = 4 * seg + (lane >> 4);
    const int phys = lane & 15;
    const int logical = phys ^ (IS_V ? v_swz(row) : k_swz(row));
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
    return *reinterpret_cast<const V8*>(kt + col * kRowBytes2 + 16 * (ch ^ k_swz(col)));
  }
  __device__ __forceinline__ V8 read_v_op(const uint8_t* vt, int db, int t) const {
    const int r1 = 16 * t + tr_row;
    const int r2 = r1 + 8;
    const int dcol = 32 * db + tr_col;
    const int ch = dcol >> 3, hb = ((dcol >> 2) & 1) * 8;
    const V4 lo = lds_read_tr<V4>(vt + r1 * kRowBytes2 + 16 * (ch ^ v_swz(r1)) + hb);
    const V4 hi = lds_read_tr<V4>(vt + r2 * kRowBytes2 + 16 * (ch ^ v_swz(r2)) + hb);
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
  wg_coords<CAUSAL, kWgPerCu>(nqb, bh, qb);
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

// ---------------------------------------------------------------------------
// Split-KV combine: one wave per query row merges the nsplit partials of the
// row (O unnormalised at stabiliser m_s, row sum l_s) at their largest m:
//   O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s,
// and writes O (fp16, lane = head dim) and, when asked, the log-sum-exp.
__device__ __forceinline__ float wave_max64(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
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
  float mx = ninf();
  for (int s = lane; s < geom.nsplit; s += 64) mx = fmaxf(mx, p0[s * split_stride + 64]);
  mx = wave_max64(mx);
  float acc = 0.0f, lsum = 0.0f;
  for (int s = 0; s < geom.nsplit; ++s) {
    const float* ps = p0 + s * split_stride;
    const float m = ps[64];
    if (m == ninf()) continue;  // no key of this chunk is visible to the row
    const float w = __builtin_amdgcn_exp2f(m - mx);
    lsum += w * ps[65];
    acc += w * ps[lane];
  }
  const int b = bh / geom.heads, h = bh - b * geom.heads;
  _Float16* orow = O + (b * geom.o_sb + h * geom.o_sh) + (long long)row * geom.o_sr;
  orow[lane] = (_Float16)(lsum > 0.0f ? acc / lsum : 0.0f);
  if (geom.lse != nullptr && lane == 0)
    geom.lse[row_id] =
        lsum > 0.0f ? 0.693147180559945309f * (mx + __builtin_amdgcn_logf(lsum)) : ninf();
}

// Q is prescaled by cq = +-min(c, 1) in the kernel; the remaining factor
// cr = c / |cq| (1 unless c > 1) is applied to the scores.
// bf16 and head_dim 128 keep Q exact (cq = +-1) and scale the fp32 scores
// instead: a bf16 rounding of the prescaled Q would cost 2^-9 of every
// score, and at D = 128 the fp16 rounding error of a score grows with
// sqrt(D) past the fp16 output tolerance at large scales (2.3e-3 measured at
// sm_scale -0.3), while one exponential per MFMA leaves the extra multiply
// room under the matrix core.
struct Scales {
  float cq, cr;
  bool scaled;
  explicit Scales(const FwdArgs& a) {
    const float c = a.scale_log2;
    const bool exact_q = a.dtype == kDtypeBF16 || a.head_dim == kD2;
    cq = (c <= 1.0f && !exact_q ? c : 1.0f) * (a.negate ? -1.0f : 1.0f);
    cr = c <= 1.0f && !exact_q ? 1.0f : c;
    scaled = cr != 1.0f;
  }
};

Geom make_geom(const FwdArgs& a) {
  Geom g;
  g.q_sb = a.q_sb;
  g.q_sh = a.q_sh;
  g.k_sb = a.k_sb;
  g.k_sh = a.k_sh;
  g.v_sb = a.v_sb;
  g.v_sh = a.v_sh;
  g.o_sb = a.o_sb;
  g.o_sh = a.o_sh;
  g.q_sr = a.q_sr;
  g.k_sr = a.k_sr;
  g.v_sr = a.v_sr;
  g.o_sr = a.o_sr;
  g.heads = a.heads;
  g.seq_q = a.seq;
  g.seq_k = a.seq_k;
  g.coff = a.seq_k - a.seq;
  g.lse = a.lse;
  g.part = nullptr;
  g.nsplit = 1;
  g.batch_heads = a.batch_heads;
  return g;
}

template <template <bool, bool> class Launcher>
hipError_t dispatch(const FwdArgs& a, hipStream_t stream, int br) {
  const int nqb = (a.seq + br - 1) / br;
  const dim3 grid((unsigned)(nqb * a.batch_heads));
  const Scales sc(a);
  const Geom g = make_geom(a);
  hipError_t e;
  if (a.causal) {
    if (sc.scaled) e = Launcher<true, true>::run(a, g, grid, nqb, sc.cq, sc.cr, stream);
    else e = Launcher<true, false>::run(a, g, grid, nqb, sc.cq, sc.cr, stream);
  } else {
    if (sc.scaled) e = Launcher<false, true>::run(a, g, grid, nqb, sc.cq, sc.cr, stream);
    else e = Launcher<false, false>::run(a, g, grid, nqb, sc.cq, sc.cr, stream);
  }
  return e != hipSuccess ? e : hipGetLastError();
}

template <int W, int D, int SPLIT>
struct PipelinedLaunch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, SPLIT, C, S>), grid, dim3(64 * W * SPLIT), 0, st,
                         static_cast<const _Float16*>(a.q), static_cast<const _Float16*>(a.k),
                         static_cast<const _Float16*>(a.v), static_cast<_Float16*>(a.o), g, nqb,
                         cq, cr);
      return hipSuccess;
    }
  };
};

template <int D>
struct PingPongLaunch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      hipLaunchKernelGGL((fa2_fwd_pp_kernel<D, C, S>), grid, dim3(512), 0, st,
                         static_cast<const _Float16*>(a.q), static_cast<const _Float16*>(a.k),
                         static_cast<const _Float16*>(a.v), static_cast<_Float16*>(a.o), g, nqb,
                         cq, cr);
      return hipSuccess;
    }
  };
};

template <int W, int FV, class T = _Float16>
struct SlotLaunch {
  template <bool C, bool S>
  struct L {
    static hipError_t run(const FwdArgs& a, const Geom& g, dim3 grid, int nqb, float cq, float cr,
                          hipStream_t st) {
      hipLaunchKernelGGL((fa2_fwd_slot_kernel<W, FV, C, S, T>), grid, dim3(64 * W), 0, st,
                         static_cast<const T*>(a.q), static_cast<const T*>(a.k),
                         static_cast<const T*>(a.v), static_cast<T*>(a.o), g, nqb, cq, cr);
      return hipSuccess;
    }
  };
};

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

// Streaming short-key kernel: one persistent work-group per CU (its two
// 64 KiB buffers take 128 KiB of the CU's 160 KiB), at most one per unit.
template <class T>
hipError_t launch_stream(const FwdArgs& a, hipStream_t st) {
  constexpr int kCus = 256;
  const int nqb = (a.seq + kStreamBr - 1) / kStreamBr;
  const int units = nqb * a.batch_heads;
  const dim3 grid((unsigned)min(units, kCus));
  const Scales sc(a);
  const Geom g = make_geom(a);
  const T *q = static_cast<const T*>(a.q), *k = static_cast<const T*>(a.k),
          *v = static_cast<const T*>(a.v);
  T* o = static_cast<T*>(a.o);
  if (a.causal) {
    if (sc.scaled)
      hipLaunchKernelGGL((fa2_fwd_stream_kernel<true, true, T>), grid, dim3(512), 0, st, q, k, v, o, g, nqb, units, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_stream_kernel<true, false, T>), grid, dim3(512), 0, st, q, k, v, o, g, nqb, units, sc.cq, sc.cr);
  } else {
    if (sc.scaled)
      hipLaunchKernelGGL((fa2_fwd_stream_kernel<false, true, T>), grid, dim3(512), 0, st, q, k, v, o, g, nqb, units, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_stream_kernel<false, false, T>), grid, dim3(512), 0, st, q, k, v, o, g, nqb, units, sc.cq, sc.cr);
  }
  return hipGetLastError();
}

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
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, 1, true, true, true>), grid, block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, 1, true, false, true>), grid, block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
  } else {
    if (sc.scaled)
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, 1, false, true, true>), grid, block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
    else
      hipLaunchKernelGGL((fa2_fwd_kernel<W, D, 1, false, false, true>), grid, block, 0, st, q, k, v, o, g, nqb, sc.cq, sc.cr);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int rows = a.batch_heads * a.seq;
  hipLaunchKernelGGL(splitkv_combine_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, o,
                     g);
  return hipGetLastError();
}

}  // namespace

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

const Fa2Config kFa2Configs[kNumFa2Configs] = {
    {1, "br32_bc64_w1"},
    {2, "br64_bc64_w2"},
    {4, "br128_bc64_w4"},
    {8, "br256_bc64_w8"},
    {8, "br256_bc64_w8_pingpong"},
    {8, "br128_bc64_w4_split2"},
    {8, "br256_bc64_w8_slot"},
    {4, "br128_bc64_w4_slot"},
    {8, "br256_kv256_w8_stream"},
};

bool stream_config_fits(const FwdArgs& a) {
  return a.seq_k <= kStreamMaxKeys && a.q_sr < kStreamMaxRowStride &&
         a.k_sr < kStreamMaxRowStride && a.v_sr < kStreamMaxRowStride &&
         a.o_sr < kStreamMaxRowStride;
}

// Fetch distance: three tiles ahead where LDS allows (64 KiB of rings per
// work-group), one tile for single-wave groups (32 KiB: five per CU).
hipError_t launch_fa2(const FwdArgs& a, int cfg, hipStream_t stream) {
  if (a.head_dim == kD2) {
    const bool bf = a.dtype == kDtypeBF16;
    if (cfg == kSlotW8Config)
      return bf ? dispatch<D128Launch<8, 5, 4, __bf16>::L>(a, stream, 256)
                : dispatch<D128Launch<8, 5, 4, _Float16>::L>(a, stream, 256);
    if (cfg == kSlotW4Config)
      return bf ? dispatch<D128Launch<4, 5, 4, __bf16>::L>(a, stream, 128)
                : dispatch<D128Launch<4, 5, 4, _Float16>::L>(a, stream, 128);
    return hipErrorInvalidValue;
  }
  if (a.dtype == kDtypeBF16) {
    if (cfg == kSlotW8Config) return dispatch<SlotLaunch<8, 4, __bf16>::L>(a, stream, 256);
    if (cfg == kSlotW4Config) return dispatch<SlotLaunch<4, 3, __bf16>::L>(a, stream, 128);
    return hipErrorInvalidValue;
  }
  switch (cfg) {
    case 0: return dispatch<PipelinedLaunch<1, 1, 1>::L>(a, stream, 32);
    case 1: return dispatch<PipelinedLaunch<2, 3, 1>::L>(a, stream, 64);
    case 2: return dispatch<PipelinedLaunch<4, 3, 1>::L>(a, stream, 128);
    case 3: return dispatch<PipelinedLaunch<8, 3, 1>::L>(a, stream, 256);
    case 4: return dispatch<PingPongLaunch<3>::L>(a, stream, 256);
    case 5: return dispatch<PipelinedLaunch<4, 3, 2>::L>(a, stream, 128);
    case 6: return dispatch<SlotLaunch<8, 4>::L>(a, stream, 256);
    case 7: return dispatch<SlotLaunch<4, 3>::L>(a, stream, 128);
    case 8: return stream_config_fits(a) ? launch_stream<_Float16>(a, stream) : hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fl
