// FlashAttention-2 forward for gfx950 (MI355X, CDNA4), fp16 (and bf16) in /
// fp32 accumulate, head_dim 64 (and 128): the device building blocks shared
// by every schedule, and the host-side launch helpers.
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
//   P rounded to fp16 before the PV product (:278-285).
//
// Work decomposition.  A wave owns 32 consecutive query rows of one
// (batch, head) (struct Rows below); a work-group owns one or more such
// blocks.  The KV sequence is walked in tiles of 64 keys staged in LDS and
// shared by the work-group's waves.
//
// MFMA formulation (v_mfma_f32_32x32x16_f16, 64 lanes, lane l: column l%32,
// k-group g = l/32):
//   GEMM1  S^T[key][query] = K . Q'^T - m   A = K rows from LDS
//                                           (ds_read_b128), B = the wave's
//                                           Q rows in VGPRs, C = -m.
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
// Softmax, at one exp per score.  As in the reference, Q enters GEMM1
// unscaled (only the sign of sm_scale is applied, exactly) and each fp32
// score is multiplied by c = |sm_scale| * log2 e (kernel_flash2.cu:188-195,
// :529-536; the factor is computed at :772) -- the SCALED template path,
// one multiply per score.  (Prescaling Q by c instead and rounding it to
// fp16 saves that multiply but measured 25% more mean error on full
// outputs.)  The running stabiliser m (in unscaled score units) enters as
// the MFMA accumulator's initial value, so GEMM1 returns s - m and
// p = v_exp_f32(c * (s - m)).  m is the exact row max of the first tile and
// later only moves when a tile would push p out of range (a stale m is
// exact math since softmax is shift invariant; m never exceeds the running
// max, so the row sum stays >= 1).  p is packed to fp16 for GEMM2.  Row
// sums: the reference sums the unrounded fp32 p (kernel_flash2.cu:268-276,
// :339), as the pipelined, streaming, key-quarter and head_dim-128 kernels
// here do (each lane sums its own keys and the two halves of a row meet
// once, in the epilogue); the slot schedules sum the rounded p that GEMM2
// multiplies, in fp32 on the matrix core (Rows::init_msum).
//
// K/V staging.  Tiles are fetched straight into LDS with buffer_load ... lds
// (no VGPRs, no LDS-store instructions; rows past N read as zeros through
// the buffer resource's bound) several tiles ahead, into rings of slots per
// tensor.  Loops are unrolled by the ring length, so every slot address is
// a constant offset.  One explicit "s_waitcnt vmcnt(n); s_barrier" per step
// makes a tile visible.
//
// Schedules (one source file each):
//   fa2_slot.hip    W = 8 or 4 waves of 32 rows, 16 fenced MFMA slots per
//                   tile, each carrying two exponentials and the LDS read of
//                   a later slot's operand.
//   fa2_pipe.hip    any W; SPLIT = 1 or 2 key-range halves; split-KV chunks
//                   and their combine kernel.
//   fa2_stream.hip  N_k <= 256: one persistent 8-wave work-group per CU
//                   walks whole units through two LDS buffers.
//   fa2_d128.hip    head_dim 128: the slot schedule over 32-key tiles.
//
// Causal.  Keys after a lane's query and keys >= N are masked to -inf on the
// diagonal and tail tiles only; work-groups are fed to each XCD heaviest
// first, with heavy and light blocks paired on a CU (wg_coords).
//
// LDS.  Rows of 128 B (64 halfs).  16-byte chunks are XOR-swizzled per row:
// K with (row&7)^((row>>3)&1), V with 2*(row&3), which makes the GEMM1
// ds_read_b128 pattern, the GEMM2 ds_read_b64_tr_b16 pattern and the
// row-contiguous tile writes conflict-free (0 SQ_LDS_BANK_CONFLICT measured
// for the D = 64 kernels).

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "fl_internal.h"

namespace fl {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
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
  int xcds, cus_per_xcd;  // the device's XCDs and CUs per XCD (wg_coords)
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

// K and V resources of head `bh` that end after row `rows` (at most N_k):
// loads of later rows return zeros without reaching memory, so fetches past
// a walk's last tile cost no L2 or HBM traffic.
template <class T, int kRowB = kRowBytes>
__device__ __forceinline__ void kv_rsrc_rows(const Geom& g, int bh, const T* K, const T* V,
                                             int rows, i32x4_t& rk, i32x4_t& rv) {
  const int b = bh / g.heads, h = bh - b * g.heads;
  const int n = min(rows, g.seq_k);
  rk = buffer_rsrc(K + (b * g.k_sb + h * g.k_sh), n > 0 ? (n - 1) * (2 * g.k_sr) + kRowB : 0);
  rv = buffer_rsrc(V + (b * g.v_sb + h * g.v_sh), n > 0 ? (n - 1) * (2 * g.v_sr) + kRowB : 0);
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

// Work-group -> (batch*head, query block).  Work-groups are dealt to the
// device's XCDs round-robin (`xcds`, 8 on an MI355X seen whole); remap so
// that the query blocks of a head land on the same XCD (shared K/V in its
// L2).  Causal work-groups differ in length, so each XCD is fed heaviest
// first (heads interleaved).  Measured dispatch on gfx950: an XCD fills its
// CUs (`cpx` of them, 32 on an MI355X) in a fixed order with its first cpx
// work-groups; with two co-resident work-groups per CU its next cpx fill the
// second slots of the same CUs in the same order; after that each goes to
// whichever CU frees first.  So with kSlotsPerCu == 2 the second cpx are
// taken in reverse (CU j pairs the j-th heaviest block with the j-th
// lightest of the first 2 cpx), and every later position keeps the
// longest-processing-time order.  With one XCD the remap is the identity
// and only the causal order remains.
template <bool CAUSAL, int kSlotsPerCu>
__device__ __forceinline__ void wg_coords(int nqb, int xcds, int cpx, int& bh, int& qb) {
  const int total = gridDim.x;
  const int i = blockIdx.x;
  const int per = total / xcds;
  const int x = i % xcds;  // the XCD this work-group runs on
  const int k = i / xcds;  // its dispatch position within the XCD
  if (per * xcds != total) {
    bh = i / nqb;
    qb = i - bh * nqb;
  } else if (!CAUSAL || per % nqb != 0) {
    const int lin = x * per + k;
    bh = lin / nqb;
    qb = lin - bh * nqb;
  } else {
    const int hx = per / nqb;  // whole heads per XCD
    const int first = cpx * kSlotsPerCu;
    int r = k;                 // work rank, 0 = heaviest
    if (kSlotsPerCu == 2 && per >= first && k >= cpx && k < first) r = first - 1 - (k - cpx);
    bh = x * hx + r % hx;
    qb = r / hx;
  }
  if (CAUSAL) qb = nqb - 1 - qb;
}

// Work-group -> (batch*head, block pair p) of the pair schedule: pairs
// p = 0 .. ceil(nqb/2) - 1 of a head, dealt so that a head's pairs run on
// one XCD (shared K/V in its L2) when the work-groups divide evenly.
__device__ __forceinline__ void pair_coords(int nqb, int xcds, int& bh, int& p) {
  const int np = (nqb + 1) / 2;
  const int total = gridDim.x;
  const int i = blockIdx.x;
  const int per = total / xcds;
  const int lin = per * xcds == total ? (i % xcds) * per + i / xcds : i;
  bh = lin / np;
  p = lin - bh * np;
}

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

// The same through a resource that ends at the walk's last row
// (kv_rsrc_rows), with tiles clamped to `tzero`, the first tile wholly past
// that row: a fetch past the walk lands as zeros with no memory traffic,
// where fetch_tile re-reads the last tile.  (Rows are at least 128 bytes
// apart, so tile tzero starts at or past the resource's end; the C ABI's
// N_k limit keeps its offset below 2^31.)
template <int kSegs>
__device__ __forceinline__ void fetch_tile_z(const i32x4_t& rs, const uint8_t* slot, int t,
                                             int tzero, int wave, const FetchOff<kSegs>& f) {
  t = min(t, tzero);
  const int tb = t * f.tile_bytes;
#pragma unroll
  for (int i = 0; i < kSegs; ++i) {
    const int seg = wave * kSegs + i;
    const int voff = tb + f.lane[i];
    const uint32_t lds_base = (uint32_t)(uintptr_t)(slot + 1024 * seg);
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(rs), "{m0}"(lds_base));
  }
}

// DMA of the 32 query rows [q, q + 32) of a head (rows >= N_q read as
// zeros) into `qblk`, laid out as the first half of a K tile (Rows::
// set_q_lds reads it): 4 fetches of 1 KiB, counted by vmcnt, or with kParts
// waves sharing the block, the 4 / kParts of them of part `part`.
template <int kParts = 1, class T>
__device__ __forceinline__ void fetch_q_block(const T* Qh, int q_sr, int q, int seq,
                                              uint8_t* qblk, int lane, int part = 0) {
  static_assert(kParts == 1 || kParts == 2 || kParts == 4, "Q block parts");
  constexpr int kSegs = 4 / kParts;
  const int rows = min(32, seq - q);
  const i32x4_t rq = buffer_rsrc(Qh + (long long)(rows > 0 ? q : 0) * q_sr,
                                 rows > 0 ? (rows - 1) * (2 * q_sr) + kRowBytes : 0);
  const FetchOff<kSegs> fq = fetch_offsets<kSegs, false>(part, lane, 2 * q_sr);
  fetch_tile_z<kSegs>(rq, qblk, 0, 1, part, fq);
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

// The 32 query rows one wave owns: Q (sign of sm_scale applied), running max, row sums and
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
  // cq = +-1 applied to a 16-bit float: exact, as a flip of the sign bits
  // (two elements per dword).
  __device__ __forceinline__ static uint32_t sign_mask(float cq) {
    return cq < 0.0f ? 0x80008000u : 0u;
  }
  __device__ __forceinline__ static V8 signed_q(const u32x4_t& raw, uint32_t m) {
    return __builtin_bit_cast(V8, raw ^ (u32x4_t){m, m, m, m});
  }
  // Q'^T from the raw 16-byte chunks Q[my_q][16s + 8g .. +7] (s = 0..3).
  __device__ __forceinline__ void set_q(const u32x4_t (&raw)[4], float cq) {
    const uint32_t m = sign_mask(cq);
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = signed_q(raw[s], m);
  }
  // The same from a 32-row Q block staged in LDS like the first half of a K
  // tile (row r's chunk c at physical chunk c ^ k_swz(r)): the B operand
  // chunks are read_k_op's reads of that block.
  __device__ __forceinline__ void set_q_lds(const uint8_t* qblk, float cq) {
    const uint32_t m = sign_mask(cq);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qf[s] = signed_q(__builtin_bit_cast(u32x4_t, read_k_op(qblk, 0, s)), m);
  }
  __device__ __forceinline__ void init(const T* Qh, int q_sr, int lane, int qw_, int seq_,
                                       int seq_k, int coff, float cq, float cr_) {
    place(lane, qw_, seq_, seq_k, coff, cr_);
    // Q'^T: lane holds cq * Q[my_q][16s + 8g .. +7] for s = 0..3.
    const uint32_t sm = sign_mask(cq);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (my_q < seq) {
        const u32x4_t raw =
            *reinterpret_cast<const u32x4_t*>(Qh + (long long)my_q * q_sr + 16 * s + 8 * g);
        qf[s] = signed_q(raw, sm);
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

  // The state after init with Q'^T read from a 32-row block staged in LDS
  // (set_q_lds).
  __device__ __forceinline__ void init_lds(const uint8_t* qblk, int lane, int qw_, int seq_,
                                           int seq_k, int coff, float cq, float cr_) {
    place(lane, qw_, seq_, seq_k, coff, cr_);
    set_q_lds(qblk, cq);
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
  // One GEMM2 MFMA outside the slot map: O[db] += V^T(key step t) . P (with
  // MS, key step t's row sums ride with db = 1, as in mfma_slot).
  template <int DB, int TS, bool MS = false>
  __device__ __forceinline__ void gemm2_step(const V8& a, const V8 (&pp)[2][2]) {
    o[DB] = E::mfma(a, pp[TS >> 1][TS & 1], o[DB]);
    if constexpr (MS && DB == 1) lacc = E::mfma16(sel, pp[TS >> 1][TS & 1], lacc);
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
  // Softmax share of slot I, in two steps for schedules that scale one slot
  // ahead: the scaled scores of slot I's pair (scores 2(I%8), 2(I%8)+1 of key
  // block I/8, times cr when SCALED) ...
  template <int I>
  __device__ __forceinline__ void scale_pair(const float16_t (&s)[2], float (&x)[2]) const {
    constexpr int kb = I >> 3, r = 2 * (I & 7);
    x[0] = SCALED ? s[kb][r] * cr : s[kb][r];
    x[1] = SCALED ? s[kb][r + 1] * cr : s[kb][r + 1];
  }
  // ... and their exponentials, packed into dword I of the P operand (the
  // row sums come from the matrix core, init_msum).
  template <int I>
  __device__ __forceinline__ void exp_pair(const float (&x)[2], V8 (&pn)[2][2]) const {
    constexpr int kb = I >> 3, r = 2 * (I & 7), h = r >> 3, e = r & 7;
    const float e0 = __builtin_amdgcn_exp2f(x[0]), e1 = __builtin_amdgcn_exp2f(x[1]);
    pn[kb][h][e] = (T)e0;
    pn[kb][h][e + 1] = (T)e1;
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
  // The slot schedule's first pass: GEMM1 of key block 0 of tile kt only,
  // and m = that block's exact row max (a row with no key there has none in
  // the tile: masks keep key prefixes), so the tile's block 1 can follow
  // against the same stabiliser inside the first iteration.
  __device__ __forceinline__ void gemm1_block0(const uint8_t* kt, float16_t (&s)[2]) const {
#pragma unroll
    for (int st = 0; st < 4; ++st) s[0] = E::mfma(read_k_op(kt, 0, st), qf[st], st == 0 ? bias : s[0]);
  }
  __device__ __forceinline__ void first_block(float16_t& s0) {
    float mx = ninf();
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s0[r]);
    mx = pair_max(mx);
    mx = mx == ninf() ? 0.0f : mx;
#pragma unroll
    for (int r = 0; r < 16; ++r) s0[r] -= mx;
    set_m(mx);
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
  // key range.  Its O, m and l go through LDS in 16-byte chunks, chunk-major
  // (part4[c * 64 + lane]: c < 8 O[c/4][4(c%4) .. +3], c = 8 {m, l}): nine
  // 128-bit accesses per lane instead of 34 32-bit ones, each chunk 1 KiB
  // contiguous over the wave.
  __device__ __forceinline__ void save_partial4(float4* part4, int lane) const {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int db = c >> 2, r = 4 * (c & 3);
      part4[c * 64 + lane] = make_float4(o[db][r], o[db][r + 1], o[db][r + 2], o[db][r + 3]);
    }
    part4[8 * 64 + lane] = make_float4(m, l, 0.0f, 0.0f);
  }
  // Symmetric in the two ranges: a row with no key in one range (l == 0
  // across the lane pair) takes the other's values.
  __device__ __forceinline__ void merge_partial4(const float4* part4, int lane) {
    const float4 ml = part4[8 * 64 + lane];
    const float m1 = ml.x, l1 = ml.y;
    const bool has0 = pair_sum(l) > 0.0f;
    const bool has1 = pair_sum(l1) > 0.0f;
    const float mm = has0 ? (has1 ? fmaxf(m, m1) : m) : m1;
    const float k = SCALED ? cr : 1.0f;
    const float a0 = has0 ? __builtin_amdgcn_exp2f(k * (m - mm)) : 0.0f;
    const float a1 = has1 ? __builtin_amdgcn_exp2f(k * (m1 - mm)) : 0.0f;
    l = a0 * l + a1 * l1;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int db = c >> 2, r = 4 * (c & 3);
      const float4 x = part4[c * 64 + lane];
      o[db][r] = a0 * o[db][r] + a1 * x.x;
      o[db][r + 1] = a0 * o[db][r + 1] + a1 * x.y;
      o[db][r + 2] = a0 * o[db][r + 2] + a1 * x.z;
      o[db][r + 3] = a0 * o[db][r + 3] + a1 * x.w;
    }
    m = mm;
  }
  // Merge of NW partials in save_partial4's layout, one of the four
  // 8-column chunks of each lane's row (chunk c = 2 db + hh: o[db][8 hh ..
  // 8 hh + 7], head dims 32 db + 16 hh + 8 g ..), normalised and stored as
  // 16 bytes per lane; the wave of chunk 0 also writes the log-sum-exp.  The
  // partials meet at their largest m; one with l = 0 across the lane pair
  // (no visible key) is skipped.  The object's own o, m, l are not used.
  template <int NW>
  __device__ __forceinline__ void merge_store_chunk(const float4* const (&parts)[NW], int c,
                                                    int lane, T* Oh, int o_sr,
                                                    float* lse) const {
    float acc[8], mm, l_tot;
    merge_chunk<NW>(parts, c, lane, acc, mm, l_tot);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (lse != nullptr && c == 0 && g == 0 && my_q < seq) {
      const float lg = mm * (SCALED ? cr : 1.0f) + __builtin_amdgcn_logf(l_tot);
      lse[my_q] = l_tot > 0.0f ? 0.693147180559945309f * lg : ninf();
    }
    if (my_q < seq) {
      V8 out;
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = (T)(acc[e] * inv);
      *reinterpret_cast<V8*>(Oh + (long long)my_q * o_sr + 32 * (c >> 1) + 16 * (c & 1) + 8 * g) =
          out;
    }
  }
  // As merge_store_chunk, for a split-KV chunk: chunk c of the merged
  // partial in store_partial's layout (O unnormalised, relative to the
  // merged stabiliser; 8 floats per lane), and with chunk 0 the stabiliser in
  // base-2 logit units and the row sum.
  template <int NW>
  __device__ __forceinline__ void merge_store_partial_chunk(const float4* const (&parts)[NW],
                                                            int c, int lane, float* part) const {
    float acc[8], mm, l_tot;
    merge_chunk<NW>(parts, c, lane, acc, mm, l_tot);
    if (my_q < seq) {
      float* r = part + (long long)my_q * kPartStride;
      float* dst = r + 32 * (c >> 1) + 16 * (c & 1) + 8 * g;
      *reinterpret_cast<float4*>(dst) = make_float4(acc[0], acc[1], acc[2], acc[3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
      if (c == 0 && g == 0) {
        r[64] = l_tot > 0.0f ? mm * (SCALED ? cr : 1.0f) : ninf();
        r[65] = l_tot;
      }
    }
  }
  // The merge itself: acc = chunk c of sum_j a_j O_j, mm = the largest m of
  // a partial with keys (-inf if none), l_tot = the row's sum_j a_j l_j.
  template <int NW>
  __device__ __forceinline__ void merge_chunk(const float4* const (&parts)[NW], int c, int lane,
                                              float (&acc)[8], float& mm, float& l_tot) const {
    float mj[NW], lj[NW];
    bool has[NW];
    mm = ninf();
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const float4 ml = parts[j][8 * 64 + lane];
      mj[j] = ml.x;
      lj[j] = ml.y;
      has[j] = pair_sum(lj[j]) > 0.0f;
      if (has[j]) mm = fmaxf(mm, mj[j]);
    }
    const float k = SCALED ? cr : 1.0f;
    float lt = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const float a = has[j] ? __builtin_amdgcn_exp2f(k * (mj[j] - mm)) : 0.0f;
      lt += a * lj[j];
      const float4 x0 = parts[j][(2 * c) * 64 + lane];
      const float4 x1 = parts[j][(2 * c + 1) * 64 + lane];
      acc[0] += a * x0.x;
      acc[1] += a * x0.y;
      acc[2] += a * x0.z;
      acc[3] += a * x0.w;
      acc[4] += a * x1.x;
      acc[5] += a * x1.y;
      acc[6] += a * x1.z;
      acc[7] += a * x1.w;
    }
    l_tot = pair_sum(lt);
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

// Head dim of the wide kernels (fa2_d128.hip); the other kernels take 64.
constexpr int kD2 = 128;

// Q enters the kernels unscaled: cq = +-1 carries the sign of sm_scale
// (exact in any element type) and every fp32 score is multiplied by
// cr = c = |sm_scale| * log2 e, as in the reference (kernel_flash2.cu:188-195).
// Only c == 1 exactly skips the multiply (the SCALED = false instances).
struct Scales {
  float cq, cr;
  bool scaled;
  explicit Scales(const FwdArgs& a) {
    cq = a.negate ? -1.0f : 1.0f;
    cr = a.scale_log2;
    scaled = cr != 1.0f;
  }
};

inline Geom make_geom(const FwdArgs& a) {
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
  g.xcds = device_xcds();
  g.cus_per_xcd = device_cus() / g.xcds;
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

}  // namespace

}  // namespace fl
