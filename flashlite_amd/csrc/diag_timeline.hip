// Diagnostic (not on the product path): the slot-scheduled kernels built
// with per-wave timeline stamps.  Each wave's lane 0 writes 8 uint64 at
// out[8 * (group * waves_per_group + wave)]:
//   [0..4] s_memrealtime at entry, first pass, loop start, loop end, store
//   [5]    s_memrealtime after the wave's last store has completed
//   [6]    s_memtime (shader clock) cycles spent in the loop
//   [7]    iterations << 48 | XCC_ID << 32 | HW_ID
// so a launch shows where its time goes (start skew, prologue, loop,
// epilogue), the clock each XCD ran the loop at, and which work-groups
// shared a CU.  The stamps add a few instructions per wave outside the loop
// and one wait for the output stores.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

namespace {
__device__ unsigned long long* g_fl_timeline;
}

#define FL_TL_STAMP(name)                                              \
  const unsigned long long name = __builtin_amdgcn_s_memrealtime();   \
  const unsigned long long name##_cyc = __builtin_amdgcn_s_memtime(); \
  (void)name##_cyc
#define FL_TL_RECORD(wpg, wave, lane, iters, t_entry, t_first, t_loop, t_loop_end, t_store)  \
  do {                                                                                      \
    __builtin_amdgcn_s_waitcnt(0);                                                          \
    const unsigned long long t_exit = __builtin_amdgcn_s_memrealtime();                     \
    if ((lane) == 0) {                                                                      \
      unsigned long long* d_ = g_fl_timeline + 8 * ((long long)blockIdx.x * (wpg) + (wave)); \
      const unsigned hw_ = __builtin_amdgcn_s_getreg((31 << 11) | 4);  /* HW_ID */          \
      const unsigned xcc_ = __builtin_amdgcn_s_getreg((31 << 11) | 20); /* XCC_ID */        \
      d_[0] = t_entry;                                                                      \
      d_[1] = t_first;                                                                      \
      d_[2] = t_loop;                                                                       \
      d_[3] = t_loop_end;                                                                   \
      d_[4] = t_store;                                                                      \
      d_[5] = t_exit;                                                                       \
      d_[6] = t_loop_end##_cyc - t_loop##_cyc;                                              \
      d_[7] = ((unsigned long long)(iters) << 48) |                                         \
              ((unsigned long long)(xcc_ & 0xff) << 32) | hw_;                              \
    }                                                                                       \
  } while (0)

// The instrumented copies get their own launcher names.
#define launch_slot diag_timeline_launch_slot
#define launch_slot_split diag_timeline_launch_slot_split
#define launch_slot_pair diag_timeline_launch_slot_pair
#include "fa2_slot.hip"
#undef launch_slot
#undef launch_slot_split
#undef launch_slot_pair

// The streaming kernel's marks: up to 64 s_memrealtime values per wave, kept
// in two registers by lane (lane j holds mark j: no memory operation, so the
// kernel's per-unit count of memory operations is unchanged) and written
// once at the end: out[64 * (group * 8 + wave) + j], j = 0 at entry,
// 1 + 3i / 2 + 3i / 3 + 3i for unit i past its barrier / after issuing the
// next unit's loads / before its stores, 63 at exit.
#define FL_ST_DECL() unsigned fl_st_lo = 0, fl_st_hi = 0
#define FL_ST_MARK(index)                                                    \
  do {                                                                       \
    const unsigned long long t_ = __builtin_amdgcn_s_memrealtime();          \
    const bool mine_ = (int)(threadIdx.x & 63) == (index);                   \
    fl_st_lo = mine_ ? (unsigned)t_ : fl_st_lo;                              \
    fl_st_hi = mine_ ? (unsigned)(t_ >> 32) : fl_st_hi;                      \
  } while (0)
#define FL_ST_FLUSH(wave, lane, count)                                                  \
  do {                                                                                  \
    __builtin_amdgcn_s_waitcnt(0);                                                      \
    FL_ST_MARK(63);                                                                     \
    if ((lane) < (count) || (lane) == 63)                                               \
      g_fl_timeline[64 * ((long long)blockIdx.x * 8 + (wave)) + (lane)] =               \
          ((unsigned long long)fl_st_hi << 32) | fl_st_lo;                              \
  } while (0)
namespace fl {
namespace {
bool diag_stream_fits(const FwdArgs& a) { return a.seq_k <= kStreamMaxKeys; }
}  // namespace
}  // namespace fl
#define launch_stream diag_timeline_launch_stream
#define stream_config_fits diag_stream_fits
#include "fa2_stream.hip"
#undef launch_stream
#undef stream_config_fits
#define launch_quarter diag_timeline_launch_quarter
#define FL_QUARTER_NO_SPLITKV
#include "fa2_short.hip"
#undef FL_QUARTER_NO_SPLITKV
#undef launch_quarter

extern "C" {

// Contiguous fp16 [B, H, N, 64] q, k, v, o; sm_scale 1/8.  mode 8 / 4: the
// br256_bc64_w8_slot / br128_bc64_w4_slot configurations; 2: the key-range
// split br128_bc64_w4x2_slot; 7: the split on 64-row groups
// br64_bc64_w2x2_slot; 9: the block pairs br128_bc64_w4x2_pair.
// `out` holds `out_entries` uint64, at least 8 per wave record of the grid
// (B*H*ceil(N/256) groups of 8 waves for mode 8, B*H*ceil(N/128) groups of
// 4 or 8 waves for modes 4 and 2, B*H*ceil(N/64) groups of 4 waves for mode
// 7, B*H*ceil(ceil(N/128)/2) groups of 8 waves
// with one record per wave and block, 16 per group, for mode 9).  Returns a
// hipError_t.
int fl_diag_slot_timeline(int mode, int causal, const void* q, const void* k, const void* v,
                          void* o, int B, int H, int N, void* out, long long out_entries,
                          void* stream) {
  if ((mode != 8 && mode != 4 && mode != 2 && mode != 7 && mode != 9) || B < 1 || H < 1 ||
      N < 1 || out == nullptr)
    return (int)hipErrorInvalidValue;
  const long long rows = mode == 8 ? 256 : mode == 7 ? 64 : 128;
  const long long blocks = (N + rows - 1) / rows;
  const long long groups = (long long)B * H * (mode == 9 ? (blocks + 1) / 2 : blocks);
  const long long records = mode == 4 || mode == 7 ? 4 : mode == 9 ? 16 : 8;
  if (out_entries < 8 * records * groups) return (int)hipErrorInvalidValue;
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_fl_timeline), &out, sizeof(out));
  if (e != hipSuccess) return (int)e;
  fl::FwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = nullptr;
  a.batch_heads = B * H;
  a.heads = H;
  a.seq = N;
  a.seq_k = N;
  a.head_dim = 64;
  a.scale_log2 = (float)(0.125 * 1.4426950408889634);  // as fl_attn_fwd_f16 computes it
  a.negate = 0;
  a.causal = causal;
  a.dtype = fl::kDtypeF16;
  a.q_sr = a.k_sr = a.v_sr = a.o_sr = 64;
  a.q_sh = a.k_sh = a.v_sh = a.o_sh = (int64_t)N * 64;
  a.q_sb = a.k_sb = a.v_sb = a.o_sb = (int64_t)H * N * 64;
  const auto st = static_cast<hipStream_t>(stream);
  e = mode == 2   ? fl::diag_timeline_launch_slot_split(a, 4, st)
      : mode == 7 ? fl::diag_timeline_launch_slot_split(a, 2, st)
      : mode == 9 ? fl::diag_timeline_launch_slot_pair(a, 4, st)
                  : fl::diag_timeline_launch_slot(a, mode, st);
  return (int)e;
}

// The streaming kernel (br256_kv256_w8_stream; contiguous fp16 [B, H, N, 64],
// N <= 256, sm_scale 1/8) with its per-wave marks; `out` holds at least
// 64 * 8 * min(B*H*ceil(N/256), 256) uint64.  Returns a hipError_t.
int fl_diag_stream_timeline(int causal, const void* q, const void* k, const void* v, void* o,
                            int B, int H, int N, void* out, long long out_entries, void* stream) {
  if (B < 1 || H < 1 || N < 1 || N > 256 || out == nullptr) return (int)hipErrorInvalidValue;
  const long long groups = std::min<long long>((long long)B * H, 256);
  if (out_entries < 64 * 8 * groups) return (int)hipErrorInvalidValue;
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_fl_timeline), &out, sizeof(out));
  if (e != hipSuccess) return (int)e;
  fl::FwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = nullptr;
  a.batch_heads = B * H;
  a.heads = H;
  a.seq = N;
  a.seq_k = N;
  a.head_dim = 64;
  a.scale_log2 = (float)(0.125 * 1.4426950408889634);
  a.negate = 0;
  a.causal = causal;
  a.dtype = fl::kDtypeF16;
  a.q_sr = a.k_sr = a.v_sr = a.o_sr = 64;
  a.q_sh = a.k_sh = a.v_sh = a.o_sh = (int64_t)N * 64;
  a.q_sb = a.k_sb = a.v_sb = a.o_sb = (int64_t)H * N * 64;
  return (int)fl::diag_timeline_launch_stream(a, static_cast<hipStream_t>(stream));
}

// The key-quarter kernel (br32_kv512_w4_quarters; contiguous fp16
// [B, H, N, 64], N <= 512, sm_scale 1/8) with per-wave marks (0 entry, 1
// loads issued, 2 loads landed, 3 tiles done, 4 merged, 63 exit, as for the
// streaming kernel); `out` holds at least 64 * 8 * B*H*ceil(N/32) uint64.
int fl_diag_quarter_timeline(int causal, const void* q, const void* k, const void* v, void* o,
                             int B, int H, int N, void* out, long long out_entries, void* stream) {
  if (B < 1 || H < 1 || N < 1 || N > 512 || out == nullptr) return (int)hipErrorInvalidValue;
  if (out_entries < 64 * 8 * (long long)B * H * ((N + 31) / 32)) return (int)hipErrorInvalidValue;
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_fl_timeline), &out, sizeof(out));
  if (e != hipSuccess) return (int)e;
  fl::FwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = nullptr;
  a.batch_heads = B * H;
  a.heads = H;
  a.seq = N;
  a.seq_k = N;
  a.head_dim = 64;
  a.scale_log2 = (float)(0.125 * 1.4426950408889634);
  a.negate = 0;
  a.causal = causal;
  a.dtype = fl::kDtypeF16;
  a.q_sr = a.k_sr = a.v_sr = a.o_sr = 64;
  a.q_sh = a.k_sh = a.v_sh = a.o_sh = (int64_t)N * 64;
  a.q_sb = a.k_sb = a.v_sb = a.o_sb = (int64_t)H * N * 64;
  return (int)fl::diag_timeline_launch_quarter(a, static_cast<hipStream_t>(stream));
}

}  // extern "C"
