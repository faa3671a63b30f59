// Internal interface between the C-ABI layer (capi.hip) and the gfx950
// kernels (fa2_*.hip, naive_fwd.hip).  Host-side only types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fl {

// Arguments shared by every forward launch.  Sizes are validated by the
// C-ABI layer before a launch function sees them.  Tensors are addressed as
// [batch][head][row][head_dim] with element strides; head_dim is unit
// stride.  The contiguous layout has row stride D, head stride N*D and
// batch stride H*N*D.
struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;        // optional [B, H, N_q] fp32 log-sum-exp (natural log), or null
  int batch_heads;   // B*H
  int heads;         // H
  int seq;           // N_q: query (and output) rows
  int seq_k;         // N_k: key / value rows
  int head_dim;      // D
  float scale_log2;  // |sm_scale| * log2(e), always > 0
  int negate;        // 1 when sm_scale < 0: the kernel flips the sign of Q
  int causal;        // key j visible to query i iff j <= i + (N_k - N_q)
  int dtype;         // element type of q, k, v, o: kDtypeF16 or kDtypeBF16
  int64_t q_sb, q_sh, k_sb, k_sh, v_sb, v_sh, o_sb, o_sh;  // batch / head strides
  int q_sr, k_sr, v_sr, o_sr;                              // row strides
};

constexpr int kDtypeF16 = 0;
constexpr int kDtypeBF16 = 1;

// One FA2 tile configuration: `waves` waves of 64 lanes, each owning 32
// query rows, so a work-group covers 32*waves queries; KV tiles of 64 keys.
struct Fa2Config {
  int waves;
  const char* name;
};

// Configuration ids (indices into kFa2Configs).
constexpr int kCfgW1 = 0;          // br32_bc64_w1: pipelined, 1 wave
constexpr int kCfgW2 = 1;          // br64_bc64_w2: pipelined, 2 waves
constexpr int kCfgSplit2 = 2;      // br128_bc64_w4x2_slot: 2 x 4 waves, key range halved
constexpr int kSlotW8Config = 3;   // br256_bc64_w8_slot
constexpr int kSlotW4Config = 4;   // br128_bc64_w4_slot
// Persistent work-groups streaming whole units of 256 query rows whose keys
// fit one LDS buffer: needs N_k <= kStreamMaxKeys and row strides below
// kStreamMaxRowStride elements (unit-relative 32-bit buffer offsets).
constexpr int kStreamConfig = 5;   // br256_kv256_w8_stream
// One 4-wave work-group per 32-row query block, each wave a quarter of at
// most kQuarterMaxKeys keys (fp16, head_dim 64).
constexpr int kQuarterConfig = 6;  // br32_kv512_w4_quarters
constexpr int kCfgSplit2W2 = 7;     // br64_bc64_w2x2_slot: 2 x 2 waves, key range halved
// Two 128-row blocks of a head per work-group (p and nqb-1-p, one after the
// other), each with its key range halved between 2 x 4 waves.
constexpr int kCfgPair = 8;         // br128_bc64_w4x2_pair
// The same with two 64-row blocks per work-group, 2 x 2 waves.
constexpr int kCfgPairW2 = 9;       // br64_bc64_w2x2_pair
constexpr int kNumFa2Configs = 10;
extern const Fa2Config kFa2Configs[kNumFa2Configs];

// Launches the FA2 kernel for configuration `cfg` on `stream`.  fp16 at
// head_dim 64 has every configuration; bf16 at head_dim 64 all but the
// pipelined ones (kCfgW1, kCfgW2); head_dim 128 the slot-scheduled ones
// (kSlotW8Config, kSlotW4Config).
hipError_t launch_fa2(const FwdArgs& a, int cfg, hipStream_t stream);
constexpr int kStreamMaxKeys = 256;
constexpr int kStreamMaxRowStride = 1 << 22;
bool stream_config_fits(const FwdArgs& a);
constexpr int kQuarterMaxKeys = 512;
// Compute units of the current device: 256 on an MI355X seen whole, fewer
// when the GPU is partitioned into several devices.  The dispatch rules
// that plan for one round of work-groups on the CUs use it.  Looked up once
// per device (hipDeviceAttributeMultiprocessorCount); 256 when no device is
// visible (host-only callers of the dispatcher, such as its CPU tests).
constexpr int kMi355xCus = 256;
inline int device_cus() {
  constexpr int kMaxDevices = 64;
  static int cached[kMaxDevices];  // 0: not looked up yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return kMi355xCus;
  int c = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
  if (c <= 0) {
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        c <= 0)
      c = kMi355xCus;
    __atomic_store_n(&cached[dev], c, __ATOMIC_RELAXED);
  }
  return c;
}
// XCDs of the current device (8 on an MI355X seen whole; 1 per partition
// when it is split into single-XCD devices), looked up once per device
// (hipDeviceAttributeNumberOfXccs).  The work-group remap that keeps a head
// on one XCD (wg_coords) follows it; a count that does not divide the CUs,
// or a failed lookup, gives 1 (no remap).  8 when no device is visible.
constexpr int kMi355xXcds = 8;
inline int device_xcds() {
  constexpr int kMaxDevices = 64;
  static int cached[kMaxDevices];  // 0: not looked up yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return kMi355xXcds;
  int x = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
  if (x <= 0) {
    if (hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || x <= 0 ||
        device_cus() % x != 0)
      x = 1;
    __atomic_store_n(&cached[dev], x, __ATOMIC_RELAXED);
  }
  return x;
}
inline bool quarter_config_fits(const FwdArgs& a) { return a.seq_k <= kQuarterMaxKeys; }

// Per-schedule launchers behind launch_fa2 (one source file each).
hipError_t launch_pipe(const FwdArgs& a, int cfg, hipStream_t stream);     // fa2_pipe.hip
hipError_t launch_slot(const FwdArgs& a, int waves, hipStream_t stream);   // fa2_slot.hip
hipError_t launch_slot_split(const FwdArgs& a, int waves, hipStream_t stream);  // fa2_slot.hip
hipError_t launch_slot_pair(const FwdArgs& a, int waves, hipStream_t stream);   // fa2_slot.hip
hipError_t launch_stream(const FwdArgs& a, hipStream_t stream);            // fa2_stream.hip
hipError_t launch_quarter(const FwdArgs& a, hipStream_t stream);           // fa2_short.hip
hipError_t launch_d128(const FwdArgs& a, int waves, hipStream_t stream);   // fa2_d128.hip

// Split-KV ("flash-decoding"): `waves` (1, 2 or 4) waves of 32 query rows
// per work-group, the key range cut into `nsplit` chunks whose partial
// results go to `part` (nsplit * B*H * N_q * 68 floats, 16-byte aligned),
// then merged by a second kernel on the same stream.
hipError_t launch_kvsplit(const FwdArgs& a, int waves, float* part, int nsplit,
                          hipStream_t stream);
// The same with single-wave query blocks (N_q <= 32) in key-quarter chunks
// of at most kQuarterMaxKeys keys: 4 waves per chunk (fa2_short.hip).
hipError_t launch_kvsplit_quarter(const FwdArgs& a, float* part, int nsplit, hipStream_t stream);
// The combine kernel alone (fa2_pipe.hip): merges the nsplit partials in
// `part` into O (and the log-sum-exp when a.lse is set).
hipError_t launch_splitkv_combine(const FwdArgs& a, float* part, int nsplit, hipStream_t stream);

// Largest seq the naive kernel can stage in LDS for this head_dim.
int64_t naive_max_seq(int64_t head_dim);
hipError_t launch_naive(const FwdArgs& a, hipStream_t stream);

}  // namespace fl
