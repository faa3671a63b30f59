// Tile configurations of the FA2 forward and their dispatch to the
// schedule that implements each (fa2_pipe.hip, fa2_slot.hip, fa2_stream.hip,
// fa2_short.hip, fa2_d128.hip).  The dispatcher that picks a configuration for a problem is
// capi.hip's select_fa2.

#include "fl_internal.h"

namespace fl {

const Fa2Config kFa2Configs[kNumFa2Configs] = {
    {1, "br32_bc64_w1"},
    {2, "br64_bc64_w2"},
    {8, "br128_bc64_w4x2_slot"},
    {8, "br256_bc64_w8_slot"},
    {4, "br128_bc64_w4_slot"},
    {8, "br256_kv256_w8_stream"},
    {4, "br32_kv512_w4_quarters"},
    {4, "br64_bc64_w2x2_slot"},
    {8, "br128_bc64_w4x2_pair"},
    {4, "br64_bc64_w2x2_pair"},
};

bool stream_config_fits(const FwdArgs& a) {
  return a.seq_k <= kStreamMaxKeys && a.q_sr < kStreamMaxRowStride &&
         a.k_sr < kStreamMaxRowStride && a.v_sr < kStreamMaxRowStride &&
         a.o_sr < kStreamMaxRowStride;
}

hipError_t launch_fa2(const FwdArgs& a, int cfg, hipStream_t stream) {
  if (a.head_dim == 128) {
    if (cfg == kSlotW8Config) return launch_d128(a, 8, stream);
    if (cfg == kSlotW4Config) return launch_d128(a, 4, stream);
    return hipErrorInvalidValue;
  }
  if (a.dtype == kDtypeBF16) {
    if (cfg == kSlotW8Config) return launch_slot(a, 8, stream);
    if (cfg == kSlotW4Config) return launch_slot(a, 4, stream);
    if (cfg == kCfgSplit2) return launch_slot_split(a, 4, stream);
    if (cfg == kCfgSplit2W2) return launch_slot_split(a, 2, stream);
    if (cfg == kCfgPair) return launch_slot_pair(a, 4, stream);
    if (cfg == kCfgPairW2) return launch_slot_pair(a, 2, stream);
    if (cfg == kStreamConfig) return launch_stream(a, stream);
    if (cfg == kQuarterConfig) return launch_quarter(a, stream);
    return hipErrorInvalidValue;
  }
  switch (cfg) {
    case kCfgW1:
    case kCfgW2: return launch_pipe(a, cfg, stream);
    case kCfgSplit2: return launch_slot_split(a, 4, stream);
    case kCfgSplit2W2: return launch_slot_split(a, 2, stream);
    case kCfgPair: return launch_slot_pair(a, 4, stream);
    case kCfgPairW2: return launch_slot_pair(a, 2, stream);
    case kSlotW8Config: return launch_slot(a, 8, stream);
    case kSlotW4Config: return launch_slot(a, 4, stream);
    case kStreamConfig: return launch_stream(a, stream);
    case kQuarterConfig: return launch_quarter(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fl
