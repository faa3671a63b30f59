// C-ABI entry points: argument checks, the sm_scale sentinel and log2 e factor,
// the adaptive tile dispatcher, and the launch.
//
// Reference host entries: csrc/kernel_flash2.cu:732-839 (flash2) and
// csrc/kernel_naive.cu:242-323 (naive).  The torch-tensor checks live in the
// binding (flash_attn.cpp); here are the checks a raw-pointer caller needs,
// plus the ones the reference skipped (64-bit sizes, alignment).  N_k may
// differ from N_q: the reference validates that shape but then indexes K and
// V with N_q (kernel_flash2.cu:84, :425, :752-755); here the keys are
// addressed with N_k and the causal diagonal is aligned bottom-right.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <cstdint>
#include <mutex>

#include "fl_internal.h"
#include "flashlite_attn.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// float(log2 e) widened to double, as the reference multiplies a double
// sm_scale by its float LOG2_E constant (kernel_flash2.cu:16, :772).
constexpr double kLog2eF = (double)1.44269504088896340736f;

// sm_scale == 0.0 -> 1/sqrt(D) computed in float (kernel_flash2.cu:769-771).
double resolve_scale(double s, int64_t d) {
  if (s == 0.0) return (double)(1.0f / std::sqrt((float)d));
  return s;
}

// Shared argument checks; fills `a` on success.
int check_common(const fl_attn_params* p, fl::FwdArgs* a, const char* who) {
  if (p == nullptr) return fail(FL_ERR_INVALID_ARGUMENT, "%s: params is NULL", who);
  if (p->batch < 0 || p->heads < 0 || p->seq_q < 0 || p->seq_k < 0 || p->head_dim < 1)
    return fail(FL_ERR_INVALID_ARGUMENT,
                "%s: sizes must be non-negative and head_dim >= 1 (got B=%lld H=%lld N_q=%lld "
                "N_k=%lld D=%lld)",
                who, (long long)p->batch, (long long)p->heads, (long long)p->seq_q,
                (long long)p->seq_k, (long long)p->head_dim);
  const double scale = resolve_scale(p->sm_scale, p->head_dim);
  const float c = (float)(std::fabs(scale) * kLog2eF);
  if (!std::isfinite(scale) || !std::isfinite(c) || c == 0.0f)
    return fail(FL_ERR_INVALID_ARGUMENT, "%s: sm_scale*log2(e) must be finite and non-zero (sm_scale=%g)",
                who, scale);
  const int64_t bh = p->batch * p->heads;
  if (p->batch != 0 && bh / p->batch != p->heads)
    return fail(FL_ERR_UNSUPPORTED, "%s: B*H overflows", who);
  if (bh > INT32_MAX || p->seq_q > INT32_MAX || p->seq_k > INT32_MAX || p->head_dim > INT32_MAX)
    return fail(FL_ERR_UNSUPPORTED, "%s: B*H, N_q, N_k and D must each fit in int32", who);
  a->q = p->q;
  a->k = p->k;
  a->v = p->v;
  a->o = p->o;
  a->lse = nullptr;
  a->batch_heads = (int)bh;
  a->heads = (int)p->heads;
  a->seq = (int)p->seq_q;
  a->seq_k = (int)p->seq_k;
  a->head_dim = (int)p->head_dim;
  a->scale_log2 = c;
  a->negate = scale < 0.0 ? 1 : 0;
  a->causal = p->causal ? 1 : 0;
  a->dtype = fl::kDtypeF16;
  // contiguous [B, H, N, D]
  const int64_t d = p->head_dim;
  a->q_sr = a->o_sr = a->k_sr = a->v_sr = (int)d;
  a->q_sh = a->o_sh = p->seq_q * d;
  a->k_sh = a->v_sh = p->seq_k * d;
  a->q_sb = a->o_sb = p->heads * p->seq_q * d;
  a->k_sb = a->v_sb = p->heads * p->seq_k * d;
  return FL_OK;
}

// No query row: nothing to write.  (N_k == 0 with rows is not empty: every
// row then has no visible key and is written as 0.)
bool empty_problem(const fl::FwdArgs& a) { return a.batch_heads == 0 || a.seq == 0; }

// With N_k == 0 (no keys: every row is written as 0) k and v are never read
// and may be NULL; the kernels then get q's address in their place.
int check_pointers(const fl_attn_params* p, fl::FwdArgs* a, const char* who, uintptr_t align) {
  const bool no_keys = p->seq_k == 0;
  if (!p->q || !p->o || (!no_keys && (!p->k || !p->v)))
    return fail(FL_ERR_INVALID_ARGUMENT, "%s: q, k, v and o must be non-NULL", who);
  const uintptr_t m = align - 1;
  const uintptr_t kv = no_keys ? 0 : ((uintptr_t)p->k | (uintptr_t)p->v);
  if (((uintptr_t)p->q | kv | (uintptr_t)p->o) & m)
    return fail(FL_ERR_MISALIGNED, "%s: q, k, v and o must be %u-byte aligned", who, (unsigned)align);
  if (no_keys) a->k = a->v = p->q;
  return FL_OK;
}

// Tile-configuration choice for the device's CUs (fl::device_cus(): 256 on
// an MI355X seen whole, where the rules below were measured; every
// configuration computes the same result).  Key ranges of at most 256 keys
// go to the streaming persistent groups (measured at least as fast as every
// other configuration from 16 to 2048 units, both masks), and of at most
// 512 with at most 512 blocks of 32 rows to the key quarters (one block per
// group up to 256 blocks, two beyond: 4-18% faster than the 128-row groups
// from 320 to 512 blocks).  Past 576
// keys, up to 256 groups of 64 rows take the key-range split on 64-row
// groups (2 x 2 waves, one per SIMD, each pair walking half the keys): one
// group per CU where the 128-row groups leave CUs idle, 1-28% faster than
// every other configuration from 16 to 256 groups (N_k 640-16384, fp16 and
// bf16; at N_k 513 the 128-row groups were 2.5% faster, and with more than
// 256 groups a second round costs 27-70%).  Other long key ranges with at most one 128-row group per
// CU take the key-range-split group of 8 waves (two per SIMD): causal
// from N_k 2048 (64 groups up; fewer fall back to smaller groups), 7-11%
// faster than the 4-wave groups, and from N_k 4096 up to two such rounds
// (2-7% faster); non-causal from N_k 2048, 4-5% faster (B2 H8 N2048 22.8
// against 23.9 us, B1 H8 N4096 39.5 against 41.1).  With more than 128 groups of 256
// rows over N_k >= 2048, non-causal takes one 256-row group of 8 waves per
// CU; otherwise
// 128-row slot-scheduled groups of 4 waves, two per CU, which also serve
// causal attention (groups of different lengths, balanced by dispatch
// order).  Smaller problems fall back to smaller groups.  Replaces the
// reference's `seq_len >= 2048 -> Br=128` rule (kernel_flash2.cu:786-789),
// which was sized for 20 SMs.
int select_fa2(const fl::FwdArgs& a) {
  const int64_t cus = fl::device_cus();
  auto wgs = [&](int64_t br) { return (a.seq + br - 1) / br * (int64_t)a.batch_heads; };
  if (fl::stream_config_fits(a)) return fl::kStreamConfig;  // br256_kv256_w8_stream
  // N_k <= 512 with few query blocks: quarter the key range (4-wave groups
  // of 32 rows, or 8-wave groups of 64 past 256 blocks; a single round).
  if (fl::quarter_config_fits(a) && wgs(32) <= 2 * cus) return fl::kQuarterConfig;
  // At most 32 query rows per head (decode-like) over at least as many
  // heads as CUs: HBM-bound; the 4-wave groups, two per CU, were 0.6-6.8%
  // faster than the 256-row groups or the 64-row split (B64 H32 N_q 1 N_k
  // 2048 181.8 against 195.1 us, B32 H32 N_k 4096 178.2 against 183.1, B8
  // H32 N_k 8192 93.4 against 94.0; within 2% of the best at B16 H32 N_k
  // 16384).
  if (a.seq <= 32 && a.batch_heads >= cus) return fl::kSlotW4Config;
  // Past 576 keys, at most one group of 64 rows per CU: the key-range split
  // on 64-row groups (2 x 2 waves) in a single round.
  if (a.seq_k > 576 && wgs(64) <= cus) return fl::kCfgSplit2W2;
  // Square causal problems over at least 4096 keys with at most one pair of
  // 64-row blocks per CU (so more than half the CUs busy, the rule above
  // having taken the rest): the 64-row block pairs, every work-group
  // carrying the same tiles in one round at one wave per SIMD.  Measured
  // 0-19% faster than the rules below would choose (B1 H2 N16384 109.2
  // against 124.6 us for the 128-row pairs and 133.8 for the one-block
  // split, B1 H1 N32768 223.7 against 239.9 and 268.6, B1 H3 N8192 55.4
  // against 60.9, B1 H8 N4096 34.8 against 35.3); slower at N 2048 (B2 H8:
  // 21.9 against 20.7) and when the pairs take a second round.
  const int64_t pairs64 = (((int64_t)a.seq + 63) / 64 + 1) / 2 * a.batch_heads;
  if (a.causal && a.seq == a.seq_k && a.seq_k >= 4096 && pairs64 <= cus) return fl::kCfgPairW2;
  const bool one_round = a.seq_k >= 2048 && wgs(128) <= cus;
  if (one_round && (!a.causal || wgs(128) >= cus / 4)) return fl::kCfgSplit2;
  // Square causal problems over 2048-4095 keys with one to two rounds of
  // 128-row groups: the one-block split up to one and a half rounds (1-9%
  // faster than the 4-wave groups: B2 H8 N3072 31.8 against 34.9 us, B1 H16
  // N3072 32.2 against 34.5, B2 H8 N2560 26.7 against 28.4), and from 2560
  // keys the block pairs beyond (B2 H10 N2560 30.8 against 34.7, B2 H8
  // N3584 42.6 against 43.8).
  if (a.causal && a.seq == a.seq_k && a.seq_k >= 2048 && a.seq_k < 4096 && wgs(128) > cus) {
    if (wgs(128) <= cus + cus / 2) return fl::kCfgSplit2;
    if (a.seq_k >= 2560 && wgs(128) <= 2 * cus) return fl::kCfgPair;
  }
  // Causal over at least 4096 keys with more than one 128-row block but at
  // most one block pair per CU: the block pairs (one round of equal
  // work-groups, each key range halved), 2-10% faster than the 4-wave
  // groups and the one-block split (B2 H8 N4096 48.3 against 50.1 and 53.7
  // us, B1 H16 N4096 43.2 against 45.5 and 45.0, B1 H8 N8192 77.3 against
  // 85.2 and 79.6); past one pair per CU the 4-wave groups win.
  if (a.causal && a.seq_k >= 4096 && wgs(128) <= 2 * cus) return fl::kCfgPair;
  if (!a.causal && a.seq_k >= 2048 && wgs(256) > cus / 2) return fl::kSlotW8Config;
  if (wgs(128) >= cus / 4) return fl::kSlotW4Config;
  if (wgs(64) >= cus / 4) return fl::kCfgW2;
  return fl::kCfgW1;
}

int check_fa2(const fl_attn_params* p, fl::FwdArgs* a, const char* who = "fl_attn_fwd_f16",
              bool wide = false) {
  int rc = check_common(p, a, who);
  if (rc != FL_OK) return rc;
  if (wide && p->head_dim != 64 && p->head_dim != 128)
    return fail(FL_ERR_UNSUPPORTED, "%s: head_dim must be 64 or 128 (got %lld)", who,
                (long long)p->head_dim);
  if (!wide && p->head_dim != 64)
    return fail(FL_ERR_UNSUPPORTED, "FlashLite WMMA kernel currently requires head_dim == 64");
  // K/V tiles are fetched through 32-bit buffer offsets within one head
  // (N_k rows of 2*D bytes, plus one tile of slack).
  const int row_bytes = 2 * a->head_dim;
  if (a->seq_k > (INT32_MAX / row_bytes) - 128)
    return fail(FL_ERR_UNSUPPORTED, "%s: N_k=%d exceeds the per-head addressing limit (%d)", who,
                a->seq_k, (INT32_MAX / row_bytes) - 128);
  // Grid = ceil(N/32) * B*H work-groups at the smallest tile; per-head
  // offsets are 64-bit in the kernel.
  if (((int64_t)a->seq + 31) / 32 * (int64_t)a->batch_heads > INT32_MAX)
    return fail(FL_ERR_UNSUPPORTED, "%s: too many work-groups (B*H*ceil(N/32) > 2^31-1)", who);
  return FL_OK;
}

// Strides of one tensor of fl_attn_fwd_f16_ex: every row 16-byte aligned
// (strides in multiples of 8 halfs), rows at least D apart, and row offsets
// that fit the kernels' 32-bit row stride.
int check_strides(const int64_t st[3], int64_t d, const char* name, const char* who) {
  for (int i = 0; i < 3; ++i)
    if (st[i] < 0 || st[i] % 8 != 0)
      return fail(FL_ERR_UNSUPPORTED, "%s: %s strides must be non-negative multiples of 8 elements "
                  "(got %lld, %lld, %lld)", who, name, (long long)st[0], (long long)st[1],
                  (long long)st[2]);
  if (st[2] < d || st[2] > INT32_MAX / 2)
    return fail(FL_ERR_UNSUPPORTED, "%s: %s row stride %lld must be in [%lld, 2^30)", who, name,
                (long long)st[2], (long long)d);
  return FL_OK;
}

// Checks of an fl_attn_params_ex and its strides; fills `a`.
int check_ex(const fl_attn_params_ex* p, fl::FwdArgs* a, const char* who, bool wide = false) {
  if (p == nullptr) return fail(FL_ERR_INVALID_ARGUMENT, "%s: params is NULL", who);
  int rc = check_fa2(&p->base, a, who, wide);
  if (rc != FL_OK) return rc;
  const int64_t* st[4] = {p->q_stride, p->k_stride, p->v_stride, p->o_stride};
  const char* names[4] = {"q", "k", "v", "o"};
  const bool no_keys = a->seq_k == 0;  // k and v are never read
  for (int i = 0; i < 4; ++i) {
    if (no_keys && (i == 1 || i == 2)) continue;
    rc = check_strides(st[i], a->head_dim, names[i], who);
    if (rc != FL_OK) return rc;
  }
  for (int i = 1; i <= 2; ++i)
    if ((a->seq_k + 128LL) * st[i][2] * 2 > INT32_MAX)
      return fail(FL_ERR_UNSUPPORTED, "%s: N_k=%d rows of stride %lld exceed the per-head "
                  "addressing limit of %s (2^31 bytes)", who, a->seq_k, (long long)st[i][2],
                  names[i]);
  if ((uintptr_t)p->lse & 3) return fail(FL_ERR_MISALIGNED, "%s: lse must be 4-byte aligned", who);
  a->q_sb = p->q_stride[0];
  a->q_sh = p->q_stride[1];
  a->q_sr = (int)p->q_stride[2];
  if (!no_keys) {
    a->k_sb = p->k_stride[0];
    a->k_sh = p->k_stride[1];
    a->k_sr = (int)p->k_stride[2];
    a->v_sb = p->v_stride[0];
    a->v_sh = p->v_stride[1];
    a->v_sr = (int)p->v_stride[2];
  }
  a->o_sb = p->o_stride[0];
  a->o_sh = p->o_stride[1];
  a->o_sr = (int)p->o_stride[2];
  a->lse = p->lse;
  return FL_OK;
}

// Split-KV plan: waves per work-group by N_q (32 query rows each), number
// of key chunks, workspace bytes.  nsplit == 0 means "do not split".
// The library's choice (requested <= 0), from decode sweeps on MI355X
// (B2 H8 and B1 H16 with N_q 1-16 over 4k-64k keys; B1-B32 with H16-H64 and
// N_q 1-128 over 2k-32k keys): with at most 128 query rows and fewer than
// half as many query-row groups as CUs, cut each key range so that the
// groups times chunks cover the CUs twice with single-wave groups (N_q <=
// 32; 2-11% faster than once, measured) and once with 2- and 4-wave groups
// (twice: +1% and +25%), keeping at least 4 key tiles per chunk (shorter
// chunks measured slower: per-work-group start-up).  Otherwise one pass:
// from 128 to 1024 groups the one-pass kernels ran 2-17% faster than 2, 4
// or 8 chunks (B4 H32 N_q 1 N_k 8192 41.2 against 46.2 us, B32 H32 N_q 1
// N_k 4096 186.6 against 196.6, B4 H32 N_q 64 N_k 8192 48.3 against 53.2,
// B8 H16 N_q 64 N_k 4096 26.0 against 31.5), while at 32-64 groups the
// chunks still won or tied (B2 H32 N_q 1 N_k 8192 27.9 against 39.0, N_q
// 64 31.2 against 43.3).  The partials of a plan with 4-wave groups can
// pass the allocation-free entry point's static scratch (4 chunks x 64
// groups x 128 rows: 8.9 MB), so that entry point plans with
// plan_kvsplit_capped, which lowers the library's chunk count to what its
// scratch holds.
//
// Single-wave groups whose chunks fit the key-quarter kernel (at most 8
// tiles) in one round of its 4-wave work-groups (at most 256) run there
// (`quarter`): the library's choice cuts such ranges into chunks of 8 tiles
// when that fits (below half as many groups as CUs: from 128 groups its 2
// chunks measured level with one pass or 9-14% slower, B8 H16 N_q 1 N_k 692
// 8.92 against 8.09 us, B2 H64 N_q 16 N_k 1000 10.96 against 9.47), and a
// requested chunk count takes it when it does.
struct KvPlan {
  int waves, nsplit;
  bool quarter;
  int64_t bytes;
};
constexpr int kMaxSplits = 256;
constexpr int64_t kPartFloats = 68;  // per row: O[64], m, l, 2 pad

KvPlan plan_kvsplit(const fl::FwdArgs& a, int32_t requested) {
  const int64_t cus = fl::device_cus();
  KvPlan p;
  p.waves = a.seq <= 32 ? 1 : (a.seq <= 64 ? 2 : 4);
  p.quarter = false;
  const int64_t nqb = (a.seq + 32 * p.waves - 1) / (32 * p.waves);
  const int64_t tiles = std::max<int64_t>(1, (a.seq_k + 63) / 64);
  const int64_t groups = nqb * a.batch_heads;
  int64_t n;
  if (requested > 0) {
    n = std::min<int64_t>({(int64_t)requested, tiles, kMaxSplits});
  } else if (a.seq > 128) {
    n = 0;  // long query ranges: the one-pass kernel's groups fill the GPU
  } else if (2 * groups < cus) {
    const int64_t cover = (p.waves == 1 ? 2 : 1) * cus;
    n = std::min<int64_t>({(cover + groups - 1) / groups, tiles / 4, kMaxSplits});
  } else {
    n = 0;  // enough groups for the one-pass kernels
  }
  if (p.waves == 1 && requested <= 0 && 2 * groups < cus) {
    const int64_t nq = (tiles + 7) / 8;  // chunks of at most 8 tiles
    if (nq >= 2 && groups * nq <= cus) {
      n = nq;
      p.quarter = true;
    }
  } else if (p.waves == 1 && requested > 0) {
    p.quarter = (tiles + n - 1) / n <= 8 && groups * n <= cus;
  }
  if (requested <= 0 && n < 2) n = 0;
  // the chunk kernel's grid (64 * waves lanes per group) must stay below 2^32 lanes
  const int64_t grid_cap = ((int64_t)UINT32_MAX / (64 * p.waves)) / (nqb * a.batch_heads);
  n = std::min(n, grid_cap);
  if (n < 1) n = 0;
  p.nsplit = (int)n;
  p.bytes = n * (int64_t)a.batch_heads * a.seq * kPartFloats * (int64_t)sizeof(float);
  return p;
}

// The plan of the allocation-free entry point, whose partials must fit
// `limit` bytes.  A requested chunk count is kept as asked (the caller then
// gets FL_ERR_UNSUPPORTED when it does not fit).  The library's own choice
// is lowered to the most chunks that fit, or to one pass when fewer than two
// do; fewer chunks are longer, so a key-quarter plan whose chunks would pass
// 8 tiles moves to the pipelined chunk kernel.
KvPlan plan_kvsplit_capped(const fl::FwdArgs& a, int32_t requested, int64_t limit) {
  KvPlan p = plan_kvsplit(a, requested);
  if (requested > 0 || p.nsplit == 0 || p.bytes <= limit) return p;
  const int64_t per_chunk = p.bytes / p.nsplit;
  const int64_t n = limit / per_chunk;
  if (n < 2) {
    p.nsplit = 0;
    p.quarter = false;
    p.bytes = 0;
    return p;
  }
  const int64_t tiles = std::max<int64_t>(1, (a.seq_k + 63) / 64);
  p.nsplit = (int)n;
  p.bytes = n * per_chunk;
  if (p.quarter && (tiles + n - 1) / n > 8) p.quarter = false;
  return p;
}

// The chunk kernel the plan names (key quarters or the pipelined kernel),
// then the combine kernel.
hipError_t run_kvsplit(const fl::FwdArgs& a, const KvPlan& plan, float* part, hipStream_t st) {
  return plan.quarter ? fl::launch_kvsplit_quarter(a, part, plan.nsplit, st)
                      : fl::launch_kvsplit(a, plan.waves, part, plan.nsplit, st);
}

// fp16 at head_dim 64 has every tile configuration; bf16 at head_dim 64
// all but the two pipelined ones; head_dim 128 the two slot-scheduled ones.
bool narrow_configs(const fl::FwdArgs& a) {
  return a.dtype != fl::kDtypeF16 || a.head_dim != 64;
}

bool config_built(const fl::FwdArgs& a, int cfg) {
  if (!narrow_configs(a) || cfg == fl::kSlotW8Config || cfg == fl::kSlotW4Config) return true;
  return a.head_dim == 64 && cfg != fl::kCfgW1 && cfg != fl::kCfgW2;
}

// bf16 at head_dim 64 follows the fp16 dispatcher where it picks the
// streaming kernel, the key quarters, a key-range split or block pairs, and
// the 4-wave groups for at most 32 query rows over at least as many heads
// as CUs (bf16 one pass: 0-5% faster than the 256-row groups, B8 H32 N_q 1
// N_k 8192 92.1 against 96.9 us); otherwise (and at head_dim 128) one of the
// slot-scheduled groups by the rule below.
int select_any(const fl::FwdArgs& a) {
  if (!narrow_configs(a)) return select_fa2(a);
  if (a.head_dim == 64) {
    const int c = select_fa2(a);
    if (c == fl::kCfgSplit2 || c == fl::kCfgSplit2W2 || c == fl::kCfgPair || c == fl::kCfgPairW2 ||
        c == fl::kStreamConfig || c == fl::kQuarterConfig)
      return c;
    if (a.seq <= 32 && a.batch_heads >= fl::device_cus()) return fl::kSlotW4Config;
  }
  const int64_t cus = fl::device_cus();
  const int64_t wgs256 = (a.seq + 255) / 256 * (int64_t)a.batch_heads;
  return (!a.causal && a.seq_k >= 4096 && wgs256 >= cus) ? fl::kSlotW8Config
                                                           : fl::kSlotW4Config;
}

int fwd_ex(const fl_attn_params_ex* p, int32_t config, void* stream, int dtype, const char* who) {
  fl::FwdArgs a;
  int rc = check_ex(p, &a, who, /*wide=*/true);
  if (rc != FL_OK) return rc;
  a.dtype = dtype;
  if (config < -1 || config >= fl::kNumFa2Configs)
    return fail(FL_ERR_BAD_CONFIG, "%s: config %d out of range [-1, %d)", who, (int)config,
                fl::kNumFa2Configs);
  if (config >= 0 && !config_built(a, config))
    return fail(FL_ERR_BAD_CONFIG,
                "%s: config %d is not built for %s at head_dim %d (use -1, %d or %d%s)", who,
                (int)config, dtype == fl::kDtypeBF16 ? "bf16" : "fp16", a.head_dim,
                fl::kSlotW8Config, fl::kSlotW4Config,
                a.head_dim == 64 ? ", 2, 5, 6, 7, 8 or 9" : "");
  if (config == fl::kStreamConfig && !fl::stream_config_fits(a))
    return fail(FL_ERR_BAD_CONFIG, "%s: config %d needs N_k <= %d and row strides below 2^22 "
                "(got N_k %d)", who, (int)config, fl::kStreamMaxKeys, a.seq_k);
  if (config == fl::kQuarterConfig && !fl::quarter_config_fits(a))
    return fail(FL_ERR_BAD_CONFIG, "%s: config %d needs N_k <= %d (got N_k %d)", who, (int)config,
                fl::kQuarterMaxKeys, a.seq_k);
  if (empty_problem(a)) return FL_OK;
  rc = check_pointers(&p->base, &a, who, 16);
  if (rc != FL_OK) return rc;
  const int cfg = config < 0 ? select_any(a) : config;
  const hipError_t e = fl::launch_fa2(a, cfg, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FL_ERR_LAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
  return FL_OK;
}

}  // namespace

// Allocation-free split-KV.  The partials live in a file-scope device
// array; every GPU the library runs on holds its own copy, so its address
// is looked up once per device (with that device current) and cached.  In
// host code the array's name is only a stand-in for the symbol: the kernels
// get the looked-up address, never the name.
static __device__ __align__(256) float scratch[FL_ATTN_SCRATCH_BYTES / sizeof(float)];
static_assert(FL_ATTN_SCRATCH_BYTES % 256 == 0, "scratch size");

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void** out, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(FL_ERR_LAUNCH, "%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FL_ERR_UNSUPPORTED, "%s: device %d beyond the %d the scratch table covers", who,
                dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(FL_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who,
                  dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FL_OK;
}

}  // namespace

extern "C" {

const char* fl_attn_last_error(void) { return g_err; }

int fl_attn_num_configs(void) { return fl::kNumFa2Configs; }

const char* fl_attn_config_name(int32_t config) {
  if (config < 0 || config >= fl::kNumFa2Configs) return nullptr;
  return fl::kFa2Configs[config].name;
}

int fl_attn_config_id(const char* name) {
  if (name == nullptr) return -1;
  for (int i = 0; i < fl::kNumFa2Configs; ++i)
    if (std::strcmp(name, fl::kFa2Configs[i].name) == 0) return i;
  return -1;
}

int fl_attn_select_config(const fl_attn_params* p) {
  fl::FwdArgs a;
  if (check_fa2(p, &a) != FL_OK) return -1;
  return select_fa2(a);
}

int fl_attn_fwd_f16_cfg(const fl_attn_params* p, int32_t config, void* stream) {
  fl::FwdArgs a;
  int rc = check_fa2(p, &a);
  if (rc != FL_OK) return rc;
  if (config < -1 || config >= fl::kNumFa2Configs)
    return fail(FL_ERR_BAD_CONFIG, "fl_attn_fwd_f16: config %d out of range [-1, %d)", (int)config,
                fl::kNumFa2Configs);
  if (config == fl::kStreamConfig && !fl::stream_config_fits(a))
    return fail(FL_ERR_BAD_CONFIG, "fl_attn_fwd_f16: config %d needs N_k <= %d (got %d)",
                (int)config, fl::kStreamMaxKeys, a.seq_k);
  if (config == fl::kQuarterConfig && !fl::quarter_config_fits(a))
    return fail(FL_ERR_BAD_CONFIG, "fl_attn_fwd_f16: config %d needs N_k <= %d (got %d)",
                (int)config, fl::kQuarterMaxKeys, a.seq_k);
  if (empty_problem(a)) return FL_OK;
  rc = check_pointers(p, &a, "fl_attn_fwd_f16", 16);
  if (rc != FL_OK) return rc;
  const int cfg = config < 0 ? select_fa2(a) : config;
  const hipError_t e = fl::launch_fa2(a, cfg, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return fail(FL_ERR_LAUNCH, "fl_attn_fwd_f16: launch failed: %s", hipGetErrorString(e));
  return FL_OK;
}

int fl_attn_fwd_f16(const fl_attn_params* p, void* stream) {
  return fl_attn_fwd_f16_cfg(p, -1, stream);
}

int fl_attn_fwd_f16_ex(const fl_attn_params_ex* p, int32_t config, void* stream) {
  return fwd_ex(p, config, stream, fl::kDtypeF16, "fl_attn_fwd_f16_ex");
}

int fl_attn_fwd_bf16_ex(const fl_attn_params_ex* p, int32_t config, void* stream) {
  return fwd_ex(p, config, stream, fl::kDtypeBF16, "fl_attn_fwd_bf16_ex");
}

int64_t fl_attn_splitkv_workspace_bytes(const fl_attn_params_ex* p, int32_t num_splits) {
  fl::FwdArgs a;
  if (check_ex(p, &a, "fl_attn_splitkv_workspace_bytes") != FL_OK) return -1;
  const KvPlan plan = plan_kvsplit(a, num_splits);
  return plan.nsplit == 0 ? 0 : plan.bytes;
}

int64_t fl_attn_splitkv_noalloc_bytes(const fl_attn_params_ex* p, int32_t num_splits) {
  fl::FwdArgs a;
  if (check_ex(p, &a, "fl_attn_splitkv_noalloc_bytes") != FL_OK) return -1;
  const KvPlan plan = plan_kvsplit_capped(a, num_splits, FL_ATTN_SCRATCH_BYTES);
  return plan.nsplit == 0 ? 0 : plan.bytes;
}

int fl_attn_fwd_f16_splitkv(const fl_attn_params_ex* p, int32_t num_splits, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  const char* who = "fl_attn_fwd_f16_splitkv";
  fl::FwdArgs a;
  int rc = check_ex(p, &a, who);
  if (rc != FL_OK) return rc;
  if (empty_problem(a)) return FL_OK;
  rc = check_pointers(&p->base, &a, who, 16);
  if (rc != FL_OK) return rc;
  const KvPlan plan = plan_kvsplit(a, num_splits);
  hipError_t e;
  if (plan.nsplit == 0) {  // the library's choice: one pass, no workspace
    e = fl::launch_fa2(a, select_fa2(a), static_cast<hipStream_t>(stream));
  } else {
    if (workspace == nullptr || workspace_bytes < plan.bytes)
      return fail(FL_ERR_INVALID_ARGUMENT, "%s: workspace of %lld bytes needed (got %lld%s)", who,
                  (long long)plan.bytes, (long long)workspace_bytes,
                  workspace == nullptr ? ", NULL" : "");
    if ((uintptr_t)workspace & 15)
      return fail(FL_ERR_MISALIGNED, "%s: workspace must be 16-byte aligned", who);
    e = run_kvsplit(a, plan, static_cast<float*>(workspace), static_cast<hipStream_t>(stream));
  }
  if (e != hipSuccess) return fail(FL_ERR_LAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
  return FL_OK;
}

int fl_attn_fwd_f16_splitkv_noalloc(const fl_attn_params_ex* p, int32_t num_splits, void* stream) {
  const char* who = "fl_attn_fwd_f16_splitkv_noalloc";
  fl::FwdArgs a;
  int rc = check_ex(p, &a, who);
  if (rc != FL_OK) return rc;
  if (empty_problem(a)) return FL_OK;
  rc = check_pointers(&p->base, &a, who, 16);
  if (rc != FL_OK) return rc;
  const KvPlan plan = plan_kvsplit_capped(a, num_splits, FL_ATTN_SCRATCH_BYTES);
  if (plan.nsplit != 0 && plan.bytes > (int64_t)FL_ATTN_SCRATCH_BYTES)
    return fail(FL_ERR_UNSUPPORTED, "%s: %d key chunks need %lld bytes of scratch, above the "
                "%lld-byte limit (use fl_attn_fwd_f16_splitkv with a workspace)", who, plan.nsplit,
                (long long)plan.bytes, (long long)FL_ATTN_SCRATCH_BYTES);
  hipError_t e;
  if (plan.nsplit == 0) {
    e = fl::launch_fa2(a, select_fa2(a), static_cast<hipStream_t>(stream));
  } else {
    void* s = nullptr;
    rc = scratch_for_current_device(&s, who);
    if (rc != FL_OK) return rc;
    e = run_kvsplit(a, plan, static_cast<float*>(s), static_cast<hipStream_t>(stream));
  }
  if (e != hipSuccess) return fail(FL_ERR_LAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
  return FL_OK;
}

int fl_attn_naive_f16(const fl_attn_params* p, void* stream) {
  const char* who = "fl_attn_naive_f16";
  fl::FwdArgs a;
  int rc = check_common(p, &a, who);
  if (rc != FL_OK) return rc;
  if (empty_problem(a)) return FL_OK;
  if (a.seq_k > fl::naive_max_seq(a.head_dim))
    return fail(FL_ERR_UNSUPPORTED, "%s: N_k=%d exceeds the LDS capacity of the naive kernel (max %lld at D=%d)",
                who, a.seq_k, (long long)fl::naive_max_seq(a.head_dim), a.head_dim);
  if (a.batch_heads > 65535)
    return fail(FL_ERR_UNSUPPORTED, "%s: B*H=%d exceeds the grid limit 65535", who, a.batch_heads);
  rc = check_pointers(p, &a, who, 2);
  if (rc != FL_OK) return rc;
  const hipError_t e = fl::launch_naive(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(FL_ERR_LAUNCH, "%s: launch failed: %s", who, hipGetErrorString(e));
  return FL_OK;
}

}  // extern "C"
