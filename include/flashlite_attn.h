/*
 * flashlite_attn.h -- C ABI of the MI355X (gfx950) FlashAttention-2 forward
 * engine.  Plain pointers and sizes only: no torch, no HIP types.  The
 * stream is passed as an opaque `void*` holding a `hipStream_t` (NULL = the
 * legacy default stream).
 *
 * Reference surface replaced (thebigblender/FlashLite):
 *   - the host entry of `flash_attn_wmma.forward_flash2`,
 *     csrc/kernel_flash2.cu:732-839 (declared csrc/includes/flash_attn.h:117-124,
 *     bound at csrc/flash_attn.cpp:18-28);
 *   - the host entry of `flash_attn_wmma.forward_naive`,
 *     csrc/kernel_naive.cu:242-323 (declared csrc/includes/flash_attn.h:100-106,
 *     bound at csrc/flash_attn.cpp:7-16).
 * The torch-side checks (device, contiguity, dtype, rank, shapes, `out=`) stay
 * in the binding (flashlite_amd/csrc/flash_attn.cpp) with the reference's
 * messages; the checks below are the ones a raw-pointer caller needs.
 *
 * Layout: q, o are fp16 [batch, heads, seq_q, head_dim] and k, v fp16
 * [batch, heads, seq_k, head_dim], contiguous (fl_attn_fwd_f16_ex takes
 * strides).
 * The library allocates nothing, never synchronises, keeps no mutable global
 * state (beyond, per GPU, the cached address of the scratch array of
 * fl_attn_fwd_f16_splitkv_noalloc) and may be called from several host
 * threads at once.  Launches are
 * asynchronous on `stream`; results are visible after the stream reaches
 * them.  `o` may alias `q` (each work-group reads its own query rows before
 * it writes them); it must not alias `k` or `v`.
 */
#ifndef FLASHLITE_ATTN_H
#define FLASHLITE_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by every entry point. */
enum fl_status {
  FL_OK = 0,
  FL_ERR_INVALID_ARGUMENT = 1, /* NULL pointer, negative size, non-finite scale */
  FL_ERR_UNSUPPORTED = 2,      /* head_dim != 64 (flash2; 64 or 128 for the _ex entries),
                                  strides or sizes past limits */
  FL_ERR_MISALIGNED = 3,       /* flash2 needs 16-byte aligned q/k/v/o */
  FL_ERR_LAUNCH = 4,           /* the HIP launch itself failed */
  FL_ERR_BAD_CONFIG = 5        /* forced tile configuration out of range */
};

typedef struct fl_attn_params {
  const void* q;      /* fp16 [B, H, N, D]; N = seq_q */
  const void* k;      /* fp16 [B, H, N_k, D] */
  const void* v;      /* fp16 [B, H, N_k, D] */
  void* o;            /* fp16 [B, H, N, D], written for rows < N */
  int64_t batch;      /* B */
  int64_t heads;      /* H */
  int64_t seq_q;      /* N (query rows) */
  int64_t seq_k;      /* N_k key/value rows (k, v are [B, H, N_k, D]); may differ from N */
  int64_t head_dim;   /* D */
  double sm_scale;    /* 0.0 means 1/sqrt(D) (kernel_flash2.cu:769-771) */
  int32_t causal;     /* non-zero: key j visible to query i iff j <= i + N_k - N (bottom-right
                         aligned; top-left when N_k == N); a row with no visible key gets 0 */
} fl_attn_params;

/*
 * FlashAttention-2 forward, fp16 in/out, fp32 accumulation, D == 64.
 * Replaces flash_attn_forward_flash2's validation tail, scale handling,
 * adaptive dispatcher and launch (csrc/kernel_flash2.cu:756-757, 769-772,
 * 786-837).  The tile configuration comes from the built-in dispatcher.
 */
int fl_attn_fwd_f16(const fl_attn_params* p, void* stream);

/*
 * Same as fl_attn_fwd_f16 with the tile configuration forced (`config` in
 * [0, fl_attn_num_configs()), or -1 for the dispatcher's choice).  Replaces
 * the reference's two hard-wired launch branches (Br=64 / Br=128,
 * csrc/kernel_flash2.cu:789-835); used by sweeps and by tests that check
 * every configuration against the oracle.  Configuration 5
 * (br256_kv256_w8_stream) takes N_k <= 256 only and configuration 6
 * (br32_kv512_w4_quarters) N_k <= 512 only; they return FL_ERR_BAD_CONFIG
 * otherwise.
 */
int fl_attn_fwd_f16_cfg(const fl_attn_params* p, int32_t config, void* stream);

/*
 * Strided layouts and the log-sum-exp output.  `base` carries the pointers,
 * sizes, scale and mask exactly as for fl_attn_fwd_f16 (its layout comment
 * aside); the strides below replace the contiguous [B, H, N, D] layout.
 * Each stride triple is {batch, head, row} in elements; head_dim is unit
 * stride.  A [B, N, H, D] tensor (the layout of the `flash_attn` package,
 * which the reference's benchmark builds by transposing,
 * benchmarks/benchmark_throughput.py:110-112) has strides
 * {N*H*D, D, H*D}.  Strides are non-negative multiples of 8 elements, row
 * strides in [64, 2^30); K and V rows must lie within 2^31 bytes of their
 * head's first row.  Output rows must not overlap each other or q, k, v
 * (o == q with equal strides is allowed, as for fl_attn_fwd_f16).
 *
 * lse: optional fp32 [B, H, N] (contiguous), written with each query row's
 * ln(sum_j exp(sm_scale * q.k_j)) over its visible keys, -inf for a row
 * with no visible key; NULL to skip.
 *
 * head_dim is 64 or 128.  At both, Q enters the MFMA unscaled and the fp32
 * scores are scaled by sm_scale*log2(e), as in the reference
 * (csrc/kernel_flash2.cu:188-195).  At 64, `config` is as for
 * fl_attn_fwd_f16_cfg;
 * at 128 it is -1 or one of the two slot-scheduled configurations
 * (3 "br256_bc64_w8_slot", 4 "br128_bc64_w4_slot"; same work-group shapes,
 * 32-key tiles), FL_ERR_BAD_CONFIG otherwise.
 *
 * No counterpart in the reference, which accepts only contiguous
 * [B, H, N, 64] tensors (csrc/kernel_flash2.cu:741-757) and returns no
 * log-sum-exp.
 */
typedef struct fl_attn_params_ex {
  fl_attn_params base;
  int64_t q_stride[3];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t o_stride[3];
  float* lse;
} fl_attn_params_ex;

int fl_attn_fwd_f16_ex(const fl_attn_params_ex* p, int32_t config, void* stream);

/*
 * bf16 q, k, v and o (same layouts, strides, lse and head_dims as
 * fl_attn_fwd_f16_ex; `config` -1 or, at head_dim 64, any configuration but
 * the pipelined 0 and 1, at head_dim 128 3 or 4).  Q enters the MFMA
 * unscaled and the fp32 scores are scaled by sm_scale*log2(e); P is rounded
 * to bf16 before the PV product and the row sums are fp32.
 *
 * No counterpart in the reference, which accepts fp16 only
 * (csrc/kernel_flash2.cu:745-747).
 */
int fl_attn_fwd_bf16_ex(const fl_attn_params_ex* p, int32_t config, void* stream);

/*
 * Split-KV forward ("flash-decoding"), fp16 at head_dim 64, for few query
 * rows over many keys:
 * the key range of every (batch, head) is cut into chunks processed by
 * separate work-groups, whose partial results (unnormalised O, stabiliser,
 * row sum) go to `workspace`; a second kernel on the same stream merges
 * them into O (and lse).  Same parameters, layouts and results as
 * fl_attn_fwd_f16_ex up to fp32 rounding.
 *
 * num_splits > 0 asks for that many chunks (at most the number of 64-key
 * tiles, and 256); num_splits <= 0 lets the library choose, which may be
 * "no split": then the one-pass kernel runs and no workspace is needed.
 * fl_attn_splitkv_workspace_bytes returns the bytes a call with the same
 * `p` and `num_splits` needs (0 when it will not split, -1 if `p` is
 * rejected).  The workspace is 16-byte aligned device memory owned by the
 * caller; calls that may overlap must not share one.
 *
 * No counterpart in the reference (one work-group per 64/128 query rows,
 * csrc/kernel_flash2.cu:786-835, which leaves a decode step with N = 1 on a
 * handful of CUs); its README advertises `out=` for serving/decode loops
 * (README.md:119-126).
 */
int64_t fl_attn_splitkv_workspace_bytes(const fl_attn_params_ex* p, int32_t num_splits);
int fl_attn_fwd_f16_splitkv(const fl_attn_params_ex* p, int32_t num_splits, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * fl_attn_fwd_f16_splitkv without a workspace argument and without any
 * allocation: the partial results go to a scratch array of
 * FL_ATTN_SCRATCH_BYTES (8 MiB) that the library holds in device memory on
 * every GPU it runs on, until the process ends.  Same parameters and
 * results as fl_attn_fwd_f16_splitkv, bit for bit, for the same chunk
 * count.  num_splits > 0 is taken as asked; a count whose partials exceed
 * the limit returns FL_ERR_UNSUPPORTED and launches nothing.
 * num_splits <= 0 lets the library choose as for fl_attn_fwd_f16_splitkv,
 * lowered to the most chunks whose partials fit the limit, or to one pass
 * (no scratch) when fewer than two fit: the library's own choice never
 * fails for lack of scratch.  fl_attn_splitkv_noalloc_bytes returns the
 * scratch bytes a call with the same `p` and `num_splits` uses (0 for one
 * pass, -1 if `p` is rejected; above FL_ATTN_SCRATCH_BYTES only for a
 * requested count that will be refused).  Launches on the
 * current device, into `stream`, which must belong to it.  Every call on a
 * GPU shares that GPU's array (each call writes every partial it reads, so
 * nothing has to start at zero): calls that may overlap on one GPU -- other
 * streams, other host threads -- race and must be serialised by the caller.
 *
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.
 */
#define FL_ATTN_SCRATCH_BYTES (8 << 20)
int fl_attn_fwd_f16_splitkv_noalloc(const fl_attn_params_ex* p, int32_t num_splits, void* stream);
int64_t fl_attn_splitkv_noalloc_bytes(const fl_attn_params_ex* p, int32_t num_splits);

/*
 * Un-fused baseline: one work-group per query row, scores staged in LDS.
 * Any head_dim >= 1; seq limited by LDS (about 40k keys at D=64).
 * Replaces flash_attn_forward_naive's scale handling and launch
 * (csrc/kernel_naive.cu:278-320), without the reference's shared-memory
 * write-after-read race between its two block reductions (:66 vs :81-83).
 */
int fl_attn_naive_f16(const fl_attn_params* p, void* stream);

/* Detail message of the last non-OK status on the calling thread. */
const char* fl_attn_last_error(void);

/* Dispatcher introspection (no counterpart in the reference, whose dispatch
 * rule is the fixed `seq_len >= 2048` test at csrc/kernel_flash2.cu:789). */
int fl_attn_num_configs(void);
const char* fl_attn_config_name(int32_t config);
/* The id of the configuration named `name` (as fl_attn_config_name returns
 * it), or -1 if no configuration has that name.  Ids can change between
 * versions of the library; names do not, so a caller that forces a
 * configuration should look its id up by name. */
int fl_attn_config_id(const char* name);
/* Returns the configuration fl_attn_fwd_f16 would launch for `p`, or -1 if
 * `p` is rejected (the reason is in fl_attn_last_error()). */
int fl_attn_select_config(const fl_attn_params* p);

#ifdef __cplusplus
}
#endif

#endif /* FLASHLITE_ATTN_H */
