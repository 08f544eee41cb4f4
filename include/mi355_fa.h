/*
 * mi355_fa.h — C ABI of the MI355X (gfx950) masked FlashAttention forward.
 *
 * One operator: O = softmax(Q·Kᵀ·(1/√d) + mask)·V over [B,H,S,d] tensors, where
 * the additive mask (0 = visible, -inf = blocked, finite = bias) is broadcast
 * over heads and K/V may carry fewer heads than Q (GQA, kv_head = h / (H/Hk)).
 *
 * Plain pointers and sizes only; no torch types cross this boundary. The
 * library never allocates device memory: split-KV partials live in a
 * caller-provided workspace whose size `mi355_fa_workspace_bytes` reports.
 * All work is enqueued on the caller's stream; nothing synchronises.
 *
 * Reference interfaces these entry points replace (Defyli/custom_ops):
 *   - mi355_fa_params        ↔ FA_mask_params           csrc/fa/common/fa_fwd_params.h:18-71
 *   - mi355_fa_fwd           ↔ mha_fwd_with_mask_cuda   csrc/fa/fa_fwd_op.cu:46-197
 *                              (validation :53-108, launch :191-194) and
 *                              fa_fwd_launch            csrc/fa/fa_fwd_launch.h:573-603
 *   - mi355_fa_num_splits    ↔ fa_mask_sm89_num_splits  csrc/fa/fa_fwd_launch.h:137-170
 *   - mi355_fa_workspace_bytes ↔ the oaccum/lseaccum torch::empty allocations
 *                              csrc/fa/fa_fwd_launch.h:289-297
 */
#ifndef MI355_FA_H
#define MI355_FA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI355_FA_ABI_VERSION 3

/* Error codes returned by the entry points (0 = success). */
enum {
  MI355_FA_OK = 0,
  MI355_FA_EINVAL = 1,     /* argument/contract violation (message filled)       */
  MI355_FA_EWORKSPACE = 2, /* workspace missing or too small for the split plan   */
  MI355_FA_ELAUNCH = 3,    /* HIP launch error (message carries hipGetErrorString) */
  MI355_FA_EDEVICE = 4     /* current device is not gfx950                        */
};

/* Element type of q/k/v/mask/out (all five share it). */
enum { MI355_FA_FP16 = 0, MI355_FA_BF16 = 1 };

/*
 * Kernel-variant selection, for parity tests and tuning only. Every field 0
 * (or mi355_fa_params.variant NULL) leaves each choice to the library's plan;
 * a nonzero field forces one choice for this call and nothing else. No
 * counterpart in the reference, whose kernel variants are compile-time
 * template choices (csrc/fa/fa_fwd_launch.h:262-309).
 */
typedef struct mi355_fa_variant {
  int32_t waves;     /* 0 | 4 | 8: waves per workgroup (128 or 256 query rows)         */
  int32_t pack;      /* 0 | 1 | 2 | 4: GQA q-heads per workgroup (capped by H/Hk)      */
  int32_t order;     /* 0 | 1 heads fastest | 2 m-blocks fastest | 3 heads, then
                        splits fastest (workgroup order)                           */
  int32_t loop;      /* 0 | 1 32-row asm loop | 2 64-row asm loop | 3 ping-pong loop
                        (fp16: the 32-row loop) | -1 compiled kernel only             */
  int32_t fuse;      /* 0 | -1: two-split launches keep the combine kernel             */
  int32_t live;      /* 0 | 1 on everywhere | -1 off: live-range narrowing             */
  int32_t deep;      /* 0 | -1: 4-wave grids keep two K/V stages                       */
  int32_t mask_mfma; /* 0 | -1: the compiled kernel widens bf16 masks on the VALU      */
  int32_t stream;    /* 0 | 1 on | -1 off: the compiled kernel loads K/V with the
                        non-temporal hint (default: when each K/V tile is read by
                        one workgroup of the launch)                               */
  int32_t live_map;  /* 0 | 1 always | -1 never: live ranges from the live-tile map
                        pre-pass instead of each workgroup's own scan (default:
                        masks with unaligned rows, and 8-wave split launches)      */
  int32_t stage;     /* 0 | -1: masks with unaligned rows are read in place
                        (through registers) instead of from an aligned staged
                        copy in the workspace (1: staged, the default)             */
} mi355_fa_variant;

/*
 * Launch parameters. Strides are in ELEMENTS. Layouts:
 *   q    [B, H,  Sq, d]   o [B, H, Sq, d]
 *   k, v [B, Hk, Sk, d]   innermost (d) stride must be 1
 *   mask [B, 1, mask_seqlen_q >= Sq, mask_seqlen_k >= Sk], innermost stride 1
 * q, k, v and o: 16-byte aligned base, every stride a multiple of 8 elements
 * (rows move as 16-byte chunks); mask: 2-byte aligned, any strides.
 * Mask columns >= seqlen_k are always treated as blocked whatever they hold;
 * mask rows >= seqlen_q are never read for output. Sk need not be a multiple
 * of 8: the kernel predicates the K/V tail and reads unaligned mask rows
 * element-wise, so no padded copy is ever made.
 */
typedef struct mi355_fa_params {
  const void* q;
  const void* k;
  const void* v;
  const void* mask;
  void* o;

  int64_t q_batch_stride, q_head_stride, q_row_stride;
  int64_t k_batch_stride, k_head_stride, k_row_stride;
  int64_t v_batch_stride, v_head_stride, v_row_stride;
  int64_t o_batch_stride, o_head_stride, o_row_stride;
  int64_t mask_batch_stride, mask_row_stride;

  int32_t b, h, h_k;
  int32_t seqlen_q, seqlen_k;
  int32_t mask_seqlen_q, mask_seqlen_k;
  int32_t d;          /* 64 or 128 */
  int32_t dtype;      /* MI355_FA_FP16 | MI355_FA_BF16 */
  float scale_softmax; /* 1/sqrt(d) in the reference op; any positive value allowed */

  /* Split-KV: 0 = let the library plan it; >= 1 forces that many splits. */
  int32_t num_splits;
  /* Device workspace for split-KV partials, the fused split tail's ticket
   * words, and for masks with unaligned rows the live-tile map and an aligned
   * staged copy of the mask (may be NULL when mi355_fa_workspace_bytes
   * reports 0; its contents need no clearing). */
  void* workspace;
  size_t workspace_bytes;
  /* Test/tuning variant selection (NULL = the library's plan); see above. */
  const mi355_fa_variant* variant;
} mi355_fa_params;

/* Run the forward pass on `stream` (a hipStream_t; NULL = legacy default stream).
 * Returns 0 on success; otherwise writes a NUL-terminated message into err. */
int mi355_fa_fwd(const mi355_fa_params* p, void* stream, char* err, size_t errlen);

/* Size of the per-GPU scratch array behind mi355_fa_fwd_noalloc. */
#define MI355_FA_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20) /* 32 MiB */

/* mi355_fa_fwd without any allocation and without a workspace argument: the
 * workspace contents (split-KV partials and tickets, the live-tile map of
 * masks with unaligned rows and their staged copy) go to a fixed per-GPU
 * device array of MI355_FA_NOALLOC_SCRATCH_BYTES (allocated when the
 * library's code is loaded onto a GPU and held until the process ends).
 * p->workspace is ignored. A staged mask that does not fit is read in place
 * instead; plans that still need more scratch fail with MI355_FA_EWORKSPACE. Calls that overlap on
 * one GPU (other streams, other threads) share the array and race: serialise
 * them. No counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). */
int mi355_fa_fwd_noalloc(const mi355_fa_params* p, void* stream, char* err, size_t errlen);

/* Number of KV splits the launcher will use for these params (after its plan,
 * the MI355_FA_NUM_SPLITS override, read once per process, and clamping). */
int mi355_fa_num_splits(const mi355_fa_params* p);

/* Bytes of workspace mi355_fa_fwd needs for these params (split partials and
 * tickets; for masks with unaligned rows the live-tile map and the staged
 * copy; 0 when none of these). */
size_t mi355_fa_workspace_bytes(const mi355_fa_params* p);

/* Pure cost model, exposed for host tests: splits for a problem of
 * total_mblocks row-tiles, num_n_blocks key-tiles, on num_cus compute units. */
int mi355_fa_cost_model_splits(int total_mblocks, int num_n_blocks, int block_m,
                               int head_dim, int num_cus);

/* ABI version (MI355_FA_ABI_VERSION) and a build string. */
int mi355_fa_abi_version(void);
const char* mi355_fa_build_info(void);

#ifdef __cplusplus
}
#endif

#endif /* MI355_FA_H */
