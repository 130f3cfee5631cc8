/*
 * attnfuse_hip.h -- C ABI of libattnfuse_hip.so, the MI355X (gfx950) kernels
 * behind the AttnFuse attention DSL.
 *
 * The reference launches Triton kernels straight from Python
 * (reference: attnfuse/runtime/dispatch.py:196-214,
 * attnfuse/runtime/flash_decode.py:150-186, attnfuse/runtime/backward.py:130-190,
 * attnfuse/runtime/block_mask.py:244-269,299-363).  This header is the
 * boundary that replaces those launch sites: plain C, plain pointers, element
 * strides and sizes, no torch or HIP types.  Any FFI (ctypes, cffi, a C++
 * extension) can bind it.
 *
 * Contract
 *  - The library never allocates or frees device memory.  Outputs and
 *    workspaces are caller-owned.
 *  - Tensors are (B, H, N, D) with arbitrary element strides, except that
 *    the innermost (head-dim) stride must be 1, base pointers must be 16-byte
 *    aligned and the batch/head/sequence strides must be multiples of 8
 *    elements (16-byte rows for 16-byte vector loads).
 *  - Every launch goes on the caller's stream (a hipStream_t passed as
 *    void*; NULL is the legacy default stream).  Launches are asynchronous.
 *  - Return value: AF_OK (0) when the kernels were enqueued; a negative
 *    af_status otherwise, with a message in af_last_error() (thread-local).
 *  - Reentrant: no mutable global state besides the immutable kernel table.
 */
#ifndef ATTNFUSE_HIP_H
#define ATTNFUSE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AF_ABI_VERSION 6

typedef enum af_status {
  AF_OK = 0,
  AF_ERR_UNSUPPORTED = -1, /* no instantiation for this specialisation key */
  AF_ERR_BAD_ARG = -2,     /* shape, stride, alignment or pointer problem  */
  AF_ERR_LAUNCH = -3,      /* the HIP runtime refused the launch           */
  AF_ERR_WORKSPACE = -4    /* workspace missing or too small               */
} af_status;

typedef enum af_dtype { AF_F16 = 0, AF_BF16 = 1, AF_F32 = 2 } af_dtype;

/* Mask kinds (reference MASK_KIND encoding, attnfuse/compiler/codegen.py:88,
 * extended with the block-sparse kind). */
typedef enum af_mask {
  AF_MASK_FULL = 0,
  AF_MASK_CAUSAL = 1,          /* key j visible to query i iff j <= i        */
  AF_MASK_SLIDING_WINDOW = 2,  /* visible iff |i - j| < window               */
  AF_MASK_BLOCK_SPARSE = 3,    /* visible iff (i/BM, j/BN) is a listed tile  */
  AF_MASK_CAUSAL_SLIDING_WINDOW = 4 /* visible iff i - window < j <= i     */
} af_mask;

typedef enum af_bias {
  AF_BIAS_NONE = 0,
  AF_BIAS_ALIBI = 1,    /* S += -slope[h] * |i - j|; decode: |(N_kv-1) - j| */
  AF_BIAS_ADDITIVE = 2  /* S += bias[b][h][i][j]                             */
} af_bias;

typedef enum af_norm { AF_NORM_SOFTMAX = 0, AF_NORM_RELU = 1 } af_norm;

/* Specialisation key: replaces the reference's Triton constexpr record
 * (attnfuse/compiler/codegen.py:391-404; attnfuse/ir/tiled.py:52-81). */
typedef struct af_spec_key {
  int32_t dtype;     /* af_dtype; AF_F32: every entry point, head dims 32/64/128 */
  int32_t head_dim;  /* instantiated: 32, 64, 128, 256 (256: fp16/bf16 only; af_query) */
  int32_t mask;      /* af_mask                   */
  int32_t bias;      /* af_bias                   */
  int32_t norm;      /* af_norm                   */
  int32_t rope;      /* 1: rotate-half RoPE fused */
} af_spec_key;

/* Block-sparse mask in CSR form: the reference BlockMask fields
 * (attnfuse/runtime/block_mask.py:84-97).  Row r of the Q-major lists names
 * the key blocks query block r visits; the K-major lists are the transpose
 * (used by the dK/dV backward).  All arrays are device int32. */
typedef struct af_blockmask {
  const int32_t* full_kv_num;   /* (n_q_blocks)                 */
  const int32_t* full_kv_idx;   /* (n_q_blocks, full_kv_stride) */
  const int32_t* kv_num_blocks; /* (n_q_blocks) partial tiles   */
  const int32_t* kv_indices;    /* (n_q_blocks, kv_stride)      */
  const int32_t* q_num_blocks;  /* (n_kv_blocks)                */
  const int32_t* q_indices;     /* (n_kv_blocks, q_stride)      */
  int64_t full_kv_stride, kv_stride, q_stride;  /* row strides = padded row widths, >= 1 */
  int32_t block_m, block_n, n_q_blocks, n_kv_blocks;
  /* Optional work plans written by af_blockmask_plan, device int32 (all
   * NULL / 0: one workgroup per query block and per key block, the
   * reference's grid).  q_*: the Q-major lists (forward, dQ); kv_*: the
   * K-major lists (dK/dV).  An item is (list, first entry, entries, partial
   * slot or -1); a split is (list, first slot, slots).  An item with slot -1
   * is a whole list and is walked to the list's count in device memory at
   * launch time, so lists may be rewritten in place between launches (graph
   * replays included); the pieces of a split list are clamped to that count,
   * and a plan must be remade after a split list changes length. */
  const int32_t* q_items;   /* (n_q_items, 4)   */
  const int32_t* q_splits;  /* (n_q_splits, 3)  */
  const int32_t* kv_items;  /* (n_kv_items, 4)  */
  const int32_t* kv_splits; /* (n_kv_splits, 3) */
  int32_t n_q_items, n_q_splits, n_q_slots;
  int32_t n_kv_items, n_kv_splits, n_kv_slots;
  /* Optional element masks of the partial tiles (kv_indices entries), all
   * three NULL or all three set.  No counterpart in the reference, which
   * visits a partial tile whole (attnfuse/runtime/block_mask.py:139-151) and
   * lists element masks as future work (PROGRESS.md:284-288).  Device
   * uint64 words, a set bit = visible:
   *   part_row_bits (n_q_blocks, kv_stride, block_m, block_n / 64): word w of
   *     row r of query block qb's partial entry e covers keys
   *     64 w .. 64 w + 63 of that entry's key block;
   *   q_col_bits (n_kv_blocks, q_stride, block_n, ceil(block_m / 64)): word w
   *     of key column c of key block kb's K-major entry e covers queries
   *     64 w .. 64 w + 63 of that entry's query block (dK/dV);
   *   q_partial (n_kv_blocks, q_stride) int32: 1 where K-major entry e of key
   *     block kb is a partial tile (its q_col_bits apply). */
  const uint64_t* part_row_bits;
  const uint64_t* q_col_bits;
  const int32_t* q_partial;
} af_blockmask;

/* Work plan of a block-sparse walk over lists of counts[i] entries (Q-major:
 * full_kv_num[i] + kv_num_blocks[i]; K-major: q_num_blocks[i]); host
 * arrays.  No counterpart in the reference, whose grids run one program per
 * query block and per key block: there a BigBird global row or column, n
 * blocks long, is a single program's serial walk behind which the rest of
 * the grid waits.  Lists longer than `chunk` entries (chunk <= 0: the
 * library's choice, twice the mean list length and at least 8) are cut into
 * near-equal pieces, each its own workgroup writing fp32 partial results to
 * a slot of the workspace that a combine kernel merges.  sizes[0..2] =
 * (n_items, n_splits, n_slots); items (n_items x 4, longest first) and
 * splits (n_splits x 3) are written when non-NULL: call once with both NULL
 * for the sizes. */
int af_blockmask_plan(const int32_t* counts, int32_t n, int32_t chunk,
                      int32_t* items, int32_t* splits, int32_t* sizes);

/* Forward attention.  Replaces the attnfuse_fwd_kernel launch
 * (reference: attnfuse/runtime/dispatch.py:69-215, kernel
 * attnfuse/compiler/codegen.py:67-381). */
typedef struct af_fwd_args {
  af_spec_key key;
  const void* q;       /* (B, H_q,  N_q,  D) */
  const void* k;       /* (B, H_kv, N_kv, D) */
  const void* v;       /* (B, H_kv, N_kv, D) */
  void* o;             /* (B, H_q,  N_q,  D), dtype of q                   */
  float* lse;          /* nullable: (B, H_q, N_q) fp32 log-sum-exp (ln)    */
  const void* cos;     /* rope: (N_rope, D) table in q's dtype             */
  const void* sin;
  const float* alibi_slopes; /* ALiBi: (H_q) fp32                          */
  const void* bias;    /* additive: (B, H_q, N_q, N_kv) in q's dtype       */
  uint32_t* coverage;  /* nullable: (B, H_q, ceil(N_q/32), ceil(N_kv/64))
                          visit counters, for mask-coverage tests          */
  int64_t q_stride[4], k_stride[4], v_stride[4], o_stride[4];
  int64_t lse_stride[3];
  int64_t rope_stride[2]; /* (n, d) */
  int64_t bias_stride[4];
  int32_t batch, heads_q, heads_kv, seqlen_q, seqlen_kv, rope_len;
  float scale;
  int32_t window;      /* sliding window size (AF_MASK_SLIDING_WINDOW)     */
} af_fwd_args;

/* Workspace bytes af_fwd / af_fwd_blocksparse need for these arguments:
 * with fused RoPE, the rotated keys k~ (B, H_kv, N_kv, D) in the input dtype,
 * written once per call so that the attention kernel streams k~ instead of
 * re-rotating every key tile in every query block; 0 without RoPE (the
 * workspace may then be NULL). */
size_t af_fwd_workspace_bytes(const af_fwd_args* args);
/* fp16 / bf16: 16-bit MFMAs with fp32 accumulation.  AF_F32: q, k, v, o,
 * tables and bias in fp32, every product in fp32 on the fp32 MFMAs (the
 * reference's Triton dots run fp32 inputs in TF32); coverage must be NULL. */
int af_fwd(const af_fwd_args* args, void* workspace, size_t workspace_bytes,
           void* stream);

/* Block-sparse forward.  Replaces attnfuse_blocksparse_fwd_kernel
 * (reference: attnfuse/runtime/block_mask.py:205-271,
 * attnfuse/compiler/codegen_blocksparse.py:34-171).  args->key.mask must be
 * AF_MASK_BLOCK_SPARSE; the tile visited per listed block is whole (no
 * element mask inside it, reference semantics).  BLOCK_M 32, 64 or 128;
 * BLOCK_N a multiple of 64 (fp16/bf16) or of 32 (fp32). */
int af_fwd_blocksparse(const af_fwd_args* args, const af_blockmask* bm,
                       void* workspace, size_t workspace_bytes, void* stream);
/* Workspace bytes af_fwd_blocksparse needs: af_fwd_workspace_bytes plus,
 * with a Q-major work plan (fp16/bf16), per partial slot and (batch, head)
 * BLOCK_M rows of fp32 (unnormalised O, running max, row sum). */
size_t af_fwd_blocksparse_workspace_bytes(const af_fwd_args* args,
                                          const af_blockmask* bm);

/* Flash-decoding (one query row per head, split-K over the cache, then a
 * log-sum-exp combine).  Replaces attnfuse_decode_split_kernel +
 * attnfuse_decode_combine_kernel (reference:
 * attnfuse/runtime/flash_decode.py:101-187,
 * attnfuse/compiler/codegen_decode.py:46-211).  key.mask must be FULL and
 * key.bias NONE or ALIBI, key.rope 0.  fp16/bf16 run the split on the
 * 16x16x32 MFMAs; fp32 (head dims 32, 64, 128) on fp32 VALU FMAs, which keep
 * up with HBM at decode's 1 FLOP per byte. */
typedef struct af_decode_args {
  af_spec_key key;
  const void* q;  /* (B, H_q, 1, D)     */
  const void* k;  /* (B, H_kv, N_kv, D) */
  const void* v;
  void* o;        /* (B, H_q, 1, D)     */
  const float* alibi_slopes;
  int64_t q_stride[4], k_stride[4], v_stride[4], o_stride[4];
  int32_t batch, heads_q, heads_kv, seqlen_kv;
  float scale;
  int32_t num_splits; /* <= 0: library default (af_decode_num_splits) */
} af_decode_args;

int32_t af_decode_num_splits(int32_t batch, int32_t heads_q, int32_t heads_kv,
                             int32_t seqlen_kv, int32_t head_dim);
size_t af_decode_workspace_bytes(int32_t batch, int32_t heads_q,
                                 int32_t head_dim, int32_t num_splits);
int af_decode(const af_decode_args* args, void* workspace,
              size_t workspace_bytes, void* stream);

/* Flash decoding that allocates nothing and takes no workspace.  It has no
 * counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  The split partials live in a library-owned device array of
 * AF_DECODE_NOALLOC_SCRATCH_BYTES per GPU, held from the first call on that
 * GPU until the process ends.  With num_splits <= 0 the split count is
 * lowered until the partials fit; an explicit num_splits whose non-empty
 * splits (after the 32-key rounding of the split length) do not fit, or a
 * batch whose single-split partials (B * H_q * (2 + D) * 4 bytes) do not
 * fit, returns AF_ERR_WORKSPACE.  Every call on one GPU shares the array:
 * calls that overlap in time on one GPU (other streams, other threads) race;
 * calls on one stream are ordered.  Results equal af_decode's for the same
 * split count.  The first call on a GPU looks up the array's device address
 * (hipGetSymbolAddress); make it before capturing a graph that calls this
 * function, after which captured calls record only the two kernel launches. */
#define AF_DECODE_NOALLOC_SCRATCH_BYTES (4u << 20)
int af_decode_noalloc(const af_decode_args* args, void* stream);

/* Backward (FA2 style: delta = rowsum(dO*O), then dK/dV, then dQ).
 * Replaces attnfuse_bwd_{preproc,dkv,dq}_kernel and the block-sparse dkv/dq
 * kernels (reference: attnfuse/runtime/backward.py:83-192,
 * attnfuse/runtime/block_mask.py:274-363).  Supports softmax with FULL,
 * CAUSAL, SLIDING_WINDOW and BLOCK_SPARSE masks, NONE/ALIBI bias and fused
 * RoPE (the gradients are rotated back to the input space).  dK/dV of a
 * key/value head are summed over its query-head group in-kernel. */
typedef struct af_bwd_args {
  af_spec_key key;
  const void *q, *k, *v, *o, *dout;
  const float* lse;  /* (B, H_q, N_q) fp32, from the forward */
  void *dq, *dk, *dv;
  const void* cos;
  const void* sin;
  const float* alibi_slopes;
  int64_t q_stride[4], k_stride[4], v_stride[4], o_stride[4], do_stride[4];
  int64_t dq_stride[4], dk_stride[4], dv_stride[4];
  int64_t lse_stride[3];
  int64_t rope_stride[2];
  int32_t batch, heads_q, heads_kv, seqlen_q, seqlen_kv, rope_len;
  float scale;
  int32_t window;
  int32_t group_split; /* dK/dV workgroups sharing one key block's GQA query
                          heads: 0 = library default (af_bwd_tile), else a
                          power of two dividing heads_q / heads_kv.  Replaces
                          the reference's _BWD_TILE override
                          (attnfuse/runtime/backward.py:26-47). */
} af_bwd_args;

/* Workspace bytes af_bwd needs for these arguments: the log2-scaled LSE and
 * delta (an fp32 pair per query row); with fused RoPE the rotated q~ and k~ in the input dtype; and when
 * the query heads of a GQA group are split over several dK/dV workgroups
 * (grids of at most two workgroups per CU), fp32 dK and dV partial sums
 * per split.  Returns 0 for a block-sparse key (key.mask
 * AF_MASK_BLOCK_SPARSE): its workspace depends on the mask's work plan, so
 * such callers use af_bwd_blocksparse_workspace_bytes. */
size_t af_bwd_workspace_bytes(const af_bwd_args* args);
/* fp16 / bf16, or AF_F32 (fp32 throughout on the fp32 MFMAs, head dims 32,
 * 64, 128).  Block-sparse (key.mask AF_MASK_BLOCK_SPARSE) needs bm with
 * BLOCK_M and BLOCK_N of 64 or 128. */
int af_bwd(const af_bwd_args* args, const af_blockmask* bm /* nullable */,
           void* workspace, size_t workspace_bytes, void* stream);
/* Workspace bytes af_bwd needs with this block mask (nullable): the above
 * plus the fp32 partials of the mask's work plans, BLOCK_M dQ rows per
 * Q-major slot and (batch, query head), BLOCK_N dK and dV rows per K-major
 * slot and (batch, key/value head).  The K-major plan is used only when the
 * GQA query heads are not split (group_split 1). */
size_t af_bwd_blocksparse_workspace_bytes(const af_bwd_args* args,
                                          const af_blockmask* bm);

/* Backward launch shape for these arguments: query rows per dQ workgroup,
 * keys per dK/dV workgroup and the GQA group split the launch uses (the
 * args' group_split, or the library's choice when it is 0).  With a block
 * mask (nullable) the block sizes are the mask's.  Any output pointer may be
 * NULL.  Replaces the reference's _pick_backward_tile
 * (attnfuse/runtime/backward.py:35-47). */
int af_bwd_tile(const af_bwd_args* args, const af_blockmask* bm,
                int32_t* block_m, int32_t* block_n, int32_t* group_split);

/* 1 if an instantiation exists for the key (forward; decode and backward
 * accept the subsets documented above), else 0. */
int af_query(const af_spec_key* key);
/* Forward tile shape used for the key: query rows per workgroup and keys per
 * stage (the coverage counters are kept per 32 query rows x 64 keys). */
int af_fwd_tile(const af_spec_key* key, int32_t* block_m, int32_t* block_n);

const char* af_last_error(void);
int af_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ATTNFUSE_HIP_H */
