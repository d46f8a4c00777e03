/*
 * dan_tree_attn.h -- C ABI of the gfx950 tree-masked prefill attention.
 *
 * One packed token sequence holds many requests ("segments"). Inside a
 * segment the new tokens are a trunk followed by contiguous branches; a
 * segment may start after `past_len` cached prefix tokens whose keys and
 * values live in separate [Hkv, P, D] tensors. A query sees a key iff the key
 * comes first and the key is past, trunk, or in the query's own branch.
 *
 * This header replaces, as one fused launch, the GPU leg of
 *   dan/attention.py:200-207   attend(q, k, v, segments, layer, scale=None)
 *   dan/attention.py:210-241   _attend_varlen: three varlen flash calls
 *                              (trunk causal, branch-vs-trunk, branch-causal)
 *                              plus the log-sum-exp merge of dan/fused.py:94-101
 * and the metadata those calls consume:
 *   dan/attention.py:72-126    Segment / segment()   -> DanSegmentDesc
 *   dan/attention.py:138-172   ReadLayout.build      -> DanWorkItem list + key_lo
 *   dan/cache.py:15            prefix-cache entry    -> DanPastDesc
 *
 * Conventions
 *  - All tensors are device memory owned by the caller. The library borrows
 *    the pointers for one stream-ordered launch, allocates nothing and keeps
 *    nothing.
 *  - Strides are in elements. The head_dim axis must have unit stride, and
 *    every row (token or head step of q, k, v, out and of each prefix-cache
 *    entry) must start 16 bytes aligned: rows move in 16-byte pieces.
 *  - Offsets inside a key tile are 32-bit: 64 * k_stride_tok * element size
 *    of k and of every prefix-cache entry's k must stay below 2^31 bytes, and
 *    so must head_dim * vt_cols * 2 (the V^T copy).
 *  - Every entry point returns 0 on success; on failure it returns a nonzero
 *    DanStatus and dan_tree_attn_last_error() describes the failure (a
 *    thread-local string, valid until the next call on the same thread).
 *  - The launch is asynchronous on `stream` (a hipStream_t); nothing here
 *    synchronizes.
 */
#ifndef DAN_TREE_ATTN_H
#define DAN_TREE_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DAN_TREE_ATTN_ABI_VERSION 8

/* Keys per key tile; the work list's key-tile indices count in these. */
#define DAN_TREE_ATTN_KEY_TILE 64

typedef enum {
  DAN_OK = 0,
  DAN_ERR_INVALID_ARGUMENT = 1,
  DAN_ERR_UNSUPPORTED = 2,
  DAN_ERR_LAUNCH = 3,
  DAN_ERR_VERSION = 4
} DanStatus;

typedef enum {
  DAN_DTYPE_BF16 = 0,
  DAN_DTYPE_F16 = 1,
  DAN_DTYPE_F32 = 2,  /* v and out only (q and k of an fp32 model are passed as fp16) */
  DAN_DTYPE_E4M3 = 3  /* OCP float8 e4m3fn inputs with per-tensor fp32 scales */
} DanDtype;

/* One request of the packed batch (dan/attention.py:72-84, :114-126).
 * New tokens are packed rows [start, start + n): the first `trunk` are the
 * trunk, the rest are branches (each contiguous). */
typedef struct {
  int32_t start;
  int32_t n;
  int32_t trunk;
  int32_t past_len; /* P: cached prefix tokens before the trunk (0: none) */
  int32_t past_idx; /* index into DanTreeAttnArgs.pasts, -1 when past_len == 0 */
  int32_t vt_col;   /* first column of this segment in the workspace's V^T copy
                       (a multiple of DAN_TREE_ATTN_KEY_TILE); the segment owns
                       roundup(past_len + n) columns from there */
  int32_t reserved[2];
} DanSegmentDesc;

/* One prefix-cache entry for the current layer: k, v each [Hkv, len, D]
 * (dan/cache.py:15, dan/attention.py:202-204, :254-257). Several segments may
 * point at the same entry. k_scale / v_scale are device fp32 scalars for
 * DAN_DTYPE_E4M3 (k ~ kq * k_scale); with fp16 q and k staged from fp32
 * (DanTreeAttnArgs.q_scale set), k_scale is the staged k's power-of-2 scale
 * and v_scale is ignored; otherwise both are ignored. */
typedef struct {
  const void *k;
  const void *v;
  int64_t k_stride_head, k_stride_tok;
  int64_t v_stride_head, v_stride_tok;
  const float *k_scale;
  const float *v_scale;
  int32_t len;
  int32_t reserved;
} DanPastDesc;

/* One query tile of one segment (replaces ReadLayout's cu_seqlens,
 * dan/attention.py:138-172). Queries are the segment's new tokens
 * [t0, t0 + tq) (segment-local). Keys are counted in "segment key
 * coordinates": 0..P-1 are the past, P.. are the new tokens. The key tiles
 * visited are [0, ja1) then [jb0, jb1) (tiles of DAN_TREE_ATTN_KEY_TILE keys;
 * jb0 >= ja1); tiles below `jfull` are visible to every query of the tile and
 * are not masked. `lo_max` is the largest key_lo of the item's queries: keys
 * in [P + trunk, lo_max) are hidden from some of its branch queries, so only
 * tiles meeting that range need the sibling-branch test; elsewhere the mask
 * is causal only. */
typedef struct {
  int32_t seg;
  int32_t t0;
  int32_t tq;
  int32_t ja1;
  int32_t jb0;
  int32_t jb1;
  int32_t jfull;
  int32_t lo_max;
} DanWorkItem;

/* One unit of the attention launch's persistent schedule: a work item for one
 * head group, with its segment's fields copied in, so that a work group
 * resolves a unit with a single 64-byte read. */
typedef struct {
  DanWorkItem item;
  int32_t start;    /* the item's segment: DanSegmentDesc.start */
  int32_t n;        /* .n */
  int32_t trunk;    /* .trunk */
  int32_t past_len; /* .past_len */
  int32_t past_idx; /* .past_idx */
  int32_t vt_col;   /* .vt_col */
  int32_t group;    /* head group: kv head + num_kv_heads * chunk, in [0, G) */
  int32_t reserved;
} DanUnit;

typedef struct {
  int32_t abi_version; /* DAN_TREE_ATTN_ABI_VERSION */
  int32_t in_dtype;    /* DanDtype of q, k and the pasts' k: bf16, f16 or e4m3 */
  int32_t out_dtype;   /* DanDtype of out: bf16, f16 or f32 (bf16 for e4m3) */
  int32_t v_dtype;     /* DanDtype of v and the pasts' v: bf16, f16, f32 or e4m3 */
  int32_t num_heads;   /* H */
  int32_t num_kv_heads;/* Hkv; query head h reads kv head h / (H / Hkv) */
  int32_t head_dim;    /* D: 64, 128 or 256 */
  int32_t num_tokens;  /* N packed tokens */
  float scale;         /* softmax scale (1/sqrt(D) when the caller passes None) */

  const void *q; int64_t q_stride_tok, q_stride_head; /* [N, H, D] view   */
  const void *k; int64_t k_stride_tok, k_stride_head; /* [N, Hkv, D] view */
  const void *v; int64_t v_stride_tok, v_stride_head; /* [N, Hkv, D] view */
  void *out;     int64_t o_stride_tok, o_stride_head; /* [N, H, D] view   */

  /* Device fp32 per-tensor scales (x ~ stored * scale). DAN_DTYPE_E4M3:
   * q_scale, k_scale and v_scale, all required. fp16 q and k with fp32 v
   * (fp32 callers): optionally q_scale and k_scale together, the power-of-2
   * scales dan_tree_attn_stage_f16 wrote, and then every prefix entry's
   * k_scale too; S is multiplied by q_scale * k_scale. NULL otherwise. */
  const float *q_scale;
  const float *k_scale;
  const float *v_scale;

  const DanSegmentDesc *segments; int32_t num_segments;
  const DanPastDesc *pasts;       int32_t num_pasts;
  const DanWorkItem *work;        int32_t num_work;
  /* [N] per packed token: for a branch token, P + (first new-token index of
   * its branch); 0 for trunk tokens. Key kc is visible to query qc iff
   *   kc <= qc  and  (kc < P + trunk  or  kc >= key_lo[query]). */
  const int32_t *key_lo;
  int32_t tile_q; /* queries per work item; must equal dan_tree_attn_tile_q() */
  int32_t vt_cols; /* columns of the V^T copy: sum over segments of roundup(past_len + n) */
  /* [vt_cols / DAN_TREE_ATTN_KEY_TILE]: the segment owning each column block */
  const int32_t *col_seg;
  /* Device scratch of at least dan_tree_attn_workspace_size() bytes, 256-byte
   * aligned, owned by the caller: it receives V (and the pasts' v) as fp16,
   * transposed to [Hkv][D][vt_cols], and after it one int32 exponent per
   * (kv head, 64-column block), before the attention kernel runs on the same
   * stream. A block holds V * 2^-e: e = 0 unless its largest |v| lies outside
   * [2^-6, 2^15], so no finite v overflows or flushes in fp16. */
  void *workspace;
  int64_t workspace_bytes;
  /* Which of the two launches to make: DAN_TREE_ATTN_PHASES_ALL (0: the V^T
   * copy, then attention), DAN_TREE_ATTN_PHASE_PACK (the copy only) or
   * DAN_TREE_ATTN_PHASE_ATTEND (attention only, reading a workspace a
   * previous call filled for the same v and pasts) -- for callers that
   * overlap the copy with other work, and for timing each launch. */
  int32_t phases;
  /* Persistent schedule of the attention launch: `num_slots` work groups
   * (about one per CU), slot s processing units[sched_off[s]] ..
   * units[sched_off[s + 1] - 1] in order. `units` holds num_work * G records,
   * G = dan_tree_attn_head_groups(num_heads, num_kv_heads): every (work item,
   * head group) pair exactly once. Slot s runs on XCD s % 8, so a planner
   * that gives slot s only units of kv head s % Hkv keeps each kv head's keys
   * and values in one XCD's L2. The attention launch reads the work items
   * and segments through `units`; `work` and `segments` keep their meaning
   * for the V^T copy and for validation. */
  const DanUnit *units;
  const int32_t *sched_off; /* [num_slots + 1], sched_off[0] = 0 */
  int32_t num_slots;
  /* Budget mode (NULL otherwise): the device int32 {S, B, W, C} a budget-mode
   * planner launch read (dan_tree_plan.h). num_work, vt_cols and num_slots
   * are then the capacities the tables were sized for (launch grids, the V^T
   * copy's row stride); the V^T copy skips column blocks from C on, and the
   * slots past this batch's are empty. The same launches, captured once,
   * serve every batch within the capacities. */
  const int32_t *counts;
} DanTreeAttnArgs;

#define DAN_TREE_ATTN_PHASES_ALL 0
#define DAN_TREE_ATTN_PHASE_PACK 1
#define DAN_TREE_ATTN_PHASE_ATTEND 2

/* Fused tree-masked attention forward: out = softmax(scale * q k^T + mask) v
 * over every (query, visible key) pair of every segment, in one launch.
 * Replaces dan/attention.py:200-241 (attend -> _attend_varlen) on gfx950. */
int dan_tree_attn_fwd(const DanTreeAttnArgs *args, void *stream);

/* Bytes of workspace dan_tree_attn_fwd needs (0 for invalid arguments). */
int64_t dan_tree_attn_workspace_size(int32_t num_kv_heads, int32_t head_dim, int32_t vt_cols);

/* fp32 -> fp16 staging of q or k for fp32 callers: out = x * 2^-e in fp16,
 * *scale = 2^e, with e = 0 while max |x| lies in [2^-6, 2^15] and otherwise
 * chosen to bring it into (2^14, 2^15] (so values beyond fp16's range neither
 * overflow nor flush). Two launches on `stream`; `partial` is device scratch
 * of DAN_TREE_ATTN_STAGE_PARTIALS floats. Replaces the reference's fp32
 * inputs to attend (dan/attention.py:200) at full range: the matrix core has
 * no fp32 product, and a plain cast to fp16 overflows beyond 65504.
 * No reference counterpart as an entry point. */
#define DAN_TREE_ATTN_STAGE_PARTIALS 1024
typedef struct {
  int32_t abi_version;          /* DAN_TREE_ATTN_ABI_VERSION */
  int32_t d0, d1, d2;           /* shape; d2 a multiple of 4, contiguous */
  const float *x;               /* 16-byte aligned */
  int64_t stride0, stride1;     /* element strides of dims 0 and 1 (multiples of 4) */
  void *out;                    /* fp16 [d0][d1][d2], contiguous */
  float *scale;                 /* device fp32 scalar: receives 2^e */
  float *partial;               /* device scratch, DAN_TREE_ATTN_STAGE_PARTIALS floats */
} DanStageF16Args;

int dan_tree_attn_stage_f16(const DanStageF16Args *args, void *stream);

/* Capacity in bytes of the library's own V^T scratch (one per GPU). */
#define DAN_TREE_ATTN_SCRATCH_BYTES (32LL << 20)

/* dan_tree_attn_fwd without a workspace: the V^T copy goes to a scratch array
 * the library keeps in each GPU's memory for the life of the process, and the
 * call allocates nothing (no hipMalloc, no allocating library routine), so it
 * can be made where allocation is not allowed: under HIP graph capture, in a
 * fixed serving loop, or in a harness that forbids it. `workspace` and
 * `workspace_bytes` of *args are ignored. It fails with
 * DAN_ERR_UNSUPPORTED when dan_tree_attn_workspace_size() exceeds
 * DAN_TREE_ATTN_SCRATCH_BYTES. Every call on one GPU shares that GPU's
 * scratch: calls that overlap in time on one GPU (different streams) race,
 * and a DAN_TREE_ATTN_PHASE_ATTEND call reads what the last pack on that GPU
 * left there. No counterpart in the reference (dan allocates through torch);
 * it exists for callers that cannot allocate. */
int dan_tree_attn_fwd_noalloc(const DanTreeAttnArgs *args, void *stream);

/* Queries per work item the kernel expects for this head configuration
 * (the tile planner's counterpart of ReadLayout, dan/attention.py:155-172):
 * the tokens per wave (32 up to head_dim 128, 16 at 256) times the waves
 * per query head of a work group of 8 waves. Returns 0 for an unsupported
 * configuration. */
int dan_tree_attn_tile_q(int32_t num_heads, int32_t num_kv_heads, int32_t head_dim);

/* Head groups G of the schedule: kv heads times the query-head chunks one
 * work group covers: num_kv_heads * ceil(rep / 4), rep = num_heads /
 * num_kv_heads. Returns 0 for an unsupported configuration. */
int dan_tree_attn_head_groups(int32_t num_heads, int32_t num_kv_heads);

/* Thread-local description of the last failure on this thread ("" if none). */
const char *dan_tree_attn_last_error(void);

/* DAN_TREE_ATTN_ABI_VERSION of the loaded library. */
int dan_tree_attn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DAN_TREE_ATTN_H */
