/*
 * dan_qkv_front.h -- C ABI of the gfx950 attention front end.
 *
 * One pass over the projected q and k of a packed token sequence:
 * optional per-head RMSNorm, rotary position embedding (rotate-half) on the
 * first `rotary_dim` dims of every head, and q, k written token-major in the
 * layout the tree-attention kernel reads ([N, H, D] / [N, Hkv, D], unit
 * stride D). In the same pass, the prefix-cache rows of saving segments are
 * copied out (k after the norm and rotation, v as is).
 *
 * This header replaces, as one launch, the GPU leg of
 *   dan/models/llama.py:78-86       qkv split, reshape, q_norm / k_norm,
 *                                   rotate(q), rotate(k), transposes
 *   dan/models/qwen3_5.py:318-326   the same with zero-centered norms and a
 *                                   partial rotary (rotate_partial)
 *   dan/fused.py:36-48              rms_norm, rms_norm_zero_centered
 *   dan/fused.py:70-76              rotate_partial (llama.py:43-45 is the
 *                                   full-width case)
 *   dan/attention.py:202-204        the prefix-save clones of k and v
 * Numerics follow those eager torch ops: fp32 arithmetic with the result of
 * every op rounded to the storage type (round to nearest even).
 *
 * Conventions: as dan_tree_attn.h (device pointers owned by the caller,
 * strides in elements, unit-stride head_dim, status codes with a
 * thread-local message from dan_tree_attn_last_error(), asynchronous on
 * `stream`, nothing allocated or kept).
 */
#ifndef DAN_QKV_FRONT_H
#define DAN_QKV_FRONT_H

#include <stdint.h>

#include "dan_tree_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define DAN_QKV_FRONT_ABI_VERSION 1

typedef enum {
  DAN_FRONT_NORM_NONE = 0,
  DAN_FRONT_NORM_RMS = 1,          /* weight * dtype(x * rsqrt(mean(x^2) + eps)) -- fused.py:36-40 */
  DAN_FRONT_NORM_RMS_ZERO_CENTERED = 2 /* dtype(x * rsqrt(mean(x^2) + eps) * (1 + weight)) -- fused.py:43-48 */
} DanFrontNorm;

/* One saving segment (dan/attention.py:202-204): rows [start, start + len)
 * of the packed sequence are copied to k_dst and v_dst, each [Hkv, len, D]
 * contiguous. */
typedef struct {
  int32_t start;
  int32_t len;
  void *k_dst;
  void *v_dst;
} DanFrontSave;

typedef struct {
  int32_t abi_version;  /* DAN_QKV_FRONT_ABI_VERSION */
  int32_t dtype;        /* DanDtype of q, k, v, cos, sin, the norm weights and the outputs: bf16 or f16 */
  int32_t num_tokens;   /* N */
  int32_t num_heads;    /* H */
  int32_t num_kv_heads; /* Hkv */
  int32_t head_dim;     /* D: 64, 128 or 256 */
  int32_t rotary_dim;   /* R: rotate the first R dims of each head; 0 (no rotation) or a multiple of 16 <= D */
  int32_t norm;         /* DanFrontNorm, the same for q and k */
  float eps;

  const void *q; int64_t q_stride_tok, q_stride_head; /* [N, H, D] view (e.g. of the fused qkv output) */
  const void *k; int64_t k_stride_tok, k_stride_head; /* [N, Hkv, D] view */
  const void *v; int64_t v_stride_tok, v_stride_head; /* [N, Hkv, D] view: read for the saves only */
  const void *cos; const void *sin; int64_t cs_stride_tok; /* [N, R] each, cs_stride_tok >= R */
  const void *q_norm_weight; /* [D], NULL when norm is NONE */
  const void *k_norm_weight; /* [D] */

  void *q_out; int64_t qo_stride_tok, qo_stride_head; /* [N, H, D] */
  void *k_out; int64_t ko_stride_tok, ko_stride_head; /* [N, Hkv, D] */

  /* Saves: save_of[t] is the index into `saves` of the segment whose saved
   * rows hold token t, or -1. Both NULL / 0 when nothing is saved. */
  const int32_t *save_of;
  const DanFrontSave *saves;
  int32_t num_saves;
} DanQkvFrontArgs;

/* q_out, k_out (and the saves) from q, k, v in one launch. Replaces the GPU
 * leg of dan/models/llama.py:78-86 and dan/models/qwen3_5.py:318-326 up to
 * the attend() call, and the clones of dan/attention.py:202-204. */
int dan_qkv_front(const DanQkvFrontArgs *args, void *stream);

/* DAN_QKV_FRONT_ABI_VERSION of the loaded library. */
int dan_qkv_front_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DAN_QKV_FRONT_H */
