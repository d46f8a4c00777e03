/*
 * dan_tree_plan.h -- C ABI of the device-side tile planner for the gfx950
 * tree-masked prefill attention (dan_tree_attn.h).
 *
 * Once per packed forward, dan turns its Segment list into the index layout
 * the attention calls read:
 *   dan/runner.py:38-64        Runner.pack -> segment() per request
 *   dan/attention.py:98-126    segment(): per-token branch structure
 *   dan/attention.py:138-172   ReadLayout.build: trunk / branch row lists and
 *                              cumulative lengths for the varlen calls
 *   dan/attention.py:211-215   the layout cached on the Batch for all layers
 * In dan this runs on the host in Python every forward. Here the host keeps
 * only O(segments) work -- each segment's first V^T column, first work item
 * and first branch, one upload -- and one launch of dan_tree_attn_plan builds
 * on the device, on the caller's stream, every table dan_tree_attn_fwd reads:
 *   key_lo [N]                 per token, the first key of its own branch
 *   col_seg [C]                the segment owning each V^T column block
 *   work [W], cost [W]         query tiles, longest first (ties: first made)
 *   units [W * G], sched_off   the persistent schedule: longest-processing-
 *                              time dealing over the slots of each head group,
 *                              then single moves and pairwise swaps out of the
 *                              most loaded slot while they lower the larger
 *                              load of the pair
 * The tables equal those of the host planner (dan_amd/plan.py) for key_lo,
 * col_seg, work and cost; the schedule is a valid one of the same kind (every
 * unit once, slot s only head group s % G, each slot's units longest first).
 *
 * Conventions are those of dan_tree_attn.h: caller-owned device memory,
 * nothing allocated or kept, asynchronous on `stream`, 0 on success and a
 * DanStatus with dan_tree_attn_last_error() on failure.
 */
#ifndef DAN_TREE_PLAN_H
#define DAN_TREE_PLAN_H

#include <stdint.h>

#include "dan_tree_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define DAN_TREE_PLAN_ABI_VERSION 2

/* Largest work list, slot count, segment count and branch count one planner
 * launch handles (its tables, sort and schedule live in one work group's
 * LDS). */
#define DAN_TREE_PLAN_MAX_WORK 4096
#define DAN_TREE_PLAN_MAX_SLOTS 256
#define DAN_TREE_PLAN_MAX_SEGMENTS 1024
#define DAN_TREE_PLAN_MAX_BRANCHES 4096

typedef struct {
  int32_t abi_version;  /* DAN_TREE_PLAN_ABI_VERSION */
  int32_t num_tokens;   /* N */
  int32_t num_segments; /* S */
  int32_t num_branches; /* B: total branches over all segments */
  int32_t num_work;     /* W = sum over segments of ceil(n / tile_q) */
  int32_t num_cols;     /* C = sum over segments of ceil((past_len + n) / 64) */
  int32_t tile_q;       /* dan_tree_attn_tile_q(H, Hkv) */
  int32_t groups;       /* G = dan_tree_attn_head_groups(H, Hkv) */
  int32_t num_cus;      /* slots per head group: k = max(1, min(num_cus / G, W)) */
  int32_t overhead;     /* schedule cost of an item: its key tiles + overhead */
  /* [S] in packed order. Besides the fields dan_tree_attn_fwd reads
   * (start, n, trunk, past_len, past_idx, vt_col), reserved[0] is the
   * segment's first work item (prefix sum of ceil(n / tile_q)) and
   * reserved[1] its first entry in branch_starts. */
  const DanSegmentDesc *segments;
  /* [B] packed row of each branch's first token, segment by segment in
   * order; a segment's branches are contiguous after its trunk and the last
   * one ends at start + n. */
  const int32_t *branch_starts;
  int32_t *key_lo;     /* out [N] (rows outside every segment: 0) */
  int32_t *col_seg;    /* out [C] */
  DanWorkItem *work;   /* out [W] */
  int32_t *cost;       /* out [W] */
  DanUnit *units;      /* out [W * G] */
  int32_t *sched_off;  /* out [k * G + 1] */
  /* Budget mode (NULL otherwise): device int32 {S, B, W, C} of this batch. The
   * counts above are then capacities (what the tables hold; the device counts
   * are clamped to them), the slots per head group are k = max(1, min(num_cus
   * / G, W)) with W the device count, and sched_off has kcap * G + 1 entries
   * for kcap = dan_tree_attn_plan_slots(capacity W, G, num_cus) / G: the
   * slots beyond k * G are empty. So a graph captured over one batch's
   * launches serves any batch within the capacities after one upload of its
   * header and one planner launch. */
  const int32_t *counts;
} DanTreePlanArgs;

/* Build the attention tables of one packed forward on the device.
 * Replaces dan/attention.py:138-172 (ReadLayout.build) and the host planner's
 * work list and schedule. */
int dan_tree_attn_plan(const DanTreePlanArgs *args, void *stream);

/* Slots of the schedule dan_tree_attn_plan writes: k * G (0 if invalid). */
int dan_tree_attn_plan_slots(int32_t num_work, int32_t groups, int32_t num_cus);

int dan_tree_attn_plan_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DAN_TREE_PLAN_H */
