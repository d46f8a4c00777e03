/*
 * dan_gdn.h -- C ABI of the gfx950 gated delta rule (Gated DeltaNet
 * recurrence) over packed runs.
 *
 * dan's hybrid models (dan/models/qwen3_5.py) run a Gated DeltaNet layer
 * over a packed tree batch in phases: trunk part 1, trunk part 2, then every
 * branch, each phase one call of
 *   dan/models/qwen3_5.py:136-158   delta_rule(q, k, v, g, beta, lengths, states)
 * over runs of consecutive packed rows, each run starting from its own state
 * (zeros, a prefix-cache state, or the trunk's final state for a branch) and
 * returning its final state (dan/models/qwen3_5.py:198-210). Per value head
 * and token, with q and k l2-normalized (eps 1e-6, fp32) and q scaled by
 * Dk^-1/2:
 *     S <- exp(g_t) S;   S <- S + k_t (beta_t (v_t - S^T k_t))^T;   o_t = S^T q_t
 * with the state S [Dk, Dv] in fp32; value head h reads key head h / (Hv / Hk).
 *
 * Conventions are those of dan_tree_attn.h: caller-owned device memory,
 * nothing allocated or kept, asynchronous on `stream`, 0 on success and a
 * DanStatus with dan_tree_attn_last_error() on failure.
 */
#ifndef DAN_GDN_H
#define DAN_GDN_H

#include <stdint.h>

#include "dan_tree_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define DAN_GDN_ABI_VERSION 1

typedef struct {
  int32_t abi_version; /* DAN_GDN_ABI_VERSION */
  int32_t dtype;       /* DanDtype of q, k, v and out: bf16 or f16 */
  int32_t num_k_heads; /* Hk */
  int32_t num_v_heads; /* Hv, a multiple of Hk */
  int32_t k_dim;       /* Dk: 128 */
  int32_t v_dim;       /* Dv: a multiple of 8, at most 256 */
  int32_t num_runs;    /* R */
  int32_t num_tokens;  /* N */
  /* Run r covers packed rows cu[r] .. cu[r + 1] - 1 (cu[0] = 0, non-decreasing). */
  const int32_t *cu;
  const void *q; int64_t q_stride_tok, q_stride_head; /* [N, Hk, Dk] */
  const void *k; int64_t k_stride_tok, k_stride_head; /* [N, Hk, Dk] */
  const void *v; int64_t v_stride_tok, v_stride_head; /* [N, Hv, Dv] */
  const float *g;    /* [N, Hv] log decay, row stride Hv */
  const float *beta; /* [N, Hv] write strength, row stride Hv */
  const float *states_in; /* [R, Hv, Dk, Dv] */
  float *states_out;      /* [R, Hv, Dk, Dv] (may equal states_in) */
  void *out; int64_t o_stride_tok, o_stride_head; /* [N, Hv, Dv] */
  /* Device scratch of at least dan_gdn_workspace_size(N, Hk) bytes, 16-byte
   * aligned: the per-token l2-norm factors of q and k. */
  void *workspace; int64_t workspace_bytes;
} DanGdnArgs;

/* The gated delta rule over every run, from states_in to states_out.
 * Replaces dan/models/qwen3_5.py:136-158 (delta_rule: fla's chunked or
 * recurrent kernel, or delta_rule_torch) on gfx950. */
int dan_gdn_fwd(const DanGdnArgs *args, void *stream);

int64_t dan_gdn_workspace_size(int32_t num_tokens, int32_t num_k_heads);

int dan_gdn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DAN_GDN_H */
