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

#define DAN_GDN_ABI_VERSION 4

/* Tokens per chunk of the chunked form. */
#define DAN_GDN_CHUNK 64
/* For fp16 inputs the chunked form walks calls whose runs average at most
 * this many tokens with a scan tuned for many short runs, other calls with
 * one tuned for the latency of long runs (same results). bf16 inputs take
 * the bf16-pair scan either way. */
#define DAN_GDN_SHORT_RUN 256

/* How dan_gdn_fwd walks a run. Both give the same recurrence within fp32
 * rounding: the token form steps token by token (a run's results do not
 * depend on how a caller splits it into calls); the chunked form steps 64
 * tokens at a time on the matrix cores, the form of the reference's own
 * CPU path (dan/models/qwen3_5.py:103-133, delta_rule_torch), and is the
 * faster one once runs are longer than a few chunks. */
typedef enum { DAN_GDN_FORM_TOKEN = 0, DAN_GDN_FORM_CHUNK = 1 } DanGdnForm;

typedef struct {
  int32_t abi_version; /* DAN_GDN_ABI_VERSION */
  int32_t dtype;       /* DanDtype of q, k, v and out: bf16 or f16 */
  int32_t num_k_heads; /* Hk */
  int32_t num_v_heads; /* Hv, a multiple of Hk */
  int32_t k_dim;       /* Dk: 128 */
  int32_t v_dim;       /* Dv: a multiple of 8 (of 32 for the chunked form), at most 256 */
  int32_t num_runs;    /* R */
  int32_t num_tokens;  /* N */
  /* Run r covers packed rows cu[r] .. cu[r + 1] - 1 (cu[0] = 0, non-decreasing). */
  const int32_t *cu;
  const void *q; int64_t q_stride_tok, q_stride_head; /* [N, Hk, Dk] */
  const void *k; int64_t k_stride_tok, k_stride_head; /* [N, Hk, Dk] */
  const void *v; int64_t v_stride_tok, v_stride_head; /* [N, Hv, Dv] */
  const float *g;    /* [N, Hv] log decay, row stride Hv */
  const float *beta; /* [N, Hv] write strength, row stride Hv */
  const float *states_in; /* [R, Hv, Dk, Dv] ([num_states_in, ...] with state_index) */
  float *states_out;      /* [R, Hv, Dk, Dv] (may equal states_in) */
  void *out; int64_t o_stride_tok, o_stride_head; /* [N, Hv, Dv] */
  /* Device scratch of at least dan_gdn_workspace_size(form, N, R, Hk, Hv, Dv)
   * bytes, 16-byte aligned: the token form's per-token l2-norm factors of q
   * and k, or the chunked form's per-chunk factors. */
  void *workspace; int64_t workspace_bytes;
  int32_t form;     /* DanGdnForm */
  int32_t reserved; /* 0 */
  /* (GDN ABI 4) NULL, or [R] int32 on the device: run r starts from
   * states_in[state_index[r]] of num_states_in entries (an index outside
   * [0, num_states_in) is clamped), the gather of dan/models/qwen3_5.py:204
   * and :211 done in the state load; states_out must not overlap states_in. */
  const int32_t *state_index;
  int32_t num_states_in;
  int32_t reserved2; /* 0 */
} DanGdnArgs;

/* The gated delta rule over every run, from states_in to states_out.
 * Replaces dan/models/qwen3_5.py:136-158 (delta_rule: fla's chunked or
 * recurrent kernel, or delta_rule_torch) on gfx950. */
int dan_gdn_fwd(const DanGdnArgs *args, void *stream);

/* Workspace bytes for dan_gdn_fwd; 0 for arguments it would reject. The
 * token form's grows as 8 N Hk bytes, the chunked form's as
 * (R + N / 64) Hv 49.25 KiB. */
int64_t dan_gdn_workspace_size(int32_t form, int32_t num_tokens, int32_t num_runs, int32_t num_k_heads,
                               int32_t num_v_heads, int32_t v_dim);

/* The input side of one DeltaNet phase, dan/models/qwen3_5.py:212-220
 * (DeltaNet._phase up to the delta rule) with the gates of
 * dan/fused.py:80-82 (delta_gates):
 *   out[i] = silu(conv_i),  conv_i[c] = sum_j weight[c][j] * X(ext[take[i] + j])[c]
 * over j < K, rounded to dtype before the silu (the reference's conv1d output),
 *   beta[i][h] = sigmoid(b[rows[i]][h]) rounded to dtype, then widened to fp32
 *   g[i][h] = -exp(a_log[h]) * softplus(a[rows[i]][h] + dt_bias[h])   (fp32)
 * X(e) is a virtual source row: packed row e of src for e < N, zeros for
 * e == N, hist row e - N - 1 above (the reference gathers from the same
 * virtual source built with torch.cat, dan/models/qwen3_5.py:191-193; here
 * the packed rows are read in place and only the cached histories are a
 * separate buffer). Indices outside these ranges read as the zero row and a
 * row index outside [0, N) gives beta = g = 0: the kernels never read out of
 * bounds. */
typedef struct {
  int32_t abi_version;   /* DAN_GDN_ABI_VERSION */
  int32_t dtype;         /* DanDtype of src, hist, weight, out, b and a: bf16 or f16 */
  int32_t channels;      /* C, the conv width (2 Hk Dk + Hv Dv), a multiple of 8 */
  int32_t kernel;        /* K, 2 to 4 */
  int32_t num_rows;      /* N: packed rows */
  int32_t num_hist_rows; /* rows of hist */
  int32_t num_ext;       /* entries of ext */
  int32_t num_out;       /* T: output rows */
  const void *src; int64_t src_stride;  /* [N, C], row stride in elements (a column slice of the projection) */
  const void *hist;                     /* [num_hist_rows, C] contiguous */
  const int32_t *ext;                   /* [num_ext] virtual source rows */
  const int32_t *take;                  /* [T] first ext entry of output row i's window */
  const void *weight;                   /* [C, K] (nn.Conv1d's [C, 1, K]), 16-byte aligned */
  void *out; int64_t out_stride;        /* [T, C] */
  int32_t num_heads;                    /* Hv; 0 skips the gates */
  int32_t reserved;
  const int32_t *rows;                  /* [T] packed row of output row i */
  const void *b; int64_t b_stride;      /* [N, Hv] */
  const void *a; int64_t a_stride;      /* [N, Hv] */
  const float *a_log;                   /* [Hv] */
  const float *dt_bias;                 /* [Hv] */
  float *beta;                          /* [T, Hv] */
  float *g;                             /* [T, Hv] */
} DanGdnConvArgs;

/* Causal depthwise conv + silu over gathered windows, and the gates, for the
 * rows of one phase. Replaces dan/models/qwen3_5.py:191-193 (the source
 * concatenation), :216-218 (index_select, conv1d, silu, index_select) and
 * the gathers of g and beta at :223, with dan/fused.py:80-82. */
int dan_gdn_conv(const DanGdnConvArgs *args, void *stream);

int dan_gdn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DAN_GDN_H */
