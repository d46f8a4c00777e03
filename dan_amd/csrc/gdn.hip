// Gated delta rule (Gated DeltaNet recurrence) over packed runs on gfx950
// (MI355X, CDNA4): dan/models/qwen3_5.py:136-158 (delta_rule), token by
// token in fp32 from each run's initial state.
//
// Two launches:
//   gdn_norms_kernel  one wave per (token, key head): 1 / sqrt(sum(x^2) + 1e-6)
//                     of q and of k (dan/models/qwen3_5.py:99-100), into the
//                     caller's workspace -- the reductions leave the
//                     sequential loop.
//   gdn_kernel        one wave per (run, value head, block of kCols = 8 state
//                     columns); lane kCols e + c owns rows kRows e ..
//                     kRows e + kRows - 1 (kRows = 16) of column c of the
//                     state S [Dk = 128, Dv], in registers, so every wave
//                     walks its run alone, without barriers. Per token:
//                       S <- exp(g) S;  u = r_k (S^T k)  (two chains of
//                       products, then the row blocks summed by VALU lane
//                       exchanges, sum_column);  S <- S + k (r_k beta (v - u))^T;
//                       o = (r_q Dk^-1/2) (S^T q); row block 0 writes o.
//                     q, k and v are loaded kAhead = 8 tokens ahead into a
//                     register FIFO, and g, beta and the norm factors once
//                     per 64 tokens (one token per lane, read back with
//                     readlane). All loads are unconditional (clamped to the
//                     run), so the compiler's waits stay per slot instead of
//                     draining every load in flight at each token.
// The recurrence is sequential in the tokens of a run; a run's output and
// final state do not depend on where a caller splits it into calls.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "dan_gdn.h"

namespace dan {
int fail(int status, const char *fmt, ...);  // tree_attn.hip: sets the thread's last-error message
extern thread_local char g_err[512];
}  // namespace dan

namespace dan_gdn {

// Workspace bytes of the norm factors [N][Hk][2], rounded to 256.
static int64_t norm_bytes(int32_t num_tokens, int32_t num_k_heads) {
  return ((int64_t)num_tokens * num_k_heads * 2 * 4 + 255) / 256 * 256;
}

constexpr int kDk = 128;
constexpr int kWavesPerGroup = 4;
constexpr int kAhead = 8;  // tokens loaded ahead (the FIFO depth)
constexpr int kCols = 8;                  // state columns per wave
constexpr int kRows = kDk * kCols / 64;   // state rows per lane
constexpr int kVecs = kRows / 8;          // 16-byte loads of q (and of k) per lane and token

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

#define DAN_GLOBAL __attribute__((address_space(1)))

template <typename T>
struct V;
template <>
struct V<__bf16> {
  typedef bf16x4 x4;
  typedef bf16x8 x8;
};
template <>
struct V<_Float16> {
  typedef f16x4 x4;
  typedef f16x8 x8;
};

template <typename T>
__device__ inline f32x4 cvt4(u32x2 raw) {
  return __builtin_convertvector(__builtin_bit_cast(typename V<T>::x4, raw), f32x4);
}
template <typename T>
__device__ inline f32x8 cvt8(u32x4 raw) {
  return __builtin_convertvector(__builtin_bit_cast(typename V<T>::x8, raw), f32x8);
}

struct Params {
  const int32_t *cu;
  const void *q, *k, *v;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh;
  const float *g, *beta, *s_in;
  float *s_out;
  void *o;
  float *norms;  // [N][Hk][2]: 1 / sqrt(sum q^2 + eps), 1 / sqrt(sum k^2 + eps)
  const int32_t *sidx;  // NULL or [R]: run r's entry of s_in (clamped to [0, nsin))
  int32_t N, Hk, Hv, Dv, R, cblocks, nsin;
};

// One wave per (token, key head): lanes 0-31 hold 4 values of q, 32-63 of k.
template <typename T>
__global__ __launch_bounds__(64 * kWavesPerGroup) void gdn_norms_kernel(const Params p) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * kWavesPerGroup + (threadIdx.x >> 6);
  if (item >= (int64_t)p.N * p.Hk) return;
  const int n = (int)(item / p.Hk), hk = (int)(item % p.Hk);
  const T *src = lane < 32 ? static_cast<const T *>(p.q) + (int64_t)n * p.q_st + (int64_t)hk * p.q_sh
                           : static_cast<const T *>(p.k) + (int64_t)n * p.k_st + (int64_t)hk * p.k_sh;
  const f32x4 x = cvt4<T>(*(const DAN_GLOBAL u32x2 *)(src + 4 * (lane & 31)));
  float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
#pragma unroll
  for (int m = 1; m <= 16; m <<= 1) ss += __shfl_xor(ss, m);
  if ((lane & 31) == 0) *(DAN_GLOBAL float *)(p.norms + item * 2 + (lane >> 5)) = 1.0f / sqrtf(ss + 1e-6f);
}

// Sum of x over the lanes l with the same l % kCols (one state column), in
// every lane, on the VALU: DPP rotations within each row of 16 lanes (by 4
// when four lanes of a row share a column, then by 8), then the row swap
// (v_permlane16_swap) and the half swap (v_permlane32_swap).
__device__ inline float sum_column(float x) {
  if (kCols == 4)
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x),
                                                               0x124, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x),
                                                             0x128, 0xf, 0xf, false));
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = __builtin_bit_cast(float, (uint32_t)r16[0]) + __builtin_bit_cast(float, (uint32_t)r16[1]);
  u = __builtin_bit_cast(uint32_t, x);
  const auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r32[0]) + __builtin_bit_cast(float, (uint32_t)r32[1]);
}

// One token's inputs, loaded ahead: the lane's kRows rows of q and of k, and v.
struct Slot {
  u32x4 q[kVecs], k[kVecs];
  float v;
};

__device__ inline float lane_value(float x, int j) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), j));
}

template <typename T>
__global__ __launch_bounds__(64 * kWavesPerGroup) void gdn_kernel(const Params p) {
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
  const int unit = blockIdx.x * kWavesPerGroup + wave;  // (run, head, column block), wave-uniform
  if (unit >= p.R * p.Hv * p.cblocks) return;           // whole waves only: no barrier follows
  const int cb = unit % p.cblocks, h = (unit / p.cblocks) % p.Hv, r = unit / (p.cblocks * p.Hv);
  const int hk = h / (p.Hv / p.Hk);
  const int re = lane / kCols, c = kCols * cb + lane % kCols;
  const int row0 = __builtin_amdgcn_readfirstlane(*(const DAN_GLOBAL int32_t *)(p.cu + r));
  const int len = __builtin_amdgcn_readfirstlane(*(const DAN_GLOBAL int32_t *)(p.cu + r + 1)) - row0;

  // state rows kRows re .. kRows re + kRows - 1 of column c
  const int64_t sbase = ((int64_t)r * p.Hv + h) * kDk * p.Dv + c;
  const int rin = p.sidx ? min(max(__builtin_amdgcn_readfirstlane(*(const DAN_GLOBAL int32_t *)(p.sidx + r)), 0), p.nsin - 1) : r;
  const int64_t sbase_in = ((int64_t)rin * p.Hv + h) * kDk * p.Dv + c;
  float s[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) s[i] = *(const DAN_GLOBAL float *)(p.s_in + sbase_in + (int64_t)(kRows * re + i) * p.Dv);

  const T *qh = static_cast<const T *>(p.q) + (int64_t)hk * p.q_sh;
  const T *kh = static_cast<const T *>(p.k) + (int64_t)hk * p.k_sh;
  const T *vh = static_cast<const T *>(p.v) + (int64_t)h * p.v_sh;
  auto load = [&](int t) __attribute__((always_inline)) {
    Slot sl;
    const int64_t row = row0 + t;
    const DAN_GLOBAL u32x4 *qs = (const DAN_GLOBAL u32x4 *)(qh + row * p.q_st + kRows * re);
    const DAN_GLOBAL u32x4 *ks = (const DAN_GLOBAL u32x4 *)(kh + row * p.k_st + kRows * re);
#pragma unroll
    for (int m = 0; m < kVecs; ++m) {
      sl.q[m] = qs[m];
      sl.k[m] = ks[m];
    }
    sl.v = (float)*(const DAN_GLOBAL T *)(vh + row * p.v_st + c);
    return sl;
  };
  // The scalars of 64 tokens from t0, one token per lane (clamped to the
  // run's last token): g, beta, 1/|q|, 1/|k|.
  auto load_gates = [&](int t0, int last, f32x4 &gv) __attribute__((always_inline)) {
    const int64_t row = row0 + min(t0 + lane, last);
    gv[0] = *(const DAN_GLOBAL float *)(p.g + row * p.Hv + h);
    gv[1] = *(const DAN_GLOBAL float *)(p.beta + row * p.Hv + h);
    const f32x2 nr = *(const DAN_GLOBAL f32x2 *)(p.norms + (row * p.Hk + hk) * 2);
    gv[2] = nr[0];
    gv[3] = nr[1];
  };
  T *oh = static_cast<T *>(p.o) + (int64_t)h * p.o_sh + c;
  const float qscale = 0.08838834764831845f;  // Dk^-1/2 (dan/models/qwen3_5.py:110)

  // The norm factors multiply the reduced sums, not the 32 elements:
  // u = r_k (S^T k), the write is k (r_k w)^T, o = (r_q Dk^-1/2) (S^T q).
  auto step = [&](int t, const Slot &sl, const f32x4 &gv) __attribute__((always_inline)) {
    const int j = t & 63;
    const float a = expf(lane_value(gv[0], j));
    const float beta = lane_value(gv[1], j), rq = lane_value(gv[2], j), rk = lane_value(gv[3], j);
    float kv[kRows], qv[kRows];
#pragma unroll
    for (int m = 0; m < kVecs; ++m) {
      const f32x8 x = cvt8<T>(sl.k[m]);
#pragma unroll
      for (int e = 0; e < 8; ++e) kv[8 * m + e] = x[e];
    }
    float u0 = 0.f, u1 = 0.f;  // two product chains
#pragma unroll
    for (int i = 0; i < kRows; i += 2) {
      s[i] *= a;
      s[i + 1] *= a;
      u0 = fmaf(kv[i], s[i], u0);
      u1 = fmaf(kv[i + 1], s[i + 1], u1);
    }
    const float u = sum_column(u0 + u1) * rk;
    const float w = (beta * (sl.v - u)) * rk;
#pragma unroll
    for (int m = 0; m < kVecs; ++m) {
      const f32x8 x = cvt8<T>(sl.q[m]);
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[8 * m + e] = x[e];
    }
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int i = 0; i < kRows; i += 2) {
      s[i] = fmaf(kv[i], w, s[i]);
      s[i + 1] = fmaf(kv[i + 1], w, s[i + 1]);
      o0 = fmaf(qv[i], s[i], o0);
      o1 = fmaf(qv[i + 1], s[i + 1], o1);
    }
    const float o = sum_column(o0 + o1) * (rq * qscale);
    if (re == 0) *(DAN_GLOBAL T *)(oh + (int64_t)(row0 + t) * p.o_st) = (T)o;
  };

  // Every load below is unconditional, with its token clamped to the run:
  // loads under a branch make the compiler wait for all memory operations
  // in flight at the join, which would serialize the loads ahead with the
  // step. A full block of kAhead tokens needs no guard; the last tokens
  // (fewer than kAhead) are the epilogue.
  if (len > 0) {
    const int last = len - 1;
    Slot f[kAhead];
#pragma unroll
    for (int j = 0; j < kAhead; ++j) f[j] = load(min(j, last));
    f32x4 gcur = {0.f, 0.f, 0.f, 0.f}, gnext = {0.f, 0.f, 0.f, 0.f};
    load_gates(0, last, gcur);
    load_gates(64, last, gnext);
    int t = 0;
    for (;;) {  // blocks of 64 tokens, each with its gate vector
      // gcur must be in registers before the token loop: a wait for it at the
      // loop header would run on every iteration and drain the loads ahead.
      asm volatile("" ::"v"(gcur[0]), "v"(gcur[1]), "v"(gcur[2]), "v"(gcur[3]));
      int k = 0;
      for (; k < 64 / kAhead && t + kAhead <= len; ++k, t += kAhead) {
#pragma unroll
        for (int j = 0; j < kAhead; ++j) {
          step(t + j, f[j], gcur);
          f[j] = load(min(t + j + kAhead, last));
        }
      }
      if (k < 64 / kAhead) break;  // fewer than kAhead tokens left, in gcur's block
      gcur = gnext;
      load_gates(t + 64, last, gnext);
    }
#pragma unroll
    for (int j = 0; j < kAhead - 1; ++j)
      if (t + j < len) step(t + j, f[j], gcur);
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) *(DAN_GLOBAL float *)(p.s_out + sbase + (int64_t)(kRows * re + i) * p.Dv) = s[i];
}

hipError_t launch_norms(const DanGdnArgs *a, float *norms, hipStream_t s) {
  Params p{};
  p.q = a->q; p.k = a->k; p.q_st = a->q_stride_tok; p.q_sh = a->q_stride_head;
  p.k_st = a->k_stride_tok; p.k_sh = a->k_stride_head;
  p.N = a->num_tokens; p.Hk = a->num_k_heads; p.norms = norms;
  const int64_t ngrid = ((int64_t)a->num_tokens * a->num_k_heads + kWavesPerGroup - 1) / kWavesPerGroup;
  if (ngrid == 0) return hipSuccess;
  const dim3 block(64 * kWavesPerGroup);
  if (a->dtype == DAN_DTYPE_BF16) hipLaunchKernelGGL(gdn_norms_kernel<__bf16>, dim3((unsigned)ngrid), block, 0, s, p);
  else hipLaunchKernelGGL(gdn_norms_kernel<_Float16>, dim3((unsigned)ngrid), block, 0, s, p);
  return hipGetLastError();
}

}  // namespace dan_gdn

// gdn_chunk.hip: the chunked form.
int64_t dan_gdn_chunk_record_bytes(int32_t num_tokens, int32_t num_runs, int32_t num_v_heads);
hipError_t dan_gdn_fwd_chunked(const DanGdnArgs *a, float *records, hipStream_t s);

extern "C" {

int dan_gdn_abi_version(void) { return DAN_GDN_ABI_VERSION; }

int64_t dan_gdn_workspace_size(int32_t form, int32_t num_tokens, int32_t num_runs, int32_t num_k_heads,
                               int32_t num_v_heads, int32_t v_dim) {
  if (num_tokens < 0 || num_runs < 0 || num_k_heads <= 0 || num_v_heads <= 0 || v_dim <= 0) return 0;
  const int64_t norms = dan_gdn::norm_bytes(num_tokens, num_k_heads);
  if (form == DAN_GDN_FORM_TOKEN) return norms;
  if (form == DAN_GDN_FORM_CHUNK) return dan_gdn_chunk_record_bytes(num_tokens, num_runs, num_v_heads);
  return 0;
}

int dan_gdn_fwd(const DanGdnArgs *a, void *stream) {
  using dan::fail;
  dan::g_err[0] = 0;
  if (!a) return fail(DAN_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != DAN_GDN_ABI_VERSION)
    return fail(DAN_ERR_VERSION, "abi_version %d, delta rule speaks %d", a->abi_version, DAN_GDN_ABI_VERSION);
  if (a->dtype != DAN_DTYPE_BF16 && a->dtype != DAN_DTYPE_F16) return fail(DAN_ERR_UNSUPPORTED, "dtype %d: bf16 or f16", a->dtype);
  if (a->k_dim != 128) return fail(DAN_ERR_UNSUPPORTED, "k_dim %d: only 128 is built", a->k_dim);
  if (a->v_dim <= 0 || a->v_dim % 8 || a->v_dim > 256) return fail(DAN_ERR_UNSUPPORTED, "v_dim %d: a multiple of 8 up to 256", a->v_dim);
  if (a->num_k_heads <= 0 || a->num_v_heads <= 0 || a->num_v_heads % a->num_k_heads)
    return fail(DAN_ERR_INVALID_ARGUMENT, "num_v_heads %d must be a positive multiple of num_k_heads %d", a->num_v_heads,
                a->num_k_heads);
  if (a->num_runs < 0 || a->num_tokens < 0) return fail(DAN_ERR_INVALID_ARGUMENT, "negative run or token count");
  if (a->num_runs == 0) return DAN_OK;
  if (!a->cu || !a->q || !a->k || !a->v || !a->g || !a->beta || !a->states_in || !a->states_out || !a->out ||
      !a->workspace)
    return fail(DAN_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (((uintptr_t)a->q & 15) || ((uintptr_t)a->k & 15) || (a->q_stride_tok % 8) || (a->q_stride_head % 8) ||
      (a->k_stride_tok % 8) || (a->k_stride_head % 8))
    return fail(DAN_ERR_INVALID_ARGUMENT, "q and k rows must be 16-byte aligned");
  if (a->form != DAN_GDN_FORM_TOKEN && a->form != DAN_GDN_FORM_CHUNK) return fail(DAN_ERR_INVALID_ARGUMENT, "form %d", a->form);
  if (a->state_index && a->num_states_in <= 0)
    return fail(DAN_ERR_INVALID_ARGUMENT, "state_index needs num_states_in > 0, got %d", a->num_states_in);
  if (a->form == DAN_GDN_FORM_CHUNK && a->v_dim % 32)
    return fail(DAN_ERR_UNSUPPORTED, "v_dim %d: the chunked form takes a multiple of 32", a->v_dim);
  const int64_t need =
      dan_gdn_workspace_size(a->form, a->num_tokens, a->num_runs, a->num_k_heads, a->num_v_heads, a->v_dim);
  if (a->workspace_bytes < need || ((uintptr_t)a->workspace & 15))
    return fail(DAN_ERR_INVALID_ARGUMENT, "workspace needs %lld bytes, 16-byte aligned", (long long)need);
  if ((int64_t)a->num_tokens * a->num_k_heads > 0x7fffffffLL * dan_gdn::kWavesPerGroup)
    return fail(DAN_ERR_INVALID_ARGUMENT, "too many tokens x heads");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float *norms = static_cast<float *>(a->workspace);
  if (a->form == DAN_GDN_FORM_CHUNK) {
    if (((int64_t)a->num_runs + a->num_tokens / DAN_GDN_CHUNK) * a->num_v_heads > 0x7fffffff ||
        ((int64_t)a->num_runs * a->num_v_heads + 7) / 8 * 8 * (a->v_dim / 32) > 0x7fffffff)
      return fail(DAN_ERR_INVALID_ARGUMENT, "too many chunks or runs x heads");
    const hipError_t err = dan_gdn_fwd_chunked(a, static_cast<float *>(a->workspace), s);
    if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "delta rule launch failed: %s", hipGetErrorString(err));
    return DAN_OK;
  }
  const int64_t units = (int64_t)a->num_runs * a->num_v_heads * (a->v_dim / dan_gdn::kCols);
  const int64_t grid = (units + dan_gdn::kWavesPerGroup - 1) / dan_gdn::kWavesPerGroup;
  if (grid > 0x7fffffff) return fail(DAN_ERR_INVALID_ARGUMENT, "too many runs x heads");
  dan_gdn::Params p;
  p.cu = a->cu; p.q = a->q; p.k = a->k; p.v = a->v;
  p.q_st = a->q_stride_tok; p.q_sh = a->q_stride_head; p.k_st = a->k_stride_tok; p.k_sh = a->k_stride_head;
  p.v_st = a->v_stride_tok; p.v_sh = a->v_stride_head; p.o_st = a->o_stride_tok; p.o_sh = a->o_stride_head;
  p.g = a->g; p.beta = a->beta; p.s_in = a->states_in; p.s_out = a->states_out; p.o = a->out;
  p.Hk = a->num_k_heads; p.Hv = a->num_v_heads; p.Dv = a->v_dim; p.R = a->num_runs;
  p.cblocks = a->v_dim / dan_gdn::kCols; p.N = a->num_tokens; p.norms = norms;
  p.sidx = a->state_index; p.nsin = a->num_states_in;
  hipError_t err = dan_gdn::launch_norms(a, norms, s);
  if (err == hipSuccess) {
    const dim3 block(64 * dan_gdn::kWavesPerGroup);
    if (a->dtype == DAN_DTYPE_BF16) hipLaunchKernelGGL(dan_gdn::gdn_kernel<__bf16>, dim3((unsigned)grid), block, 0, s, p);
    else hipLaunchKernelGGL(dan_gdn::gdn_kernel<_Float16>, dim3((unsigned)grid), block, 0, s, p);
    err = hipGetLastError();
  }
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "delta rule launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}

}  // extern "C"
