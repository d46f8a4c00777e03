// The input side of one Gated DeltaNet phase on gfx950 (MI355X, CDNA4):
// dan/models/qwen3_5.py:212-220 (DeltaNet._phase up to the delta rule) and
// dan/fused.py:80-82 (delta_gates).
//
// Two launches, both HBM-bound streaming work:
//   gdn_conv_kernel   one thread per (strip of kStrip output rows, 8 channels).
//                     Consecutive threads take consecutive 16-byte channel
//                     groups of the same rows, so every row load is coalesced.
//                     A strip's window starts, ext entries and rows are each
//                     loaded as one batch (all in flight), not one memory
//                     round trip per row. Along a strip the K-row window
//                     slides: output row i + 1 of a run starts one ext entry
//                     after row i, so one new row is loaded per output row
//                     and a full window only at a run boundary. Sum in fp32 (j = 0 .. K-1, fused
//                     multiply-adds), rounded to the I/O type as the
//                     reference's conv1d output is, then silu in fp32 (hardware
//                     exp2 and reciprocal: the kernel is otherwise VALU-bound
//                     on a full-precision exp and divide).
//   gdn_gates_kernel  one thread per (output row, head): beta and g.
// The packed projection rows are read in place through the virtual row index
// (no concatenated copy of the source).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "dan_gdn.h"

namespace dan {
int fail(int status, const char *fmt, ...);  // tree_attn.hip: sets the thread's last-error message
extern thread_local char g_err[512];
}  // namespace dan

namespace dan_conv {

constexpr int kStrip = 8;  // output rows per thread (16 held too many loads' registers: 2 waves per SIMD)
constexpr int kBlock = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

#define DAN_GLOBAL __attribute__((address_space(1)))

template <typename T>
struct V;
template <>
struct V<__bf16> {
  typedef bf16x8 x8;
};
template <>
struct V<_Float16> {
  typedef f16x8 x8;
};

template <typename T>
__device__ inline f32x8 cvt8(u32x4 raw) {
  return __builtin_convertvector(__builtin_bit_cast(typename V<T>::x8, raw), f32x8);
}
template <typename T>
__device__ inline u32x4 pack8(f32x8 x) {
  return __builtin_bit_cast(u32x4, __builtin_convertvector(x, typename V<T>::x8));
}

struct Params {
  const void *src, *hist, *weight, *b, *a;
  const int32_t *ext, *take, *rows;
  const float *a_log, *dt_bias;
  void *out;
  float *beta, *g;
  int64_t src_stride, out_stride, b_stride, a_stride;
  int32_t C, N, hist_rows, num_ext, T, Hv, groups;  // groups = C / 8
};

// 8 channels of virtual source row e (zeros outside the packed and history rows).
template <typename T>
__device__ inline f32x8 load_row(const Params &p, int e, int cg) {
  const T *row = nullptr;
  if (e >= 0 && e < p.N)
    row = static_cast<const T *>(p.src) + (int64_t)e * p.src_stride;
  else if (e > p.N && e - p.N - 1 < p.hist_rows)
    row = static_cast<const T *>(p.hist) + (int64_t)(e - p.N - 1) * p.C;
  if (!row) return f32x8{0, 0, 0, 0, 0, 0, 0, 0};
  return cvt8<T>(*(const DAN_GLOBAL u32x4 *)(row + 8 * cg));
}

template <typename T, int K>
__global__ __launch_bounds__(kBlock) void gdn_conv_kernel(const Params p) {
  const int64_t gid = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int cg = (int)(gid % p.groups);
  const int64_t i0 = gid / p.groups * kStrip;
  if (i0 >= p.T) return;
  const int nr = (int)min((int64_t)p.T - i0, (int64_t)kStrip);  // output rows of this strip
  f32x8 w[K];
  const T *wp = static_cast<const T *>(p.weight) + (int64_t)cg * 8 * K;
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int j = 0; j < K; ++j) w[j][c] = (float)wp[c * K + j];
  T *out = static_cast<T *>(p.out) + i0 * p.out_stride + 8 * cg;
  auto emit = [&](int r, const f32x8(&x)[K]) __attribute__((always_inline)) {
    f32x8 y;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float acc = w[0][c] * x[0][c];
#pragma unroll
      for (int j = 1; j < K; ++j) acc = fmaf(w[j][c], x[j][c], acc);
      const float r = (float)(T)acc;  // the conv output in the I/O type
      // silu(r) = r / (1 + e^-r) with the hardware exp2 and reciprocal (about
      // one fp32 ulp each, far below the output type's spacing)
      y[c] = r * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(r * -1.4426950408889634f));
    }
    *(DAN_GLOBAL u32x4 *)(out + (int64_t)r * p.out_stride) = pack8<T>(y);
  };
  // With no source row or too few ext entries every window reads as zeros.
  if (!((p.N > 0 || p.hist_rows > 0) && p.num_ext >= K)) {
    f32x8 x[K];
#pragma unroll
    for (int j = 0; j < K; ++j) x[j] = f32x8{0, 0, 0, 0, 0, 0, 0, 0};
    for (int r = 0; r < nr; ++r) emit(r, x);
    return;
  }
  // Virtual source row e: a packed row, a history row, or zeros. Every load is
  // issued unconditionally -- a zero row reads a row that exists (packed row
  // 0, else history row 0) and is masked -- so a strip's loads are in flight
  // together instead of one memory round trip per branch.
  const T *src = static_cast<const T *>(p.src), *hist = static_cast<const T *>(p.hist);
  const T *stand = p.N > 0 ? src : hist;
  auto row_at = [&](int e, bool &ok) __attribute__((always_inline)) {
    const bool in_src = e >= 0 && e < p.N, in_hist = e > p.N && e - p.N - 1 < p.hist_rows;
    ok = in_src || in_hist;
    const T *row = in_src ? src + (int64_t)e * p.src_stride : in_hist ? hist + (int64_t)(e - p.N - 1) * p.C : stand;
    return *(const DAN_GLOBAL u32x4 *)(row + 8 * cg);
  };
  // 1. The strip's window starts (rows past the strip repeat its last row and
  //    are not stored). A start outside [0, num_ext - K] reads as zeros.
  int t[kStrip];
  bool tv[kStrip];
#pragma unroll
  for (int r = 0; r < kStrip; ++r) t[r] = p.take[i0 + min(r, nr - 1)];
#pragma unroll
  for (int r = 0; r < kStrip; ++r) {
    tv[r] = t[r] >= 0 && t[r] <= p.num_ext - K;
    t[r] = tv[r] ? t[r] : 0;
  }
  // 2. Each row's newest window entry, and the first row's older ones.
  int en[kStrip], ep[K - 1];
#pragma unroll
  for (int r = 0; r < kStrip; ++r) en[r] = p.ext[t[r] + K - 1];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) ep[j] = p.ext[t[0] + j];
  // 3. Their rows.
  u32x4 rn[kStrip], rp[K - 1];
  bool okn[kStrip], okp[K - 1];
#pragma unroll
  for (int r = 0; r < kStrip; ++r) rn[r] = row_at(en[r], okn[r]);
#pragma unroll
  for (int j = 0; j < K - 1; ++j) rp[j] = row_at(ep[j], okp[j]);
  const f32x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
  // 4. The outputs. Along a run the window slides one entry per output row;
  //    at a run boundary (rare) the row's older entries are loaded then.
  f32x8 x[K];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) x[j] = tv[0] && okp[j] ? cvt8<T>(rp[j]) : zero;
  x[K - 1] = tv[0] && okn[0] ? cvt8<T>(rn[0]) : zero;
  emit(0, x);
#pragma unroll
  for (int r = 1; r < kStrip; ++r) {
    // (rows past nr repeat the strip's last row: computed, not stored)
    if (tv[r] && tv[r - 1] && t[r] == t[r - 1] + 1) {
#pragma unroll
      for (int j = 0; j < K - 1; ++j) x[j] = x[j + 1];
    } else {
#pragma unroll
      for (int j = 0; j < K - 1; ++j) {
        bool ok = false;
        const u32x4 raw = tv[r] ? row_at(p.ext[t[r] + j], ok) : u32x4{0, 0, 0, 0};
        x[j] = ok ? cvt8<T>(raw) : zero;
      }
    }
    x[K - 1] = tv[r] && okn[r] ? cvt8<T>(rn[r]) : zero;
    if (r < nr) emit(r, x);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void gdn_gates_kernel(const Params p) {
  const int64_t gid = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (gid >= (int64_t)p.T * p.Hv) return;
  const int i = (int)(gid / p.Hv), h = (int)(gid % p.Hv);
  const int r = p.rows[i];
  float beta = 0.0f, g = 0.0f;
  if (r >= 0 && r < p.N) {
    const float bb = (float)static_cast<const T *>(p.b)[(int64_t)r * p.b_stride + h];
    const float aa = (float)static_cast<const T *>(p.a)[(int64_t)r * p.a_stride + h];
    beta = (float)(T)(1.0f / (1.0f + expf(-bb)));
    const float z = aa + p.dt_bias[h];
    const float sp = z > 20.0f ? z : log1pf(expf(z));  // softplus, threshold 20
    g = -expf(p.a_log[h]) * sp;
  }
  p.beta[gid] = beta;
  p.g[gid] = g;
}

template <typename T, int K>
void launch_conv(const Params &p, int64_t grid, hipStream_t s) {
  hipLaunchKernelGGL((gdn_conv_kernel<T, K>), dim3((unsigned)grid), dim3(kBlock), 0, s, p);
}

template <typename T>
void launch(const Params &p, int K, int64_t grid, int64_t ggrid, hipStream_t s) {
  if (grid) {
    if (K == 2) launch_conv<T, 2>(p, grid, s);
    else if (K == 3) launch_conv<T, 3>(p, grid, s);
    else launch_conv<T, 4>(p, grid, s);
  }
  if (ggrid) hipLaunchKernelGGL(gdn_gates_kernel<T>, dim3((unsigned)ggrid), dim3(kBlock), 0, s, p);
}

}  // namespace dan_conv

extern "C" int dan_gdn_conv(const DanGdnConvArgs *a, void *stream) {
  using dan::fail;
  dan::g_err[0] = 0;
  if (!a) return fail(DAN_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != DAN_GDN_ABI_VERSION)
    return fail(DAN_ERR_VERSION, "abi_version %d, delta rule speaks %d", a->abi_version, DAN_GDN_ABI_VERSION);
  if (a->dtype != DAN_DTYPE_BF16 && a->dtype != DAN_DTYPE_F16) return fail(DAN_ERR_UNSUPPORTED, "dtype %d: bf16 or f16", a->dtype);
  if (a->kernel < 2 || a->kernel > 4) return fail(DAN_ERR_UNSUPPORTED, "kernel %d: 2 to 4", a->kernel);
  if (a->channels <= 0 || a->channels % 8) return fail(DAN_ERR_UNSUPPORTED, "channels %d: a positive multiple of 8", a->channels);
  if (a->num_rows < 0 || a->num_hist_rows < 0 || a->num_ext < 0 || a->num_out < 0 || a->num_heads < 0)
    return fail(DAN_ERR_INVALID_ARGUMENT, "negative count");
  if (a->num_out == 0) return DAN_OK;
  if (!a->ext || !a->take || !a->weight || !a->out || (a->num_rows && !a->src) || (a->num_hist_rows && !a->hist))
    return fail(DAN_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (((uintptr_t)a->src & 15) || ((uintptr_t)a->hist & 15) || ((uintptr_t)a->out & 15) || a->src_stride % 8 ||
      a->out_stride % 8 || a->src_stride < a->channels || a->out_stride < a->channels)
    return fail(DAN_ERR_INVALID_ARGUMENT, "src, hist and out rows must be 16-byte aligned and hold the channels");
  if (a->num_heads && (!a->rows || !a->b || !a->a || !a->a_log || !a->dt_bias || !a->beta || !a->g))
    return fail(DAN_ERR_INVALID_ARGUMENT, "NULL gate pointer");
  dan_conv::Params p;
  p.src = a->src; p.hist = a->hist; p.weight = a->weight; p.b = a->b; p.a = a->a;
  p.ext = a->ext; p.take = a->take; p.rows = a->rows; p.a_log = a->a_log; p.dt_bias = a->dt_bias;
  p.out = a->out; p.beta = a->beta; p.g = a->g;
  p.src_stride = a->src_stride; p.out_stride = a->out_stride; p.b_stride = a->b_stride; p.a_stride = a->a_stride;
  p.C = a->channels; p.N = a->num_rows; p.hist_rows = a->num_hist_rows; p.num_ext = a->num_ext; p.T = a->num_out;
  p.Hv = a->num_heads; p.groups = a->channels / 8;
  const int64_t threads = (int64_t)(a->num_out + dan_conv::kStrip - 1) / dan_conv::kStrip * p.groups;
  const int64_t grid = (threads + dan_conv::kBlock - 1) / dan_conv::kBlock;
  const int64_t ggrid = ((int64_t)a->num_out * a->num_heads + dan_conv::kBlock - 1) / dan_conv::kBlock;
  if (grid > 0x7fffffff || ggrid > 0x7fffffff) return fail(DAN_ERR_INVALID_ARGUMENT, "too many rows x channels");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->dtype == DAN_DTYPE_BF16) dan_conv::launch<__bf16>(p, a->kernel, grid, ggrid, s);
  else dan_conv::launch<_Float16>(p, a->kernel, grid, ggrid, s);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "conv launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}
