// The input side of one Gated DeltaNet phase on gfx950 (MI355X, CDNA4):
// dan/models/qwen3_5.py:212-220 (DeltaNet._phase up to the delta rule) and
// dan/fused.py:80-82 (delta_gates).
//
// One launch of HBM-bound streaming work, gdn_conv_kernel:
//   - its first work groups compute the gates, one thread per (output row,
//     head): beta and g;
//   - then one wave per (strip of kStrip output rows, 64 channel groups of 8
//     channels). The lanes take consecutive 16-byte channel groups of the same
//     rows, so every row load is coalesced, and the strip's window starts, ext
//     entries and row bases are wave-uniform (scalar loads). A strip's window
//     starts, ext entries and rows are each loaded as one batch (all in
//     flight), not one memory round trip per row. Along a strip the K-row
//     window slides: output row i + 1 of a run starts one ext entry after row
//     i, so one new row is loaded per output row and a full window only at a
//     run boundary. Sum in fp32 (j = 0 .. K-1, fused multiply-adds), rounded to
//     the I/O type as the reference's conv1d output is, then silu in fp32
//     (hardware exp2 and reciprocal: the kernel is otherwise VALU-bound on a
//     full-precision exp and divide).
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

// Output rows per wave. With the XCD-major order (shared window rows hit in
// L2) and streaming stores, c3 trunk / branch phase: 4 rows 25.4 / 11.8 us,
// 6 rows 25.4 / 12.5, 8 rows 25.6 / 12.9; 16 rows held too many registers.
constexpr int kStrip = 4;
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
  int32_t cblocks, gate_blocks;  // ceil(groups / 64) waves per strip; work groups of gates
};

// A wave-uniform int32 table entry through the scalar unit (the tables are
// read-only during the launch).
__device__ inline int sload(const int32_t *p) {
  return __builtin_amdgcn_readfirstlane(*(const __attribute__((address_space(4))) int32_t *)p);
}

// beta and g of output row i and value head h (one work item of the gates).
template <typename T>
__device__ inline void gates(const Params &p, int64_t gid) {
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

// The first gate_blocks work groups compute the gates (they are dispatched
// first and overlap the conv's streaming); every other wave takes one strip of
// kStrip output rows and 64 consecutive channel groups, so its window starts,
// ext entries and row bases are wave-uniform: scalar loads, and row loads on a
// scalar base plus the lane's channel offset.
template <typename T, int K>
__global__ __launch_bounds__(kBlock) void gdn_conv_kernel(const Params p) {
  if ((int)blockIdx.x < p.gate_blocks) {
    gates<T>(p, (int64_t)blockIdx.x * kBlock + threadIdx.x);
    return;
  }
  // Work groups go to the 8 XCDs (each with its own L2) in turn: XCD-major
  // order gives each XCD a contiguous range of strips, so the K - 1 window
  // rows that a strip shares with the one before it are L2 hits.
  const int i = (int)blockIdx.x - p.gate_blocks, nb = (int)gridDim.x - p.gate_blocks;
  const int blk = i % 8 * (nb / 8) + min(i % 8, nb % 8) + i / 8;
  const int wave = __builtin_amdgcn_readfirstlane(blk * (kBlock / 64) + (int)(threadIdx.x >> 6));
  const int i0 = wave / p.cblocks * kStrip;
  const int cg = wave % p.cblocks * 64 + (int)(threadIdx.x & 63);
  if (i0 >= p.T || cg >= p.groups) return;
  const int nr = min(p.T - i0, kStrip);  // output rows of this strip
  // The 8 channels' taps, [channel][tap] as stored, kept packed (converted
  // where used: registers are what limits the waves per SIMD here).
  T wr[8 * K] __attribute__((aligned(16)));
  const T *wp = static_cast<const T *>(p.weight) + (int64_t)cg * 8 * K;
#pragma unroll
  for (int i = 0; i < K; ++i)  // 16 bytes = 8 values per load
    *reinterpret_cast<u32x4 *>(wr + 8 * i) = *(const DAN_GLOBAL u32x4 *)(wp + 8 * i);
  T *out = static_cast<T *>(p.out) + (int64_t)i0 * p.out_stride + 8 * cg;
  // x: the window's K rows as raw packed values, converted here.
  auto emit = [&](int r, const u32x4(&x)[K]) __attribute__((always_inline)) {
    f32x8 xs[K];
#pragma unroll
    for (int j = 0; j < K; ++j) xs[j] = cvt8<T>(x[j]);
    f32x8 y;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float acc = (float)wr[c * K] * xs[0][c];
#pragma unroll
      for (int j = 1; j < K; ++j) acc = fmaf((float)wr[c * K + j], xs[j][c], acc);
      const float r = (float)(T)acc;  // the conv output in the I/O type
      // silu(r) = r / (1 + e^-r) with the hardware exp2 and reciprocal (about
      // one fp32 ulp each, far below the output type's spacing)
      y[c] = r * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(r * -1.4426950408889634f));
    }
    // streaming store: nothing in this launch reads the output
    __builtin_nontemporal_store(pack8<T>(y), (DAN_GLOBAL u32x4 *)(out + (int64_t)r * p.out_stride));
  };
  const u32x4 zero = {0, 0, 0, 0};
  // With no source row or too few ext entries every window reads as zeros.
  if (!((p.N > 0 || p.hist_rows > 0) && p.num_ext >= K)) {
    u32x4 x[K];
#pragma unroll
    for (int j = 0; j < K; ++j) x[j] = zero;
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
  for (int r = 0; r < kStrip; ++r) t[r] = sload(p.take + i0 + min(r, nr - 1));
#pragma unroll
  for (int r = 0; r < kStrip; ++r) {
    tv[r] = t[r] >= 0 && t[r] <= p.num_ext - K;
    t[r] = tv[r] ? t[r] : 0;
  }
  // 2. Each row's newest window entry, and the first row's older ones.
  int en[kStrip], ep[K - 1];
#pragma unroll
  for (int r = 0; r < kStrip; ++r) en[r] = sload(p.ext + t[r] + K - 1);
#pragma unroll
  for (int j = 0; j < K - 1; ++j) ep[j] = sload(p.ext + t[0] + j);
  // 3. Their rows.
  u32x4 rn[kStrip], rp[K - 1];
  bool okn[kStrip], okp[K - 1];
#pragma unroll
  for (int r = 0; r < kStrip; ++r) rn[r] = row_at(en[r], okn[r]);
#pragma unroll
  for (int j = 0; j < K - 1; ++j) rp[j] = row_at(ep[j], okp[j]);
  // 4. The outputs. Along a run the window slides one entry per output row;
  //    at a run boundary (rare) the row's older entries are loaded then.
  u32x4 x[K];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) x[j] = tv[0] && okp[j] ? rp[j] : zero;
  x[K - 1] = tv[0] && okn[0] ? rn[0] : zero;
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
        const u32x4 raw = tv[r] ? row_at(sload(p.ext + t[r] + j), ok) : zero;
        x[j] = ok ? raw : zero;
      }
    }
    x[K - 1] = tv[r] && okn[r] ? rn[r] : zero;
    if (r < nr) emit(r, x);
  }
}

template <typename T>
void launch(const Params &p, int K, int64_t grid, hipStream_t s) {
  if (K == 2) hipLaunchKernelGGL((gdn_conv_kernel<T, 2>), dim3((unsigned)grid), dim3(kBlock), 0, s, p);
  else if (K == 3) hipLaunchKernelGGL((gdn_conv_kernel<T, 3>), dim3((unsigned)grid), dim3(kBlock), 0, s, p);
  else hipLaunchKernelGGL((gdn_conv_kernel<T, 4>), dim3((unsigned)grid), dim3(kBlock), 0, s, p);
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
  if ((uintptr_t)a->weight & 15) return fail(DAN_ERR_INVALID_ARGUMENT, "weight must be 16-byte aligned");
  if (a->num_heads && (!a->rows || !a->b || !a->a || !a->a_log || !a->dt_bias || !a->beta || !a->g))
    return fail(DAN_ERR_INVALID_ARGUMENT, "NULL gate pointer");
  dan_conv::Params p;
  p.src = a->src; p.hist = a->hist; p.weight = a->weight; p.b = a->b; p.a = a->a;
  p.ext = a->ext; p.take = a->take; p.rows = a->rows; p.a_log = a->a_log; p.dt_bias = a->dt_bias;
  p.out = a->out; p.beta = a->beta; p.g = a->g;
  p.src_stride = a->src_stride; p.out_stride = a->out_stride; p.b_stride = a->b_stride; p.a_stride = a->a_stride;
  p.C = a->channels; p.N = a->num_rows; p.hist_rows = a->num_hist_rows; p.num_ext = a->num_ext; p.T = a->num_out;
  p.Hv = a->num_heads; p.groups = a->channels / 8;
  p.cblocks = (p.groups + 63) / 64;
  const int64_t waves = (int64_t)(a->num_out + dan_conv::kStrip - 1) / dan_conv::kStrip * p.cblocks;
  const int64_t gate_blocks = ((int64_t)a->num_out * a->num_heads + dan_conv::kBlock - 1) / dan_conv::kBlock;
  const int64_t grid = gate_blocks + (waves + dan_conv::kBlock / 64 - 1) / (dan_conv::kBlock / 64);
  if (grid > 0x7fffffff / (dan_conv::kBlock / 64) || a->num_out > 0x7fffffff - dan_conv::kStrip)
    return fail(DAN_ERR_INVALID_ARGUMENT, "too many rows x channels");
  p.gate_blocks = (int32_t)gate_blocks;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->dtype == DAN_DTYPE_BF16) dan_conv::launch<__bf16>(p, a->kernel, grid, s);
  else dan_conv::launch<_Float16>(p, a->kernel, grid, s);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "conv launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}
