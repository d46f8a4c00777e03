// e4m3 quantizer for dan's FP8 decoder linears on gfx950 (MI355X, CDNA4):
// dan/fused.py:85-91 (fp8_quantize) as one pass over x per row.
//
//   amax  = max |x| over a row (rowwise) or the tensor
//   scale = max(amax, 1e-12) / 448               fp32, correctly rounded
//   xq    = e4m3fn(x / scale)                     fp32 divide, then v_cvt_pk_fp8_f32
//                                                 (gfx950: OCP e4m3, round to
//                                                 nearest even)
// |x / scale| <= 448 (up to the divide's rounding, which rounds back to 448),
// so no code saturates.
//
// Rowwise: one work group of 256 threads per row; each thread takes 8
// consecutive values (one 16-byte load for 16-bit inputs) per 2048 of the
// row, reduces |x| (wave shuffles, then LDS across the 4 waves), and on a
// second pass over the row (now in L2) writes 8 codes per 8 values.
// Per tensor: a zero fill, the same per-row amax folded into one fp32 by a
// vector atomic max on its bits (non-negative floats and NaN order as
// integers),
// the scale, then the quantizing pass with the one scale.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dan_fp8.h"

namespace dan {
int fail(int status, const char *fmt, ...);  // tree_attn.hip: sets the thread's last-error message
extern thread_local char g_err[512];
}  // namespace dan

namespace dan_fp8 {

constexpr int kThreads = 256;
constexpr float kE4m3Max = 448.0f;  // torch.finfo(torch.float8_e4m3fn).max (dan/quant.py:16)

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

#define DAN_GLOBAL __attribute__((address_space(1)))

template <typename T>
__device__ inline f32x8 load8(const T *p);
template <>
__device__ inline f32x8 load8<__bf16>(const __bf16 *p) {
  return __builtin_convertvector(__builtin_bit_cast(bf16x8, *(const DAN_GLOBAL u32x4 *)p), f32x8);
}
template <>
__device__ inline f32x8 load8<_Float16>(const _Float16 *p) {
  return __builtin_convertvector(__builtin_bit_cast(f16x8, *(const DAN_GLOBAL u32x4 *)p), f32x8);
}
template <>
__device__ inline f32x8 load8<float>(const float *p) {
  const f32x4 a = __builtin_bit_cast(f32x4, *(const DAN_GLOBAL u32x4 *)p);
  const f32x4 b = __builtin_bit_cast(f32x4, *(const DAN_GLOBAL u32x4 *)(p + 4));
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// |x| as its fp32 bit pattern. Non-negative floats order as unsigned
// integers and every NaN pattern lies above +inf's, so an integer max over
// these propagates NaN as torch's amax does (dan/fused.py:88): a row holding
// a NaN gets a NaN scale and NaN codes. (A float max would skip the NaN.)
__device__ inline uint32_t abs_bits(float x) { return __builtin_bit_cast(uint32_t, x) & 0x7fffffffu; }

// max |x| over the work group (as bits), in every thread.
__device__ inline uint32_t block_amax(uint32_t v, uint32_t *red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, m));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  v = max(max(red[0], red[1]), max(red[2], red[3]));
  __syncthreads();  // red is reused by the next call
  return v;
}

template <typename T>
__device__ inline uint32_t row_amax(const T *row, int cols) {
  uint32_t a = 0;
  for (int c = 8 * threadIdx.x; c < cols; c += 8 * kThreads) {
    const f32x8 x = load8<T>(row + c);
#pragma unroll
    for (int i = 0; i < 8; ++i) a = max(a, abs_bits(x[i]));
  }
  return a;
}

// max(amax, 1e-12) / 448 from amax's bits; a NaN amax gives a NaN scale
// (torch's clamp keeps NaN).
__device__ inline float scale_of(uint32_t amax_bits) {
  const float amax = __builtin_bit_cast(float, amax_bits);
  return amax_bits > 0x7f800000u ? amax : fmaxf(amax, 1e-12f) / kE4m3Max;
}

struct Params {
  const void *x;
  int64_t x_stride;
  uint8_t *xq;
  float *scale;
  int32_t rows, cols;
  int32_t tiled;  // DAN_FP8_LAYOUT_TILED: codes in the GEMM's panel layout
  int32_t kt;     // 64-byte k-steps per row (tiled)
};

// Byte offset of the 8 codes of row r, columns c .. c + 7 (c a multiple of 8).
// Tiled: 256-row panels, each a run of 16 KB k-steps; a k-step is 16 blocks
// of 16 rows x 64 bytes, row i of a block at 64 i, its 16-byte chunk j at
// position j ^ (((i >> 1) & 3) ^ ((i >> 3) & 1)) (include/dan_fp8.h).
__device__ inline int64_t code_offset(const Params &p, int r, int c) {
  if (!p.tiled) return (int64_t)r * p.cols + c;
  const int i = r & 15, chunk = (c >> 4) & 3;
  const int pos = chunk ^ (((i >> 1) & 3) ^ ((i >> 3) & 1));
  return ((((int64_t)(r >> 8) * p.kt + (c >> 6)) * 16 + ((r >> 4) & 15)) << 10) + 64 * i + 16 * pos + (c & 8);
}

template <typename T>
__device__ inline u32x2 codes8(f32x8 x, float scale) {
  u32x2 q;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * h] / scale, x[4 * h + 1] / scale, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * h + 2] / scale, x[4 * h + 3] / scale, w, true);
    q[h] = (uint32_t)w;
  }
  return q;
}

template <typename T>
__device__ inline void quantize_row(const Params &p, const T *row, int r, float scale) {
  for (int c = 8 * threadIdx.x; c < p.cols; c += 8 * kThreads)
    *(DAN_GLOBAL u32x2 *)(p.xq + code_offset(p, r, c)) = codes8<T>(load8<T>(row + c), scale);
}

// Tiled: zeros past the row's last column, up to its last k-step's end.
__device__ inline void zero_row_tail(const Params &p, int r) {
  if (!p.tiled) return;
  for (int c = p.cols + 8 * threadIdx.x; c < 64 * p.kt; c += 8 * kThreads)
    *(DAN_GLOBAL u32x2 *)(p.xq + code_offset(p, r, c)) = (u32x2){0u, 0u};
}

// Tiled: the padding rows of the last panel are zeros. Returns true for such
// a row (the whole work group).
__device__ inline bool pad_row(const Params &p, int r) {
  if (r < p.rows) return false;
  for (int c = 8 * threadIdx.x; c < 64 * p.kt; c += 8 * kThreads)
    *(DAN_GLOBAL u32x2 *)(p.xq + code_offset(p, r, c)) = (u32x2){0u, 0u};
  return true;
}

// Rowwise: the row's scale, then its codes.
template <typename T>
__global__ __launch_bounds__(kThreads) void quant_rows_kernel(const Params p) {
  __shared__ uint32_t red[4];
  const int r = blockIdx.x;
  if (pad_row(p, r)) return;
  const T *row = static_cast<const T *>(p.x) + (int64_t)r * p.x_stride;
  const float s = scale_of(block_amax(row_amax<T>(row, p.cols), red));
  if (threadIdx.x == 0) *(DAN_GLOBAL float *)(p.scale + r) = s;
  quantize_row<T>(p, row, r, s);
  zero_row_tail(p, r);
}

// Rowwise, for rows of at most NC * 8 * kThreads values: the row stays in
// registers between the amax and the quantization, so it is read from HBM
// once and not again from L2. Loads are unconditional (clamped to the row's
// last 8 values, then masked), so all NC are in flight together.
template <typename T, int NC>
__global__ __launch_bounds__(kThreads) void quant_rows_reg_kernel(const Params p) {
  __shared__ uint32_t red[4];
  const int r = blockIdx.x;
  if (pad_row(p, r)) return;
  const T *row = static_cast<const T *>(p.x) + (int64_t)r * p.x_stride;
  f32x8 x[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) x[j] = load8<T>(row + min(8 * (int)threadIdx.x + j * 8 * kThreads, p.cols - 8));
  uint32_t a = 0;
#pragma unroll
  for (int j = 0; j < NC; ++j)
    if (8 * (int)threadIdx.x + j * 8 * kThreads < p.cols) {
#pragma unroll
      for (int i = 0; i < 8; ++i) a = max(a, abs_bits(x[j][i]));
    }
  const float s = scale_of(block_amax(a, red));
  if (threadIdx.x == 0) *(DAN_GLOBAL float *)(p.scale + r) = s;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = 8 * threadIdx.x + j * 8 * kThreads;
    if (c < p.cols) *(DAN_GLOBAL u32x2 *)(p.xq + code_offset(p, r, c)) = codes8<T>(x[j], s);
  }
  zero_row_tail(p, r);
}

// Per tensor, step 1: zero the accumulator (scale[0] holds amax's bits until step 3).
__global__ void zero_kernel(float *scale) { *(DAN_GLOBAL uint32_t *)scale = 0u; }

// Per tensor, step 2: each row's amax into the accumulator.
template <typename T>
__global__ __launch_bounds__(kThreads) void amax_rows_kernel(const Params p) {
  __shared__ uint32_t red[4];
  const T *row = static_cast<const T *>(p.x) + (int64_t)blockIdx.x * p.x_stride;
  const uint32_t a = block_amax(row_amax<T>(row, p.cols), red);
  if (threadIdx.x == 0) atomicMax(reinterpret_cast<unsigned int *>(p.scale), a);
}

// Per tensor, step 3: amax -> scale.
__global__ void finalize_kernel(float *scale) {
  DAN_GLOBAL float *s = (DAN_GLOBAL float *)scale;
  *s = scale_of(*(DAN_GLOBAL uint32_t *)scale);
}

// Per tensor, step 4: every row with the one scale.
template <typename T>
__global__ __launch_bounds__(kThreads) void quant_tensor_kernel(const Params p) {
  const float s = *(const DAN_GLOBAL float *)p.scale;
  const int r = blockIdx.x;
  if (pad_row(p, r)) return;
  quantize_row<T>(p, static_cast<const T *>(p.x) + (int64_t)r * p.x_stride, r, s);
  zero_row_tail(p, r);
}

// rows of codes written: the tiled layout pads to whole 256-row panels
inline int out_rows(const Params &p) { return p.tiled ? (p.rows + 255) / 256 * 256 : p.rows; }

template <typename T>
hipError_t launch(const Params &p, int mode, hipStream_t s) {
  if (mode == DAN_FP8_SCALE_ROW) {
    const int chunks = (p.cols + 8 * kThreads - 1) / (8 * kThreads);
    const dim3 grid(out_rows(p));
    if (chunks <= 1) hipLaunchKernelGGL((quant_rows_reg_kernel<T, 1>), grid, dim3(kThreads), 0, s, p);
    else if (chunks <= 2) hipLaunchKernelGGL((quant_rows_reg_kernel<T, 2>), grid, dim3(kThreads), 0, s, p);
    else if (chunks <= 4) hipLaunchKernelGGL((quant_rows_reg_kernel<T, 4>), grid, dim3(kThreads), 0, s, p);
    else if (chunks <= 8) hipLaunchKernelGGL((quant_rows_reg_kernel<T, 8>), grid, dim3(kThreads), 0, s, p);
    else hipLaunchKernelGGL(quant_rows_kernel<T>, grid, dim3(kThreads), 0, s, p);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(1), 0, s, p.scale);
  hipLaunchKernelGGL(amax_rows_kernel<T>, dim3(p.rows), dim3(kThreads), 0, s, p);
  hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(1), 0, s, p.scale);
  hipLaunchKernelGGL(quant_tensor_kernel<T>, dim3(out_rows(p)), dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace dan_fp8

extern "C" {

int dan_fp8_abi_version(void) { return DAN_FP8_ABI_VERSION; }

int64_t dan_fp8_tiled_bytes(int32_t rows, int32_t cols) {
  if (rows < 0 || cols < 0) return -1;
  return (int64_t)((rows + 255) / 256) * 256 * ((cols + 63) / 64) * 64;
}

int dan_fp8_quantize(const DanFp8QuantArgs *a, void *stream) {
  using dan::fail;
  dan::g_err[0] = 0;
  if (!a) return fail(DAN_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != DAN_FP8_ABI_VERSION)
    return fail(DAN_ERR_VERSION, "abi_version %d, quantizer speaks %d", a->abi_version, DAN_FP8_ABI_VERSION);
  if (a->dtype != DAN_DTYPE_BF16 && a->dtype != DAN_DTYPE_F16 && a->dtype != DAN_DTYPE_F32)
    return fail(DAN_ERR_UNSUPPORTED, "dtype %d: bf16, f16 or f32", a->dtype);
  if (a->mode != DAN_FP8_SCALE_TENSOR && a->mode != DAN_FP8_SCALE_ROW)
    return fail(DAN_ERR_INVALID_ARGUMENT, "mode %d: 0 (tensor) or 1 (row)", a->mode);
  if (a->layout != DAN_FP8_LAYOUT_ROWS && a->layout != DAN_FP8_LAYOUT_TILED)
    return fail(DAN_ERR_INVALID_ARGUMENT, "layout %d: 0 (rows) or 1 (tiled)", a->layout);
  if (a->rows < 0 || a->cols < 0) return fail(DAN_ERR_INVALID_ARGUMENT, "negative shape");
  if (a->cols % 16) return fail(DAN_ERR_INVALID_ARGUMENT, "cols %d must be a multiple of 16", a->cols);
  if (a->rows == 0 || a->cols == 0) {  // torch's amax of an empty tensor raises; an empty row list is a no-op
    if (a->mode == DAN_FP8_SCALE_TENSOR) return fail(DAN_ERR_INVALID_ARGUMENT, "an empty tensor has no per-tensor scale");
    return DAN_OK;
  }
  if (!a->x || !a->xq || !a->scale) return fail(DAN_ERR_INVALID_ARGUMENT, "NULL pointer");
  const int es = a->dtype == DAN_DTYPE_F32 ? 4 : 2;
  if (a->x_stride < a->cols || ((uintptr_t)a->x & 15) || (a->x_stride * es) % 16 || ((uintptr_t)a->xq & 15) ||
      ((uintptr_t)a->scale & 3))
    return fail(DAN_ERR_INVALID_ARGUMENT, "x rows must be 16-byte aligned with x_stride >= cols, xq 16-byte aligned");
  dan_fp8::Params p;
  p.x = a->x; p.x_stride = a->x_stride; p.xq = a->xq; p.scale = a->scale; p.rows = a->rows; p.cols = a->cols;
  p.tiled = a->layout == DAN_FP8_LAYOUT_TILED;
  p.kt = (a->cols + 63) / 64;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  if (a->dtype == DAN_DTYPE_BF16) err = dan_fp8::launch<__bf16>(p, a->mode, s);
  else if (a->dtype == DAN_DTYPE_F16) err = dan_fp8::launch<_Float16>(p, a->mode, s);
  else err = dan_fp8::launch<float>(p, a->mode, s);
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "quantizer launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}

}  // extern "C"
