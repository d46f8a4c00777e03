// Attention front end for gfx950 (MI355X, CDNA4): per-head RMSNorm and
// rotate-half RoPE of q and k, written token-major for the tree-attention
// kernel, with the prefix-cache rows of saving segments copied out in the
// same pass. One launch replaces the eager chain of dan/models/llama.py:78-86
// (dan/models/qwen3_5.py:318-326 for zero-centered norms and a partial
// rotary) and the clones of dan/attention.py:202-204.
//
// Work decomposition: a head vector (one token, one head: D values, 2 D
// bytes) is handled by D / 8 consecutive lanes, 16 bytes each; a work group
// of 256 threads takes 256 / (D / 8) consecutive vectors of the flattened
// [token][q heads, then kv heads] order, so q and k rows are read and written
// as whole 256-byte (D = 128) lines. The row's sum of squares is a butterfly
// over those lanes; the rotate-half partner of a lane's 8 values sits R / 16
// lanes away (R = rotary dims) and is fetched with a lane permute.
//
// Numerics are those of the eager torch ops the reference runs: fp32
// arithmetic, each op's result rounded to the storage type (RNE):
//   RMS:            n = rnd(w * rnd(x * r)),   r = rsqrt(sum(x^2) / D + eps)
//   zero-centered:  n = rnd(x * r * (1 + w))
//   rotate-half:    o = rnd(rnd(n * cos) + rnd(rot(n) * sin)),
//                   rot(n)[i] = -n[i + R/2] for i < R/2, n[i - R/2] for R/2 <= i < R
// The differences from torch are the summation order of sum(x^2) and r,
// which is the hardware rsqrt (within 1 ulp of the fp32 1 / sqrt): without a
// norm the outputs are bit-identical, with one an element moves by at most
// one unit of the storage type, rarely (a few per million at the Llama shape).
//
// The kernel is HBM-bound: it reads q, k (and the saved v rows) and cos /
// sin once and writes q, k (and the saves) once.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dan_qkv_front.h"

// Every eager op rounds its result to the storage type, so a product followed
// by a sum must not be fused: contraction would drop the rounding of the
// product (rnd(n * cos) + rnd(rot * sin) would become fma(n, cos, ...)).
#pragma clang fp contract(off)

namespace dan {
int fail(int status, const char *fmt, ...);  // tree_attn.hip: sets the thread's last-error message
bool finite_nonnegative(float x);             // tree_attn.hip: decided from the float's bits
extern thread_local char g_err[512];
}  // namespace dan

namespace dan_front {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

#define DAN_GLOBAL __attribute__((address_space(1)))

template <typename T>
struct Vec8;
template <>
struct Vec8<__bf16> {
  typedef bf16x8 type;
};
template <>
struct Vec8<_Float16> {
  typedef f16x8 type;
};

// 8 stored values (16 bytes) <-> 8 fp32 values; fp32 -> storage is RNE.
template <typename T>
__device__ inline f32x8 to_f32(u32x4 raw) {
  return __builtin_convertvector(__builtin_bit_cast(typename Vec8<T>::type, raw), f32x8);
}
template <typename T>
__device__ inline u32x4 from_f32(f32x8 x) {
  return __builtin_bit_cast(u32x4, __builtin_convertvector(x, typename Vec8<T>::type));
}
// The result of one eager op on 8 values: fp32 rounded to the storage type
// (two values per conversion instruction) and widened back.
template <typename T>
__device__ inline f32x8 rnd8(f32x8 x) {
  return to_f32<T>(from_f32<T>(x));
}

template <typename T>
__device__ inline u32x4 load16(const T *p) {
  return *(const DAN_GLOBAL u32x4 *)p;
}
template <typename T>
__device__ inline void store16(T *p, u32x4 v) {
  *(DAN_GLOBAL u32x4 *)p = v;
}

// Lane l's value from lane l ^ 1 / l ^ 2 of its quad, lane 7 - l of its
// 8-lane half-row, lane 15 - l of its 16-lane row (DPP: no LDS round trip).
#define DAN_DPP(x, ctrl) __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), ctrl, 0xF, 0xF, false))
// The sum of v over the L lanes of a head vector (L = 8, 16 or 32 consecutive
// lanes from a multiple of L), in every one of them. Once a quad holds its sum
// in every lane, the half-row mirror reads the other quad of the half-row and
// the row mirror the other half of the row, so each step adds the same pair
// as an xor butterfly over lane ^ 1, ^ 2, ^ 4, ^ 8 (^ 16 across rows).
template <int L>
__device__ inline float vec_sum(float v) {
  v += DAN_DPP(v, 0xB1);   // quad_perm 1, 0, 3, 2
  v += DAN_DPP(v, 0x4E);   // quad_perm 2, 3, 0, 1
  v += DAN_DPP(v, 0x141);  // row_half_mirror
  if constexpr (L >= 16) v += DAN_DPP(v, 0x140);  // row_mirror
  if constexpr (L >= 32) v += __shfl_xor(v, 16, 32);
  return v;
}

struct Params {
  const void *q, *k, *v, *cos, *sin, *qw, *kw;
  void *qo, *ko;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, cs_st, qo_st, qo_sh, ko_st, ko_sh;
  const int32_t *save_of;
  const DanFrontSave *saves;
  int32_t N, H, Hkv, R, norm;
  float eps;
};

// Head vectors per lane (qkv_front_kernel).
constexpr int kVecs = 2;

template <typename T, int D, int NORM>
__global__ __launch_bounds__(256) void qkv_front_kernel(const Params p) {
  constexpr int L = D / 8;      // lanes per head vector
  constexpr int VPB = 256 / L;  // head vectors per work group and pass
  const int slot = threadIdx.x / L, j = threadIdx.x % L;
  const int HV = p.H + p.Hkv;
  // A lane takes kVecs head vectors VPB apart, all loaded before any math, so
  // a wave keeps twice the bytes in flight through the norm's reduction.
  const int64_t v0 = (int64_t)blockIdx.x * (kVecs * VPB) + slot;
  // Whole vectors (all L lanes of one) leave together, so the lane
  // exchanges below only ever involve lanes of a live vector. A later vector
  // past the end is computed on a stand-in (the last vector) and not stored.
  if (v0 >= (int64_t)p.N * HV) return;
  int tv[kVecs], headv[kVecs];
  bool isqv[kVecs], okv[kVecs];
  u32x4 xraw[kVecs], wraw[kVecs], craw[kVecs], sraw[kVecs];
  {
    int t = (int)(v0 / HV), hv = (int)(v0 % HV);
#pragma unroll
    for (int k = 0; k < kVecs; ++k) {
      bool ok = true;
      if (k > 0) {
        hv += VPB;
        t += hv / HV;
        hv %= HV;
        ok = t < p.N;
      }
      const int tc = ok ? t : p.N - 1, hc = ok ? hv : HV - 1;
      const bool isq = hc < p.H;
      const int head = isq ? hc : hc - p.H;
      tv[k] = tc;
      headv[k] = head;
      isqv[k] = isq;
      okv[k] = ok;
      const T *src = isq ? static_cast<const T *>(p.q) + tc * p.q_st + head * p.q_sh
                         : static_cast<const T *>(p.k) + tc * p.k_st + head * p.k_sh;
      // Every operand is loaded here, unconditionally (a stand-in row, the
      // lane's own x, where the norm weight or the rotary tables are unused):
      // loads under branches would make the compiler wait for each in turn.
      const T *row = src + 8 * j;
      const T *wrow = NORM != DAN_FRONT_NORM_NONE ? static_cast<const T *>(isq ? p.qw : p.kw) + 8 * j : row;
      const int64_t cs_off = (int64_t)tc * p.cs_st + min(8 * j, p.R - 8);
      const T *crow = p.R > 0 ? static_cast<const T *>(p.cos) + cs_off : row;
      const T *srow = p.R > 0 ? static_cast<const T *>(p.sin) + cs_off : row;
      xraw[k] = load16(row);
      wraw[k] = load16(wrow);
      craw[k] = load16(crow);
      sraw[k] = load16(srow);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // the scheduler would issue the weight loads after the norm's math

#pragma unroll
  for (int k = 0; k < kVecs; ++k) {
    const int t = tv[k], head = headv[k];
    const bool isq = isqv[k];
    const f32x8 x = to_f32<T>(xraw[k]), w = to_f32<T>(wraw[k]), cs = to_f32<T>(craw[k]), sn = to_f32<T>(sraw[k]);

    f32x8 n = x;
    if constexpr (NORM != DAN_FRONT_NORM_NONE) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
      ss = vec_sum<L>(ss);
      // rsqrt on the transcendental unit (within 1 ulp of 1 / sqrt, as torch's GPU rsqrt)
      const float r = __builtin_amdgcn_rsqf(ss * (1.0f / (float)D) + p.eps);
      const f32x8 y = x * r;
      n = NORM == DAN_FRONT_NORM_RMS ? rnd8<T>(w * rnd8<T>(y)) : rnd8<T>(y * (1.0f + w));
    }

    f32x8 o = n;
    if (8 * j < p.R) {
      const int half = p.R / 16;  // lanes per rotary half
      const int partner = j < half ? j + half : j - half;
      const u32x4 np = from_f32<T>(n);  // exact: n is already rounded to T
      // rot(n): the partner's values, negated in the first half (the sign
      // bit of each 16-bit value, exact)
      const uint32_t sign = j < half ? 0x80008000u : 0u;
      u32x4 pp;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t word = np[c];
        pp[c] = (uint32_t)__shfl((int)word, partner, L) ^ sign;  // lane `partner` of this vector's L lanes
      }
      o = rnd8<T>(n * cs) + rnd8<T>(to_f32<T>(pp) * sn);  // rounded once more at the store
    }
    if (!okv[k]) continue;
    const u32x4 out = from_f32<T>(o);
    T *dst = isq ? static_cast<T *>(p.qo) + t * p.qo_st + head * p.qo_sh
                 : static_cast<T *>(p.ko) + t * p.ko_st + head * p.ko_sh;
    store16(dst + 8 * j, out);

    // Prefix save: the kv-head vector of a saved token also writes its k row
    // and copies its v row.
    if (!isq && p.save_of) {
      const int si = p.save_of[t];
      if (si >= 0) {
        const DanFrontSave sv = p.saves[si];
        const int64_t row = (int64_t)head * sv.len + (t - sv.start);
        store16(static_cast<T *>(sv.k_dst) + row * D + 8 * j, out);
        const T *vs = static_cast<const T *>(p.v) + t * p.v_st + head * p.v_sh;
        store16(static_cast<T *>(sv.v_dst) + row * D + 8 * j, load16(vs + 8 * j));
      }
    }
  }
}

template <typename T, int D>
hipError_t launch(const Params &p, hipStream_t s) {
  constexpr int VPB = kVecs * (256 / (D / 8));  // head vectors per work group
  const int64_t vectors = (int64_t)p.N * (p.H + p.Hkv);
  const dim3 grid((unsigned)((vectors + VPB - 1) / VPB));
  if (p.norm == DAN_FRONT_NORM_RMS) hipLaunchKernelGGL((qkv_front_kernel<T, D, DAN_FRONT_NORM_RMS>), grid, dim3(256), 0, s, p);
  else if (p.norm == DAN_FRONT_NORM_RMS_ZERO_CENTERED)
    hipLaunchKernelGGL((qkv_front_kernel<T, D, DAN_FRONT_NORM_RMS_ZERO_CENTERED>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((qkv_front_kernel<T, D, DAN_FRONT_NORM_NONE>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

static bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace dan_front

extern "C" {

int dan_qkv_front_abi_version(void) { return DAN_QKV_FRONT_ABI_VERSION; }

int dan_qkv_front(const DanQkvFrontArgs *a, void *stream) {
  using namespace dan_front;
  using dan::fail;
  dan::g_err[0] = 0;
  if (!a) return fail(DAN_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != DAN_QKV_FRONT_ABI_VERSION)
    return fail(DAN_ERR_VERSION, "abi_version %d, library speaks %d", a->abi_version, DAN_QKV_FRONT_ABI_VERSION);
  const int N = a->num_tokens, H = a->num_heads, Hkv = a->num_kv_heads, D = a->head_dim, R = a->rotary_dim;
  if (N < 0 || H <= 0 || Hkv <= 0) return fail(DAN_ERR_INVALID_ARGUMENT, "need num_tokens >= 0 and positive head counts");
  if (D != 64 && D != 128 && D != 256) return fail(DAN_ERR_UNSUPPORTED, "head_dim %d: only 64, 128 and 256 are built", D);
  if (a->dtype != DAN_DTYPE_BF16 && a->dtype != DAN_DTYPE_F16) return fail(DAN_ERR_UNSUPPORTED, "dtype %d: bf16 or f16", a->dtype);
  if (R < 0 || R > D || R % 16) return fail(DAN_ERR_INVALID_ARGUMENT, "rotary_dim %d must be a multiple of 16 in [0, %d]", R, D);
  if (a->norm < DAN_FRONT_NORM_NONE || a->norm > DAN_FRONT_NORM_RMS_ZERO_CENTERED)
    return fail(DAN_ERR_INVALID_ARGUMENT, "norm %d is not a DanFrontNorm", a->norm);
  if (a->norm != DAN_FRONT_NORM_NONE && (!a->q_norm_weight || !a->k_norm_weight || !dan::finite_nonnegative(a->eps)))
    return fail(DAN_ERR_INVALID_ARGUMENT, "a norm needs q_norm_weight, k_norm_weight and a finite eps >= 0");
  if (a->num_saves < 0 || (a->num_saves > 0 && (!a->save_of || !a->saves || !a->v)))
    return fail(DAN_ERR_INVALID_ARGUMENT, "saves need save_of, saves and v");
  if (N == 0) return DAN_OK;
  if (!a->q || !a->k || !a->q_out || !a->k_out || (R > 0 && (!a->cos || !a->sin)))
    return fail(DAN_ERR_INVALID_ARGUMENT, "NULL tensor pointer");
  if (R > 0 && a->cs_stride_tok < R) return fail(DAN_ERR_INVALID_ARGUMENT, "cs_stride_tok %lld < rotary_dim", (long long)a->cs_stride_tok);
  // 16-byte accesses: every row start must be 16-byte aligned.
  const int64_t strides[] = {a->q_stride_tok, a->q_stride_head, a->k_stride_tok, a->k_stride_head, a->qo_stride_tok,
                             a->qo_stride_head, a->ko_stride_tok, a->ko_stride_head, R > 0 ? a->cs_stride_tok : 0,
                             a->num_saves > 0 ? a->v_stride_tok : 0, a->num_saves > 0 ? a->v_stride_head : 0};
  for (int64_t st : strides)
    if (st % 8) return fail(DAN_ERR_INVALID_ARGUMENT, "strides must be multiples of 8 elements (16-byte rows)");
  const void *ptrs[] = {a->q, a->k, a->q_out, a->k_out, a->cos, a->sin, a->q_norm_weight, a->k_norm_weight, a->v};
  for (const void *ptr : ptrs)
    if (!aligned16(ptr)) return fail(DAN_ERR_INVALID_ARGUMENT, "tensor pointers must be 16-byte aligned");
  if ((int64_t)N * (H + Hkv) / (256 / (D / 8)) >= (int64_t)1 << 31) return fail(DAN_ERR_INVALID_ARGUMENT, "too many head vectors");

  Params p;
  p.q = a->q; p.k = a->k; p.v = a->v; p.cos = a->cos; p.sin = a->sin;
  p.qw = a->q_norm_weight; p.kw = a->k_norm_weight; p.qo = a->q_out; p.ko = a->k_out;
  p.q_st = a->q_stride_tok; p.q_sh = a->q_stride_head; p.k_st = a->k_stride_tok; p.k_sh = a->k_stride_head;
  p.v_st = a->v_stride_tok; p.v_sh = a->v_stride_head; p.cs_st = a->cs_stride_tok;
  p.qo_st = a->qo_stride_tok; p.qo_sh = a->qo_stride_head; p.ko_st = a->ko_stride_tok; p.ko_sh = a->ko_stride_head;
  p.save_of = a->num_saves > 0 ? a->save_of : nullptr;
  p.saves = a->saves;
  p.N = N; p.H = H; p.Hkv = Hkv; p.R = R; p.norm = a->norm; p.eps = a->eps;

  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  const bool bf16 = a->dtype == DAN_DTYPE_BF16;
  if (D == 64) err = bf16 ? launch<__bf16, 64>(p, s) : launch<_Float16, 64>(p, s);
  else if (D == 128) err = bf16 ? launch<__bf16, 128>(p, s) : launch<_Float16, 128>(p, s);
  else err = bf16 ? launch<__bf16, 256>(p, s) : launch<_Float16, 256>(p, s);
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "front-end launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}

}  // extern "C"
