// Fused tree-masked prefill attention for gfx950 (MI355X, CDNA4).
//
// One launch computes, for every segment of a packed batch, what
// dan/attention.py:210-241 computes with three varlen flash calls, six gathers
// and a log-sum-exp merge: trunk queries attend causally over [past; trunk],
// branch queries attend to [past; trunk] and causally to their own branch.
// Here every (query tile, kv head) work group walks only the key tiles its
// queries can see, in one online-softmax pass, so there is no merge.
//
// Work decomposition
//   - A work group (4 waves of 64 lanes) owns one work item (a tile of query
//     tokens of one segment) for one kv head. With rep = H / Hkv query heads
//     per kv head, wave w takes query head (w % hpw) of the kv group and the
//     (w / hpw)-th run of 64 tokens of the tile, so the K/V tiles staged in LDS
//     serve every query head that shares them (GQA head packing).
//   - blockIdx.x = item * (Hkv * chunks) + kv head + Hkv * chunk: consecutive
//     blocks land on different XCDs, so with Hkv = 8 each XCD's L2 holds one
//     kv head's keys and values.
//
// Per wave, per key tile of 64 keys (bf16 / fp16 matrix cores):
//   S^T[key, query] = K Q^T      v_mfma_f32_32x32x16: A = K rows from LDS,
//                                B = Q held in registers. Queries sit on the
//                                lanes, so each lane owns its query's softmax
//                                state and the row max/sum need one cross-half
//                                exchange only.
//   online softmax in fp32 with exp2 (scale * log2 e folded in); the running
//   max is raised lazily (only when it grows by more than kLazyRescale) so the
//   O accumulators are rarely rescaled.
//   O^T[d, query] += V^T P^T     A = V^T rows from LDS (V is transposed while
//                                it is staged), B = P^T straight from the S^T
//                                registers: K rows are staged in a permuted
//                                order so that the S^T accumulator layout is
//                                already the B-operand layout of P^T.
// K and V tiles are double-buffered in LDS in padded rows (no bank conflicts).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "dan_tree_attn.h"

#ifndef DAN_TREE_ATTN_SKEW
#define DAN_TREE_ATTN_SKEW 1
#endif

namespace dan {

constexpr int kKeyTile = DAN_TREE_ATTN_KEY_TILE;  // keys per tile
constexpr int kWaves = 8;                         // 2 per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kWaveQ = 32;                        // queries per wave
constexpr float kLazyRescale = 8.0f;              // log2 units: p <= 2^8

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
constexpr f16x2 kOnes2 = {(_Float16)1.0f, (_Float16)1.0f};

struct KParams {
  const void *q, *k, *v;
  void *o;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh;
  const DanSegmentDesc *segs;
  const DanPastDesc *pasts;
  const DanWorkItem *work;
  const int32_t *key_lo;
  int32_t num_kv_heads, rep, hpw, chunks;
  float c;  // softmax scale * log2(e)
};

// ---------------------------------------------------------------- element I/O
// Kernel pointers arrive inside a struct, so the compiler cannot prove they are
// global memory; casting to address space 1 gives global_load instead of flat
// loads (which would also count against the LDS wait counter).
#define DAN_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ inline const DAN_GLOBAL T *gbl(const T *p) {
  return (const DAN_GLOBAL T *)p;
}
template <typename T>
__device__ inline DAN_GLOBAL T *gbl_mut(T *p) {
  return (DAN_GLOBAL T *)p;
}

// A small table entry read from global memory (dword by dword; the compiler
// merges the loads).
template <typename T>
__device__ inline T load_entry(const T *p) {
  static_assert(sizeof(T) % 4 == 0, "table entries are dword multiples");
  struct Raw {
    uint32_t w[sizeof(T) / 4];
  } raw;
  const DAN_GLOBAL uint32_t *src = gbl(reinterpret_cast<const uint32_t *>(p));
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) raw.w[i] = src[i];
  return __builtin_bit_cast(T, raw);
}

// 8 consecutive input elements -> 8 compute-type elements (16 bytes).
template <typename TIn, typename TC>
__device__ inline u32x4 load8(const TIn *p);

template <>
__device__ inline u32x4 load8<__bf16, __bf16>(const __bf16 *p) {
  return *gbl(reinterpret_cast<const u32x4 *>(p));
}
template <>
__device__ inline u32x4 load8<_Float16, _Float16>(const _Float16 *p) {
  return *gbl(reinterpret_cast<const u32x4 *>(p));
}
template <>
__device__ inline u32x4 load8<float, _Float16>(const float *p) {
  const f32x4 a = *gbl(reinterpret_cast<const f32x4 *>(p));
  const f32x4 b = *gbl(reinterpret_cast<const f32x4 *>(p + 4));
  const f32x8 x = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return __builtin_bit_cast(u32x4, __builtin_convertvector(x, f16x8));
}
// bf16 -> fp16 is exact for magnitudes in fp16's normal range [2^-14, 65504].
template <>
__device__ inline u32x4 load8<__bf16, _Float16>(const __bf16 *p) {
  const u32x4 v = *gbl(reinterpret_cast<const u32x4 *>(p));
  f32x8 x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __builtin_bit_cast(float, v[i] << 16);
    x[2 * i + 1] = __builtin_bit_cast(float, v[i] & 0xffff0000u);
  }
  return __builtin_bit_cast(u32x4, __builtin_convertvector(x, f16x8));
}

template <typename TC>
__device__ inline u32x4 pack8(f32x8 x);
template <>
__device__ inline u32x4 pack8<__bf16>(f32x8 x) {
  return __builtin_bit_cast(u32x4, __builtin_convertvector(x, bf16x8));
}
template <>
__device__ inline u32x4 pack8<_Float16>(f32x8 x) {
  return __builtin_bit_cast(u32x4, __builtin_convertvector(x, f16x8));
}

template <typename TOut>
__device__ inline void store4(TOut *p, f32x4 x);
template <>
__device__ inline void store4<__bf16>(__bf16 *p, f32x4 x) {
  *gbl_mut(reinterpret_cast<u32x2 *>(p)) = __builtin_bit_cast(u32x2, __builtin_convertvector(x, bf16x4));
}
template <>
__device__ inline void store4<_Float16>(_Float16 *p, f32x4 x) {
  *gbl_mut(reinterpret_cast<u32x2 *>(p)) = __builtin_bit_cast(u32x2, __builtin_convertvector(x, f16x4));
}
template <>
__device__ inline void store4<float>(float *p, f32x4 x) {
  *gbl_mut(reinterpret_cast<f32x4 *>(p)) = x;
}

template <typename TC>
__device__ inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);
template <>
__device__ inline f32x16 mfma32<__bf16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ inline f32x16 mfma32<_Float16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 16-bit element `e` (0..7) of a 16-byte vector, as the low half of a dword.
__device__ inline uint32_t half_of(u32x4 v, int e) {
  const uint32_t d = v[e >> 1];
  return (e & 1) ? (d >> 16) : (d & 0xffffu);
}

// LDS row of key `r` (0..63) in the K tile: bits 2 and 3 swapped, which makes
// the S^T accumulator of lane l, register i hold key 16*(i/8) + 8*(l/32) + i%8
// of its 32-key block -- exactly the k-order of the P^T B operand.
__device__ inline int k_row(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

// LDS layout: two K buffers (rows [64][D]) and three V^T buffers (rows
// [D][64]); three V buffers let the second wave group run one phase behind
// the first (see the kernel). Rows are padded by 16 bytes so the 32 rows one
// MFMA operand read touches fall in distinct banks, and every read of a wave
// is one base address plus a compile-time offset.
template <int D>
struct LdsLayout {
  static constexpr int kRow = D * 2 + 16;
  static constexpr int vRow = kKeyTile * 2 + 16;
  static constexpr int kBytes = kKeyTile * kRow;
  static constexpr int vBytes = D * vRow;
  static constexpr int kBase = 0;
  static constexpr int vBase = 2 * kBytes;
  static constexpr int total = 2 * kBytes + 3 * vBytes;
};

// ---------------------------------------------------------------- kernel
// TIn: q/k/v element type. TQK: matrix-core type of S = K Q^T (bf16 for bf16
// inputs, fp16 otherwise). P V always runs in fp16: P in [0, 2^8] keeps 11
// significant bits instead of bf16's 8, and bf16 V converts to fp16 exactly
// inside fp16's range.
// kSkew: the second wave group (waves 4-7, one per SIMD next to a wave of the
// first group) runs each iteration as [P V of the previous tile, S = K Q^T,
// softmax] while the first runs [S, softmax, P V], so on every SIMD one wave
// feeds the matrix core while the other runs its softmax.
template <typename TIn, typename TOut, typename TQK, int D, bool kSkew>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads), amdgpu_waves_per_eu(2, 2)))
void tree_attn_fwd_kernel(const KParams p) {
  using TPV = _Float16;
  constexpr int CPR = D / 8;                      // 16-byte chunks per K row
  constexpr int ROWS_PER_PASS = kThreads / CPR;   // K rows one pass loads
  constexpr int KCH = kKeyTile / ROWS_PER_PASS;   // passes (= V keys per thread)
  constexpr int ND = D / 32;                      // 32-row d blocks of O^T
  constexpr int NK = D / 16;                      // k-steps of Q K^T
  constexpr int NKG = kKeyTile / KCH;             // V key groups of KCH keys
  constexpr int KROW = LdsLayout<D>::kRow;
  constexpr int VROW = LdsLayout<D>::vRow;
  constexpr int KBYTES = LdsLayout<D>::kBytes;
  constexpr int VBYTES = LdsLayout<D>::vBytes;
  constexpr int VBASE = LdsLayout<D>::vBase;
  static_assert(KCH == 1 || KCH == 2, "head_dim must be 64 or 128");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, hl = lane >> 5, lq = lane & 31;
  const bool lagging = kSkew && wave >= kWaves / 2;

  const int groups = p.num_kv_heads * p.chunks;
  const DanWorkItem w = load_entry(p.work + blockIdx.x / groups);
  const int g = blockIdx.x % groups;
  const int kvh = g % p.num_kv_heads, chunk = g / p.num_kv_heads;
  const DanSegmentDesc sg = load_entry(p.segs + w.seg);
  const int P = sg.past_len, PT = P + sg.trunk, PN = P + sg.n;
  const int H = p.num_kv_heads * p.rep;

  const int hig = chunk * p.hpw + (wave % p.hpw);
  const int head = kvh * p.rep + hig;
  const int qw0 = w.t0 + (wave / p.hpw) * kWaveQ;  // wave's first query (segment-local)
  const int qend = w.t0 + w.tq;
  const bool wave_work = hig < p.rep && qw0 < qend;

  const TIn *qp = static_cast<const TIn *>(p.q);
  const TIn *kp = static_cast<const TIn *>(p.k) + (int64_t)kvh * p.k_sh;
  const TIn *vp = static_cast<const TIn *>(p.v) + (int64_t)kvh * p.v_sh;
  const TIn *pkp = nullptr, *pvp = nullptr;
  int64_t pk_st = 0, pv_st = 0;
  if (P > 0) {
    const DanPastDesc pd = load_entry(p.pasts + sg.past_idx);
    pkp = static_cast<const TIn *>(pd.k) + (int64_t)kvh * pd.k_stride_head;
    pvp = static_cast<const TIn *>(pd.v) + (int64_t)kvh * pd.v_stride_head;
    pk_st = pd.k_stride_tok;
    pv_st = pd.v_stride_tok;
  }

  // Per-lane query state: lane owns query column lq of its wave. Padding
  // columns (past the tile, or an idle wave) read a clamped valid row and see
  // every key, so they stay finite; they are never stored.
  const int ql = qw0 + lq;
  const bool qvalid = wave_work && ql < qend;
  const int qrow = sg.start + min(ql, qend - 1);
  const int qk = qvalid ? P + ql : 0x3fffffff;
  const int qlo = qvalid ? *gbl(p.key_lo + qrow) : 0;
  u32x4 qf[NK];
  {
    const TIn *row = qp + (int64_t)qrow * p.q_st + (int64_t)min(head, H - 1) * p.q_sh + 8 * hl;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) qf[kk] = load8<TIn, TQK>(row + 16 * kk);
  }

  // Staging registers for the next key tile.
  u32x4 kreg[KCH], vreg[KCH];
  const int kc = tid % CPR;         // K: 16-byte chunk of the row
  const int kr0 = tid / CPR;        // K: first row, then + ROWS_PER_PASS
  const int vkg = tid % NKG;        // V: key group of KCH keys
  const int vdc = tid / NKG;        // V: d chunk (8 values of d)
  // Element offsets of this thread's rows from the tile's first row, for the
  // new-token and the past tensors (a tile lying wholly in one of them is
  // loaded from a wave-uniform base plus these loop-invariant offsets).
  uint32_t koff_new[KCH], koff_past[KCH], voff_new[KCH], voff_past[KCH];
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    koff_new[i] = (uint32_t)((kr0 + i * ROWS_PER_PASS) * p.k_st + 8 * kc);
    koff_past[i] = (uint32_t)((kr0 + i * ROWS_PER_PASS) * pk_st + 8 * kc);
    voff_new[i] = (uint32_t)((vkg * KCH + i) * p.v_st + 8 * vdc);
    voff_past[i] = (uint32_t)((vkg * KCH + i) * pv_st + 8 * vdc);
  }

  auto key_src = [&](const TIn *newp, int64_t new_st, const TIn *pastp, int64_t past_st, int key) -> const TIn * {
    return key < P ? pastp + (int64_t)key * past_st : newp + (int64_t)(sg.start + key - P) * new_st;
  };
  // Key rows past the segment's end (ragged last tile) are clamped to its last
  // row: they lie beyond every query's causal limit, so the mask zeroes their
  // probabilities, and finite rows keep 0 * v finite.
  auto load_tile = [&](int j) {
    const int kb = j * kKeyTile;
    const bool in_past = kb + kKeyTile <= P;
    if (in_past || (kb >= P && kb + kKeyTile <= PN)) {  // wave-uniform fast path
      const TIn *kt = in_past ? pkp + (int64_t)kb * pk_st : kp + (int64_t)(sg.start + kb - P) * p.k_st;
      const TIn *vt = in_past ? pvp + (int64_t)kb * pv_st : vp + (int64_t)(sg.start + kb - P) * p.v_st;
#pragma unroll
      for (int i = 0; i < KCH; ++i) kreg[i] = load8<TIn, TQK>(kt + (in_past ? koff_past[i] : koff_new[i]));
#pragma unroll
      for (int i = 0; i < KCH; ++i) vreg[i] = load8<TIn, TPV>(vt + (in_past ? voff_past[i] : voff_new[i]));
      return;
    }
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int key = kb + kr0 + i * ROWS_PER_PASS;
      kreg[i] = load8<TIn, TQK>(key_src(kp, p.k_st, pkp, pk_st, min(key, PN - 1)) + 8 * kc);
    }
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int key = kb + vkg * KCH + i;
      vreg[i] = load8<TIn, TPV>(key_src(vp, p.v_st, pvp, pv_st, min(key, PN - 1)) + 8 * vdc);
    }
  };
  auto store_tile = [&](int it) {
    uint8_t *kb = smem + (it & 1) * KBYTES;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int m = k_row(kr0 + i * ROWS_PER_PASS);
      *reinterpret_cast<u32x4 *>(kb + m * KROW + kc * 16) = kreg[i];
    }
    uint8_t *vb = smem + VBASE + (it % 3) * VBYTES;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = vdc * 8 + e;
      if constexpr (KCH == 2) {
        *reinterpret_cast<uint32_t *>(vb + d * VROW + vkg * 4) = half_of(vreg[0], e) | (half_of(vreg[1], e) << 16);
      } else {
        *reinterpret_cast<uint16_t *>(vb + d * VROW + vkg * 2) = (uint16_t)half_of(vreg[0], e);
      }
    }
  };

  f32x16 o[ND];
#pragma unroll
  for (int db = 0; db < ND; ++db) o[db] = f32x16{};
  float mrun = -1e30f, lsum = 0.f;
  u32x4 pf[4];  // P^T B operands (fp16), one per 16 keys of the tile
#pragma unroll
  for (int kj = 0; kj < 4; ++kj) pf[kj] = u32x4{0, 0, 0, 0};

  // S^T = K Q^T for 64 keys x 32 queries: two 32-key blocks.
  auto qk_phase = [&](int it, f32x16 (&s)[2]) {
    const uint8_t *kb = smem + (it & 1) * KBYTES;
    s[0] = f32x16{};
    s[1] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const int m = 32 * mb + lq;
        const u32x4 a = *reinterpret_cast<const u32x4 *>(kb + m * KROW + (2 * kk + hl) * 16);
        s[mb] = mfma32<TQK>(a, qf[kk], s[mb]);
      }
    }
  };
  // Mask (boundary tiles only), online-softmax update, P^T in fp16.
  auto softmax_phase = [&](int j, f32x16 (&s)[2]) {
    if (j >= w.jfull) {
      // Key index of register r relative to the tile start: 32*mb + 16*(r/8) +
      // 8*hl + r%8. Causal limit and sibling-branch gap become per-lane bounds
      // on that index; the gap test runs only on tiles meeting [PT, lo_max).
      const int kb = j * kKeyTile;
      const int lim = qk - kb - 8 * hl;  // visible: rel <= lim
      if (kb + kKeyTile > PT && kb < w.lo_max) {
        const int g0 = PT - kb - 8 * hl, g1 = qlo - kb - 8 * hl;  // hidden: g0 <= rel < g1
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int rel = 32 * mb + 16 * (r >> 3) + (r & 7);
            const bool vis = rel <= lim && (rel < g0 || rel >= g1);
            s[mb][r] = vis ? s[mb][r] : -INFINITY;
          }
      } else {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int rel = 32 * mb + 16 * (r >> 3) + (r & 7);
            s[mb][r] = rel <= lim ? s[mb][r] : -INFINITY;
          }
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[mb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mc = mx * p.c;
    if (__any(mc > mrun + kLazyRescale)) {
      const float mnew = fmaxf(mrun, mc);
      const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
      mrun = mnew;
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < ND; ++db) o[db] *= alpha;
    }
    const float mneg = -mrun;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      f32x8 x0, x1;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        x0[r] = __builtin_amdgcn_exp2f(fmaf(s[mb][r], p.c, mneg));
        x1[r] = __builtin_amdgcn_exp2f(fmaf(s[mb][r + 8], p.c, mneg));
      }
      pf[2 * mb] = pack8<TPV>(x0);
      pf[2 * mb + 1] = pack8<TPV>(x1);
    }
    // The normalizer sums the fp16-rounded probabilities that P V uses (exact
    // fp16 products, fp32 accumulation), so rounding P mostly cancels in O / l.
    // (Pairs are taken with a shuffle of the whole vector: clang 22 miscompiles
    // __builtin_bit_cast applied to a single element of an ext_vector.)
    float acc = 0.f;
#pragma unroll
    for (int kj = 0; kj < 4; ++kj) {
      const f16x8 h = __builtin_bit_cast(f16x8, pf[kj]);
      acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 0, 1), kOnes2, acc, false);
      acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 2, 3), kOnes2, acc, false);
      acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 4, 5), kOnes2, acc, false);
      acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 6, 7), kOnes2, acc, false);
    }
    lsum += acc;
  };
  // O^T += V^T P^T over the tile's 64 keys.
  auto pv_phase = [&](int it) {
    const uint8_t *vb = smem + VBASE + (it % 3) * VBYTES;
#pragma unroll
    for (int kj = 0; kj < 4; ++kj) {
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const int d = 32 * db + lq;
        const u32x4 a = *reinterpret_cast<const u32x4 *>(vb + d * VROW + (2 * kj + hl) * 16);
        o[db] = mfma32<TPV>(a, pf[kj], o[db]);
      }
    }
  };

  const int ntile = w.ja1 + (w.jb1 - w.jb0);
  auto tile_of = [&](int i) { return i < w.ja1 ? i : w.jb0 + (i - w.ja1); };

  if (ntile > 0) {
    load_tile(tile_of(0));
    store_tile(0);
  }
  __syncthreads();

  // Idle waves compute on clamped rows too: no divergent control flow around
  // the barriers.
  for (int it = 0; it < ntile; ++it) {
    const int j = tile_of(it);
    if (it + 1 < ntile) load_tile(tile_of(it + 1));
    f32x16 s[2];
    if (lagging) {
      if (it > 0) pv_phase(it - 1);
      qk_phase(it, s);
      softmax_phase(j, s);
    } else {
      qk_phase(it, s);
      softmax_phase(j, s);
      pv_phase(it);
    }
    if (it + 1 < ntile) store_tile(it + 1);
    __syncthreads();
  }
  if (lagging && ntile > 0) pv_phase(ntile - 1);

  // Epilogue: O = O^T / l, written token-major [N, H, D].
  const float l = lsum + __shfl_xor(lsum, 32);
  const float linv = l > 0.f ? 1.0f / l : 0.f;
  if (!qvalid) return;
  TOut *row = static_cast<TOut *>(p.o) + (int64_t)(sg.start + ql) * p.o_st + (int64_t)head * p.o_sh + 4 * hl;
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const f32x4 x = {o[db][4 * r4] * linv, o[db][4 * r4 + 1] * linv, o[db][4 * r4 + 2] * linv,
                       o[db][4 * r4 + 3] * linv};
      store4<TOut>(row + 32 * db + 8 * r4, x);
    }
}

// ---------------------------------------------------------------- host side
thread_local char g_err[512];

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return status;
}

// Heads of one kv group that one work group covers: 4 waves split over them.
int heads_per_group(int rep) { return rep >= 3 ? 4 : rep; }  // of kWaves / 2 per group

template <typename TIn, typename TOut, typename TQK, int D>
hipError_t launch(const KParams &kp, int grid, hipStream_t stream) {
  constexpr bool kSkew = DAN_TREE_ATTN_SKEW;
  auto kernel = tree_attn_fwd_kernel<TIn, TOut, TQK, D, kSkew>;
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, LdsLayout<D>::total);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), LdsLayout<D>::total, stream, kp);
  return hipGetLastError();
}

}  // namespace dan

extern "C" {

int dan_tree_attn_abi_version(void) { return DAN_TREE_ATTN_ABI_VERSION; }

const char *dan_tree_attn_last_error(void) { return dan::g_err; }

int dan_tree_attn_tile_q(int32_t num_heads, int32_t num_kv_heads) {
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  return dan::kWaveQ * dan::kWaves / dan::heads_per_group(num_heads / num_kv_heads);
}

int dan_tree_attn_fwd(const DanTreeAttnArgs *a, void *stream) {
  using namespace dan;
  g_err[0] = 0;
  if (!a) return fail(DAN_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != DAN_TREE_ATTN_ABI_VERSION)
    return fail(DAN_ERR_VERSION, "abi_version %d, library speaks %d", a->abi_version, DAN_TREE_ATTN_ABI_VERSION);
  const int H = a->num_heads, Hkv = a->num_kv_heads, D = a->head_dim;
  if (H <= 0 || Hkv <= 0 || H % Hkv)
    return fail(DAN_ERR_INVALID_ARGUMENT, "num_heads %d must be a positive multiple of num_kv_heads %d", H, Hkv);
  if (D != 64 && D != 128) return fail(DAN_ERR_UNSUPPORTED, "head_dim %d: only 64 and 128 are built", D);
  const int rep = H / Hkv;
  const int tq = dan_tree_attn_tile_q(H, Hkv);
  if (a->tile_q != tq) return fail(DAN_ERR_INVALID_ARGUMENT, "tile_q %d, the kernel needs %d", a->tile_q, tq);
  if (a->num_work < 0 || a->num_segments < 0 || a->num_pasts < 0 || a->num_tokens < 0)
    return fail(DAN_ERR_INVALID_ARGUMENT, "negative count");
  if (a->num_work == 0) return DAN_OK;
  if (!a->q || !a->k || !a->v || !a->out || !a->segments || !a->work || !a->key_lo)
    return fail(DAN_ERR_INVALID_ARGUMENT, "NULL tensor or table pointer");
  if (a->num_pasts > 0 && !a->pasts) return fail(DAN_ERR_INVALID_ARGUMENT, "num_pasts > 0 with NULL pasts");
  if (!(a->scale > 0.f) || !isfinite(a->scale)) return fail(DAN_ERR_INVALID_ARGUMENT, "scale must be finite and > 0");
  // Per-thread row offsets inside a 64-key tile are kept in 32 bits.
  const int64_t max_tok_stride = a->k_stride_tok > a->v_stride_tok ? a->k_stride_tok : a->v_stride_tok;
  if (max_tok_stride < 0 || max_tok_stride * kKeyTile >= (int64_t(1) << 31))
    return fail(DAN_ERR_UNSUPPORTED, "k/v token stride %lld is too large", (long long)max_tok_stride);
  const int hpw = heads_per_group(rep);
  const int chunks = (rep + hpw - 1) / hpw;
  const int64_t grid = (int64_t)a->num_work * Hkv * chunks;
  if (grid > 0x7fffffff) return fail(DAN_ERR_INVALID_ARGUMENT, "grid of %lld work groups is too large", (long long)grid);

  KParams kp;
  kp.q = a->q; kp.k = a->k; kp.v = a->v; kp.o = a->out;
  kp.q_st = a->q_stride_tok; kp.q_sh = a->q_stride_head;
  kp.k_st = a->k_stride_tok; kp.k_sh = a->k_stride_head;
  kp.v_st = a->v_stride_tok; kp.v_sh = a->v_stride_head;
  kp.o_st = a->o_stride_tok; kp.o_sh = a->o_stride_head;
  kp.segs = a->segments; kp.pasts = a->pasts; kp.work = a->work; kp.key_lo = a->key_lo;
  kp.num_kv_heads = Hkv; kp.rep = rep; kp.hpw = hpw; kp.chunks = chunks;
  kp.c = a->scale * 1.4426950408889634f;

  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  const int in = a->in_dtype, out = a->out_dtype;
  if (in == DAN_DTYPE_BF16 && out == DAN_DTYPE_BF16) {
    err = D == 128 ? launch<__bf16, __bf16, __bf16, 128>(kp, (int)grid, s) : launch<__bf16, __bf16, __bf16, 64>(kp, (int)grid, s);
  } else if (in == DAN_DTYPE_F16 && out == DAN_DTYPE_F16) {
    err = D == 128 ? launch<_Float16, _Float16, _Float16, 128>(kp, (int)grid, s)
                   : launch<_Float16, _Float16, _Float16, 64>(kp, (int)grid, s);
  } else if (in == DAN_DTYPE_F32 && out == DAN_DTYPE_F32) {
    err = D == 128 ? launch<float, float, _Float16, 128>(kp, (int)grid, s)
                   : launch<float, float, _Float16, 64>(kp, (int)grid, s);
  } else {
    return fail(DAN_ERR_UNSUPPORTED, "dtype combination in=%d out=%d is not built", in, out);
  }
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}

}  // extern "C"
