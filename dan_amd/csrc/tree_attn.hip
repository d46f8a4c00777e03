// Fused tree-masked prefill attention for gfx950 (MI355X, CDNA4).
//
// One dan_tree_attn_fwd call computes, for every segment of a packed batch,
// what dan/attention.py:210-241 computes with three varlen flash calls, six
// gathers and a log-sum-exp merge: trunk queries attend causally over
// [past; trunk], branch queries attend to [past; trunk] and causally to their
// own branch. Each (query tile, kv head) work group walks only the key tiles
// its queries can see, in one online-softmax pass, so there is no merge.
//
// Two kernels run on the caller's stream:
//   vt_pack_kernel     V (and each prefix-cache entry's v) -> fp16 V^T in the
//                      caller's workspace, [Hkv][D][columns], one 64-aligned
//                      column range per segment holding [past; new] keys.
//   tree_attn_kernel   the attention itself.
//
// Work decomposition of tree_attn_kernel
//   - A unit is one work item (a tile of query tokens of one segment) for one
//     head group (kv head + Hkv * chunk). A work group (8 waves, 2 per SIMD)
//     runs units one after another. Wave w takes query head (w % hpw) of the
//     kv group and the (w / hpw)-th run of 32 tokens (16 at head_dim 256,
//     on 16x16 products with two stage buffers), so the K / V^T tiles
//     staged in LDS serve every query head that shares them (GQA head
//     packing).
//   - The grid is persistent: about one work group per CU, each walking a
//     host-planned list of units with balanced key-tile counts (one launch
//     wave, no tail of short work groups). Work group b runs on XCD b % 8
//     and gets only units of head group b % groups, so with Hkv = 8 each
//     XCD's L2 holds one kv head's keys and values.
//
// Per wave and key tile of 64 keys:
//   S^T[key, query] = K Q^T      v_mfma_f32_32x32x16 (bf16 or fp16): A = K rows
//                                from LDS, B = Q held in registers. Queries sit
//                                on the lanes, so each lane owns its query's
//                                softmax state; row max/sum need one cross-half
//                                exchange.
//   online softmax in fp32 with exp2 (scale * log2 e folded in); the running
//   max is not recomputed per tile. It stays at the first tile's max unless a
//   later p overflows fp16, in which case the unit runs again raising m per
//   tile whenever a score would put p above 2^kLog2Limit, so the O
//   accumulators are rarely rescaled and most tiles skip the max altogether.
//   O^T[d, query] += V^T P^T     v_mfma_f32_32x32x16_f16: A = V^T rows from LDS,
//                                B = P^T straight from the S^T registers: K rows
//                                are staged in a permuted order that makes the
//                                S^T accumulator layout the B-operand layout.
// Staging: K and V^T tiles go from global memory straight into LDS
// (global_load_lds_dwordx4, no registers, no VALU), four buffers deep, each
// K row's 16-byte chunks XOR-swizzled (conflict-free operand reads).
// Pipelining: while the softmax of tile j runs on the VALU, the wave already
// issues S = K Q^T of tile j+1 on the matrix core (into the same registers,
// each as soon as the softmax has read it); the tile two ahead is in flight
// from memory.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "dan_tree_attn.h"

namespace dan {

constexpr int kKeyTile = DAN_TREE_ATTN_KEY_TILE;  // keys per tile
// Work-group shape of the attention launch: 8 waves, 2 per SIMD. A wave
// takes 32 queries on 32x32 products up to D = 128, and 16 queries on 16x16
// products at D = 256, where 32 queries' O^T (128 registers) and Q
// fragments (64) would not fit a wave's 256 registers next to the scores.
template <int D>
struct Shape {
  static constexpr int waves = 8;
  static constexpr int threads = 64 * waves;
  static constexpr int waves_per_simd = 2;
  static constexpr int wave_q = D == 256 ? 16 : 32;  // queries per wave
};
inline int wave_q_for(int head_dim) { return head_dim == 256 ? Shape<256>::wave_q : Shape<128>::wave_q; }
// Up to head_dim 128, waves 0-3 (one per SIMD) issue every direct load of
// the stage buffers; their SIMD partners only compute. The loads queue at the
// CU's address unit; a queued wave cannot issue anything else, so the stall
// is given to the wave that has slack (the older wave of each SIMD wins issue
// arbitration and otherwise waits at the step barrier), and its partner runs
// its S products alone meanwhile: the two waves of a SIMD settle half a phase
// apart. At head_dim 256 the tiles are twice as large and all eight waves
// issue (8 loads of 1 KB per issuing wave and tile either way).
template <int D>
struct Issuers {
  static constexpr int n = D == 256 ? 8 : 4;
};
constexpr float kLog2Limit = 15.0f;  // p = exp2(S c - m) <= 2^15: P stays inside fp16's range
constexpr int kVoteBytes = 16;       // LDS past the stage ring: the work group's overflow votes

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
constexpr f16x2 kOnes2 = {(_Float16)1.0f, (_Float16)1.0f};
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));

// OCP float8 e4m3fn (the format of torch.float8_e4m3fn), as stored.
struct E4M3 {
  uint8_t bits;
};

// Operand traits of S = K Q^T on the matrix core. A lane's fragment of one
// k-step is `chunks` 16-byte pieces: 8 values of a 16-bit type
// (v_mfma_f32_32x32x16_{bf16,f16}, k-step 16) or 32 e4m3 values
// (v_mfma_f32_32x32x64_f8f6f4, k-step 64). Lane l holds row l % 32 and the
// k-range [step/2 * (l / 32), +step/2) of the step.
template <typename T>
struct QK {
  static constexpr int step = 16, chunks = 1;
};
template <>
struct QK<E4M3> {
  static constexpr int step = 64, chunks = 2;
};
template <typename T>
struct Frag {
  u32x4 c[QK<T>::chunks];
};

struct KParams {
  const void *q, *k;
  void *o;
  const _Float16 *vt;
  const int32_t *vexp;  // per V^T column block: the copy holds V * 2^-vexp
  int64_t q_st, q_sh, k_st, k_sh, o_st, o_sh;
  const DanPastDesc *pasts;
  const int32_t *key_lo;
  int32_t num_kv_heads, rep, hpw, chunks, vt_cols;
  float c;  // softmax scale * log2(e)
  // e4m3 only: per-tensor scales of q and k (device fp32 scalars); S is
  // scaled by q_scale * k_scale (a prefix-cache entry has its own k scale).
  const float *q_scale, *k_scale;
  // Persistent schedule: work group b runs units[sched_off[b]] ..
  // units[sched_off[b + 1] - 1] (work items with their segment's fields).
  const DanUnit *units;
  const int32_t *sched_off;
  int32_t num_units;
};

typedef const __attribute__((address_space(4))) KParams *KArgPtr;

struct PackParams {
  const void *v;
  int64_t v_st, v_sh;
  const DanSegmentDesc *segs;
  const DanPastDesc *pasts;
  const int32_t *col_seg;
  _Float16 *vt;
  int32_t *vexp;  // [Hkv][vt_cols / 64]: power-of-2 exponent of each column block (V^T = V * 2^-e)
  int32_t num_kv_heads, vt_cols;
  const float *v_scale;  // e4m3 only: per-tensor scale of v (prefix-cache entries carry their own)
  const int32_t *counts; // budget mode: device {S, B, W, C}; column blocks from C on are skipped
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

// The same for an entry every lane reads at the same address: each dword is
// made visibly wave-uniform (SGPRs), so control flow that depends on it stays
// scalar.
template <typename T>
__device__ inline T load_uniform(const T *p) {
  static_assert(sizeof(T) % 4 == 0, "table entries are dword multiples");
  struct Raw {
    uint32_t w[sizeof(T) / 4];
  } raw;
  const DAN_GLOBAL uint32_t *src = gbl(reinterpret_cast<const uint32_t *>(p));
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) raw.w[i] = __builtin_amdgcn_readfirstlane(src[i]);
  return __builtin_bit_cast(T, raw);
}

// A small table entry every lane reads at the same address, read through the
// constant address space: scalar loads (counted by lgkmcnt), so a wait for it
// never drains the vector-memory loads in flight (the stage buffers' direct
// loads). The entry must not change while the kernel runs.
template <typename T>
__device__ inline T load_scalar(const T *p) {
  static_assert(sizeof(T) % 4 == 0, "table entries are dword multiples");
  struct Raw {
    uint32_t w[sizeof(T) / 4];
  } raw;
  const __attribute__((address_space(4))) uint32_t *src = (const __attribute__((address_space(4))) uint32_t *)p;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) raw.w[i] = __builtin_amdgcn_readfirstlane(src[i]);
  return __builtin_bit_cast(T, raw);
}

// 8 e4m3 values (8 bytes) -> 8 fp32 values.
__device__ inline f32x8 e4m3x8_to_f32(u32x2 v) {
  f32x8 x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(v[i], false), hi = __builtin_amdgcn_cvt_pk_f32_fp8(v[i], true);
    const float a = lo[0], b = lo[1], c = hi[0], d = hi[1];
    x[4 * i] = a;
    x[4 * i + 1] = b;
    x[4 * i + 2] = c;
    x[4 * i + 3] = d;
  }
  return x;
}

// A lane's operand fragment of one k-step: `chunks` consecutive 16-byte
// pieces starting at p.
template <typename T>
__device__ inline Frag<T> load_frag(const T *p) {
  Frag<T> f;
#pragma unroll
  for (int i = 0; i < QK<T>::chunks; ++i) f.c[i] = *gbl(reinterpret_cast<const u32x4 *>(p) + i);
  return f;
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

// Four output values of one register group, converted to the output type
// and held as 32-bit words (2 for 16-bit outputs, 4 for fp32).
template <typename TOut>
struct Out4 {
  static constexpr int kWords = (int)sizeof(TOut);
  uint32_t w[kWords];
};
template <typename TOut>
__device__ inline Out4<TOut> pack_out(const f32x16 &o, int first, float scale) {
  const f32x4 x = {o[first] * scale, o[first + 1] * scale, o[first + 2] * scale, o[first + 3] * scale};
  Out4<TOut> r;
  if constexpr (std::is_same<TOut, float>::value) {
    // (the whole vector is bit-cast: clang 22 bit-casts an ext_vector element
    // by reading element 0)
    const u32x4 u = __builtin_bit_cast(u32x4, x);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.w[i] = u[i];
  } else {
    using V4 = TOut __attribute__((ext_vector_type(4)));
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_convertvector(x, V4));
    r.w[0] = v[0];
    r.w[1] = v[1];
  }
  return r;
}
// Eight consecutive output values (a then b) at p.
template <typename TOut>
__device__ inline void store8(TOut *p, const Out4<TOut> &a, const Out4<TOut> &b) {
  if constexpr (std::is_same<TOut, float>::value) {
    *gbl_mut(reinterpret_cast<u32x4 *>(p)) = u32x4{a.w[0], a.w[1], a.w[2], a.w[3]};
    *gbl_mut(reinterpret_cast<u32x4 *>(p + 4)) = u32x4{b.w[0], b.w[1], b.w[2], b.w[3]};
  } else {
    *gbl_mut(reinterpret_cast<u32x4 *>(p)) = u32x4{a.w[0], a.w[1], b.w[0], b.w[1]};
  }
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

// Dot product of two vectors of 8 16-bit values, accumulated in fp32.
template <typename TC>
__device__ inline float dot8(u32x4 a, u32x4 b, float acc);
template <>
__device__ inline float dot8<__bf16>(u32x4 a, u32x4 b, float acc) {
  const bf16x8 x = __builtin_bit_cast(bf16x8, a), y = __builtin_bit_cast(bf16x8, b);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 0, 1), __builtin_shufflevector(y, y, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 2, 3), __builtin_shufflevector(y, y, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 4, 5), __builtin_shufflevector(y, y, 4, 5), acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 6, 7), __builtin_shufflevector(y, y, 6, 7), acc, false);
}
template <>
__device__ inline float dot8<_Float16>(u32x4 a, u32x4 b, float acc) {
  const f16x8 x = __builtin_bit_cast(f16x8, a), y = __builtin_bit_cast(f16x8, b);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 0, 1), __builtin_shufflevector(y, y, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 2, 3), __builtin_shufflevector(y, y, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 4, 5), __builtin_shufflevector(y, y, 4, 5), acc, false);
  return __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 6, 7), __builtin_shufflevector(y, y, 6, 7), acc, false);
}

template <typename T>
__device__ inline f32x16 mfma_qk(const Frag<T> &a, const Frag<T> &b, f32x16 c) {
  return mfma32<T>(a.c[0], b.c[0], c);
}
template <>
__device__ inline f32x16 mfma_qk<E4M3>(const Frag<E4M3> &a, const Frag<E4M3> &b, f32x16 c) {
  const i32x8 x = __builtin_bit_cast(i32x8, a), y = __builtin_bit_cast(i32x8, b);
  // Format codes 0, 0: both operands OCP e4m3; no block scales.
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(x, y, c, 0, 0, 0, 0, 0, 0);
}
template <typename T>
__device__ inline float dot_frag(const Frag<T> &a, const Frag<T> &b, float acc) {
  return dot8<T>(a.c[0], b.c[0], acc);
}
template <>
__device__ inline float dot_frag<E4M3>(const Frag<E4M3> &a, const Frag<E4M3> &b, float acc) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const u32x4 x4 = a.c[i], y4 = b.c[i];
    const u32x2 xl = {x4[0], x4[1]}, xh = {x4[2], x4[3]}, yl = {y4[0], y4[1]}, yh = {y4[2], y4[3]};
    const f32x8 x0 = e4m3x8_to_f32(xl), x1 = e4m3x8_to_f32(xh), y0 = e4m3x8_to_f32(yl), y1 = e4m3x8_to_f32(yh);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = fmaf(x0[j], y0[j], fmaf(x1[j], y1[j], acc));
  }
  return acc;
}

// 16x16 products (head_dim 256, 16 queries per wave): A is 16 rows x one
// k-step, B one k-step x 16 columns, lane l holding row / column l % 16 and
// the k-range part l / 16 of the step; the accumulator of lane l holds rows
// 4 (l / 16) .. + 3 of column l % 16.
template <typename TC>
__device__ inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ inline f32x4 mfma16<__bf16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ inline f32x4 mfma16<_Float16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <typename T>
__device__ inline f32x4 mfma16_qk(const Frag<T> &a, const Frag<T> &b, f32x4 c) {
  return mfma16<T>(a.c[0], b.c[0], c);
}
template <>
__device__ inline f32x4 mfma16_qk<E4M3>(const Frag<E4M3> &a, const Frag<E4M3> &b, f32x4 c) {
  const i32x8 x = __builtin_bit_cast(i32x8, a), y = __builtin_bit_cast(i32x8, b);
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(x, y, c, 0, 0, 0, 0, 0, 0);  // OCP e4m3 x e4m3, no block scales
}

// Key held in LDS row r of a K tile (0..63), head_dim 256: within each 32-row
// group, row 16 h + 4 q + e holds key 8 q + 4 h + e. The 16x16 product of
// row block 2 g + h then gives lane l (q = l / 16) keys 32 g + 8 q + 4 h + e,
// so across blocks 2 g and 2 g + 1 a lane holds keys 32 g + 8 q .. + 7 of its
// query: exactly its part of the P^T B operand of the next product.
__host__ __device__ constexpr int k_row16(int r) {
  return (r & ~31) | (((r >> 2) & 3) << 3) | (((r >> 4) & 1) << 2) | (r & 3);
}

// Key held in LDS row r of a K tile (0..63), head_dim <= 128: bits 2 and 3
// swapped, which makes the S^T accumulator of lane l, register i hold key
// 16*(i/8) + 8*(l/32) + i%8 of its 32-key block -- exactly the k-order of
// the P^T B operand.
template <int D>
__device__ inline int k_row(int r) {
  if constexpr (D == 256) return k_row16(r);
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}


// The value of lane l and of lane l ^ 32 (v_permlane32_swap on a copy). The
// elements of the result are copied out before the bit casts: clang 22
// bit-casts an element of an ext_vector by reading element 0.
struct LanePair {
  float self, other;
};
__device__ inline LanePair lane_pair(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t a = sw[0], b = sw[1];
  return {__builtin_bit_cast(float, a), __builtin_bit_cast(float, b)};
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left alone).
template <int N>
__device__ inline void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Work-group barrier without the memory fence __syncthreads() adds: the fence
// makes the compiler drain every outstanding direct load (vmcnt(0)), while a
// stage buffer only needs its own loads counted down (wait_vmem) before the
// barrier. LDS reads are drained so no wave still reads a buffer that the next
// loads overwrite; the "memory" clobber keeps the compiler from moving memory
// accesses across the barrier.
__device__ inline void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

#define DAN_LDS __attribute__((address_space(3)))
// One 16-byte direct load per lane into LDS (global_load_lds_dwordx4: lane l
// writes lds + 16 * l; M0 holds the LDS address). Issued from inline asm:
// the compiler's wait-count pass treats an in-flight LDS DMA it can see as an
// LDS event of unknown order and then makes every wait on an LDS read a full
// lgkmcnt(0), serializing the operand reads of the matrix products. The
// stage buffers' completion is waited for explicitly (wait_vmem), and the
// "memory" clobber keeps compiler memory accesses from moving across.
// `lds` is the LDS byte address (an integer: no generic-pointer conversion
// and its null check per load). A load that reads M0 needs one wait state
// after the SALU write of M0 (s_nop 0); the compiler's hazard pass does not
// look inside inline asm.
// Uniform base address (an SGPR pair) plus a per-lane 32-bit byte offset:
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// (The base is made visibly uniform here: it is uniform by construction, and
// readfirstlane of a value the compiler already holds in SGPRs costs nothing.)
__device__ inline void dma16(const void *base_any, uint32_t off, uint32_t lds) {
  const uint64_t bv = (uint64_t)(uintptr_t)base_any;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)bv), hi = __builtin_amdgcn_readfirstlane((uint32_t)(bv >> 32));
  const void *base = (const void *)(uintptr_t)(((uint64_t)hi << 32) | lo);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
// A per-lane 64-bit address:
__device__ inline void dma16(const void *addr, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(addr), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wave-uniform integers, made visibly uniform (SGPRs).
__device__ inline int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ inline int64_t uni64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)x),
                 hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// A wave-uniform pointer, made visibly uniform (SGPRs) for an "s" operand.
template <typename T>
__device__ inline const T *uniform_ptr(const T *p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const T *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// LDS layout of one of four stage buffers, without padding:
//  - K rows [64][D] (row m holds key k_row(m)), each row's 16-byte chunks
//    XOR-swizzled: chunk c of row m sits at slot c ^ kswz(m). The 16 lanes a
//    ds_read_b128 serves together read one chunk of 16 consecutive rows, which
//    the swizzle spreads over all 64 banks; the direct loads still move whole
//    rows (1 KB = 64 lanes x 16 bytes of contiguous rows).
//  - V^T as the P V operand fragments themselves: block (kj, db) holds, for
//    lane l, d = 32 db + l % 32 and keys 16 kj + 8 (l / 32) .. + 8 (fp16), in
//    lane order. The V^T copy in the workspace has the same order, so every
//    direct load of V^T is 1 KB of contiguous memory and every operand read
//    is 1 KB of contiguous LDS.
template <int D, int KB = 2>  // KB: bytes per K element
struct Lds {
  static constexpr int kRowBytes = D * KB;
  static constexpr int kChunks = kRowBytes / 16;          // 16-byte chunks per K row
  static constexpr int kBytes = kKeyTile * kRowBytes;
  static constexpr int kBlocks = kBytes / 1024;
  static constexpr int vBytes = D * kKeyTile * 2;         // fp16 V^T tile
  static constexpr int vBlocks = vBytes / 1024;
  static constexpr int blocks = kBlocks + vBlocks;
  static constexpr int kIssuers = Issuers<D>::n;
  static_assert(kBlocks % kIssuers == 0 && vBlocks % kIssuers == 0, "blocks divide evenly among the issuing waves");
  static constexpr int slots = blocks / kIssuers;  // direct loads per issuing wave per tile
  static constexpr int buf = kBytes + vBytes;
  // Stage buffers: a ring of four where they fit (the S product of tile j+1
  // overlaps the softmax of tile j, tile j+2 is in flight), else two (tile
  // j+1 in flight while tile j is processed: head_dim 256).
  static constexpr int nbuf = 4 * buf <= 160 * 1024 ? 4 : 2;
  static constexpr int total = nbuf * buf;
  // Swizzle: rows per 256-byte bank period, and the width of the chunk XOR.
  static constexpr int kRowsPerPeriod = kRowBytes >= 256 ? 1 : 256 / kRowBytes;
  static constexpr int kSwizzle = kChunks < 16 ? kChunks : 16;
  static_assert(kBytes % 1024 == 0 && vBytes % 1024 == 0, "whole 1 KB blocks");
  static_assert(total + kVoteBytes <= 160 * 1024, "LDS");
  // Operand reads XOR the chunk into (buffer offset + lane offset): the
  // buffer offsets must leave the lane offset's bits (32 rows) untouched.
  static_assert(buf % (32 * kRowBytes) == 0, "buffer alignment");
};

// Slot of chunk c of K row m (see Lds).
template <int D, int KB>
__host__ __device__ constexpr int kswz(int m) {
  return (m / Lds<D, KB>::kRowsPerPeriod) % Lds<D, KB>::kSwizzle;
}

// ---------------------------------------------------------------- V^T packing
// One work group per (64-column block of the V^T copy, kv head): reads the 64
// keys of the block (past rows from the segment's prefix-cache entry, new rows
// from v; zero past the segment's end), converts them to fp16 and writes them
// transposed, as the P V operand fragments of the block (16 KB contiguous per
// block and kv head at D = 128; see Lds).
// 8 consecutive values of v (times `scale`, e4m3 only) as fp32.
template <typename TV>
__device__ inline f32x8 load8_f32(const TV *p, float scale);
template <>
__device__ inline f32x8 load8_f32<__bf16>(const __bf16 *p, float) {
  const u32x4 v = *gbl(reinterpret_cast<const u32x4 *>(p));
  f32x8 x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __builtin_bit_cast(float, v[i] << 16);
    x[2 * i + 1] = __builtin_bit_cast(float, v[i] & 0xffff0000u);
  }
  return x;
}
template <>
__device__ inline f32x8 load8_f32<_Float16>(const _Float16 *p, float) {
  return __builtin_convertvector(__builtin_bit_cast(f16x8, *gbl(reinterpret_cast<const u32x4 *>(p))), f32x8);
}
template <>
__device__ inline f32x8 load8_f32<float>(const float *p, float) {
  const f32x4 a = *gbl(reinterpret_cast<const f32x4 *>(p));
  const f32x4 b = *gbl(reinterpret_cast<const f32x4 *>(p + 4));
  return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
template <>
__device__ inline f32x8 load8_f32<E4M3>(const E4M3 *p, float scale) {
  return e4m3x8_to_f32(*gbl(reinterpret_cast<const u32x2 *>(p))) * scale;
}

// Power-of-2 exponent e of a V^T column block from its largest magnitude:
// the copy holds V * 2^-e in fp16. e = 0 while the largest |v| lies in
// [2^-6, 2^15] (bf16 and fp16 inputs there convert exactly, or lose only
// fp16 subnormal bits far below the block's largest value); otherwise e
// brings it into (2^14, 2^15], so fp16 neither overflows nor flushes the
// block. A zero, inf or NaN maximum keeps e = 0 (NaN and inf propagate).
// e is clamped to [-60, 60]: blocks with |v| up to 2^75 stay finite.
__host__ __device__ inline int vt_exponent(float amax) {
  uint32_t b;
  memcpy(&b, &amax, 4);
  const int bexp = (int)((b >> 23) & 0xff);
  if (bexp == 0xff || b == 0 || (amax >= 0x1p-6f && amax <= 0x1p15f)) return 0;
  const int ceil_log2 = bexp == 0 ? -126 : (bexp - 127) + ((b & 0x7fffff) != 0);
  const int e = ceil_log2 - 15;
  return e < -60 ? -60 : e > 60 ? 60 : e;  // any two differ by at most 120: 2^(e1 - e2) stays a normal fp32
}
// 2^e as an fp32 (exact for e in [-126, 127]).
__device__ inline float exp2i(int e) { return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23); }

template <typename TV, int D>
__global__ __launch_bounds__(256) void vt_pack_kernel(const PackParams p) {
  constexpr bool kF8 = std::is_same<TV, E4M3>::value;
  constexpr int kPasses = D / 64;  // (8-value d chunk, key pair) items per thread
  // tile: row d = 32 dwords, dword kp holding keys 2 kp and 2 kp + 1 (fp16) at
  // position kp ^ 4 * ((d / 8) % 8). The swizzle keeps every 16-byte group of
  // a row together and makes both phases conflict-free: each half-wave writes
  // 8 d chunks x 4 key pairs to 32 distinct banks, and 8 lanes read one row.
  __shared__ __attribute__((aligned(16))) uint32_t tile[D * 32];
  __shared__ float wave_max[4];
  const int kvh = blockIdx.x % p.num_kv_heads, cb = blockIdx.x / p.num_kv_heads;
  if (p.counts && cb >= load_scalar(p.counts + 3)) return;  // past this batch's columns (the grid covers the capacity)
  const DanSegmentDesc sg = load_scalar(p.segs + load_scalar(p.col_seg + cb));
  const int key0 = cb * kKeyTile - sg.vt_col;
  const int P = sg.past_len, PN = P + sg.n;
  const TV *vp = static_cast<const TV *>(p.v) + (int64_t)kvh * p.v_sh;
  const TV *pvp = nullptr;
  int64_t pv_st = 0;
  float vs = 1.f, pvs = 1.f;
  if (kF8) vs = load_scalar(p.v_scale);
  if (P > 0) {
    const DanPastDesc pd = load_scalar(p.pasts + sg.past_idx);
    pvp = static_cast<const TV *>(pd.v) + (int64_t)kvh * pd.v_stride_head;
    pv_st = pd.v_stride_tok;
    if (kF8) pvs = load_scalar(pd.v_scale);
  }
  // 8 values of key `key` (segment key coordinates) from d chunk c, as fp32.
  // Branch-free: a key past the segment reads a stand-in row (the segment's
  // first past or new row, which exists since the column block does) and is
  // zeroed, so every thread's loads are in flight together (a load under a
  // branch makes the compiler drain all loads at the join).
  const TV *first = P > 0 ? pvp : vp + (int64_t)sg.start * p.v_st;
  auto row8 = [&](int key, int c) __attribute__((always_inline)) {
    const bool past = key < P, valid = key < PN;
    const TV *src = !valid ? first : past ? pvp + (int64_t)key * pv_st : vp + (int64_t)(sg.start + key - P) * p.v_st;
    const f32x8 x = load8_f32<TV>(src + 8 * c, past ? pvs : vs);
    return valid ? x : f32x8{};
  };
  const int hw = threadIdx.x >> 5, j = threadIdx.x & 31;  // half-wave, lane in it
  const int c_lo = j >> 2, kp_lo = j & 3;
  f32x8 r0[kPasses], r1[kPasses];
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) {  // all loads in flight first
    const int item = hw + 8 * pass;
    const int c = c_lo + 8 * (item / 8), kp = kp_lo + 4 * (item % 8);
    r0[pass] = row8(key0 + 2 * kp, c);
    r1[pass] = row8(key0 + 2 * kp + 1, c);
  }
  __builtin_amdgcn_sched_barrier(0);
  // The block's largest magnitude (NaN-ignoring max) -> its exponent.
  float m = 0.f;
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass)
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, fmaxf(fabsf(r0[pass][e]), fabsf(r1[pass][e])));
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) m = fmaxf(m, __shfl_xor(m, w));
  if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = m;
  __syncthreads();
  const int ex = vt_exponent(fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3])));
  const float down = exp2i(-ex);
  if (threadIdx.x == 0) p.vexp[(int64_t)kvh * (p.vt_cols / kKeyTile) + cb] = ex;
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) {
    const int item = hw + 8 * pass;
    const int c = c_lo + 8 * (item / 8), kp = kp_lo + 4 * (item % 8);
    const f16x8 a = __builtin_convertvector(r0[pass] * down, f16x8), b = __builtin_convertvector(r1[pass] * down, f16x8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const f16x2 pr = {a[e], b[e]};
      tile[(8 * c + e) * 32 + (kp ^ (4 * c_lo))] = __builtin_bit_cast(uint32_t, pr);
    }
  }
  __syncthreads();
  // Out in operand-fragment order: chunk o = (kj * ND + db) * 64 + lane holds
  // d = 32 db + lane % 32, keys 8 q .. 8 q + 7 with q = 2 kj + lane / 32.
  constexpr int ND = D / 32;
  _Float16 *dst = p.vt + ((int64_t)kvh * (p.vt_cols / kKeyTile) + cb) * (D * kKeyTile);
#pragma unroll
  for (int o = threadIdx.x; o < D * 8; o += 256) {
    const int lane = o & 63, db = (o >> 6) % ND, kj = (o >> 6) / ND;
    const int d = 32 * db + (lane & 31), q = 2 * kj + (lane >> 5);
    *gbl_mut(reinterpret_cast<u32x4 *>(dst + 8 * o)) =
        *reinterpret_cast<const u32x4 *>(&tile[d * 32 + 4 * (q ^ ((d >> 3) & 7))]);
  }
}

// ---------------------------------------------------------------- attention
// TQK: matrix-core type of S = K Q^T (q, k and the pasts' k): bf16, fp16 or
// e4m3. P V always runs in fp16: P keeps 11 significant bits instead of
// bf16's 8 (or e4m3's 4), and the V^T copy is fp16.
template <typename TQK, typename TOut, int D>
__global__ __attribute__((amdgpu_flat_work_group_size(Shape<D>::threads, Shape<D>::threads),
                          amdgpu_waves_per_eu(Shape<D>::waves_per_simd, Shape<D>::waves_per_simd)))
void tree_attn_kernel(const KParams args) {
  using L = Lds<D, (int)sizeof(TQK)>;
  constexpr int NB = L::nbuf;
  // Two stage buffers (head_dim 256): 16 queries per wave on 16x16 products,
  // every wave issues, and each step processes one tile while the next one
  // loads.
  constexpr bool kTwoStage = NB == 2;
  static_assert(NB == 4 || (NB == 2 && D == 256), "ring of 4, or 2 at head_dim 256");
  constexpr int WQ = Shape<D>::wave_q;  // queries per wave
  constexpr int kIssuers = Issuers<D>::n;  // waves that issue the stage loads
  constexpr bool kF8 = std::is_same<TQK, E4M3>::value;
  constexpr int KS = QK<TQK>::step;                   // k-step of Q K^T
  constexpr int NK = D / KS;                          // k-steps of Q K^T
  constexpr int CE = 16 / (int)sizeof(TQK);           // K / Q elements per 16-byte chunk
  constexpr int CH = QK<TQK>::chunks;                 // 16-byte chunks per lane per k-step
  constexpr int ND = D / 32;   // 32-row d blocks of O^T
  constexpr int SLOTS = L::slots;
  constexpr int NC = L::kChunks;
  constexpr int RB = L::kRowBytes;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t smem_lds = (uint32_t)(uintptr_t)(DAN_LDS uint8_t *)smem;  // its LDS byte address

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, hl = lane >> 5, lq = lane & 31;
  // The lane's query within the wave, and which part of a k-step of S it
  // holds (32x32 products: two halves; 16x16: four quarters).
  const int lqq = WQ == 16 ? (lane & 15) : lq, kpart = WQ == 16 ? (lane >> 4) : hl;
  // LDS byte offsets of this lane's operand reads (see Lds). K: row lq of a
  // 32-row block with its chunk swizzle and half-step folded in; the chunk
  // of each k-step is XOR'd in per read (it only touches the low bits).
  // V^T: the lane's 16 bytes of each operand fragment block.
  const uint32_t k_lane = (uint32_t)(lq * RB + kswz<D, (int)sizeof(TQK)>(lq) * 16) ^ (uint32_t)(hl * CH * 16);
  const uint32_t v_lane = (uint32_t)(L::kBytes + lane * 16);

  // units holds num_units records: clamping the range keeps a malformed
  // offset table from reading past it.
  const int u_begin = max(load_scalar(args.sched_off + blockIdx.x), 0);
  const int u_end = min(load_scalar(args.sched_off + blockIdx.x + 1), args.num_units);
  // `args` is the first (and only) explicit kernel argument, at the start of
  // the kernarg segment. Each unit reads its fields through an opaque copy
  // of that address, so they are reloaded per unit (scalar loads) instead of
  // being hoisted out of the unit loop and held in SGPRs across the key
  // loop, where they would spill.
  const KArgPtr kseg = (KArgPtr)__builtin_amdgcn_kernarg_segment_ptr();

  // Where a unit's key tiles come from: its segment's new-token keys (kp, in
  // packed rows from `start`), its prefix-cache keys (pkp), and its V^T
  // column blocks (vtp; tile j at vtp + j * D * 64). Tiles are counted along
  // the unit's visit order: [0, ja1) then [jb0, jb1).
  struct Src {
    const TQK *kp, *pkp;
    const _Float16 *vtp;
    int64_t k_st, pk_st;
    int start, P, PN, ja1, jb0, ntile;
  };
  auto make_src = [&](const KParams &p, const DanUnit &un) __attribute__((always_inline)) {
    const int kvh = un.group % p.num_kv_heads;
    Src r;
    r.kp = static_cast<const TQK *>(p.k) + (int64_t)kvh * p.k_sh;
    r.k_st = p.k_st;
    r.pkp = nullptr;
    r.pk_st = 0;
    if (un.past_len > 0) {
      const DanPastDesc pd = load_scalar(p.pasts + un.past_idx);
      r.pkp = static_cast<const TQK *>(pd.k) + (int64_t)kvh * pd.k_stride_head;
      r.pk_st = pd.k_stride_tok;
    }
    r.vtp = p.vt + ((int64_t)kvh * (p.vt_cols / kKeyTile) + un.vt_col / kKeyTile) * (D * kKeyTile);
    r.start = un.start;
    r.P = un.past_len;
    r.PN = un.past_len + un.n;
    r.ja1 = un.item.ja1;
    r.jb0 = un.item.jb0;
    r.ntile = un.item.ja1 + (un.item.jb1 - un.item.jb0);
    return r;
  };
  // A unit record is usable when its head group exists and it visits at
  // least one key tile (every query sees its own key, so a planner never
  // makes an empty item).
  auto valid_unit = [&](const KParams &p, const DanUnit &un) __attribute__((always_inline)) {
    return un.group >= 0 && un.group < p.num_kv_heads * p.chunks && un.item.ja1 >= 0 && un.item.jb1 >= un.item.jb0 &&
           un.item.ja1 + (un.item.jb1 - un.item.jb0) > 0;
  };

  // Direct-load slots. A stage buffer is kBlocks 1 KB blocks of K rows then
  // vBlocks of V^T fragments; issuing wave w loads blocks w, w + kIssuers, ...
  // (SLOTS per tile). Both block counts are multiples of kIssuers, so the
  // first SK slots of every issuing wave are K blocks and the rest V^T blocks.
  // K offsets are per source layout (new tokens / past) and include the row
  // swizzle; V^T offsets are relative to the tile's block of the copy.
  constexpr int SK = L::kBlocks / kIssuers;
  auto k_offset = [&](int blk, int64_t st) __attribute__((always_inline)) {  // bytes
    const int pos = blk * 64 + lane, m = pos / NC;
    const int c = (pos % NC) ^ kswz<D, (int)sizeof(TQK)>(m);
    return (uint32_t)((k_row<D>(m) * st + c * CE) * (int64_t)sizeof(TQK));
  };
  uint32_t off_a[SLOTS];  // K: new-token offsets; V^T: offsets in the copy
  {
    const KParams &p = *(const KParams *)kseg;
#pragma unroll
    for (int sl = 0; sl < SLOTS; ++sl) {
      const int blk = wave + kIssuers * sl;
      off_a[sl] = sl < SK ? k_offset(blk, p.k_st) : (uint32_t)((blk - L::kBlocks) * 1024 + lane * 16);
    }
  }
  // K offsets for a prefix-cache layout of token stride st (zero elsewhere).
  auto past_offsets = [&](int64_t st, uint32_t(&off)[SLOTS]) __attribute__((always_inline)) {
#pragma unroll
    for (int sl = 0; sl < SLOTS; ++sl) {
      const int blk = wave + kIssuers * sl;
      off[sl] = sl < SK ? k_offset(blk, st) : 0u;
    }
  };

  // Issue the direct loads of tile i (visit order) of source u into stage
  // buffer b: the K slots from the tile's source layout (chosen once per
  // tile), then the V^T slots. Every field is wave-uniform; saying so keeps
  // the address arithmetic on the scalar unit (readfirstlane of a value
  // already in SGPRs costs nothing).
  auto issue = [&](const Src &u_any, const uint32_t(&off_b)[SLOTS], int i_any, int b_any) __attribute__((always_inline)) {
    const int i = uni(i_any), b = uni(b_any), P = uni(u_any.P), PN = uni(u_any.PN);
    const int ja1 = uni(u_any.ja1), jb0 = uni(u_any.jb0);
    const int j = i < ja1 ? i : jb0 + (i - ja1);
    const int kb = j * kKeyTile;
    const uint32_t dst = smem_lds + (uint32_t)(b * L::buf + wave * 1024);  // LDS address of slot 0; slot sl + sl * kIssuers KB
    if (kb + kKeyTile <= P) {  // prefix-cache keys
      const TQK *tb = uniform_ptr(uniform_ptr(u_any.pkp) + (int64_t)kb * uni64(u_any.pk_st));
#pragma unroll
      for (int sl = 0; sl < SK; ++sl) dma16(tb, off_b[sl], dst + (uint32_t)(sl * kIssuers * 1024));
    } else if (kb >= P && kb + kKeyTile <= PN) {  // new-token keys
      const TQK *tb = uniform_ptr(uniform_ptr(u_any.kp) + (int64_t)(uni(u_any.start) + kb - P) * uni64(u_any.k_st));
#pragma unroll
      for (int sl = 0; sl < SK; ++sl) dma16(tb, off_a[sl], dst + (uint32_t)(sl * kIssuers * 1024));
    } else {  // the tile straddles the past/new boundary or the segment's end: per-lane rows
      const TQK *kp = uniform_ptr(u_any.kp), *pkp = uniform_ptr(u_any.pkp);
      const int64_t k_st = uni64(u_any.k_st), pk_st = uni64(u_any.pk_st);
      const int start = uni(u_any.start);
#pragma unroll
      for (int sl = 0; sl < SK; ++sl) {
        const int pos = (wave + kIssuers * sl) * 64 + lane, m = pos / NC;
        const int col = CE * ((pos % NC) ^ kswz<D, (int)sizeof(TQK)>(m));
        const int key = min(kb + k_row<D>(m), PN - 1);
        dma16(key < P ? pkp + (int64_t)key * pk_st + col : kp + (int64_t)(start + key - P) * k_st + col,
              dst + (uint32_t)(sl * kIssuers * 1024));
      }
    }
    const _Float16 *vtt = uniform_ptr(uniform_ptr(u_any.vtp) + (int64_t)j * (D * kKeyTile));
#pragma unroll
    for (int sl = SK; sl < SLOTS; ++sl) dma16(vtt, off_a[sl], dst + (uint32_t)(sl * kIssuers * 1024));
  };

  // The stage-buffer ring runs across units: the work group's k-th tile
  // overall (in unit order) uses buffer k % 4. A unit's first three tiles
  // are issued during the previous unit's last three steps, so the tile
  // pipeline does not drain between units. `pre` counts the current unit's
  // tiles the previous unit issued.
  int gbase = 0, pre = 0;
  // Passes over units (a unit run again with the check is a second pass);
  // each pass votes in LDS word pass % 2, past the stage ring.
  int pass = 0;
  bool check = false;
  auto vote_word = [&](int k) __attribute__((always_inline)) -> volatile DAN_LDS uint32_t & {
    return *(volatile DAN_LDS uint32_t *)(uintptr_t)(smem_lds + (uint32_t)L::total + 4u * (uint32_t)(k & 1));
  };
  if constexpr (!kTwoStage) {
    if (tid == 0) {
      vote_word(0) = 0u;
      vote_word(1) = 0u;
    }
  }
  // A wave's q fragments and key_lo for a unit: loaded in the unit's
  // prologue, or, when the previous unit ran here, during that unit's last
  // step (where they are no longer used), so the prologue does not wait a
  // whole memory round trip for them.
  Frag<TQK> qf[NK];
  int qlo = 0;
  bool q_ready = false;
  auto load_q = [&](const KParams &p, const DanUnit &un) __attribute__((always_inline)) {
    const int g = un.group, kvh = g % p.num_kv_heads, chunk = g / p.num_kv_heads;
    const int hig = chunk * p.hpw + (wave % p.hpw), head = kvh * p.rep + hig;
    const int qw0 = un.item.t0 + (wave / p.hpw) * WQ, qend = un.item.t0 + un.item.tq;
    const int ql = qw0 + lqq;
    const bool qvalid = hig < p.rep && qw0 < qend && ql < qend;
    const int qrow = un.start + min(ql, qend - 1);
    qlo = qvalid ? *gbl(p.key_lo + qrow) : 0;
    const TQK *row = static_cast<const TQK *>(p.q) + (int64_t)qrow * p.q_st +
                     (int64_t)min(head, p.num_kv_heads * p.rep - 1) * p.q_sh + KS / 2 * kpart;
    // 16x16 products take k-steps twice as long as the 32x32 ones
    constexpr int QS = WQ == 16 ? 2 * KS : KS;
#pragma unroll
    for (int kk = 0; kk < D / QS; ++kk) qf[kk] = load_frag<TQK>(row + QS * kk);
  };
  for (int u = u_begin; u < u_end; ++u) {
    KArgPtr kp_u = kseg;
    asm volatile("" : "+s"(kp_u));
    const KParams &p = *(const KParams *)kp_u;
    const DanUnit un = load_scalar(p.units + u);  // one read resolves the unit
    if (!valid_unit(p, un)) {  // a malformed unit record: skip it (the previous unit prefetched nothing for it)
      pre = 0;
      continue;
    }
    const int g = un.group;
    const DanWorkItem &w = un.item;
    const int kvh = g % p.num_kv_heads, chunk = g / p.num_kv_heads;
    const Src cur = make_src(p, un);
    const int P = cur.P, PT = P + un.trunk, ntile = cur.ntile;
    // exponents of this unit's V^T column blocks (tile j: vexp_u[j])
    const int32_t *vexp_u = p.vexp + ((int64_t)kvh * (p.vt_cols / kKeyTile) + un.vt_col / kKeyTile);
    uint32_t off_b[SLOTS];
    past_offsets(cur.pk_st, off_b);
    // The next unit, whose first tiles (nn of them) this unit's last steps
    // prefetch. Only its tile count stays live; the few steps that issue its
    // tiles re-read its record (scalar loads).
    int nn = 0;
    if (u + 1 < u_end) {
      const DanUnit un2 = load_scalar(p.units + u + 1);
      if (valid_unit(p, un2)) nn = min(un2.item.ja1 + (un2.item.jb1 - un2.item.jb0), 3);
    }
    // Tile i of the concatenation [this unit; the next unit's first nn tiles].
    auto issue_cat = [&](int i) __attribute__((always_inline)) {
      if (i < ntile) {
        issue(cur, off_b, i, (gbase + i) & (NB - 1));
      } else if (i - ntile < nn) {
        const Src nxt = make_src(p, load_scalar(p.units + u + 1));
        uint32_t off_nb[SLOTS];
        past_offsets(nxt.pk_st, off_nb);
        issue(nxt, off_nb, i - ntile, (gbase + i) & (NB - 1));
      }
    };
    auto issued_cat = [&](int i) __attribute__((always_inline)) { return i < ntile + nn; };

    const int hig = chunk * p.hpw + (wave % p.hpw);
    const int head = kvh * p.rep + hig;
    const int qw0 = w.t0 + (wave / p.hpw) * WQ;  // wave's first query (segment-local)
    const int qend = w.t0 + w.tq;
    const bool wave_work = hig < p.rep && qw0 < qend;

    // Softmax exponent factor c of S: scale * log2(e), times q_scale * k_scale
    // for scaled inputs -- e4m3, and fp32 q / k staged to fp16 with power-of-2
    // scales (the prefix-cache entry's k has its own scale, c_past).
    float c_new = p.c, c_past = p.c;
    if (kF8 || p.q_scale) {
      const float qs = load_scalar(p.q_scale);
      c_new = c_past = p.c * qs * load_scalar(p.k_scale);
      if (P > 0) c_past = p.c * qs * load_scalar(load_scalar(p.pasts + un.past_idx).k_scale);
    }

    // Per-lane query state: lane owns query column lq of its wave. Padding
    // columns (past the tile, or an idle wave) read a clamped valid row and see
    // every key, so they stay finite; they are never stored.
    const int ql = qw0 + lqq;
    const bool qvalid = wave_work && ql < qend;
    const int qk = qvalid ? P + ql : 0x3fffffff;

    f32x16 o[ND];
#pragma unroll
    for (int db = 0; db < ND; ++db) o[db] = f32x16{};
    float mneg, lsum = 0.f;  // exponent offset -m of the running max m
    // O holds O_true * 2^-vE: the exponent of the V^T blocks it was last
    // accumulated from (0 unless a block of this unit needed one).
    int vE = 0;
    u32x4 pf[4];  // P^T B operands (fp16), one per 16 keys of the tile

    // S^T = K Q^T for the 64 keys of stage buffer b x this wave's 32 queries.
    auto qk_phase = [&](int b, f32x16(&s)[2], auto &&after_kstep) {
      // LDS address of this lane's row in buffer b. The dynamic LDS block is
      // the kernel's only LDS object and starts at address 0, and buffer
      // offsets are multiples of 32 rows, so XOR-ing a chunk into the address
      // only changes the lane's row offset: one v_xor per k-step.
      const uint32_t kbase = (uint32_t)(uintptr_t)(DAN_LDS uint8_t *)(smem + b * L::buf) + k_lane;
      s[0] = f32x16{};
      s[1] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        Frag<TQK> a[2];
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          const uint32_t off = kbase ^ (uint32_t)((2 * kk * CH + i) * 16);
#pragma unroll
          for (int mb = 0; mb < 2; ++mb)
            a[mb].c[i] = *reinterpret_cast<const DAN_LDS u32x4 *>((uintptr_t)(off + mb * 32 * RB));
        }
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) s[mb] = mfma_qk<TQK>(a[mb], qf[kk], s[mb]);
        after_kstep(kk);
      }
    };
    // Tree mask on boundary tiles. Key index of register r relative to the tile
    // start: 32*mb + 16*(r/8) + 8*hl + r%8. The causal limit and the
    // sibling-branch gap are per-lane bounds on it; the gap test runs only on
    // tiles meeting [PT, lo_max).
    auto mask_phase = [&](int j, f32x16(&s)[2]) {
      if (j < w.jfull) return;
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
    };
    // Exponent factor of tile j's scores, and (scaled inputs) the fix-up of a
    // tile that holds both prefix-cache and new keys: the prefix keys' scores
    // are brought to the new keys' k scale, and the tile then uses c_new.
    auto tile_c = [&](int j) __attribute__((always_inline)) { return j * kKeyTile + kKeyTile <= P ? c_past : c_new; };
    auto fix_straddle = [&](int j, f32x16(&s)[2]) __attribute__((always_inline)) {
      const int kb = j * kKeyTile;
      if (c_past == c_new || !(kb < P && kb + kKeyTile > P)) return;
      const float ratio = c_past / c_new;
      const int lim = P - kb - 8 * hl;  // prefix key: rel < lim
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rel = 32 * mb + 16 * (r >> 3) + (r & 7);
          s[mb][r] = rel < lim ? s[mb][r] * ratio : s[mb][r];
        }
    };
    // Softmax of one tile (VALU): P = exp2(S * c - m) in fp16 and the lane's
    // partial row sum of the fp16-rounded values that P V uses (exact products,
    // fp32 accumulation), so rounding P mostly cancels in O / l. The running
    // max m is not recomputed per tile. A unit's first pass keeps m at the
    // first tile's max: p may then exceed 2^15 (fine) or overflow fp16 to inf,
    // which the row sum shows at the unit's end, and the work group runs the
    // unit again with the check (two ring-of-four passes; the two-buffer
    // instantiation always checks). With the check, a lane score above
    // m + kLog2Limit (or a NaN) in any lane raises m to the tile's max (O and l
    // rescaled) before the tile's exponentials, so every p stays below 2^15;
    // the check reads S only, so P V does not wait on the row sum. A lane
    // holds half of its query's keys and the other half sits in lane ^ 32;
    // both keep the same m.
    // max S over the lane's 32 keys: a tree of three-input maxima (v_max3_f32,
    // two values per instruction): 32 -> 12 -> 4 -> 1 in 16 instructions.
    auto lane_max = [&](const f32x16(&s)[2]) __attribute__((always_inline)) {
      auto e = [&](int i) __attribute__((always_inline)) { return s[i >> 4][i & 15]; };
      auto max3 = [](float a, float b, float c) __attribute__((always_inline)) { return fmaxf(fmaxf(a, b), c); };
      float m12[12];
#pragma unroll
      for (int i = 0; i < 10; ++i) m12[i] = max3(e(3 * i), e(3 * i + 1), e(3 * i + 2));
      m12[10] = e(30);
      m12[11] = e(31);
      float m4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) m4[i] = max3(m12[3 * i], m12[3 * i + 1], m12[3 * i + 2]);
      return fmaxf(max3(m4[0], m4[1], m4[2]), m4[3]);
    };
    auto s_max = [&](const f32x16(&s)[2]) __attribute__((always_inline)) {  // max S over the query's keys
      const LanePair mp = lane_pair(lane_max(s));
      return fmaxf(mp.self, mp.other);
    };
    auto exp_phase = [&](const f32x16(&s)[2], float c) __attribute__((always_inline)) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        f32x8 x0, x1;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          x0[r] = __builtin_amdgcn_exp2f(fmaf(s[mb][r], c, mneg));
          x1[r] = __builtin_amdgcn_exp2f(fmaf(s[mb][r + 8], c, mneg));
        }
        pf[2 * mb] = pack8<_Float16>(x0);
        pf[2 * mb + 1] = pack8<_Float16>(x1);
      }
      float acc[4];
#pragma unroll
      for (int kj = 0; kj < 4; ++kj) {  // four short chains instead of one long one
        const f16x8 h = __builtin_bit_cast(f16x8, pf[kj]);
        acc[kj] = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 0, 1), kOnes2, 0.f, false);
        acc[kj] = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 2, 3), kOnes2, acc[kj], false);
        acc[kj] = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 4, 5), kOnes2, acc[kj], false);
        acc[kj] = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 6, 7), kOnes2, acc[kj], false);
      }
      return (acc[0] + acc[1]) + (acc[2] + acc[3]);
    };
    // Before a tile's softmax: raise m to the tile's max if some score would
    // put p above 2^kLog2Limit, and bring O to the scale of the tile's V^T
    // block (2^ve) if it differs from O's (2^vE). Both are rare and share one
    // branch.
    // Without the check (kCheck false) no score raises m: a p that overflows
    // fp16 becomes inf, which the row sum carries to the unit's end, where
    // the work group then runs the unit again with the check (see the vote).
    auto begin_tile = [&](bool chk, const f32x16(&s)[2], float c, int ve) __attribute__((always_inline)) {
      bool raise = false;
      if (chk) raise = __any(!(fmaf(lane_max(s), c, mneg) <= kLog2Limit));
      if (raise || ve != vE) {
        float f = exp2i(vE - ve);
        if (raise) {
          const float mold = -mneg;
          const float mnew = fmaxf(mold, s_max(s) * c);
          const float alpha = __builtin_amdgcn_exp2f(mold - mnew);
          mneg = -mnew;
          lsum *= alpha;
          f *= alpha;
        }
#pragma unroll
        for (int db = 0; db < ND; ++db) o[db] *= f;
        vE = ve;
      }
    };
    // O^T += V^T P^T over the 64 keys of stage buffer b (its V^T block is at
    // O's scale: begin_tile).
    auto pv_phase = [&](int b) __attribute__((always_inline)) {
      const uint8_t *vbuf = smem + b * L::buf + v_lane;
#pragma unroll
      for (int kj = 0; kj < 4; ++kj) {
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          const u32x4 a = *reinterpret_cast<const u32x4 *>(vbuf + (kj * ND + db) * 1024);
          o[db] = mfma32<_Float16>(a, pf[kj], o[db]);
        }
      }
    };

    auto tile_of = [&](int i) __attribute__((always_inline)) { return i < w.ja1 ? i : w.jb0 + (i - w.ja1); };

    if constexpr (kTwoStage) {
      // head_dim 256: 16 queries per wave on 16x16 products, two waves per
      // SIMD, two stage buffers. Each step waits for its tile, passes the
      // barrier (after which the other buffer, last used by the previous step,
      // is free), the issuing waves load the next tile there, and every wave
      // processes its own: S, mask, softmax, then O += V P. The running max
      // starts at the first tile's largest visible score and is raised per
      // tile when a score would put p above 2^kLog2Limit.
      static_assert(L::kRowsPerPeriod == 1 && L::kSwizzle == 16, "the K row swizzle of the 16x16 reads");
      constexpr int NK2 = D / (2 * KS);   // k-steps of S (16x16 products)
      constexpr int CPK = 2 * KS / CE;    // 16-byte chunks per k-step and row
      constexpr int NDB = D / 16;         // 16-row d blocks of O^T
      const int q4 = lane >> 4, l16 = lane & 15;
      f32x4 o4[NDB];
#pragma unroll
      for (int db = 0; db < NDB; ++db) o4[db] = f32x4{};
      u32x4 pf2[2];  // P^T of the tile (fp16): keys 32 g + 8 q4 .. + 7
      // S^T = K Q^T: block bb of 16 keys (LDS rows 16 bb .. + 15), lane row
      // 16 bb + l16 whose swizzle is l16, k-step kk's chunks kk CPK + q4 CH + i.
      auto qk16 = [&](int b, f32x4(&s)[4], auto &&after_kstep) __attribute__((always_inline)) {
        const uint32_t base = smem_lds + (uint32_t)(b * L::buf + l16 * RB);
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) s[bb] = f32x4{};
        constexpr int W = 1;  // k-steps of operand fragments read ahead
        Frag<TQK> a[NK2][4];
        auto rd = [&](int kk) __attribute__((always_inline)) {
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            const uint32_t off = base + (uint32_t)(((kk * CPK + q4 * CH + i) ^ l16) * 16);
#pragma unroll
            for (int bb = 0; bb < 4; ++bb)
              a[kk][bb].c[i] = *reinterpret_cast<const DAN_LDS u32x4 *>((uintptr_t)(off + bb * 16 * RB));
          }
        };
#pragma unroll
        for (int kk = 0; kk < W; ++kk) rd(kk);
#pragma unroll
        for (int kk = 0; kk < NK2; ++kk) {
          if (kk + W < NK2) rd(kk + W);
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) s[bb] = mfma16_qk<TQK>(a[kk][bb], qf[kk], s[bb]);
          after_kstep(kk);
        }
      };
      // key (within the tile) of register e of block bb in this lane
      auto rel16 = [&](int bb, int e) __attribute__((always_inline)) { return 32 * (bb >> 1) + 8 * q4 + 4 * (bb & 1) + e; };
      auto mask16 = [&](int j, f32x4(&s)[4]) __attribute__((always_inline)) {
        if (j < w.jfull) return;
        const int kb = j * kKeyTile;
        const int lim = qk - kb;  // visible: rel <= lim
        if (kb + kKeyTile > PT && kb < w.lo_max) {
          const int g0 = PT - kb, g1 = qlo - kb;  // hidden: g0 <= rel < g1
#pragma unroll
          for (int bb = 0; bb < 4; ++bb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int rel = rel16(bb, e);
              s[bb][e] = rel <= lim && (rel < g0 || rel >= g1) ? s[bb][e] : -INFINITY;
            }
        } else {
#pragma unroll
          for (int bb = 0; bb < 4; ++bb)
#pragma unroll
            for (int e = 0; e < 4; ++e) s[bb][e] = rel16(bb, e) <= lim ? s[bb][e] : -INFINITY;
        }
      };
      auto fix16 = [&](int j, f32x4(&s)[4]) __attribute__((always_inline)) {
        const int kb = j * kKeyTile;
        if (c_past == c_new || !(kb < P && kb + kKeyTile > P)) return;
        const float ratio = c_past / c_new;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb)
#pragma unroll
          for (int e = 0; e < 4; ++e) s[bb][e] = rel16(bb, e) < P - kb ? s[bb][e] * ratio : s[bb][e];
      };
      // the lane's largest score (16), and its query's (the lanes l16 + 16 q)
      auto lmax16 = [&](const f32x4(&s)[4]) __attribute__((always_inline)) {
        auto max3 = [](float a, float b, float c) __attribute__((always_inline)) { return fmaxf(fmaxf(a, b), c); };
        const float a0 = max3(s[0][0], s[0][1], s[0][2]), a1 = max3(s[0][3], s[1][0], s[1][1]);
        const float a2 = max3(s[1][2], s[1][3], s[2][0]), a3 = max3(s[2][1], s[2][2], s[2][3]);
        const float a4 = max3(s[3][0], s[3][1], s[3][2]);
        return fmaxf(max3(a0, a1, a2), max3(a3, a4, s[3][3]));
      };
      auto qmax16 = [&](const f32x4(&s)[4]) __attribute__((always_inline)) {
        float m = lmax16(s);
        m = fmaxf(m, __shfl_xor(m, 16));
        return fmaxf(m, __shfl_xor(m, 32));
      };
      auto begin16 = [&](const f32x4(&s)[4], float c, int ve) __attribute__((always_inline)) {
        const bool raise = __any(!(fmaf(lmax16(s), c, mneg) <= kLog2Limit));
        if (raise || ve != vE) {
          float f = exp2i(vE - ve);
          if (raise) {
            const float mold = -mneg;
            const float mnew = fmaxf(mold, qmax16(s) * c);
            const float alpha = __builtin_amdgcn_exp2f(mold - mnew);
            mneg = -mnew;
            lsum *= alpha;
            f *= alpha;
          }
#pragma unroll
          for (int db = 0; db < NDB; ++db) o4[db] *= f;
          vE = ve;
        }
      };
      auto exp16 = [&](const f32x4(&s)[4], float c) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          f32x8 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x[e] = __builtin_amdgcn_exp2f(fmaf(s[2 * g][e], c, mneg));
            x[4 + e] = __builtin_amdgcn_exp2f(fmaf(s[2 * g + 1][e], c, mneg));
          }
          pf2[g] = pack8<_Float16>(x);
        }
        float acc[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const f16x8 h = __builtin_bit_cast(f16x8, pf2[g]);
          acc[g] = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 0, 1), kOnes2, 0.f, false);
          acc[g] = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 2, 3), kOnes2, acc[g], false);
          acc[g] = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 4, 5), kOnes2, acc[g], false);
          acc[g] = __builtin_amdgcn_fdot2(__builtin_shufflevector(h, h, 6, 7), kOnes2, acc[g], false);
        }
        return acc[0] + acc[1];
      };
      // O^T += V^T P^T: the A fragment of d block dbb (16 rows) and key group g
      // (32 keys) is read from the copy's 32x32 fragments: lane (l16, q4)
      // holds d 16 dbb + l16, keys 32 g + 8 q4 .. + 7, which is lane
      // 32 (q4 % 2) + 16 (dbb % 2) + l16 of fragment (key group 2 g + q4 / 2,
      // d block dbb / 2).
      const uint32_t vlane16 = (uint32_t)(L::kBytes + (q4 >> 1) * ND * 1024 + (32 * (q4 & 1) + l16) * 16);
      auto pv16 = [&](int b) __attribute__((always_inline)) {
        const uint32_t vb = smem_lds + (uint32_t)(b * L::buf) + vlane16;
        constexpr int NV = 2 * NDB, WV = 2;
        u32x4 a[NV];
        auto rd = [&](int i) __attribute__((always_inline)) {
          const int g = i / NDB, db = i % NDB;
          a[i] = *reinterpret_cast<const DAN_LDS u32x4 *>((uintptr_t)(vb + (uint32_t)((2 * g * ND + db / 2) * 1024 + (db & 1) * 256)));
        };
#pragma unroll
        for (int i = 0; i < WV; ++i) rd(i);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          if (i + WV < NV) rd(i + WV);
          o4[i % NDB] = mfma16<_Float16>(a[i], pf2[i / NDB], o4[i % NDB]);
        }
      };

      if (wave < kIssuers) issue(cur, off_b, 0, gbase & (NB - 1));
      load_q(p, un);
      f32x4 s[4];
      for (int it = 0; it < ntile; ++it) {
        wait_vmem<0>();
        barrier_lds();
        const int ve = load_scalar(vexp_u + tile_of(it));
        // The next tile's loads go out over this tile's S products (two per
        // k-step); a tile straddling the past/new boundary issues them all now.
        int kind = 2;
        const TQK *sp_tb = cur.kp;
        const _Float16 *sp_vtt = cur.vtp;
        uint32_t sp_dst = 0;
        if (it + 1 < ntile) {
          const int i = it + 1, j = tile_of(i), kb = j * kKeyTile;
          kind = kb + kKeyTile <= P ? 0 : (kb >= P && kb + kKeyTile <= cur.PN) ? 1 : 2;
          sp_tb = kind == 0 ? cur.pkp + (int64_t)kb * cur.pk_st : cur.kp + (int64_t)(cur.start + kb - P) * cur.k_st;
          sp_vtt = cur.vtp + (int64_t)j * (D * kKeyTile);
          sp_dst = smem_lds + (uint32_t)(((gbase + i) & (NB - 1)) * L::buf + wave * 1024);
          if (kind == 2 && wave < kIssuers) issue(cur, off_b, i, (gbase + i) & (NB - 1));
        }
        if (kind != 2 && wave < kIssuers) {
          qk16((gbase + it) & (NB - 1), s, [&](int kk) __attribute__((always_inline)) {
#pragma unroll
            for (int sl = kk * SLOTS / NK2; sl < (kk + 1) * SLOTS / NK2; ++sl) {
              if (sl < SK) dma16(sp_tb, kind == 0 ? off_b[sl] : off_a[sl], sp_dst + (uint32_t)(sl * kIssuers * 1024));
              else dma16(sp_vtt, off_a[sl], sp_dst + (uint32_t)(sl * kIssuers * 1024));
            }
          });
        } else {
          qk16((gbase + it) & (NB - 1), s, [](int) {});
        }
        mask16(tile_of(it), s);
        fix16(tile_of(it), s);
        const float c = tile_c(tile_of(it));
        if (it == 0) mneg = -fmaxf(qmax16(s) * c, -3.0e38f);
        begin16(s, c, ve);
        lsum += exp16(s, c);
        pv16((gbase + it) & (NB - 1));
      }
      // Epilogue: O = O^T / l, the query's l summed over its four lanes.
      // Lane (l16, q4) holds d 16 db + 4 q4 .. + 3 of block db.
      float l = lsum + __shfl_xor(lsum, 16);
      l += __shfl_xor(l, 32);
      const float linv = l > 0.f ? exp2i(vE) / l : 0.f;
      TOut *orow = static_cast<TOut *>(p.o) + (int64_t)(cur.start + ql) * p.o_st + (int64_t)head * p.o_sh;
      if (qvalid) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) store4<TOut>(orow + 16 * db + 4 * q4, o4[db] * linv);
      }
      nn = 0;
    } else {
      // Prologue: the tiles 0..2 the previous unit did not prefetch, and the
      // next unit's tiles that fall within three of this unit's start (when this
      // unit is shorter than three tiles), then q and key_lo. The buffers they
      // go to held tiles that every wave finished before the previous unit's
      // last barrier. Waiting for q (a load the compiler sees, issued last)
      // also completes every direct load issued before it.
      if (wave < kIssuers) {
  #pragma unroll
        for (int t = 0; t < 3; ++t)
          if (t >= pre && t < ntile) issue(cur, off_b, t, (gbase + t) & (NB - 1));
        for (int t = ntile; t < 3; ++t) issue_cat(t);
      }
      if (!q_ready) load_q(p, un);
      q_ready = false;
      wait_vmem<0>();
      barrier_lds();
      // Every wave has read the previous pass's vote: its word is the next
      // pass's, cleared now.
      if (tid == 0) vote_word(pass + 1) = 0u;
      f32x16 sc[2];  // S of the current tile
      // The running max m starts at the largest visible score of the first
      // tile (exact, so that tile's largest p is 1). A query that sees no key
      // of the first tile (only when the segment has neither past nor trunk)
      // starts from m = -3e38: its p stay 0 while its keys are hidden, and its
      // first visible key scores far above m + kLog2Limit, which overflows
      // without the check and, with it, raises m to that tile's max (O and l
      // are still 0, scaled by exp2(-3e38 - m) = 0). Finite throughout, so no
      // inf - inf.
      qk_phase(gbase & (NB - 1), sc, [](int) {});
      mask_phase(tile_of(0), sc);
      fix_straddle(tile_of(0), sc);
      mneg = -fmaxf(s_max(sc) * tile_c(tile_of(0)), -3.0e38f);

      // Step `it`: P of tile it (VALU) while S of tile it+1 runs on the matrix
      // core, then O += V P of tile it while the VALU masks S(it+1). S(it+1)
      // goes to the registers of S(it): each product starts once the softmax
      // has read the scores it overwrites. The last step of the unit has no
      // next tile. Every step starts with a barrier,
      // after which tile it+3 of the concatenation (this unit, then the next
      // unit's first tiles) is issued into the buffer that tile it-1 used:
      // every wave has finished tile it-1 before the barrier.
      int it = 0;
      auto step = [&](auto last, f32x16(&s)[2]) {
        constexpr bool kLast = decltype(last)::value;
        if (!kLast && wave < kIssuers) {
          if (issued_cat(it + 2)) wait_vmem<SLOTS>();  // tile it+1 landed; it+2 may be in flight
          else wait_vmem<0>();
        }
        barrier_lds();
        const int ve = load_scalar(vexp_u + tile_of(it));  // the tile's V^T exponent (begin_tile)
        // The issuing waves load tile it+3 now (see kIssuers).
        if (wave < kIssuers) issue_cat(it + 3);
        if (kLast && nn > 0) {  // q and key_lo of the next unit (this unit's are no longer used)
          load_q(p, load_scalar(p.units + u + 1));
          q_ready = true;
        }
        const float c = tile_c(tile_of(it));
        begin_tile(check, s, c, ve);
        const float ts = exp_phase(s, c);
        if (!kLast) qk_phase((gbase + it + 1) & (NB - 1), s, [](int) {});
        lsum += ts;
        pv_phase((gbase + it) & (NB - 1));
        if (!kLast) {
          mask_phase(tile_of(it + 1), s);
          fix_straddle(tile_of(it + 1), s);
        }
        ++it;
      };
      using NotLast = std::integral_constant<bool, false>;
      using Last = std::integral_constant<bool, true>;
      while (it + 1 < ntile) step(NotLast{}, sc);
      step(Last{}, sc);
      // The overflow vote. A pass without the check is exact unless some p
      // overflowed fp16 (a score about 16 above the running max, or a NaN):
      // then that query's row sum is inf or NaN. If any valid query of the
      // work group has one, the work group runs the unit again with the
      // check, after its loads have landed (the next unit's first tiles are
      // issued again by that pass).
      if (!check) {
        const float lt = lsum + __shfl_xor(lsum, 32);
        const bool bad = qvalid && (__builtin_bit_cast(uint32_t, lt) & 0x7f800000u) == 0x7f800000u;
        if (__any(bad) && lane == 0) vote_word(pass) = 1u;
        barrier_lds();
        const bool replay = __builtin_amdgcn_readfirstlane(vote_word(pass)) != 0u;
        ++pass;
        if (replay) {
          wait_vmem<0>();
          barrier_lds();
          check = true;
          q_ready = false;
          gbase += ntile;
          pre = 0;
          --u;
          continue;
        }
      } else {
        ++pass;
        check = false;
      }
    }

    if constexpr (!kTwoStage) {
      // Epilogue: O = O^T / l, written token-major [N, H, D]. Register group
      // r4 of block db holds d = 32 db + 8 r4 + 4 hl + (0..3); lanes l and
      // l ^ 32 (the same query) trade halves so that each stores 8 contiguous
      // d: lane hl = 0 the even groups, hl = 1 the odd ones.
      const float l = lsum + __shfl_xor(lsum, 32);
      const float linv = l > 0.f ? exp2i(vE) / l : 0.f;
      TOut *orow = static_cast<TOut *>(p.o) + (int64_t)(cur.start + ql) * p.o_st + (int64_t)head * p.o_sh;
  #pragma unroll
      for (int db = 0; db < ND; ++db)
  #pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
          const Out4<TOut> e = pack_out<TOut>(o[db], 8 * jp, linv), od = pack_out<TOut>(o[db], 8 * jp + 4, linv);
          // v_permlane32_swap(e, od) leaves lanes below 32 (e, partner's e) and lanes from 32
          // (partner's od, od): each lane's 8 contiguous d in order, with no select.
          Out4<TOut> first, second;
  #pragma unroll
          for (int w4 = 0; w4 < Out4<TOut>::kWords; ++w4) {
            const auto sw = __builtin_amdgcn_permlane32_swap(e.w[w4], od.w[w4], false, false);
            first.w[w4] = sw[0];
            second.w[w4] = sw[1];
          }
          if (qvalid) store8<TOut>(orow + 32 * db + 8 * (2 * jp + hl), first, second);
        }
    }
    gbase += ntile;
    pre = nn;
  }  // units
}

// ---------------------------------------------------------------- fp32 -> fp16 staging
// q and k of fp32 callers become fp16 for the matrix core with a per-tensor
// power-of-2 scale (x = out * scale, exact), so magnitudes beyond fp16's
// range neither overflow nor flush. Two launches over the same grid: the
// partial maxima, then every work group reduces them, takes the exponent
// (vt_exponent's rule) and converts its share.
struct StageParams {
  const float *x;
  int64_t s0, s1;  // strides of dims 0 and 1 (dim 2 contiguous)
  int32_t d0, d1, d2;
  _Float16 *out;   // [d0][d1][d2] contiguous
  float *scale;    // receives 2^e
  float *partial;  // [gridDim.x] partial maxima
};

__device__ inline float block_max256(float m, float *red) {
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) m = fmaxf(m, __shfl_xor(m, w));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__global__ __launch_bounds__(256) void stage_max_kernel(const StageParams p) {
  __shared__ float red[4];
  const int c4 = p.d2 / 4;
  const int64_t n = (int64_t)p.d0 * p.d1 * c4;
  float m = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / c4;
    const f32x4 v = *gbl(reinterpret_cast<const f32x4 *>(p.x + (r / p.d1) * p.s0 + (r % p.d1) * p.s1 + 4 * (i % c4)));
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  }
  m = block_max256(m, red);
  if (threadIdx.x == 0) p.partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(256) void stage_convert_kernel(const StageParams p) {
  __shared__ float red[4];
  float m = 0.f;
  for (int i = threadIdx.x; i < (int)gridDim.x; i += 256) m = fmaxf(m, *gbl(p.partial + i));
  const int ex = vt_exponent(block_max256(m, red));
  const float down = exp2i(-ex);
  if (blockIdx.x == 0 && threadIdx.x == 0) *gbl_mut(p.scale) = exp2i(ex);
  const int c4 = p.d2 / 4;
  const int64_t n = (int64_t)p.d0 * p.d1 * c4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / c4;
    const f32x4 v = *gbl(reinterpret_cast<const f32x4 *>(p.x + (r / p.d1) * p.s0 + (r % p.d1) * p.s1 + 4 * (i % c4)));
    *gbl_mut(reinterpret_cast<u32x2 *>(p.out + 4 * i)) = __builtin_bit_cast(u32x2, __builtin_convertvector(v * down, f16x4));
  }
}

// ---------------------------------------------------------------- host side
thread_local char g_err[512];

// Argument checks on float values read their bits: the library's device code
// is built with -fno-honor-nans, under which the compiler may fold a NaN
// comparison (x != x, !(x > 0)) to a constant.
bool finite_positive(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  return b != 0 && b < 0x7f800000u;  // +0, negatives (sign bit), inf and NaN fail
}
bool finite_nonnegative(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  return b < 0x7f800000u || b == 0x80000000u;  // +-0 or a finite positive
}

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return status;
}

// Bytes of the fp16 V^T copy at the start of the workspace; the column
// blocks' int32 exponents follow it.
int64_t vt_bytes(int32_t num_kv_heads, int32_t head_dim, int32_t vt_cols) {
  return (int64_t)num_kv_heads * head_dim * vt_cols * 2;
}

// Heads of one kv group that one work group covers: the 4 waves of a SIMD
// pair's group split over them.
int heads_per_group(int rep) { return rep >= 3 ? 4 : rep; }

// The V^T scratch of dan_tree_attn_fwd_noalloc: a device array in every GPU's
// memory for the life of the process. In host code `scratch` names a host-side
// stand-in, never the device memory: kernels get the per-device address that
// hipGetSymbolAddress returns (scratch_address below).
static __device__ __align__(256) uint8_t scratch[DAN_TREE_ATTN_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the device `stream` launches on, looked up once
// per device with that device current. 0 on success.
int scratch_address(hipStream_t stream, void **out) {
  int dev = -1;
  hipError_t err = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "cannot find the stream's device: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices) return fail(DAN_ERR_UNSUPPORTED, "device %d: the library serves devices 0..%d", dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if ((err = hipGetDevice(&cur)) != hipSuccess) return fail(DAN_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(err));
    if (cur != dev && (err = hipSetDevice(dev)) != hipSuccess)
      return fail(DAN_ERR_LAUNCH, "hipSetDevice(%d): %s", dev, hipGetErrorString(err));
    void *ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (err != hipSuccess || !ptr)
      return fail(DAN_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(err));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return DAN_OK;
}

template <typename TV, int D>
hipError_t launch_pack(const PackParams &pp, int blocks, hipStream_t stream) {
  hipLaunchKernelGGL((vt_pack_kernel<TV, D>), dim3(blocks), dim3(256), 0, stream, pp);
  return hipGetLastError();
}

template <typename TQK, typename TOut, int D>
hipError_t launch_attn(const KParams &kp, int grid, hipStream_t stream) {
  auto kernel = tree_attn_kernel<TQK, TOut, D>;
  constexpr int lds = Lds<D, (int)sizeof(TQK)>::total + kVoteBytes;
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(Shape<D>::threads), lds, stream, kp);
  return hipGetLastError();
}

}  // namespace dan

extern "C" {

int dan_tree_attn_abi_version(void) { return DAN_TREE_ATTN_ABI_VERSION; }

const char *dan_tree_attn_last_error(void) { return dan::g_err; }

int dan_tree_attn_tile_q(int32_t num_heads, int32_t num_kv_heads, int32_t head_dim) {
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
  return dan::wave_q_for(head_dim) * dan::Shape<128>::waves / dan::heads_per_group(num_heads / num_kv_heads);
}

int dan_tree_attn_head_groups(int32_t num_heads, int32_t num_kv_heads) {
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  const int rep = num_heads / num_kv_heads, hpw = dan::heads_per_group(rep);
  return num_kv_heads * ((rep + hpw - 1) / hpw);
}

int64_t dan_tree_attn_workspace_size(int32_t num_kv_heads, int32_t head_dim, int32_t vt_cols) {
  if (num_kv_heads <= 0 || head_dim <= 0 || vt_cols < 0 || vt_cols % dan::kKeyTile) return 0;
  return dan::vt_bytes(num_kv_heads, head_dim, vt_cols) + ((int64_t)num_kv_heads * (vt_cols / dan::kKeyTile) * 4 + 255) / 256 * 256;
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
  if (D != 64 && D != 128 && D != 256) return fail(DAN_ERR_UNSUPPORTED, "head_dim %d: only 64, 128 and 256 are built", D);
  const int rep = H / Hkv;
  const int tq = dan_tree_attn_tile_q(H, Hkv, D);
  if (a->tile_q != tq) return fail(DAN_ERR_INVALID_ARGUMENT, "tile_q %d, the kernel needs %d", a->tile_q, tq);
  const int in = a->in_dtype, vd = a->v_dtype, out = a->out_dtype;
  const bool bf16 = in == DAN_DTYPE_BF16 && vd == DAN_DTYPE_BF16 && out == DAN_DTYPE_BF16;
  const bool f16 = in == DAN_DTYPE_F16 && vd == DAN_DTYPE_F16 && out == DAN_DTYPE_F16;
  const bool f32 = in == DAN_DTYPE_F16 && vd == DAN_DTYPE_F32 && out == DAN_DTYPE_F32;
  const bool f8 = in == DAN_DTYPE_E4M3 && vd == DAN_DTYPE_E4M3 && out == DAN_DTYPE_BF16;
  if (!bf16 && !f16 && !f32 && !f8)
    return fail(DAN_ERR_UNSUPPORTED, "dtype combination q/k=%d v=%d out=%d is not built", in, vd, out);
  if (a->num_work < 0 || a->num_segments < 0 || a->num_pasts < 0 || a->num_tokens < 0 || a->vt_cols < 0)
    return fail(DAN_ERR_INVALID_ARGUMENT, "negative count");
  if (a->num_work == 0) return DAN_OK;
  if (!a->q || !a->k || !a->v || !a->out || !a->segments || !a->work || !a->key_lo || !a->col_seg)
    return fail(DAN_ERR_INVALID_ARGUMENT, "NULL tensor or table pointer");
  if (a->num_pasts > 0 && !a->pasts) return fail(DAN_ERR_INVALID_ARGUMENT, "num_pasts > 0 with NULL pasts");
  if (f8 && (!a->q_scale || !a->k_scale || !a->v_scale))
    return fail(DAN_ERR_INVALID_ARGUMENT, "e4m3 inputs need q_scale, k_scale and v_scale");
  if (!f8 && (!a->q_scale != !a->k_scale || (a->q_scale && !f32)))
    return fail(DAN_ERR_INVALID_ARGUMENT, "q_scale and k_scale go together, and only with e4m3 or fp32-staged inputs");
  if (!finite_positive(a->scale)) return fail(DAN_ERR_INVALID_ARGUMENT, "scale must be finite and > 0");
  if (a->phases < DAN_TREE_ATTN_PHASES_ALL || a->phases > DAN_TREE_ATTN_PHASE_ATTEND)
    return fail(DAN_ERR_INVALID_ARGUMENT, "phases %d: 0 (all), 1 (pack) or 2 (attend)", a->phases);
  const int64_t need = dan_tree_attn_workspace_size(Hkv, D, a->vt_cols);
  if (a->vt_cols <= 0 || need <= 0) return fail(DAN_ERR_INVALID_ARGUMENT, "vt_cols %d must be a positive multiple of %d", a->vt_cols, kKeyTile);
  if (!a->workspace || a->workspace_bytes < need || ((uintptr_t)a->workspace & 255))
    return fail(DAN_ERR_INVALID_ARGUMENT, "workspace needs %lld bytes, 256-byte aligned", (long long)need);
  // Rows are read and written in 16-byte pieces: every row start must be
  // 16-byte aligned (the wrapper passes a contiguous copy otherwise).
  {
    const int es_in = in == DAN_DTYPE_E4M3 ? 1 : 2, es_v = vd == DAN_DTYPE_F32 ? 4 : vd == DAN_DTYPE_E4M3 ? 1 : 2;
    const int es_out = out == DAN_DTYPE_F32 ? 4 : 2;
    const int64_t row_bytes[] = {a->q_stride_tok * es_in, a->q_stride_head * es_in, a->k_stride_tok * es_in,
                                 a->k_stride_head * es_in, a->v_stride_tok * es_v, a->v_stride_head * es_v,
                                 a->o_stride_tok * es_out, a->o_stride_head * es_out};
    for (int64_t b : row_bytes)
      if (b % 16) return fail(DAN_ERR_INVALID_ARGUMENT, "strides must keep rows 16-byte aligned");
    const void *ptrs[] = {a->q, a->k, a->v, a->out};
    for (const void *ptr : ptrs)
      if ((uintptr_t)ptr & 15) return fail(DAN_ERR_INVALID_ARGUMENT, "q, k, v and out must be 16-byte aligned");
  }
  // Per-lane offsets inside a tile are kept in 32 bits.
  if (a->k_stride_tok < 0 || a->k_stride_tok * kKeyTile >= (int64_t(1) << 31) || (int64_t)D * a->vt_cols >= (int64_t(1) << 31))
    return fail(DAN_ERR_UNSUPPORTED, "k token stride %lld or vt_cols %d is too large", (long long)a->k_stride_tok, a->vt_cols);
  const int hpw = heads_per_group(rep);
  const int chunks = (rep + hpw - 1) / hpw;
  const int64_t units = (int64_t)a->num_work * Hkv * chunks;
  const int64_t pack_grid = (int64_t)(a->vt_cols / kKeyTile) * Hkv;
  if (units > 0x7fffffff || pack_grid > 0x7fffffff) return fail(DAN_ERR_INVALID_ARGUMENT, "grid is too large");
  if (a->phases != DAN_TREE_ATTN_PHASE_PACK && (!a->units || !a->sched_off || a->num_slots <= 0 || a->num_slots > units))
    return fail(DAN_ERR_INVALID_ARGUMENT, "schedule: need units, sched_off and 1 <= num_slots <= %lld units",
                (long long)units);

  PackParams pp;
  pp.v = a->v; pp.v_st = a->v_stride_tok; pp.v_sh = a->v_stride_head;
  pp.segs = a->segments; pp.pasts = a->pasts; pp.col_seg = a->col_seg;
  pp.vt = static_cast<_Float16 *>(a->workspace);
  pp.vexp = reinterpret_cast<int32_t *>(static_cast<uint8_t *>(a->workspace) + vt_bytes(Hkv, D, a->vt_cols));
  pp.num_kv_heads = Hkv; pp.vt_cols = a->vt_cols;
  pp.v_scale = a->v_scale;
  pp.counts = a->counts;

  KParams kp;
  kp.q = a->q; kp.k = a->k; kp.o = a->out; kp.vt = pp.vt; kp.vexp = pp.vexp;
  kp.q_st = a->q_stride_tok; kp.q_sh = a->q_stride_head;
  kp.k_st = a->k_stride_tok; kp.k_sh = a->k_stride_head;
  kp.o_st = a->o_stride_tok; kp.o_sh = a->o_stride_head;
  kp.pasts = a->pasts; kp.key_lo = a->key_lo;
  kp.num_kv_heads = Hkv; kp.rep = rep; kp.hpw = hpw; kp.chunks = chunks; kp.vt_cols = a->vt_cols;
  kp.c = a->scale * 1.4426950408889634f;
  kp.q_scale = a->q_scale; kp.k_scale = a->k_scale;
  kp.units = a->units; kp.sched_off = a->sched_off; kp.num_units = (int32_t)units;
  const int grid = a->num_slots;

  hipStream_t s = static_cast<hipStream_t>(stream);
  // One instantiation per (input types, head_dim).
  auto by_d = [&](auto f64, auto f128, auto f256) { return D == 64 ? f64() : D == 128 ? f128() : f256(); };
#define DAN_PACK(TV) by_d([&] { return launch_pack<TV, 64>(pp, (int)pack_grid, s); }, \
                          [&] { return launch_pack<TV, 128>(pp, (int)pack_grid, s); }, \
                          [&] { return launch_pack<TV, 256>(pp, (int)pack_grid, s); })
#define DAN_ATTN(TQK, TO) by_d([&] { return launch_attn<TQK, TO, 64>(kp, grid, s); }, \
                               [&] { return launch_attn<TQK, TO, 128>(kp, grid, s); }, \
                               [&] { return launch_attn<TQK, TO, 256>(kp, grid, s); })
  hipError_t err = hipSuccess;
  if (a->phases != DAN_TREE_ATTN_PHASE_ATTEND) {
    if (bf16) err = DAN_PACK(__bf16);
    else if (f16) err = DAN_PACK(_Float16);
    else if (f8) err = DAN_PACK(E4M3);
    else err = DAN_PACK(float);
    if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "V^T pack launch failed: %s", hipGetErrorString(err));
  }
  if (a->phases == DAN_TREE_ATTN_PHASE_PACK) return DAN_OK;

  if (bf16) err = DAN_ATTN(__bf16, __bf16);
  else if (f16) err = DAN_ATTN(_Float16, _Float16);
  else if (f8) err = DAN_ATTN(E4M3, __bf16);
  else err = DAN_ATTN(_Float16, float);
#undef DAN_PACK
#undef DAN_ATTN
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "attention launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}

int dan_tree_attn_stage_f16(const DanStageF16Args *a, void *stream) {
  using namespace dan;
  g_err[0] = 0;
  if (!a) return fail(DAN_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != DAN_TREE_ATTN_ABI_VERSION)
    return fail(DAN_ERR_VERSION, "abi_version %d, library speaks %d", a->abi_version, DAN_TREE_ATTN_ABI_VERSION);
  if (a->d0 < 0 || a->d1 < 0 || a->d2 < 0 || a->d2 % 4)
    return fail(DAN_ERR_INVALID_ARGUMENT, "shape [%d, %d, %d]: the last dimension must be a multiple of 4", a->d0, a->d1, a->d2);
  if (!a->x || !a->out || !a->scale || !a->partial) return fail(DAN_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (((uintptr_t)a->x & 15) || ((uintptr_t)a->out & 7) || ((a->stride0 | a->stride1) & 3) || a->stride0 < 0 || a->stride1 < 0)
    return fail(DAN_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned with strides that keep rows 16-byte aligned, out 8-byte aligned");
  StageParams sp;
  sp.x = a->x; sp.s0 = a->stride0; sp.s1 = a->stride1; sp.d0 = a->d0; sp.d1 = a->d1; sp.d2 = a->d2;
  sp.out = static_cast<_Float16 *>(a->out); sp.scale = a->scale; sp.partial = a->partial;
  const int64_t n4 = (int64_t)a->d0 * a->d1 * (a->d2 / 4);
  const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(DAN_TREE_ATTN_STAGE_PARTIALS, (n4 + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(stage_max_kernel, dim3(grid), dim3(256), 0, s, sp);
  hipLaunchKernelGGL(stage_convert_kernel, dim3(grid), dim3(256), 0, s, sp);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "staging launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}

int dan_tree_attn_fwd_noalloc(const DanTreeAttnArgs *a, void *stream) {
  using namespace dan;
  g_err[0] = 0;
  if (!a) return fail(DAN_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != DAN_TREE_ATTN_ABI_VERSION)
    return fail(DAN_ERR_VERSION, "abi_version %d, library speaks %d", a->abi_version, DAN_TREE_ATTN_ABI_VERSION);
  if (a->num_work == 0) return DAN_OK;
  const int64_t need = dan_tree_attn_workspace_size(a->num_kv_heads, a->head_dim, a->vt_cols);
  if (need > DAN_TREE_ATTN_SCRATCH_BYTES)
    return fail(DAN_ERR_UNSUPPORTED, "the V^T copy needs %lld bytes; the library's scratch holds %lld (use dan_tree_attn_fwd "
                "with a workspace)", (long long)need, (long long)DAN_TREE_ATTN_SCRATCH_BYTES);
  DanTreeAttnArgs b = *a;
  const int rc = scratch_address(static_cast<hipStream_t>(stream), &b.workspace);
  if (rc != DAN_OK) return rc;
  b.workspace_bytes = DAN_TREE_ATTN_SCRATCH_BYTES;
  return dan_tree_attn_fwd(&b, stream);
}

}  // extern "C"
