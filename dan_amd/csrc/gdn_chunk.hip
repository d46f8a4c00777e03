// Gated delta rule in chunked form (gfx950): the recurrence of gdn.hip
// (dan/models/qwen3_5.py:136-158) restated over chunks of 64 tokens, the
// form of the reference's own CPU path (delta_rule_torch,
// dan/models/qwen3_5.py:103-133).
//
// Within a chunk (rows i = 0..63 from the chunk's first token; rows past the
// run's end are padding with g = beta = 0), with r_q, r_k the l2-norm
// factors of q and k, G_i = g_0 + .. + g_i and gamma_i = exp(G_i):
//   L[i][j] = beta_i r_k,i r_k,j (k_i . k_j) exp(G_i - G_j)            j < i
//   A[i][j] = r_q,i Dk^-1/2 r_k,j (q_i . k_j) exp(G_i - G_j)           j <= i
//   T = (I + L)^-1
// and then, in chunk order, from the run's state S [Dk][Dv]:
//   D = T (diag(beta) V - diag(beta gamma r_k) K S)     (the chunk's updates)
//   O = diag(r_q Dk^-1/2 gamma) Q S + A D
//   S <- gamma_63 S + K^T diag(exp(G_63 - G) r_k) D
// Two launches:
//   chunk_prep_kernel  every (chunk, value head) at once: the chunk's q and k
//                      rows into LDS in coalesced loads, the l2-norm factors
//                      of the rows, K K^T and Q K^T on v_mfma_f32_32x32x16
//                      (exact bf16/fp16 products, fp32 sums; the norm factors
//                      and decays are applied after, in fp32), then T by
//                      forward substitution, one column per four lanes; T, A
//                      and the per-row factors (and for bf16 inputs K^T) go
//                      to the chunk records of the workspace, T and A staged
//                      in LDS for 16-byte stores.
//   chunk_scan_bf16_kernel  (bf16 inputs) one work group per (run, value
//                      head, 32 state columns), the state slice in LDS; the
//                      run's chunks in order, each the five products above on
//                      v_mfma_f32_16x16x32_bf16, fp32 operands as bf16 pairs
//                      (hi + lo, ~16 significant bits) against an fp32 master
//                      copy of the state; q, k and v read in place.
//   chunk_scan_kernel  (fp16 inputs) the same on v_mfma_f32_16x16x4_f32 (fp32
//                      operands), 16 state columns per work group for long
//                      runs, 32 for many short ones.
// The sequential critical path is one chunk step per 64 tokens.
//
// Chunk records: run r's chunks are slots r + cu[r] / 64 + j, j = 0, 1, ..;
// r + cu[r] / 64 increases strictly with r, so the slots of different runs
// never meet, and every slot is below num_runs + num_tokens / 64.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "dan_gdn.h"

namespace dan_gdnc {

constexpr int kC = DAN_GDN_CHUNK;  // tokens per chunk
constexpr int kDk = 128;
constexpr int kThreads = 256;
// State columns per scan work group (a template argument of the scan: 32 or
// 16) for phases of long and of short runs.
constexpr int kLongCols = 16, kShortCols = 32;
// Chunk record per (slot, value head), two layouts:
// - fp16 inputs (the fp32 scan): T [64][64] and A [64][64] in fp32, then the
//   five rows of 64 floats below, at float kVecF32;
// - bf16 inputs (the bf16 scan): T and A as bf16 pairs (hi = bf16(x), lo =
//   bf16(x - hi): x to ~16 significant bits), each [64][64] row-major, then
//   K^T [128][64] bf16 (exact), then the five rows at float kVecBf.
// The five rows: beta gamma r_k, beta, r_q Dk^-1/2 gamma, exp(G_63 - G) r_k,
// {gamma_63, 0, ..}.
constexpr int kVecF32 = 2 * kC * kC;
constexpr int kVecBf = (4 * kC * kC * 2 + kDk * kC * 2) / 4;
constexpr int kRec = kVecBf + 5 * kC;  // floats; the fp32 layout uses the first kVecF32 + 5 * kC
// bf16 layout: byte offsets of T hi / lo, A hi / lo and K^T.
constexpr int kThiB = 0, kTloB = kC * kC * 2, kAhiB = 2 * kC * kC * 2, kAloB = 3 * kC * kC * 2, kKtB = 4 * kC * kC * 2;
constexpr float kQs = 0.08838834764831845f;  // Dk^-1/2

#define DAN_GLOBAL __attribute__((address_space(1)))

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct Params {
  const int32_t *cu;
  const void *q, *k, *v;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh;
  const float *g, *beta, *s_in;
  float *s_out, *rec;
  void *o;
  const int32_t *sidx;  // NULL or [R]: run r's entry of s_in (clamped to [0, nsin))
  int32_t Hk, Hv, Dv, R, ncb, units, nsin;
};

// Run r's entry of s_in (wave-uniform).
__device__ inline int state_in_of(const Params &p, int r) {
  return p.sidx ? min(max(__builtin_amdgcn_readfirstlane(*(const __attribute__((address_space(1))) int32_t *)(p.sidx + r)), 0), p.nsin - 1) : r;
}

template <typename T>
__device__ inline f32x16 mfma_in(u32x4 a, u32x4 b, f32x16 c);
template <>
__device__ inline f32x16 mfma_in<__bf16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ inline f32x16 mfma_in<_Float16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Element `half` (0: low 16 bits) of a word holding two T.
template <typename T>
__device__ inline float half_of(uint32_t w, int half);
template <>
__device__ inline float half_of<__bf16>(uint32_t w, int half) {
  return __builtin_bit_cast(float, half ? (w & 0xffff0000u) : (w << 16));
}
template <>
__device__ inline float half_of<_Float16>(uint32_t w, int half) {
  return (float)__builtin_bit_cast(f16x2, w)[half];
}

// Sum of squares of the 8 T in x, in fp32.
template <typename T>
__device__ inline float sumsq8(u32x4 x) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float y = half_of<T>(x[e >> 1], e & 1);
    s = fmaf(y, y, s);
  }
  return s;
}

__device__ inline int slot_of(const int32_t *cu, int r) { return r + *(const DAN_GLOBAL int32_t *)(cu + r) / kC; }

// ---------------------------------------------------------------- chunk preparation
// A work-group barrier that waits for this wave's LDS operations only:
// __syncthreads() also waits for every global access in flight (the scan's
// next-chunk operand loads, the prep's record stores).
__device__ inline void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The prep's LDS: the chunk's k and q rows, 16 threads per row loading 16
// bytes each (coalesced; the products then read their operands here). Rows
// are kTileRow bytes apart: 16 rows reading 16 bytes of one column hit all 64
// banks. After the products the q tile holds L [64][kC + 4] (the same bytes)
// and the k tile stages A, then T: 16 KB each, written to the record in
// coalesced 16-byte stores.
constexpr int kTileRow = kDk * 2 + 16;
constexpr int kTileBytes = kC * kTileRow;
static_assert(kTileBytes == kC * (kC + 4) * 4, "L fits the q tile");
static_assert(kC * kC * 4 <= kTileBytes, "A or T staging fits the k tile");

// Rows 16 W .. kC - 1 of the forward substitution (rows above 16 W are 0 in
// wave W's columns), as one straight-line block.
template <int W>
__device__ inline void tsolve_rows(const float (*sL)[kC + 4], float (&xm)[kC / 4], int j, int part) {
#pragma unroll
  for (int i = 16 * W; i < kC; ++i) {
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < (i + 3) / 4; ++k) acc = fmaf(sL[i][4 * k + part], xm[k], acc);
    acc += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0xB1, 0xf, 0xf, false));
    acc += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x4E, 0xf, 0xf, false));
    const float xi = (i == j ? 1.f : 0.f) - acc;
    if (part == (i & 3)) xm[i >> 2] = xi;
  }
}

// Grid: slots x Hv; a slot past its run's last chunk exits at once.
template <typename T>
__global__ __launch_bounds__(kThreads) void chunk_prep_kernel(const Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t sKt[kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t sQt[kTileBytes];
  __shared__ float sG[kC], sF[3][kC];  // G; per row beta r_k, r_q Dk^-1/2 and r_k
  float(*sL)[kC + 4] = reinterpret_cast<float(*)[kC + 4]>(sQt);
  const int s = blockIdx.x / p.Hv, h = blockIdx.x % p.Hv;
  // The run of slot s: the largest r with slot_of(r) <= s. slot_of increases
  // strictly with r (slot_of(0) = 0), so r + 1 is the number of runs whose
  // slot is at most s: each wave counts them 64 runs at a time with one load
  // per lane, all in flight, instead of a binary search's chain of loads.
  // The same pass loads cu[r] and cu[r + 1] (the lane of run r holds them).
  int r = 0, cu_r = 0, cu_r1 = 0;
  {
    const int ln = threadIdx.x & 63;
    int last0 = 0, last1 = 0;  // cu[base - 1], cu[base]: lane 63 of the pass before
    for (int base = 0; base < p.R; base += 64) {
      const int rr = min(base + ln, p.R - 1);
      const int c0 = *(const DAN_GLOBAL int32_t *)(p.cu + rr), c1 = *(const DAN_GLOBAL int32_t *)(p.cu + rr + 1);
      const bool le = base + ln < p.R && rr + c0 / kC <= s;
      const uint64_t m = __ballot(le);
      const int n = __popcll(m);
      r = base + n - 1;
      cu_r = n > 0 ? __shfl(c0, n - 1) : last0;
      cu_r1 = n > 0 ? __shfl(c1, n - 1) : last1;
      last0 = __shfl(c0, 63);
      last1 = __shfl(c1, 63);
      if (m != ~0ull) break;  // a run of this block starts past s (or the runs end here)
    }
  }
  const int t0 = cu_r + kC * (s - (r + cu_r / kC));
  const int end = cu_r1;
  if (t0 >= end) return;  // the whole group, before any barrier
  const int L = min(kC, end - t0);
  const int hk = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  constexpr bool kBf = std::is_same<T, __bf16>::value;
  float *rec = p.rec + ((int64_t)s * p.Hv + h) * kRec;
  float *vec = rec + (kBf ? kVecBf : kVecF32);
  uint8_t *recb = reinterpret_cast<uint8_t *>(rec);

  // 1. The k and q rows (rows past the run repeat its last row; the scan
  //    multiplies padding by zero), and wave 0's gates of row `lane`.
  {
    const T *kb = static_cast<const T *>(p.k) + (int64_t)hk * p.k_sh + 8 * (tid & 15);
    const T *qb = static_cast<const T *>(p.q) + (int64_t)hk * p.q_sh + 8 * (tid & 15);
    u32x4 kx[4], qx[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int64_t t = t0 + min(16 * m + (tid >> 4), L - 1);
      kx[m] = *(const DAN_GLOBAL u32x4 *)(kb + t * p.k_st);
      qx[m] = *(const DAN_GLOBAL u32x4 *)(qb + t * p.q_st);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int at = (16 * m + (tid >> 4)) * kTileRow + 16 * (tid & 15);
      *reinterpret_cast<u32x4 *>(sKt + at) = kx[m];
      *reinterpret_cast<u32x4 *>(sQt + at) = qx[m];
    }
  }
  float G = 0.f, b = 0.f;
  if (wave == 0) {
    const bool ok = lane < L;
    const int64_t t = t0 + min(lane, L - 1);
    G = ok ? *(const DAN_GLOBAL float *)(p.g + t * p.Hv + h) : 0.f;
    b = ok ? *(const DAN_GLOBAL float *)(p.beta + t * p.Hv + h) : 0.f;
  }
  barrier_lds();

  // 2. Wave 0: the row factors of row `lane`: 1 / sqrt(sum x^2 + 1e-6) of its
  //    q and k rows (dan/models/qwen3_5.py:99-100), G by a prefix sum over the
  //    lanes, the record's five rows.
  if (wave == 0) {
    const int i = lane;
    const bool ok = i < L;
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int j = 0; j < kDk / 8; ++j) {
      sq += sumsq8<T>(*reinterpret_cast<const u32x4 *>(sQt + i * kTileRow + 16 * j));
      sk += sumsq8<T>(*reinterpret_cast<const u32x4 *>(sKt + i * kTileRow + 16 * j));
    }
    const float rq = ok ? 1.0f / sqrtf(sq + 1e-6f) : 0.f;
    const float rk = ok ? 1.0f / sqrtf(sk + 1e-6f) : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(G, off);
      if (lane >= off) G += y;
    }
    const float Glast = __shfl(G, 63);  // padding rows add 0: the decay through the run's last row
    const float gam = expf(G);
    sG[i] = G;
    vec[0 * kC + i] = b * gam * rk;
    vec[1 * kC + i] = b;
    vec[2 * kC + i] = rq * kQs * gam;
    vec[3 * kC + i] = expf(Glast - G) * rk;
    vec[4 * kC + i] = i == 0 ? expf(Glast) : 0.f;
    sF[0][i] = b * rk;
    sF[1][i] = rq * kQs;
    sF[2][i] = rk;
  }

  // K K^T and Q K^T, 32 x 32 block (bi, bj) per wave: lane l reads 16 bytes
  // of row 32 b + l % 32 at element 16 kk + 8 (l / 32).
  const int bi = wave >> 1, bj = wave & 1;
  const uint8_t *ki = sKt + (32 * bi + (lane & 31)) * kTileRow + 16 * (lane >> 5);
  const uint8_t *kj = sKt + (32 * bj + (lane & 31)) * kTileRow + 16 * (lane >> 5);
  const uint8_t *qi = sQt + (32 * bi + (lane & 31)) * kTileRow + 16 * (lane >> 5);
  f32x16 P = {}, QK = {};
#pragma unroll
  for (int kk = 0; kk < kDk / 16; ++kk) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(ki + 32 * kk);
    const u32x4 bb = *reinterpret_cast<const u32x4 *>(kj + 32 * kk);
    const u32x4 aq = *reinterpret_cast<const u32x4 *>(qi + 32 * kk);
    P = mfma_in<T>(a, bb, P);
    QK = mfma_in<T>(aq, bb, QK);
  }
  if constexpr (kBf) {
    // K^T [Dk][kC] for the bf16 scan: thread t writes d rows 2 dp and 2 dp + 1,
    // tokens 8 oc .. 8 oc + 7, from 8 dwords (d 2 dp, 2 dp + 1) of 8 tile rows.
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int dp = (tid >> 3) + 32 * n, oc = tid & 7;
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = *reinterpret_cast<const uint32_t *>(sKt + (8 * oc + e) * kTileRow + 4 * dp);
      u32x4 lo, hi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo[e] = (w[2 * e] & 0xffffu) | (w[2 * e + 1] << 16);
        hi[e] = (w[2 * e] >> 16) | (w[2 * e + 1] & 0xffff0000u);
      }
      *(DAN_GLOBAL u32x4 *)(recb + kKtB + 2 * ((2 * dp) * kC + 8 * oc)) = lo;
      *(DAN_GLOBAL u32x4 *)(recb + kKtB + 2 * ((2 * dp + 1) * kC + 8 * oc)) = hi;
    }
  }
  barrier_lds();  // sG, the row factors; every read of the tiles is done

  // 3. L into the q tile's bytes, A staged in the k tile's (the record's A
  //    block layout: bf16 hi and lo planes, or fp32).
#pragma unroll
  for (int rr = 0; rr < 16; ++rr) {  // accumulator: row 8 (rr / 4) + 4 (lane / 32) + rr % 4, column lane % 32
    const int i = 32 * bi + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3), j = 32 * bj + (lane & 31);
    const float e = (i >= j && i < L) ? expf(sG[i] - sG[j]) : 0.f;
    const float rkj = sF[2][j];
    sL[i][j] = i > j ? sF[0][i] * rkj * P[rr] * e : 0.f;
    const float av = sF[1][i] * rkj * QK[rr] * e;
    if constexpr (kBf) {
      const __bf16 hi = (__bf16)av;
      *reinterpret_cast<__bf16 *>(sKt + 2 * (i * kC + j)) = hi;
      *reinterpret_cast<__bf16 *>(sKt + kC * kC * 2 + 2 * (i * kC + j)) = (__bf16)(av - (float)hi);
    } else {
      *reinterpret_cast<float *>(sKt + 4 * (i * kC + j)) = av;
    }
  }
  barrier_lds();

  // 4. A out (16 KB from the stage), then T = (I + L)^-1 by forward
  //    substitution, x_i = [i == j] - sum_{m < i} L[i][m] x_m for column j:
  //    wave w solves columns 16 w .. 16 w + 15, four lanes per column (lane
  //    4 c + p: column 16 w + c, the terms m = p mod 4), the four partial sums
  //    added by two quad swaps. Rows above 16 w are 0 in these columns;
  //    L[i][m] = 0 for m >= i, so whole groups of four are summed.
  constexpr int kBlockBytes = kC * kC * 4;  // the T block, then the A block, of the record
  static_assert(kAhiB == kBlockBytes && kThiB == 0, "record layout");
#pragma unroll
  for (int m = 0; m < kBlockBytes / (16 * kThreads); ++m) {
    const int off = 16 * (kThreads * m + tid);
    *(DAN_GLOBAL u32x4 *)(recb + kBlockBytes + off) = *reinterpret_cast<const u32x4 *>(sKt + off);
  }
  const int j = 16 * wave + (lane >> 2), part = lane & 3;
  float xm[kC / 4];  // x_{4 k + part}
#pragma unroll
  for (int k = 0; k < kC / 4; ++k) xm[k] = 0.f;
  switch (wave) {  // wave-uniform
    case 0: tsolve_rows<0>(sL, xm, j, part); break;
    case 1: tsolve_rows<1>(sL, xm, j, part); break;
    case 2: tsolve_rows<2>(sL, xm, j, part); break;
    default: tsolve_rows<3>(sL, xm, j, part); break;
  }
  barrier_lds();  // every wave's A reads of the stage are done
#pragma unroll
  for (int k = 0; k < kC / 4; ++k) {
    const int i = 4 * k + part;
    if constexpr (kBf) {
      const __bf16 hi = (__bf16)xm[k];
      *reinterpret_cast<__bf16 *>(sKt + 2 * (i * kC + j)) = hi;
      *reinterpret_cast<__bf16 *>(sKt + kC * kC * 2 + 2 * (i * kC + j)) = (__bf16)(xm[k] - (float)hi);
    } else {
      *reinterpret_cast<float *>(sKt + 4 * (i * kC + j)) = xm[k];
    }
  }
  barrier_lds();
#pragma unroll
  for (int m = 0; m < kBlockBytes / (16 * kThreads); ++m) {
    const int off = 16 * (kThreads * m + tid);
    *(DAN_GLOBAL u32x4 *)(recb + off) = *reinterpret_cast<const u32x4 *>(sKt + off);
  }
}

// ---------------------------------------------------------------- the scan over chunks
// LDS (floats) of a COLS-column scan: the state slice twice (the chunk's S
// and the next), [128][COLS + 2] each; Y, D and diag(exp(G_63 - G) r_k) D,
// [64][COLS + 4] each. With these row strides every B-operand read of
// v_mfma_f32_16x16x4_f32 (4 rows x 16 columns: rows 8 apart in S, 4 apart in
// the others) hits 64 distinct banks: 8 (COLS + 2) and 4 (COLS + 4) are 16
// modulo 64 for COLS = 16 and 32.
template <int COLS>
struct ScanLds {
  static constexpr int kSS = COLS + 2, kSB = COLS + 4;
  static constexpr int floats = 2 * kDk * kSS + 3 * kC * kSB;
  static_assert((8 * kSS) % 64 == 16 && (4 * kSB) % 64 == 16, "conflict-free operand reads");
};
// Long runs, where a chunk step's latency sets the pace: 4 waves on 16 state
// columns (one 16 x 16 tile each), so a (run, head) spreads over 8 work groups.
// Many short runs, where the per-group fixed cost does: 4 waves on 32 columns
// (16 x 32 each). Both leave room for two work groups per CU. (The kernel
// also runs as 8 waves on 32 columns, one tile each, which took 11 % longer on
// a trunk phase of 5 runs of 286 to 1843 tokens.)
constexpr int kScanLongWaves = 4, kScanShortWaves = 4;

__device__ inline f32x4 mma(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }


// Contraction orders: the 128-long sums over the state rows take k-index
// 32 (kk / 8) + 8 q + kk % 8 at step kk in lane group q = lane / 16 (a lane's
// q or k elements for 8 steps are 16 contiguous bytes); the 64-long sums over
// the chunk rows take 16 (kk / 4) + 4 q + kk % 4 (4 contiguous floats of T or
// A), so steps 4 j .. 4 j + 3 cover chunk rows 16 j .. 16 j + 15.
__device__ inline int kidx128(int kk, int q) { return 32 * (kk >> 3) + 8 * q + (kk & 7); }
__device__ inline int kidx64(int kk, int q) { return 16 * (kk >> 2) + 4 * q + (kk & 3); }

// One wave's operands of one chunk, loaded a chunk ahead: each group is
// loaded right after its last use in the chunk before. NC: the wave's
// 16-column halves of the slice.
template <typename T, int NC>
struct Ops {
  u32x4 ka[4], qa[4];     // k, q row 16 rb + l16 (the A operands of K S and Q S)
  f32x4 va, vb, vq, vs;   // the row factors of rows 16 rb + 4 q4 .. + 3
  float vv[NC][4];        // v of those rows, the wave's columns
  f32x4 ta[4], aa[4];     // T, A row 16 rb + l16
  uint32_t kt[16];        // k[kidx64(kk, q4)][32 rb + 2 l16 .. + 1]: the A operands of K^T D
  float glast;
};

// Work group: one (run, value head, 32 state columns). Wave w computes rows
// 16 rb .. 16 rb + 15 of Y, D and O in its NC column halves, and state rows
// 32 rb .. 32 rb + 31 of those columns: with 8 waves, half nb = w / 4 and
// rb = w % 4 or 3 - w % 4 (waves w and w + 4 share a SIMD, so every SIMD
// carries the same share of the triangular products); with 4 waves, rb = w
// and both halves. Per chunk, with jmax = (L - 1) / 16 the last row block
// holding run tokens:
//   phase 0  K S and Q S together (one read of S), Y to LDS        barrier
//   phase 1  D = T Y over row blocks j <= min(rb, jmax) (T is lower
//            triangular, blocks past jmax are padding), D and Ds to LDS  barrier
//   phase 2  O = (Q S) + A D (blocks j <= min(rb, jmax)), S <- gamma S + K^T Ds
//            (blocks j <= jmax) into the other state buffer        barrier
// A wave whose rows are all padding skips phases 0-1 and the O products.
template <typename T, int W, int COLS>
__global__ __launch_bounds__(64 * W) void chunk_scan_kernel(const Params p) {
  // 16-column halves per wave: 8 waves x 1 (32 columns), 4 x 2 (32), 4 x 1 (16)
  constexpr int NC = COLS / 16 * 4 / W;
  static_assert(NC >= 1 && (W == 4 || (W == 8 && COLS == 32)), "scan shapes");
  constexpr int kCols = COLS, kSS = ScanLds<COLS>::kSS, kSB = ScanLds<COLS>::kSB;
  __shared__ __attribute__((aligned(16))) float smem[ScanLds<COLS>::floats];
  // work group b -> (unit u = r Hv + h, column block cb); the ncb groups of a
  // unit share b % 8 and so an XCD, whose L2 then serves their common reads
  const int b = blockIdx.x;
  const int u = (b / (8 * p.ncb)) * 8 + (b & 7), cb = (b >> 3) % p.ncb;
  if (u >= p.units) return;  // the whole group, before any barrier
  const int r = u / p.Hv, h = u % p.Hv, hk = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, q4 = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb0 = W == 8 ? w >> 2 : 0, rb = W == 8 ? (nb0 ? 3 - (w & 3) : (w & 3)) : w;
  float *sY = smem + 2 * kDk * kSS, *sD = sY + kC * kSB, *sDs = sD + kC * kSB;
  const int col0 = kCols * cb;
  int col[NC];
#pragma unroll
  for (int n = 0; n < NC; ++n) col[n] = 16 * (nb0 + n) + l16;
  const int64_t sbase = ((int64_t)r * p.Hv + h) * kDk * p.Dv + col0;
  const int64_t sbase_in = ((int64_t)state_in_of(p, r) * p.Hv + h) * kDk * p.Dv + col0;
  {  // the state slice: every load in flight before the first LDS write
    constexpr int kSt = kDk * kCols / (64 * W);
    float sv[kSt];
#pragma unroll
    for (int m = 0; m < kSt; ++m) {
      const int x = tid + 64 * W * m;
      sv[m] = *(const DAN_GLOBAL float *)(p.s_in + sbase_in + (int64_t)(x / kCols) * p.Dv + x % kCols);
    }
#pragma unroll
    for (int m = 0; m < kSt; ++m) {
      const int x = tid + 64 * W * m;
      smem[(x / kCols) * kSS + x % kCols] = sv[m];
    }
  }
  const int row0 = *(const DAN_GLOBAL int32_t *)(p.cu + r), end = *(const DAN_GLOBAL int32_t *)(p.cu + r + 1);
  const T *qh = static_cast<const T *>(p.q) + (int64_t)hk * p.q_sh;
  const T *kh = static_cast<const T *>(p.k) + (int64_t)hk * p.k_sh;
  const T *vh = static_cast<const T *>(p.v) + (int64_t)h * p.v_sh + col0;
  T *oh = static_cast<T *>(p.o) + (int64_t)h * p.o_sh + col0;
  const int ri = 16 * rb + l16;   // the A-operand row of the 64-row products
  const int ro = 16 * rb + 4 * q4;  // the first of the lane's accumulator rows

  // Loads of chunk (t0, slot s), rows clamped to the run (padding rows carry zero factors).
  auto rec_of = [&](int s) __attribute__((always_inline)) { return p.rec + ((int64_t)s * p.Hv + h) * kRec; };
  auto load0 = [&](Ops<T, NC> &o, int t0, int s) __attribute__((always_inline)) {
    const int L = min(kC, end - t0);
    const int64_t tr = t0 + min(ri, L - 1);
    const float *vec = rec_of(s) + kVecF32;
#pragma unroll
    for (int j = 0; j < 4; ++j) o.ka[j] = *(const DAN_GLOBAL u32x4 *)(kh + tr * p.k_st + 32 * j + 8 * q4);
#pragma unroll
    for (int j = 0; j < 4; ++j) o.qa[j] = *(const DAN_GLOBAL u32x4 *)(qh + tr * p.q_st + 32 * j + 8 * q4);
    o.va = *(const DAN_GLOBAL f32x4 *)(vec + 0 * kC + ro);
    o.vb = *(const DAN_GLOBAL f32x4 *)(vec + 1 * kC + ro);
#pragma unroll
    for (int n = 0; n < NC; ++n)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        o.vv[n][rr] = (float)*(const DAN_GLOBAL T *)(vh + (int64_t)(t0 + min(ro + rr, L - 1)) * p.v_st + col[n]);
  };
  auto load1 = [&](Ops<T, NC> &o, int s) __attribute__((always_inline)) {
    const float *rec = rec_of(s);
#pragma unroll
    for (int j = 0; j < 4; ++j) o.ta[j] = *(const DAN_GLOBAL f32x4 *)(rec + ri * kC + 16 * j + 4 * q4);
    o.vs = *(const DAN_GLOBAL f32x4 *)(rec + kVecF32 + 3 * kC + ro);
  };
  auto load2 = [&](Ops<T, NC> &o, int t0, int s) __attribute__((always_inline)) {
    const int L = min(kC, end - t0);
    const float *rec = rec_of(s);
#pragma unroll
    for (int j = 0; j < 4; ++j) o.aa[j] = *(const DAN_GLOBAL f32x4 *)(rec + kC * kC + ri * kC + 16 * j + 4 * q4);
    o.vq = *(const DAN_GLOBAL f32x4 *)(rec + kVecF32 + 2 * kC + ro);
    o.glast = *(const DAN_GLOBAL float *)(rec + kVecF32 + 4 * kC);
#pragma unroll
    for (int kk = 0; kk < 16; ++kk)
      o.kt[kk] = *(const DAN_GLOBAL uint32_t *)(kh + (int64_t)(t0 + min(kidx64(kk, q4), L - 1)) * p.k_st + 32 * rb + 2 * l16);
  };

  Ops<T, NC> op;
  int s = r + row0 / kC;
  if (row0 < end) {
    load0(op, row0, s);
    load1(op, s);
    load2(op, row0, s);
  }
  int cur = 0;
  __syncthreads();
  for (int t0 = row0; t0 < end; t0 += kC, ++s) {
    const int L = min(kC, end - t0), jmax = (L - 1) >> 4;
    const bool rows = 16 * rb < L;  // the wave's tile holds run tokens
    const int jtop = min(rb, jmax);
    // the next chunk (this one again after the last: the loads stay in bounds)
    const bool more = t0 + kC < end;
    const int tn = more ? t0 + kC : t0, sn = more ? s + 1 : s;
    float *sS = smem + cur * kDk * kSS, *sN = smem + (cur ^ 1) * kDk * kSS;

    // phase 0: K S and Q S; Y = diag(beta) V - diag(beta gamma r_k) K S
    f32x4 x[NC], o1[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) x[n] = o1[n] = f32x4{};
    if (rows) {
#pragma unroll
      for (int kk = 0; kk < 32; ++kk) {
        const float ak = half_of<T>(op.ka[kk >> 3][(kk & 7) >> 1], kk & 1);
        const float aq = half_of<T>(op.qa[kk >> 3][(kk & 7) >> 1], kk & 1);
#pragma unroll
        for (int n = 0; n < NC; ++n) {
          const float bs = sS[kidx128(kk, q4) * kSS + col[n]];
          x[n] = mma(ak, bs, x[n]);
          o1[n] = mma(aq, bs, o1[n]);
        }
      }
#pragma unroll
      for (int n = 0; n < NC; ++n)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sY[(ro + rr) * kSB + col[n]] = op.vb[rr] * op.vv[n][rr] - op.va[rr] * x[n][rr];
    }
    load0(op, tn, sn);
    barrier_lds();

    // phase 1: D = T Y
    if (rows) {
      f32x4 d[NC];
#pragma unroll
      for (int n = 0; n < NC; ++n) d[n] = f32x4{};
#pragma unroll
      for (int j = 0; j < 4; ++j)  // static indices keep op in registers; the guard is wave-uniform
        if (j <= jtop) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int n = 0; n < NC; ++n) d[n] = mma(op.ta[j][e], sY[(16 * j + 4 * q4 + e) * kSB + col[n]], d[n]);
        }
#pragma unroll
      for (int n = 0; n < NC; ++n)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          sD[(ro + rr) * kSB + col[n]] = d[n][rr];
          sDs[(ro + rr) * kSB + col[n]] = op.vs[rr] * d[n][rr];
        }
    }
    load1(op, sn);
    barrier_lds();

    // phase 2: O = diag(r_q Dk^-1/2 gamma) Q S + A D; S <- gamma_63 S + K^T Ds
    if (rows) {
      f32x4 o2[NC];
#pragma unroll
      for (int n = 0; n < NC; ++n) o2[n] = f32x4{};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j <= jtop) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int n = 0; n < NC; ++n) o2[n] = mma(op.aa[j][e], sD[(16 * j + 4 * q4 + e) * kSB + col[n]], o2[n]);
        }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        if (ro + rr < L) {
#pragma unroll
          for (int n = 0; n < NC; ++n)
            *(DAN_GLOBAL T *)(oh + (int64_t)(t0 + ro + rr) * p.o_st + col[n]) = (T)(op.vq[rr] * o1[n][rr] + o2[n][rr]);
        }
    }
    // the wave's state rows are 32 rb + 2 m + mb for row m of block mb (one
    // 4-byte load of k gives both blocks' A operands)
    f32x4 sn0[NC], sn1[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        sn0[n][rr] = op.glast * sS[(32 * rb + 2 * (4 * q4 + rr)) * kSS + col[n]];
        sn1[n][rr] = op.glast * sS[(32 * rb + 2 * (4 * q4 + rr) + 1) * kSS + col[n]];
      }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j <= jmax) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a0 = half_of<T>(op.kt[4 * j + e], 0), a1 = half_of<T>(op.kt[4 * j + e], 1);
#pragma unroll
          for (int n = 0; n < NC; ++n) {
            const float bd = sDs[(16 * j + 4 * q4 + e) * kSB + col[n]];
            sn0[n] = mma(a0, bd, sn0[n]);
            sn1[n] = mma(a1, bd, sn1[n]);
          }
        }
      }
#pragma unroll
    for (int n = 0; n < NC; ++n)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        sN[(32 * rb + 2 * (4 * q4 + rr)) * kSS + col[n]] = sn0[n][rr];
        sN[(32 * rb + 2 * (4 * q4 + rr) + 1) * kSS + col[n]] = sn1[n][rr];
      }
    load2(op, tn, sn);
    barrier_lds();  // the new state is whole, and every read of this chunk's Y, D and S is done
    cur ^= 1;
  }
  const float *sS = smem + cur * kDk * kSS;
#pragma unroll
  for (int m = 0; m < kDk * kCols / (64 * W); ++m) {
    const int x = tid + 64 * W * m;
    *(DAN_GLOBAL float *)(p.s_out + sbase + (int64_t)(x / kCols) * p.Dv + x % kCols) = sS[(x / kCols) * kSS + x % kCols];
  }
}

// ---------------------------------------------------------------- the bf16 scan
// bf16 inputs: the same chunk step as chunk_scan_kernel, its products on
// v_mfma_f32_16x16x32_bf16, eight times the fp32 product's rate. Every fp32
// operand goes in as a bf16 pair (hi = bf16(x), lo = bf16(x - hi): ~16
// significant bits); q, k and K^T are bf16 already. Per pair of operands:
// K S, Q S, K^T Ds take two products (x hi, x lo), T Y and A D three (the lo
// x lo term, ~2^-17 relative, is dropped). Sums stay fp32, and the state's
// fp32 master copy carries the decay and the updates; the bf16 pairs of S are
// rewritten from it every chunk.
// LDS (bytes): the state's fp32 master [128][COLS + 2]; the state as bf16
// planes (hi, lo) of [COLS][128 + 8] (one state column per row, so the B
// operand's 8 consecutive state rows are 16 contiguous bytes); Y, D and
// diag(exp(G_63 - G) r_k) D as planes of [COLS][64 + 8]. The 8-element pads
// spread a B-operand read's 16 columns over the banks.
template <int COLS>
struct BfLds {
  static constexpr int kSS = COLS + 2, kPS = kDk + 8, kPC = kC + 8;
  static constexpr int sHi = kDk * kSS * 4, sLo = sHi + COLS * kPS * 2;
  static constexpr int yHi = sLo + COLS * kPS * 2, yLo = yHi + COLS * kPC * 2;
  static constexpr int dHi = yLo + COLS * kPC * 2, dLo = dHi + COLS * kPC * 2;
  static constexpr int eHi = dLo + COLS * kPC * 2, eLo = eHi + COLS * kPC * 2;
  static constexpr int bytes = eLo + COLS * kPC * 2;
  static_assert(sHi % 16 == 0 && (kPS * 2) % 16 == 0 && (kPC * 2) % 16 == 0, "16-byte operand reads");
};

// State columns per work group of the bf16 scan, long and short runs alike:
// its per-chunk operands (q, k, T, A, K^T) are loaded by every column group
// of a (run, head), and with 16 columns the CUs' address units were the
// limit (trunk phase of 5 runs of 286 to 1843 tokens: 0.209 ms on 16
// columns, 0.164 on 32, 0.226 on 64 with one group per CU).
constexpr int kBfCols = 32;

__device__ inline f32x4 mma_bf(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
// x as a bf16 pair, the hi and lo halves' bits.
__device__ inline void split_bf(float x, uint32_t &hi, uint32_t &lo) {
  const __bf16 h = (__bf16)x;
  const __bf16 l = (__bf16)(x - (float)h);
  hi = __builtin_bit_cast(uint16_t, h);
  lo = __builtin_bit_cast(uint16_t, l);
}
// Four consecutive rows of one plane column (8 bytes, hi and lo planes).
__device__ inline void put4_bf(uint8_t *hi_plane, uint8_t *lo_plane, int off, const f32x4 &x) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) split_bf(x[i], h[i], l[i]);
  *reinterpret_cast<u32x2 *>(hi_plane + off) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  *reinterpret_cast<u32x2 *>(lo_plane + off) = u32x2{l[0] | (l[1] << 16), l[2] | (l[3] << 16)};
}

// One wave's operands of one chunk, loaded a chunk ahead (each group right
// after its last use in the chunk before).
template <int NC>
struct OpsBf {
  u32x4 ka[4], qa[4];   // k, q row 16 rb + l16, d 32 j + 8 g4 .. + 7 (A operands of K S, Q S)
  f32x4 va, vb, vq, vs; // the row factors of rows 16 rb + 4 g4 .. + 3
  float vv[NC][4];      // v of those rows, the wave's columns
  u32x4 th[2], tl[2];   // T row 16 rb + l16, chunk rows 32 j + 8 g4 .. + 7 (hi, lo)
  u32x4 ah[2], al[2];   // A, the same
  u32x4 kt[2][2];       // K^T row 32 rb + 16 mb + l16, chunk rows 32 j + 8 g4 .. + 7
  float glast;
};

// Work group: one (run, value head, COLS state columns), 4 waves. Wave rb
// computes rows 16 rb .. + 15 of Y, D and O and state rows 32 rb .. + 31,
// all COLS columns (NC tiles of 16). Per chunk, with jmax = (L - 1) / 32:
//   phase 0  K S and Q S (the S planes), Y to its planes                barrier
//   phase 1  D = T Y (chunk-row blocks j <= rb / 2: T is lower triangular),
//            D and Ds to their planes                                   barrier
//   phase 2  O = (Q S) + A D; S <- gamma_63 S + K^T Ds (blocks j <= jmax)
//            into the master and the S planes                           barrier
// Padding rows (past the run) come out as zeros in Y, D and Ds (their row
// factors are zero), so every wave runs every phase.
template <int COLS>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2)))
void chunk_scan_bf16_kernel(const Params p) {
  constexpr int NC = COLS / 16;
  using LB = BfLds<COLS>;
  constexpr int kSS = LB::kSS, kPS = LB::kPS, kPC = LB::kPC;
  __shared__ __attribute__((aligned(16))) uint8_t lds[LB::bytes];
  float *sS = reinterpret_cast<float *>(lds);
  const int b = blockIdx.x;
  const int u = (b / (8 * p.ncb)) * 8 + (b & 7), cb = (b >> 3) % p.ncb;
  if (u >= p.units) return;  // the whole group, before any barrier
  const int r = u / p.Hv, h = u % p.Hv, hk = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, g4 = lane >> 4;
  const int rb = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col0 = COLS * cb;
  const int64_t sbase = ((int64_t)r * p.Hv + h) * kDk * p.Dv + col0;
  const int64_t sbase_in = ((int64_t)state_in_of(p, r) * p.Hv + h) * kDk * p.Dv + col0;
  {  // the state slice: every load in flight before the first LDS write
    constexpr int kSt = kDk * COLS / 256;
    float sv[kSt];
#pragma unroll
    for (int m = 0; m < kSt; ++m) {
      const int x = tid + 256 * m;
      sv[m] = *(const DAN_GLOBAL float *)(p.s_in + sbase_in + (int64_t)(x / COLS) * p.Dv + x % COLS);
    }
#pragma unroll
    for (int m = 0; m < kSt; ++m) {
      const int x = tid + 256 * m, row = x / COLS, c = x % COLS;
      sS[row * kSS + c] = sv[m];
      uint32_t hi, lo;
      split_bf(sv[m], hi, lo);
      *reinterpret_cast<uint16_t *>(lds + LB::sHi + 2 * (c * kPS + row)) = (uint16_t)hi;
      *reinterpret_cast<uint16_t *>(lds + LB::sLo + 2 * (c * kPS + row)) = (uint16_t)lo;
    }
  }
  const int row0 = *(const DAN_GLOBAL int32_t *)(p.cu + r), end = *(const DAN_GLOBAL int32_t *)(p.cu + r + 1);
  const __bf16 *qh = static_cast<const __bf16 *>(p.q) + (int64_t)hk * p.q_sh;
  const __bf16 *kh = static_cast<const __bf16 *>(p.k) + (int64_t)hk * p.k_sh;
  const __bf16 *vh = static_cast<const __bf16 *>(p.v) + (int64_t)h * p.v_sh + col0;
  __bf16 *oh = static_cast<__bf16 *>(p.o) + (int64_t)h * p.o_sh + col0;
  const int ri = 16 * rb + l16;     // the A-operand row of the 64-row products
  const int ro = 16 * rb + 4 * g4;  // the first of the lane's accumulator rows

  auto recb = [&](int s) __attribute__((always_inline)) {
    return reinterpret_cast<const uint8_t *>(p.rec + ((int64_t)s * p.Hv + h) * kRec);
  };
  auto ld16 = [&](const uint8_t *q) __attribute__((always_inline)) { return *(const DAN_GLOBAL u32x4 *)q; };
  auto load0 = [&](OpsBf<NC> &o, int t0, int s) __attribute__((always_inline)) {
    const int L = min(kC, end - t0);
    const int64_t tr = t0 + min(ri, L - 1);
    const float *vec = reinterpret_cast<const float *>(recb(s)) + kVecBf;
#pragma unroll
    for (int j = 0; j < 4; ++j) o.ka[j] = *(const DAN_GLOBAL u32x4 *)(kh + tr * p.k_st + 32 * j + 8 * g4);
#pragma unroll
    for (int j = 0; j < 4; ++j) o.qa[j] = *(const DAN_GLOBAL u32x4 *)(qh + tr * p.q_st + 32 * j + 8 * g4);
    o.va = *(const DAN_GLOBAL f32x4 *)(vec + 0 * kC + ro);
    o.vb = *(const DAN_GLOBAL f32x4 *)(vec + 1 * kC + ro);
#pragma unroll
    for (int n = 0; n < NC; ++n)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        o.vv[n][rr] = (float)*(const DAN_GLOBAL __bf16 *)(vh + (int64_t)(t0 + min(ro + rr, L - 1)) * p.v_st + 16 * n + l16);
  };
  auto load1 = [&](OpsBf<NC> &o, int s) __attribute__((always_inline)) {
    const uint8_t *rc = recb(s);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      o.th[j] = ld16(rc + kThiB + 2 * (ri * kC + 32 * j + 8 * g4));
      o.tl[j] = ld16(rc + kTloB + 2 * (ri * kC + 32 * j + 8 * g4));
    }
    o.vs = *(const DAN_GLOBAL f32x4 *)(reinterpret_cast<const float *>(rc) + kVecBf + 3 * kC + ro);
  };
  auto load2 = [&](OpsBf<NC> &o, int s) __attribute__((always_inline)) {
    const uint8_t *rc = recb(s);
    const float *vec = reinterpret_cast<const float *>(rc) + kVecBf;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      o.ah[j] = ld16(rc + kAhiB + 2 * (ri * kC + 32 * j + 8 * g4));
      o.al[j] = ld16(rc + kAloB + 2 * (ri * kC + 32 * j + 8 * g4));
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int j = 0; j < 2; ++j) o.kt[mb][j] = ld16(rc + kKtB + 2 * ((32 * rb + 16 * mb + l16) * kC + 32 * j + 8 * g4));
    o.vq = *(const DAN_GLOBAL f32x4 *)(vec + 2 * kC + ro);
    o.glast = *(const DAN_GLOBAL float *)(vec + 4 * kC);
  };
  // the 16 bytes of plane column c, rows k0 .. k0 + 7
  auto rd = [&](int plane, int stride, int c, int k0) __attribute__((always_inline)) {
    return *reinterpret_cast<const u32x4 *>(lds + plane + 2 * (c * stride + k0));
  };

  OpsBf<NC> op;
  int s = r + row0 / kC;
  if (row0 < end) {
    load0(op, row0, s);
    load1(op, s);
    load2(op, s);
  }
  __syncthreads();
  for (int t0 = row0; t0 < end; t0 += kC, ++s) {
    const int L = min(kC, end - t0), jmax = (L - 1) >> 5;
    const int jt = min(rb >> 1, jmax);  // the wave's last 32-row block of T Y and A D
    const bool more = t0 + kC < end;    // the next chunk (this one again after the last: the loads stay in bounds)
    const int tn = more ? t0 + kC : t0, sn = more ? s + 1 : s;

    // phase 0: K S and Q S; Y = diag(beta) V - diag(beta gamma r_k) K S
    f32x4 x[NC], o1[NC];
#pragma unroll
    for (int n = 0; n < NC; ++n) x[n] = o1[n] = f32x4{};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        const u32x4 bh = rd(LB::sHi, kPS, 16 * n + l16, 32 * j + 8 * g4);
        const u32x4 bl = rd(LB::sLo, kPS, 16 * n + l16, 32 * j + 8 * g4);
        x[n] = mma_bf(op.ka[j], bh, x[n]);
        o1[n] = mma_bf(op.qa[j], bh, o1[n]);
        x[n] = mma_bf(op.ka[j], bl, x[n]);
        o1[n] = mma_bf(op.qa[j], bl, o1[n]);
      }
#pragma unroll
    for (int n = 0; n < NC; ++n) {
      f32x4 y;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) y[rr] = op.vb[rr] * op.vv[n][rr] - op.va[rr] * x[n][rr];
      put4_bf(lds + LB::yHi, lds + LB::yLo, 2 * ((16 * n + l16) * kPC + ro), y);
    }
    load0(op, tn, sn);
    barrier_lds();

    // phase 1: D = T Y
    {
      f32x4 d[NC];
#pragma unroll
      for (int n = 0; n < NC; ++n) d[n] = f32x4{};
#pragma unroll
      for (int j = 0; j < 2; ++j)  // static indices keep op in registers; the guard is wave-uniform
        if (j <= jt) {
#pragma unroll
          for (int n = 0; n < NC; ++n) {
            const u32x4 bh = rd(LB::yHi, kPC, 16 * n + l16, 32 * j + 8 * g4);
            const u32x4 bl = rd(LB::yLo, kPC, 16 * n + l16, 32 * j + 8 * g4);
            d[n] = mma_bf(op.th[j], bh, d[n]);
            d[n] = mma_bf(op.th[j], bl, d[n]);
            d[n] = mma_bf(op.tl[j], bh, d[n]);
          }
        }
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        put4_bf(lds + LB::dHi, lds + LB::dLo, 2 * ((16 * n + l16) * kPC + ro), d[n]);
        f32x4 e;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) e[rr] = op.vs[rr] * d[n][rr];
        put4_bf(lds + LB::eHi, lds + LB::eLo, 2 * ((16 * n + l16) * kPC + ro), e);
      }
    }
    load1(op, sn);
    barrier_lds();

    // phase 2: O = diag(r_q Dk^-1/2 gamma) Q S + A D; S <- gamma_63 S + K^T Ds
    {
      f32x4 o2[NC];
#pragma unroll
      for (int n = 0; n < NC; ++n) o2[n] = f32x4{};
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (j <= jt) {
#pragma unroll
          for (int n = 0; n < NC; ++n) {
            const u32x4 bh = rd(LB::dHi, kPC, 16 * n + l16, 32 * j + 8 * g4);
            const u32x4 bl = rd(LB::dLo, kPC, 16 * n + l16, 32 * j + 8 * g4);
            o2[n] = mma_bf(op.ah[j], bh, o2[n]);
            o2[n] = mma_bf(op.ah[j], bl, o2[n]);
            o2[n] = mma_bf(op.al[j], bh, o2[n]);
          }
        }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        if (ro + rr < L) {
#pragma unroll
          for (int n = 0; n < NC; ++n)
            *(DAN_GLOBAL __bf16 *)(oh + (int64_t)(t0 + ro + rr) * p.o_st + 16 * n + l16) = (__bf16)(op.vq[rr] * o1[n][rr] + o2[n][rr]);
        }
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int sr = 32 * rb + 16 * mb + 4 * g4;  // the lane's first state row of block mb
      f32x4 acc[NC];
#pragma unroll
      for (int n = 0; n < NC; ++n)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) acc[n][rr] = op.glast * sS[(sr + rr) * kSS + 16 * n + l16];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (j <= jmax) {
#pragma unroll
          for (int n = 0; n < NC; ++n) {
            const u32x4 bh = rd(LB::eHi, kPC, 16 * n + l16, 32 * j + 8 * g4);
            const u32x4 bl = rd(LB::eLo, kPC, 16 * n + l16, 32 * j + 8 * g4);
            acc[n] = mma_bf(op.kt[mb][j], bh, acc[n]);
            acc[n] = mma_bf(op.kt[mb][j], bl, acc[n]);
          }
        }
#pragma unroll
      for (int n = 0; n < NC; ++n) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sS[(sr + rr) * kSS + 16 * n + l16] = acc[n][rr];
        put4_bf(lds + LB::sHi, lds + LB::sLo, 2 * ((16 * n + l16) * kPS + sr), acc[n]);
      }
    }
    load2(op, sn);
    barrier_lds();  // the new state is whole, and every read of this chunk's Y, D and S is done
  }
#pragma unroll
  for (int m = 0; m < kDk * COLS / 256; ++m) {
    const int x = tid + 256 * m;
    *(DAN_GLOBAL float *)(p.s_out + sbase + (int64_t)(x / COLS) * p.Dv + x % COLS) = sS[(x / COLS) * kSS + x % COLS];
  }
}

int64_t slots(int32_t num_tokens, int32_t num_runs) { return (int64_t)num_runs + num_tokens / kC; }

}  // namespace dan_gdnc

// Bytes of chunk records that follow the norm factors in the workspace.
int64_t dan_gdn_chunk_record_bytes(int32_t num_tokens, int32_t num_runs, int32_t num_v_heads) {
  return dan_gdnc::slots(num_tokens, num_runs) * num_v_heads * dan_gdnc::kRec * 4;
}

// The chunked form; arguments already checked by dan_gdn_fwd, `records` the
// workspace (16-byte aligned).
hipError_t dan_gdn_fwd_chunked(const DanGdnArgs *a, float *records, hipStream_t s) {
  dan_gdnc::Params p;
  p.cu = a->cu; p.q = a->q; p.k = a->k; p.v = a->v;
  p.q_st = a->q_stride_tok; p.q_sh = a->q_stride_head; p.k_st = a->k_stride_tok; p.k_sh = a->k_stride_head;
  p.v_st = a->v_stride_tok; p.v_sh = a->v_stride_head; p.o_st = a->o_stride_tok; p.o_sh = a->o_stride_head;
  p.g = a->g; p.beta = a->beta; p.s_in = a->states_in; p.s_out = a->states_out; p.o = a->out;
  p.rec = records;
  p.Hk = a->num_k_heads; p.Hv = a->num_v_heads; p.Dv = a->v_dim; p.R = a->num_runs;
  p.units = a->num_runs * a->num_v_heads;
  p.sidx = a->state_index; p.nsin = a->num_states_in;
  const int64_t prep = dan_gdnc::slots(a->num_tokens, a->num_runs) * a->num_v_heads;
  // Runs of DAN_GDN_SHORT_RUN tokens or fewer on average: the short-run scan;
  // longer: the long-run scan.
  const bool shortrun = (int64_t)a->num_tokens <= (int64_t)DAN_GDN_SHORT_RUN * a->num_runs;
  const dim3 block(dan_gdnc::kThreads);
  auto scan = [&](auto kernel, int waves, int cols) {
    p.ncb = a->v_dim / cols;
    const int64_t groups = ((int64_t)p.units + 7) / 8 * 8 * p.ncb;
    hipLaunchKernelGGL(kernel, dim3((unsigned)groups), dim3(64 * waves), 0, s, p);
  };
  constexpr int LW = dan_gdnc::kScanLongWaves, LC = dan_gdnc::kLongCols;
  constexpr int SW = dan_gdnc::kScanShortWaves, SC = dan_gdnc::kShortCols;
  if (a->dtype == DAN_DTYPE_BF16) {
    if (prep) hipLaunchKernelGGL(dan_gdnc::chunk_prep_kernel<__bf16>, dim3((unsigned)prep), block, 0, s, p);
    scan(dan_gdnc::chunk_scan_bf16_kernel<dan_gdnc::kBfCols>, 4, dan_gdnc::kBfCols);
  } else {
    if (prep) hipLaunchKernelGGL(dan_gdnc::chunk_prep_kernel<_Float16>, dim3((unsigned)prep), block, 0, s, p);
    if (shortrun) scan(dan_gdnc::chunk_scan_kernel<_Float16, SW, SC>, SW, SC);
    else scan(dan_gdnc::chunk_scan_kernel<_Float16, LW, LC>, LW, LC);
  }
  return hipGetLastError();
}
