// e4m3 GEMM for dan's FP8 decoder linears on gfx950 (MI355X, CDNA4).
//
// dan's FP8Linear.forward (dan/quant.py:36-42) multiplies the per-call
// quantized activation with the quantized weight through torch._scaled_mm:
//
//   y[m, n] = (sum_k xq[m, k] * wq[n, k]) * x_scale[m] * w_scale[n] + bias[n]
//
// rounded to the model dtype, with fp32 accumulation; scales are per row
// (x_scale [M, 1], w_scale [1, N]) or per tensor ([1, 1] each). This kernel
// computes exactly that product.
//
// Shape of the computation (one work group per 256 x 256 tile of y, four
// waves, each wave a 128 x 128 quarter):
// - Both operands are K-major: xq [M, K] and wq [N, K] as dan stores them
//   (the weight is never transposed), either as byte rows at a stride or in
//   the tiled layout of include/dan_fp8.h, where each 256-row panel's 64-byte
//   k-step is 16 contiguous KB already in the LDS order below, so every direct
//   load reads one contiguous KB.
// - Products run on v_mfma_f32_32x32x64_f8f6f4 (OCP e4m3 x e4m3, fp32
//   accumulate; 64 k per instruction). The matrix core's A operand is a
//   32-row block of w and its B operand a 32-row block of x, so each lane's
//   accumulators hold 4 consecutive n of one m: the epilogue stores 4 outputs
//   per lane and instruction. A wave's 16 accumulator blocks (256 fp32 per
//   lane) live in the accumulation registers.
// - K advances 64 bytes per step through a ring of four LDS stages of 32 KB
//   (the w tile's 256 rows x 64 bytes, then the x tile's). Stages are filled
//   by direct loads (buffer_load_dwordx4 ... lds: 16 bytes per lane straight
//   into LDS, no registers): 32 loads of 1 KB per stage, 8 per wave, issued
//   three steps before the stage is read.
// - Out-of-range reads return zero: each wave's buffer resource spans only
//   its tile's valid rows, and in the last step of a K that is not a multiple
//   of 64 the chunks past K get an offset beyond the resource. Rows past M or
//   N and k past K therefore add nothing, and the epilogue skips their stores.
// - LDS rows are 64 bytes (4 chunks of 16); chunk c of row r sits at
//   position c ^ f(r), f(r) = ((r >> 1) & 3) ^ ((r >> 3) & 1), so the
//   16-byte operand reads of any 8 (and any 16) consecutive lanes, one row
//   each, fall into distinct bank groups.
// - One step per wave: wait for the next stage's loads and a barrier, then
//   16 products on the fragments read in the previous step, with the next
//   stage's fragment reads (2 x 16 bytes per lane and block) and the new
//   stage's 8 direct loads interleaved between them.
// - Work-group order is XCD-aware: consecutive work-group ids go to the 8
//   XCDs in turn, so ids are remapped so that each XCD takes a contiguous
//   range of tiles, walked 8 tile rows (of x) at a time; the 32 tiles an XCD
//   runs at once then share 12 operand panels in its L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "dan_fp8.h"

namespace dan {
int fail(int status, const char *fmt, ...);  // tree_attn.hip: sets the thread's last-error message
extern thread_local char g_err[512];
}  // namespace dan

namespace dan_gemm {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define DAN_LDS __attribute__((address_space(3)))
#define DAN_GLOBAL __attribute__((address_space(1)))

constexpr int kTile = 256;                     // rows of x and of w per work group
constexpr int kBK = 64;                        // k bytes per stage
constexpr int kStages = 4;
constexpr int kOpBytes = kTile * kBK;          // one operand's stage: 16 KB
constexpr int kStageBytes = 2 * kOpBytes;      // w rows, then x rows
constexpr int kOutPitch = 128 * 2 + 16;        // a wave's 128 16-bit outputs per row, padded (LDS staging)
constexpr int kBodyLds = kStages * kStageBytes > 4 * 128 * kOutPitch ? kStages * kStageBytes : 4 * 128 * kOutPitch;
constexpr int kEpiLds = 3 * kTile * 4;         // the tile's x scales, w scales and bias (fp32)
constexpr int kLds = kBodyLds + kEpiLds;       // 139 KB
constexpr int kThreads = 256;
constexpr int kLoadsPerWave = kStageBytes / 1024 / (kThreads / 64);  // 8
constexpr uint32_t kOutOfRange = 0x80000000u;  // a buffer offset past every resource
#ifndef DAN_GEMM_GROUP_M
#define DAN_GEMM_GROUP_M 8
#endif
constexpr int kGroupM = DAN_GEMM_GROUP_M;      // tile rows of x walked together
// Slots of a k-step (one product each) that also read a fragment of the next
// step (8 of 16) or issue a direct load (8 of 16): bit i = slot i.
#ifndef DAN_GEMM_READ_SLOTS
#define DAN_GEMM_READ_SLOTS 0x00ff
#endif
#ifndef DAN_GEMM_LOAD_SLOTS
#define DAN_GEMM_LOAD_SLOTS 0xff00
#endif
constexpr uint32_t kReadSlots = DAN_GEMM_READ_SLOTS, kLoadSlots = DAN_GEMM_LOAD_SLOTS;
static_assert(__builtin_popcount(kReadSlots) == 8 && __builtin_popcount(kLoadSlots) == 8, "8 reads and 8 loads per step");
constexpr int before(uint32_t mask, int slot) { return __builtin_popcount(mask & ((1u << slot) - 1)); }

struct Params {
  const uint8_t *x, *w;  // e4m3 codes: x [M, K], w [N, K]
  int64_t x_st, w_st;    // row strides in bytes
  const float *xs, *ws;  // fp32 scales
  int32_t xs_inc, ws_inc;  // 1: one per row; 0: one for the tensor
  const void *bias;        // [N] of the output type, or null
  void *y;                 // [M, N] of the output type
  int64_t y_st;            // row stride in elements
  int32_t m, n, k;
  int32_t tiles_m, tiles_n;
  int32_t x_tiled, w_tiled;  // operand in the tiled layout (include/dan_fp8.h)
};

__device__ inline uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// chunk position of row r (the LDS swizzle)
__device__ inline int swz(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }

// Raw buffer resource (gfx9 layout): base, stride 0, num_records bytes.
__device__ inline i32x4 resource(const void *base, uint32_t bytes) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  i32x4 r;
  r[0] = (int32_t)uniform((uint32_t)b);
  r[1] = (int32_t)(uniform((uint32_t)(b >> 32)) & 0xffff);
  r[2] = (int32_t)uniform(bytes);
  r[3] = 0x00020000;
  return r;
}

// Where a wave's direct loads read: a tile's operand panel as a buffer
// resource, each load's per-lane offset, and the offset step per k-step.
// Rows: the panel's valid rows at their stride; a k-step is 64 bytes further.
// Tiled: the panel's run of 16 KB k-steps; load i of the wave reads block
// (row block) b, 16 bytes per lane, already in LDS order.
struct Panel {
  i32x4 rsrc;
  uint32_t kstep;  // offset of the next k-step
};
__device__ inline Panel panel_of(const Params &p, bool w, int row0, int kt) {
  const bool tiled = w ? p.w_tiled : p.x_tiled;
  const uint8_t *ptr = w ? p.w : p.x;
  if (tiled) return Panel{resource(ptr + (int64_t)(row0 / kTile) * kt * 16384, (uint32_t)kt * 16384u), 16384u};
  const int64_t st = w ? p.w_st : p.x_st;
  const int rows = min(kTile, (w ? p.n : p.m) - row0);
  return Panel{resource(ptr + (int64_t)row0 * st, (uint32_t)(rows * st)), (uint32_t)kBK};
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One 16-byte direct load per lane into LDS: lane l writes lds + 16 l (M0
// holds the LDS byte address; one wait state after the SALU write of M0,
// which the compiler's hazard pass does not see inside inline asm). Issued
// from inline asm so that the compiler's wait-count pass does not treat the
// in-flight LDS write as an unordered LDS event (it would then wait for every
// LDS read with lgkmcnt(0)); completion is waited for explicitly (vmcnt).
__device__ inline void dma16(i32x4 rsrc, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(off), "s"(rsrc),
               "s"(uniform(lds))
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ inline void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// every wave's LDS reads done, then the barrier
__device__ inline void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Staged LDS writes: the LDS may read a write's data registers after the
// instruction issued (lanes delayed by bank conflicts read theirs later), and
// the compiler reuses a data register as soon as the write has issued. So a
// batch of writes ends with a wait for the LDS (lgkmcnt(0)), and every data
// register is used again after that wait, which keeps its value in place
// until the LDS has read it.
template <int N>
__device__ inline void lds_writes_done(const u32x2 (&data)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" ::"v"(data[i]));
}

__device__ inline f32x16 mfma(const i32x8 &a, const i32x8 &b, f32x16 c) {
  // Format codes 0, 0: both operands OCP e4m3; no block scales.
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

struct Frags {
  i32x8 w[4], x[4];
};

template <typename T>
struct Out;
template <>
struct Out<__bf16> {
  __device__ static void store4(__bf16 *p, f32x4 v) {
    typedef __bf16 v4 __attribute__((ext_vector_type(4)));
    const v4 o = __builtin_convertvector(v, v4);
    *(DAN_GLOBAL u32x2 *)p = __builtin_bit_cast(u32x2, o);
  }
  __device__ static u32x2 pack4(f32x4 v) {
    typedef __bf16 v4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(u32x2, __builtin_convertvector(v, v4));
  }
};
template <>
struct Out<_Float16> {
  __device__ static void store4(_Float16 *p, f32x4 v) {
    typedef _Float16 v4 __attribute__((ext_vector_type(4)));
    const v4 o = __builtin_convertvector(v, v4);
    *(DAN_GLOBAL u32x2 *)p = __builtin_bit_cast(u32x2, o);
  }
  __device__ static u32x2 pack4(f32x4 v) {
    typedef _Float16 v4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(u32x2, __builtin_convertvector(v, v4));
  }
};
template <>
struct Out<float> {
  __device__ static void store4(float *p, f32x4 v) { *(DAN_GLOBAL f32x4 *)p = v; }
};

template <typename TOut, bool kTail>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void fp8_gemm_kernel(Params p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);

  // work group -> tile: XCD-contiguous ranges, then groups of kGroupM tile rows
  const int tiles = p.tiles_m * p.tiles_n;
  int t = blockIdx.x;
#ifndef DAN_GEMM_NO_XCD_REMAP
  if (tiles % 8 == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);
#endif
  const int per_group = kGroupM * p.tiles_n;
  const int first_m = (t / per_group) * kGroupM;
  const int group_m = min(p.tiles_m - first_m, kGroupM);
  const int in_group = t % per_group;
  const int m0 = (first_m + in_group % group_m) * kTile;
  const int n0 = (in_group / group_m) * kTile;

  // The epilogue's operands for the tile (x scale per row, w scale and bias
  // per column, as fp32) are fetched now, one value per thread and array, so
  // that their latency passes under the main loop; the epilogue parks them in
  // LDS past the stages for every lane to read.
  const uint32_t lds_base = (uint32_t)(uintptr_t)smem;
  const uint32_t epi = lds_base + kBodyLds;  // x scales, then w scales, then bias: kTile fp32 each
  const TOut *bias = static_cast<const TOut *>(p.bias);
  const int tid = threadIdx.x;
  const float e_xs = p.xs[(int64_t)min(m0 + tid, p.m - 1) * p.xs_inc];
  const float e_ws = p.ws[(int64_t)min(n0 + tid, p.n - 1) * p.ws_inc];
  // (without a bias the load reads the first bytes of w_scale, always valid, and is discarded:
  // a branch would make the compiler convert, and so wait for, the value right here)
  const TOut e_b = *(bias ? bias + min(n0 + tid, p.n - 1) : reinterpret_cast<const TOut *>(p.ws));

  // Direct loads: waves 0-1 fill the w rows of each stage, waves 2-3 the x rows.
  // Load i of wave v moves 16 rows (1 KB): block b = 8 v + i of the stage; lane
  // l writes row 16 (b % 16) + l / 4 at position l % 4, holding chunk (l % 4) ^ f(row).
  const bool loads_w = wave < 2;
  const bool tiled = loads_w ? p.w_tiled : p.x_tiled;
  const int64_t st = loads_w ? p.w_st : p.x_st;
  const Panel pan = panel_of(p, loads_w, loads_w ? n0 : m0, (p.k + kBK - 1) / kBK);
  const i32x4 rsrc = pan.rsrc;
  const int rl = lane >> 2;
  const int chunk = (lane & 3) ^ swz(rl);
  uint32_t voff[kLoadsPerWave];
#pragma unroll
  for (int i = 0; i < kLoadsPerWave; ++i) {
    const int blk = (wave * kLoadsPerWave + i) & 15;
    voff[i] = tiled ? (uint32_t)(blk * 1024 + 16 * lane) : (uint32_t)((16 * blk + rl) * st + 16 * chunk);
  }
  const uint32_t lds_load = lds_base + wave * kLoadsPerWave * 1024;

  const int kt = (p.k + kBK - 1) / kBK;
  // Issue the loads of k-step s into its stage (s % 4). Advancing the
  // resource base by 64 bytes per step keeps the per-lane offsets fixed; the
  // shortened resource still ends at the last valid row's end.
  auto issue = [&](int s) __attribute__((always_inline)) {
    const uint32_t k0 = (uint32_t)s * kBK, adv = (uint32_t)s * pan.kstep;
    i32x4 r = rsrc;
    const uint64_t b = ((uint64_t)(uint32_t)r[0] | ((uint64_t)(uint32_t)(r[1] & 0xffff) << 32)) + adv;
    r[0] = (int32_t)(uint32_t)b;
    r[1] = (int32_t)((uint32_t)(b >> 32) & 0xffff);
    r[2] = (int32_t)((uint32_t)r[2] - adv);
    const uint32_t lds = lds_load + (s & (kStages - 1)) * kStageBytes;
    const bool full = !kTail || tiled || (int)k0 + kBK <= p.k;  // tiled padding holds zeros
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) {
      uint32_t off = voff[i];
      if (kTail && !full && (int)k0 + 16 * chunk >= p.k) off = kOutOfRange;
      dma16(r, off, lds + i * 1024);
    }
  };

  // Fragment reads: lane l reads row l % 32 of a 32-row block, bytes
  // [32 (l / 32), +32) of the stage's 64 (chunks 2 (l / 32) and 2 (l / 32) + 1).
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, h = lane >> 5;
  const uint32_t f_lo = fr * kBK + 16 * ((2 * h) ^ swz(fr)), f_hi = fr * kBK + 16 * ((2 * h + 1) ^ swz(fr));
  const uint32_t w_rows = lds_base + wn * 128 * kBK, x_rows = lds_base + kOpBytes + wm * 128 * kBK;
  auto read_frag = [&](i32x8 &f, uint32_t blk) __attribute__((always_inline)) {
    const u32x4 lo = *(const DAN_LDS u32x4 *)(uintptr_t)(blk + f_lo);
    const u32x4 hi = *(const DAN_LDS u32x4 *)(uintptr_t)(blk + f_hi);
    f = __builtin_bit_cast(i32x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = (f32x16){};

  // One k-step: products on `cur`, fragment reads of step s + 1 into `nxt`,
  // direct loads of step s + 4. Each of the 16 slots issues one product, then
  // a fragment read and/or a direct load as kReadSlots and kLoadSlots place them.
  auto step = [&](int s, Frags &cur, Frags &nxt, bool do_read, bool do_issue) __attribute__((always_inline)) {
    const uint32_t stage = (uint32_t)((s + 1) & (kStages - 1)) * kStageBytes;
    const uint32_t k0 = (uint32_t)(s + 4) * kBK, adv = (uint32_t)(s + 4) * pan.kstep;
    i32x4 r = rsrc;
    const uint64_t b64 = ((uint64_t)(uint32_t)r[0] | ((uint64_t)(uint32_t)(r[1] & 0xffff) << 32)) + adv;
    r[0] = (int32_t)(uint32_t)b64;
    r[1] = (int32_t)((uint32_t)(b64 >> 32) & 0xffff);
    r[2] = (int32_t)((uint32_t)r[2] - adv);
    const uint32_t lds = lds_load + (s & (kStages - 1)) * kStageBytes;
    const bool full = !kTail || tiled || (int)k0 + kBK <= p.k;
#pragma unroll
    for (int slot = 0; slot < 16; ++slot) {
      const int a = slot >> 2, bb = slot & 3;
      acc[a][bb] = mfma(cur.w[a], cur.x[bb], acc[a][bb]);
      if ((kReadSlots >> slot) & 1) {
        const int f = before(kReadSlots, slot);  // fragments w0-w3, then x0-x3
        if (do_read) {
          if (f < 4) read_frag(nxt.w[f], w_rows + stage + f * 32 * kBK);
          else read_frag(nxt.x[f - 4], x_rows + stage + (f - 4) * 32 * kBK);
        }
      }
      if ((kLoadSlots >> slot) & 1) {
        const int i = before(kLoadSlots, slot);
        if (do_issue) {
          uint32_t off = voff[i];
          if (kTail && !full && (int)k0 + 16 * chunk >= p.k) off = kOutOfRange;
          dma16(r, off, lds + i * 1024);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  if (kt > 0) {
    // prologue: steps 0-3 in flight, step 0's fragments read
#pragma unroll
    for (int s = 0; s < kStages; ++s)
      if (s < kt) issue(s);
    if (kt >= 4) wait_vm<3 * kLoadsPerWave>();
    else if (kt == 3) wait_vm<2 * kLoadsPerWave>();
    else if (kt == 2) wait_vm<kLoadsPerWave>();
    else wait_vm<0>();
    barrier_lds();
    Frags f0, f1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      read_frag(f0.w[i], w_rows + i * 32 * kBK);
      read_frag(f0.x[i], x_rows + i * 32 * kBK);
    }
    // Steady state: before step s, the loads of steps s + 2 and s + 3 may
    // still be in flight; step s + 1's must have landed.
    int s = 0;
    for (; s + 1 < kt - 4; s += 2) {
      wait_vm<2 * kLoadsPerWave>();
      barrier_lds();
      step(s, f0, f1, true, true);
      wait_vm<2 * kLoadsPerWave>();
      barrier_lds();
      step(s + 1, f1, f0, true, true);
    }
    if (s < kt - 4) {
      wait_vm<2 * kLoadsPerWave>();
      barrier_lds();
      step(s, f0, f1, true, true);
      f0 = f1;
      ++s;
    }
    // Tail: no loads left to issue; in flight before step s are the steps
    // after s + 1 up to kt - 1.
    for (; s < kt; ++s) {
      const int after = kt - 2 - s;
      if (after >= 2) wait_vm<2 * kLoadsPerWave>();
      else if (after == 1) wait_vm<kLoadsPerWave>();
      else wait_vm<0>();
      if (s + 1 < kt) barrier_lds();
      step(s, f0, f1, s + 1 < kt, false);
      f0 = f1;
    }
  }

  // Epilogue: lane l holds, in block (a, b) and register 4 g + i,
  // n = n0 + 128 wn + 32 a + 8 g + 4 (l / 32) + i and m = m0 + 128 wm + 32 b + l % 32.
  TOut *y = static_cast<TOut *>(p.y);
  *(DAN_LDS float *)(uintptr_t)(epi + 4 * tid) = e_xs;
  *(DAN_LDS float *)(uintptr_t)(epi + 4 * (kTile + tid)) = e_ws;
  *(DAN_LDS float *)(uintptr_t)(epi + 4 * (2 * kTile + tid)) = bias ? (float)e_b : 0.0f;
  // Every wave has read its last operands (the 16-bit path reuses the stages)
  // and parked its epilogue values.
  barrier_lds();
  float xsv[4];
  int mrow[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    mrow[b] = m0 + 128 * wm + 32 * b + fr;
    xsv[b] = *(const DAN_LDS float *)(uintptr_t)(epi + 4 * (128 * wm + 32 * b + fr));
  }
  // Column groups are 8 wide and N is a multiple of 16, so a group is in or
  // out for the whole wave (a uniform test).
  auto col = [&](int a, int g) __attribute__((always_inline)) { return n0 + 128 * wn + 32 * a + 8 * g; };
  auto value = [&](int a, int b, int g) __attribute__((always_inline)) {
    const uint32_t c = 4 * (128 * wn + 32 * a + 8 * g + 4 * h);
    const f32x4 ws = *(const DAN_LDS f32x4 *)(uintptr_t)(epi + 4 * kTile + c);
    const f32x4 bv = *(const DAN_LDS f32x4 *)(uintptr_t)(epi + 8 * kTile + c);
    f32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __builtin_fmaf(acc[a][b][4 * g + i] * xsv[b], ws[i], bv[i]);
    return v;
  };
  if constexpr (sizeof(TOut) == 2) {
    // 16-bit outputs go through LDS: a store straight from the accumulator
    // layout writes 16 bytes into each of 32 rows (32 cache lines per
    // instruction); staged, each instruction writes 4 rows of 256 contiguous
    // bytes. The wave's 128 x 128 outputs take rows of kOutPitch bytes in its
    // own LDS quarter.
    const uint32_t stage = lds_base + wave * 128 * kOutPitch;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      u32x2 pk[16];
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          pk[4 * g + b] = Out<TOut>::pack4(value(a, b, g));
          *(DAN_LDS u32x2 *)(uintptr_t)(stage + (32 * b + fr) * kOutPitch + (32 * a + 8 * g + 4 * h) * 2) = pk[4 * g + b];
        }
      lds_writes_done(pk);
    }
    const int r0 = lane >> 4, c = lane & 15;  // 16 lanes per 256-byte row, 4 rows per instruction
    const int ncol = n0 + 128 * wn + 8 * c;
#pragma unroll 8
    for (int it = 0; it < 32; ++it) {
      const int r = 4 * it + r0;
      const u32x4 v = *(const DAN_LDS u32x4 *)(uintptr_t)(stage + r * kOutPitch + 16 * c);
      const int row = m0 + 128 * wm + r;
      if (row < p.m && ncol < p.n) *(DAN_GLOBAL u32x4 *)(y + (int64_t)row * p.y_st + ncol) = v;
    }
  } else {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (col(a, g) >= p.n) continue;
        const int n = col(a, g) + 4 * h;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          if (mrow[b] >= p.m) continue;
          Out<TOut>::store4(y + (int64_t)mrow[b] * p.y_st + n, value(a, b, g));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent form (16-bit outputs, an even number >= 6 of k-steps): one work
// group per CU walks its tiles, and the ring of stages runs on across tile
// boundaries: the next tile's first three stages load while the current tile
// finishes, and the stores drain while the next tile's products run.
//
// A tile's last step holds back its direct loads (the next tile's step 3):
// the stage it would fill, the one that step consumed, is the epilogue's
// staging area. Each wave stages its 128 x 128 outputs 32 rows at a time in
// the 8 KB of that stage its own direct loads fill, then issues those loads.
//
// Every wave issues a fixed pattern of vector-memory operations, so its waits
// (vmcnt counts loads and stores in issue order) are constants:
// - each step but a tile's last: 8 direct loads (the step 4 ahead; past the
//   last tile they read out of range, which writes zeros into the stage just
//   consumed);
// - each tile boundary: 32 stores (out-of-range rows and columns are dropped
//   by the buffer resource), 3 direct loads of the next tile's x scales, w
//   scales and bias (into an LDS operand area kept per tile parity), then the
//   8 held-back direct loads.
// Before step s of a tile, step s + 1 must have landed. In flight may be
// steps s + 2 and s + 3 (16 loads); before steps 0 and 1 of every tile but
// the first, also the boundary's 35 stores and operand loads, which were
// issued after step s + 1's loads.
constexpr int kPStageLds = kStages * kStageBytes;              // 128 KB ring
constexpr int kPOpsBytes = 2 * kTile * 4 + kTile * 2;          // x scales, w scales (fp32), bias (16-bit)
constexpr int kPOpsLds = 2 * 2560;                             // two tiles' operands, 2.5 KB each
constexpr int kPLds = kPStageLds + kPOpsLds;                   // 133 KB
constexpr int kPBoundaryOps = 32 + 3;
static_assert(kPOpsBytes <= 2560, "operand area");
static_assert(kLoadsPerWave * 1024 == 32 * 256, "a wave's share of a stage holds its 32 staged output rows");

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void dma4(i32x4 rsrc, uint32_t off, uint32_t lds) {  // 4 bytes per lane: lane l writes lds + 4 l
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(off), "s"(rsrc),
               "s"(uniform(lds))
               : "memory", "m0");
}
// A store of more than 8 bytes needs a wait state before a VALU instruction
// may overwrite its data registers; the compiler does not see inside the asm.
__device__ inline void store16(i32x4 rsrc, uint32_t off, u32x4 v) {
  asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen\n\ts_nop 1" ::"v"(v), "v"(off), "s"(rsrc) : "memory");
}
#pragma clang diagnostic pop

struct PTile {
  int m0, n0;
};

template <typename TOut, bool kTail>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void fp8_gemm_persistent(Params p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const uint32_t lds_base = (uint32_t)(uintptr_t)smem;
  const uint32_t ops_lds = lds_base + kPStageLds;

  // This work group's tiles: XCD-contiguous ranges of tiles (work groups go
  // to the 8 XCDs in turn), each XCD's work groups taking every (G / 8)-th
  // tile of its range, grouped kGroupM tile rows at a time.
  const int tiles = p.tiles_m * p.tiles_n, G = gridDim.x, b = blockIdx.x;
  const bool xcd = tiles % 8 == 0 && G % 8 == 0;
  const int stride = xcd ? G / 8 : G, first = xcd ? (b & 7) * (tiles / 8) + (b >> 3) : b;
  const int range_end = xcd ? ((b & 7) + 1) * (tiles / 8) : tiles;
  const int my_tiles = first < range_end ? (range_end - first + stride - 1) / stride : 0;
  auto tile_at = [&](int j) __attribute__((always_inline)) {
    const int t = first + j * stride;
    const int per_group = kGroupM * p.tiles_n;
    const int first_m = (t / per_group) * kGroupM;
    const int group_m = min(p.tiles_m - first_m, kGroupM);
    const int in_group = t % per_group;
    return PTile{(first_m + in_group % group_m) * kTile, (in_group / group_m) * kTile};
  };

  // direct-load geometry (as in fp8_gemm_kernel)
  const bool loads_w = wave < 2;
  const bool tiled = loads_w ? p.w_tiled : p.x_tiled;
  const int64_t st = loads_w ? p.w_st : p.x_st;
  const int rl = lane >> 2;
  const int chunk = (lane & 3) ^ swz(rl);
  // load i's offset: vbase + (row block (wave % 2) * 8 + i) * (16 rows or one
  // 1 KB tiled block); only the per-lane base stays in a register over the loop
  const uint32_t vbase = tiled ? (uint32_t)(16 * lane) : (uint32_t)(rl * st + 16 * chunk);
  const uint32_t blk_step = uniform(tiled ? 1024u : (uint32_t)(16 * st));
  const uint32_t rows16 = blk_step, wrows = uniform((uint32_t)(wave & 1) * 8 * blk_step);
  const uint32_t lds_load = lds_base + wave * kLoadsPerWave * 1024;
  const int kt = (p.k + kBK - 1) / kBK;
  const uint32_t kstep = tiled ? 16384u : (uint32_t)kBK;
  auto operand_rsrc = [&](int j) __attribute__((always_inline)) {
    if (j >= my_tiles) return resource(p.x, 0);  // past the last tile: every read out of range
    const PTile tl = tile_at(j);
    return panel_of(p, loads_w, loads_w ? tl.n0 : tl.m0, kt).rsrc;
  };
  // the direct loads of step s of tile j (tile j past the last: zeros)
  auto issue = [&](i32x4 rsrc, int s, uint32_t lds, bool ok) __attribute__((always_inline)) {
    const uint32_t k0 = (uint32_t)s * kBK, adv = (uint32_t)s * kstep;
    i32x4 r = rsrc;
    const uint64_t bb = ((uint64_t)(uint32_t)r[0] | ((uint64_t)(uint32_t)(r[1] & 0xffff) << 32)) + adv;
    r[0] = (int32_t)(uint32_t)bb;
    r[1] = (int32_t)((uint32_t)(bb >> 32) & 0xffff);
    r[2] = ok ? (int32_t)((uint32_t)r[2] - adv) : 0;
    const bool full = !kTail || tiled || (int)k0 + kBK <= p.k;  // tiled padding holds zeros
    return [=](int i) __attribute__((always_inline)) {
      uint32_t off = vbase + (wrows + i * rows16);
      if (kTail && !full && (int)k0 + 16 * chunk >= p.k) off = kOutOfRange;
      dma16(r, off, lds + i * 1024);
    };
  };
  // the epilogue operands of tile j into the operand area of its parity
  auto issue_ops = [&](int j) __attribute__((always_inline)) {
    const uint32_t area = ops_lds + (j & 1) * 2560;
    const bool ok = j < my_tiles;
    const PTile tl = ok ? tile_at(j) : PTile{0, 0};
    const int w4 = wave * 64 + lane;  // 256 threads: one x scale and one w scale each
    dma4(resource(p.xs, ok ? (uint32_t)(p.xs_inc ? p.m : 1) * 4 : 0), (uint32_t)((tl.m0 + w4) * p.xs_inc) * 4,
         area + wave * 256);
    dma4(resource(p.ws, ok ? (uint32_t)(p.ws_inc ? p.n : 1) * 4 : 0), (uint32_t)((tl.n0 + w4) * p.ws_inc) * 4,
         area + 1024 + wave * 256);
    // bias: 256 16-bit values, two per lane; waves 0-1 and 2-3 load the same halves
    const int half = wave & 1;
    dma4(resource(p.bias, ok && p.bias ? (uint32_t)p.n * 2 : 0), (uint32_t)(tl.n0 + 128 * half + 2 * lane) * 2,
         area + 2048 + half * 256);
  };

  // fragment reads (as in fp8_gemm_kernel)
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, h = lane >> 5;
  const uint32_t f_lo = fr * kBK + 16 * ((2 * h) ^ swz(fr)), f_hi = fr * kBK + 16 * ((2 * h + 1) ^ swz(fr));
  const uint32_t w_rows = lds_base + wn * 128 * kBK, x_rows = lds_base + kOpBytes + wm * 128 * kBK;
  auto read_frag = [&](i32x8 &f, uint32_t blk) __attribute__((always_inline)) {
    const u32x4 lo = *(const DAN_LDS u32x4 *)(uintptr_t)(blk + f_lo);
    const u32x4 hi = *(const DAN_LDS u32x4 *)(uintptr_t)(blk + f_hi);
    f = __builtin_bit_cast(i32x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16 acc[4][4];
  Frags f0, f1;
  if (my_tiles == 0) return;

  // issue pointer: the step 4 ahead of the current one
  int ij = 0, is = 0;
  i32x4 irsrc = operand_rsrc(0);
  auto advance = [&]() __attribute__((always_inline)) {
    if (++is == kt) {
      is = 0;
      ++ij;
      irsrc = operand_rsrc(ij);
    }
  };

  // prologue: tile 0's operands, steps 0-3; step 0 landed
  issue_ops(0);
#pragma unroll
  for (int g = 0; g < kStages; ++g) {
    auto ld = issue(irsrc, is, lds_load + g * kStageBytes, ij < my_tiles);
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) ld(i);
    advance();
  }
  wait_vm<3 * kLoadsPerWave>();
  barrier_lds();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    read_frag(f0.w[i], w_rows + i * 32 * kBK);
    read_frag(f0.x[i], x_rows + i * 32 * kBK);
  }

  // One step (global step g): products on `cur` (into zeroed accumulators on
  // a tile's first step), fragment reads of step g + 1 into `nxt`, direct
  // loads of step g + 4 into the stage of step g.
  auto step = [&](int g, Frags &cur, Frags &nxt, auto first_of_tile, auto issues) __attribute__((always_inline)) {
    const uint32_t stage = (uint32_t)((g + 1) & (kStages - 1)) * kStageBytes;
    auto ld = issue(irsrc, is, lds_load + (g & (kStages - 1)) * kStageBytes, ij < my_tiles);
#pragma unroll
    for (int slot = 0; slot < 16; ++slot) {
      const int a = slot >> 2, bb = slot & 3;
      if constexpr (decltype(first_of_tile)::value) acc[a][bb] = mfma(cur.w[a], cur.x[bb], (f32x16){});
      else acc[a][bb] = mfma(cur.w[a], cur.x[bb], acc[a][bb]);
      if ((kReadSlots >> slot) & 1) {  // (after the last step these read a stage nobody uses)
        const int f = before(kReadSlots, slot);
        if (f < 4) read_frag(nxt.w[f], w_rows + stage + f * 32 * kBK);
        else read_frag(nxt.x[f - 4], x_rows + stage + (f - 4) * 32 * kBK);
      }
      if constexpr (decltype(issues)::value)
        if ((kLoadSlots >> slot) & 1) ld(before(kLoadSlots, slot));
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (decltype(issues)::value) advance();
  };
  // the loads a tile's last step held back (after the epilogue)
  auto issue_held = [&](int g) __attribute__((always_inline)) {
    auto ld = issue(irsrc, is, lds_load + (g & (kStages - 1)) * kStageBytes, ij < my_tiles);
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) ld(i);
    advance();
  };

  // Epilogue of tile j: scale and bias, then the 16-bit outputs staged 32
  // rows at a time in the wave's 8 KB of stage `stg` and stored 16 bytes per
  // lane (256 contiguous bytes per row). Row r's 16-byte chunk c sits at
  // position c ^ (r % 16) with its two 8-byte halves swapped for r >= 16, so
  // the 32 rows written by one instruction fall into distinct banks.
  auto epilogue = [&](int j, uint32_t stg) __attribute__((always_inline)) {
    // The lane index passes through an empty asm, so that the compiler
    // computes the epilogue's per-lane addresses here instead of hoisting
    // them out of the tile loop (where they would stay live over every step).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int fr = ln & 31, h = ln >> 5;
    const PTile tl = tile_at(j);
    const uint32_t area = ops_lds + (j & 1) * 2560;
    const uint32_t out = stg + wave * kLoadsPerWave * 1024;
    TOut *const y0 = static_cast<TOut *>(p.y) + (int64_t)tl.m0 * p.y_st;
    const i32x4 yr = resource(y0, (uint32_t)(min(kTile, p.m - tl.m0) * p.y_st * (int64_t)sizeof(TOut)));
    const bool has_bias = p.bias != nullptr;
    const uint32_t wpos = fr * 256 + 8 * (h ^ (fr >> 4));  // the lane's row and half in the staging area
#pragma unroll
    for (int b = 0; b < 4; ++b) {  // rows 32 b .. 32 b + 31 of the wave's 128
      const float xs = *(const DAN_LDS float *)(uintptr_t)(area + 4 * (128 * wm + 32 * b + fr));
      u32x2 pk[16];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int c = 128 * wn + 32 * a + 8 * g + 4 * h;  // tile column of the lane's 4 outputs
          const f32x4 ws = *(const DAN_LDS f32x4 *)(uintptr_t)(area + 1024 + 4 * c);
          f32x4 bv = {};
          if (has_bias) {
            typedef TOut v4 __attribute__((ext_vector_type(4)));
            bv = __builtin_convertvector(__builtin_bit_cast(v4, *(const DAN_LDS u32x2 *)(uintptr_t)(area + 2048 + 2 * c)), f32x4);
          }
          f32x4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = __builtin_fmaf(acc[a][b][4 * g + i] * xs, ws[i], bv[i]);
          pk[4 * a + g] = Out<TOut>::pack4(v);
          *(DAN_LDS u32x2 *)(uintptr_t)(out + wpos + 16 * ((4 * a + g) ^ (fr & 15))) = pk[4 * a + g];
        }
      lds_writes_done(pk);
      const int rr = ln >> 4, c = ln & 15;
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int r = 4 * it + rr;
        u32x4 v = *(const DAN_LDS u32x4 *)(uintptr_t)(out + r * 256 + 16 * (c ^ (r & 15)));
        if (r >= 16) v = __builtin_shufflevector(v, v, 2, 3, 0, 1);
        const int row = 128 * wm + 32 * b + r, col = tl.n0 + 128 * wn + 8 * c;
        const uint32_t off = col < p.n ? (uint32_t)(row * p.y_st + col) * (uint32_t)sizeof(TOut) : kOutOfRange;
        store16(yr, off, v);
      }
    }
  };

  const std::integral_constant<bool, true> zeroed, yes;
  const std::integral_constant<bool, false> later, no;
  auto wait = [&](bool boundary) __attribute__((always_inline)) {
    if (boundary) wait_vm<2 * kLoadsPerWave + kPBoundaryOps>();
    else wait_vm<2 * kLoadsPerWave>();
    barrier_lds();
  };
  int g = 0;
  for (int j = 0; j < my_tiles; ++j) {
    const bool b = j > 0;  // steps 0 and 1 wait across the previous tile's boundary operations
    wait(b);
    step(g, f0, f1, zeroed, yes);
    wait(b);
    step(g + 1, f1, f0, later, yes);
    g += 2;
    for (int s = 2; s < kt - 2; s += 2, g += 2) {
      wait(false);
      step(g, f0, f1, later, yes);
      wait(false);
      step(g + 1, f1, f0, later, yes);
    }
    wait(false);
    step(g, f0, f1, later, yes);
    wait(false);
    step(g + 1, f1, f0, later, no);  // the tile's last step: its stage becomes the staging area
    epilogue(j, lds_base + ((g + 1) & (kStages - 1)) * kStageBytes);
    issue_ops(j + 1);
    issue_held(g + 1);
    g += 2;
  }
  wait_vm<0>();
}

template <typename TOut, bool kTail>
hipError_t launch(const Params &p, hipStream_t s) {
  auto kernel = fp8_gemm_kernel<TOut, kTail>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(kernel, dim3(p.tiles_m * p.tiles_n), dim3(kThreads), kLds, s, p);
  return hipGetLastError();
}

template <typename TOut, bool kTail>
hipError_t launch_persistent(const Params &p, int grid, hipStream_t s) {
  auto kernel = fp8_gemm_persistent<TOut, kTail>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, kPLds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), kPLds, s, p);
  return hipGetLastError();
}

int num_cus() {  // of the current device, cached per device
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

template <typename TOut>
hipError_t launch(const Params &p, hipStream_t s) {
  const int kt = (p.k + kBK - 1) / kBK, tiles = p.tiles_m * p.tiles_n, cus = num_cus();
  // The persistent form: 16-bit outputs, an even number of k-steps >= 6, and
  // 256 output rows spanning less than 2 GiB (its stores use a buffer resource).
  if constexpr (sizeof(TOut) == 2) {
    if (kt >= 6 && kt % 2 == 0 && cus > 0 && (int64_t)kTile * p.y_st * (int64_t)sizeof(TOut) < ((int64_t)1 << 31)) {
      const int grid = tiles < cus ? tiles : cus;
      return p.k % kBK ? launch_persistent<TOut, true>(p, grid, s) : launch_persistent<TOut, false>(p, grid, s);
    }
  }
  return p.k % kBK ? launch<TOut, true>(p, s) : launch<TOut, false>(p, s);
}

}  // namespace dan_gemm

extern "C" {

int dan_fp8_gemm(const DanFp8GemmArgs *a, void *stream) {
  using dan::fail;
  dan::g_err[0] = 0;
  if (!a) return fail(DAN_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != DAN_FP8_ABI_VERSION)
    return fail(DAN_ERR_VERSION, "abi_version %d, the fp8 library speaks %d", a->abi_version, DAN_FP8_ABI_VERSION);
  if (a->out_dtype != DAN_DTYPE_BF16 && a->out_dtype != DAN_DTYPE_F16 && a->out_dtype != DAN_DTYPE_F32)
    return fail(DAN_ERR_UNSUPPORTED, "out_dtype %d: bf16, f16 or f32", a->out_dtype);
  if (a->m < 0 || a->n < 0 || a->k < 0) return fail(DAN_ERR_INVALID_ARGUMENT, "negative shape");
  if (a->k % 16 || a->n % 16)
    return fail(DAN_ERR_INVALID_ARGUMENT, "k %d and n %d must be multiples of 16", a->k, a->n);
  if (a->flags & ~(DAN_FP8_GEMM_X_SCALE_TENSOR | DAN_FP8_GEMM_W_SCALE_TENSOR | DAN_FP8_GEMM_X_TILED | DAN_FP8_GEMM_W_TILED))
    return fail(DAN_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", a->flags);
  if (a->m == 0 || a->n == 0) return DAN_OK;
  if (!a->xq || !a->wq || !a->x_scale || !a->w_scale || !a->y) return fail(DAN_ERR_INVALID_ARGUMENT, "NULL pointer");
  const int es = a->out_dtype == DAN_DTYPE_F32 ? 4 : 2;
  const bool xt = a->flags & DAN_FP8_GEMM_X_TILED, wt = a->flags & DAN_FP8_GEMM_W_TILED;
  if (((uintptr_t)a->xq & 15) || ((uintptr_t)a->wq & 15))
    return fail(DAN_ERR_INVALID_ARGUMENT, "xq and wq must be 16-byte aligned");
  if ((!xt && (a->xq_stride % 16 || a->xq_stride < a->k)) || (!wt && (a->wq_stride % 16 || a->wq_stride < a->k)))
    return fail(DAN_ERR_INVALID_ARGUMENT, "row-major xq and wq need strides >= k, multiples of 16 bytes");
  // a panel (256 rows) must span less than 2 GiB: its buffer resource counts bytes in 31 bits
  const int64_t span = (int64_t)256 * ((a->k + 63) / 64 * 64);
  if ((xt ? span : (int64_t)256 * a->xq_stride) >= ((int64_t)1 << 31) ||
      (wt ? span : (int64_t)256 * a->wq_stride) >= ((int64_t)1 << 31))
    return fail(DAN_ERR_UNSUPPORTED, "256 rows of xq or wq span 2 GiB or more");
  if (((uintptr_t)a->y & 15) || (a->y_stride * es) % 16 || a->y_stride < a->n)
    return fail(DAN_ERR_INVALID_ARGUMENT, "y rows must be 16-byte aligned, with y_stride >= n");
  if (((uintptr_t)a->x_scale & 3) || ((uintptr_t)a->w_scale & 15) || ((uintptr_t)a->bias & 15))
    return fail(DAN_ERR_INVALID_ARGUMENT, "x_scale 4-byte, w_scale and bias 16-byte aligned");
  dan_gemm::Params p;
  p.x = a->xq; p.w = a->wq; p.x_st = a->xq_stride; p.w_st = a->wq_stride;
  p.x_tiled = (a->flags & DAN_FP8_GEMM_X_TILED) != 0;
  p.w_tiled = (a->flags & DAN_FP8_GEMM_W_TILED) != 0;
  p.xs = a->x_scale; p.ws = a->w_scale;
  p.xs_inc = (a->flags & DAN_FP8_GEMM_X_SCALE_TENSOR) ? 0 : 1;
  p.ws_inc = (a->flags & DAN_FP8_GEMM_W_SCALE_TENSOR) ? 0 : 1;
  p.bias = a->bias; p.y = a->y; p.y_st = a->y_stride;
  p.m = a->m; p.n = a->n; p.k = a->k;
  p.tiles_m = (a->m + dan_gemm::kTile - 1) / dan_gemm::kTile;
  p.tiles_n = (a->n + dan_gemm::kTile - 1) / dan_gemm::kTile;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  if (a->out_dtype == DAN_DTYPE_BF16) err = dan_gemm::launch<__bf16>(p, s);
  else if (a->out_dtype == DAN_DTYPE_F16) err = dan_gemm::launch<_Float16>(p, s);
  else err = dan_gemm::launch<float>(p, s);
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "fp8 GEMM launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}

}  // extern "C"
