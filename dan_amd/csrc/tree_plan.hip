// Device-side tile planner for the gfx950 tree-masked attention (MI355X,
// CDNA4): one launch per packed forward builds key_lo, col_seg, the work list
// and the persistent schedule that dan_tree_attn_fwd reads, from the segment
// table and the branch starts (O(segments) on the host). It replaces, on the
// device, what dan/attention.py:138-172 (ReadLayout.build) computes on the
// host every forward, and the host planner of this package (dan_amd/plan.py).
//
// One work group of 1024 threads; the segment table and the branch starts are
// first copied to LDS, where every search below runs:
//   1. key_lo (zero, then every branch's rows, one thread per branch) and
//      col_seg
//   2. work items; their costs (key tiles) sorted longest first, ties by
//      creation order (bitonic sort of 64-bit keys in LDS)
//   3. one wave deals the sorted items to the k slots of a head-group class,
//      each to the least loaded slot (ties: lowest slot), then repeatedly
//      moves one item out of the most loaded slot, or swaps one of its items
//      with a lighter item elsewhere, choosing the option with the lowest
//      resulting larger load of the pair, while that is below the maximum
//   4. a sort by (slot, rank) gives each slot's items longest first; slot s
//      of the k * G slots runs class s / G for head group s % G
// Every loop has a fixed bound (the rebalance stops after 2 W + 64 rounds).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dan_tree_plan.h"

namespace dan {
int fail(int status, const char *fmt, ...);  // tree_attn.hip: sets the thread's last-error message
extern thread_local char g_err[512];
}  // namespace dan

namespace dan_plan {

constexpr int kThreads = 1024;
constexpr int kMaxWork = DAN_TREE_PLAN_MAX_WORK;
constexpr int kMaxSlots = DAN_TREE_PLAN_MAX_SLOTS;
constexpr int kMaxSegs = DAN_TREE_PLAN_MAX_SEGMENTS;
constexpr int kMaxBranches = DAN_TREE_PLAN_MAX_BRANCHES;
constexpr int kTile = DAN_TREE_ATTN_KEY_TILE;

#define DAN_GLOBAL __attribute__((address_space(1)))

// Table pointers arrive inside a struct, so the compiler cannot prove they
// are global memory; reading through address space 1 gives global loads.
template <typename T>
__device__ inline T ld(const T *p) {
  static_assert(sizeof(T) % 4 == 0, "table entries are dword multiples");
  struct Raw {
    uint32_t w[sizeof(T) / 4];
  } raw;
  const DAN_GLOBAL uint32_t *src = (const DAN_GLOBAL uint32_t *)p;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) raw.w[i] = src[i];
  return __builtin_bit_cast(T, raw);
}

struct Params {
  int32_t N, S, B, W, C, tile_q, G, k, overhead, max_rounds;
  int32_t kcap;             // slots per head group the sched_off table covers (== k unless counts)
  const int32_t *counts;    // budget mode: device {S, B, W, C} (capacities in S, B, W, C)
  const DanSegmentDesc *segs;  // LDS copies (the kernel repoints these at its own)
  const int32_t *bstart;
  int32_t *key_lo, *col_seg, *cost;
  DanWorkItem *work;
  DanUnit *units;
  int32_t *sched_off;
};

// Dynamic LDS layout.
struct Smem {
  DanSegmentDesc seg[kMaxSegs];
  int32_t bst[kMaxBranches];
  uint64_t keys[kMaxWork];  // sort keys
  int32_t w[kMaxWork];      // schedule weight of the item at each rank
  int16_t slot[kMaxWork];   // slot of each rank
  int16_t alist[kMaxWork];  // ranks held by the most loaded slot
  int32_t load[kMaxSlots];
  int32_t start[kMaxSlots + 1];  // first position of each slot's run after the (slot, rank) sort
};

__device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

__device__ inline DanSegmentDesc seg_at(const Params &p, int i) {
  return p.segs[i];
}
__device__ inline int branch_end_idx(const Params &p, int i) {  // one past segment i's last branch
  return i + 1 < p.S ? seg_at(p, i + 1).reserved[1] : p.B;
}

// The last segment whose field `f` (a prefix sum over segments) is <= x.
template <typename F>
__device__ inline int find_seg(const Params &p, int x, F f) {
  int lo = 0, hi = p.S - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (f(seg_at(p, mid)) <= x) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// key_lo of packed row `row` in branch region of segment s: P + (first row of
// its branch - start), the first row being the last branch start <= row.
__device__ inline int branch_key_lo(const Params &p, const DanSegmentDesc &s, int b0, int b1, int row) {
  int lo = max(b0, 0), hi = min(b1, p.B) - 1;
  if (hi < lo) return s.past_len + s.trunk;  // no branch entry: the region starts at the trunk's end
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.bstart[mid] <= row) lo = mid;
    else hi = mid - 1;
  }
  const int a = max(p.bstart[lo], s.start + s.trunk);
  return s.past_len + (a - s.start);
}

// Work item `w` in creation order (segment by segment, query tiles in order)
// and its cost in key tiles, as dan_amd/plan.py build_tables makes it.
__device__ inline DanWorkItem make_item(const Params &p, int w, int &cost) {
  const int i = find_seg(p, w, [](const DanSegmentDesc &s) { return s.reserved[0]; });
  const DanSegmentDesc s = seg_at(p, i);
  const int n = s.n, t = s.trunk, P = s.past_len, pt = P + t;
  const int t0 = min(max(w - s.reserved[0], 0) * p.tile_q, max(n - 1, 0));
  const int tq = min(p.tile_q, n - t0);
  const int top = P + t0 + tq;
  const int kfull = min(P + t0 + 1, pt);
  const int ja1 = ceil_div(min(pt, top), kTile);
  int jb0 = ja1, jb1 = ja1, lo_max = 0;
  if (t0 + tq > t) {
    const int b0 = s.reserved[1], b1 = branch_end_idx(p, i);
    const int first = s.start + max(t0, t);
    jb0 = max(branch_key_lo(p, s, b0, b1, first) / kTile, ja1);
    jb1 = max(ceil_div(top, kTile), jb0);
    lo_max = branch_key_lo(p, s, b0, b1, s.start + t0 + tq - 1);
  }
  cost = ja1 + jb1 - jb0;
  DanWorkItem it;
  it.seg = i; it.t0 = t0; it.tq = tq; it.ja1 = ja1; it.jb0 = jb0; it.jb1 = jb1;
  it.jfull = kfull / kTile; it.lo_max = lo_max;
  return it;
}

// Ascending bitonic sort of keys[0, n), n a power of two.
__device__ inline void bitonic(uint64_t *keys, int n) {
  for (int size = 2; size <= n; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < n / 2; i += kThreads) {
        const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t a = keys[lo], b = keys[hi];
        if ((a > b) == up) {
          keys[lo] = b;
          keys[hi] = a;
        }
      }
      __syncthreads();
    }
}

// Minimum (maximum) of x over the wave's 64 lanes, returned in every lane.
// DPP lane moves: quad permutes [1,0,3,2] and [2,3,0,1], rotations by 4 and 8
// within each row of 16 lanes (every lane then holds its row's result), and
// the broadcasts of lane 15 to the next row and of lane 31 to rows 2 and 3:
// lane 63 ends with the wave's result. A lane without a source keeps x.
template <bool kMax>
__device__ inline uint32_t wave_reduce(uint32_t x) {
  auto step = [](uint32_t v, int moved) {
    const uint32_t m = (uint32_t)moved;
    return kMax ? (m > v ? m : v) : (m < v ? m : v);
  };
  x = step(x, __builtin_amdgcn_update_dpp((int)x, (int)x, 0xb1, 0xf, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp((int)x, (int)x, 0x4e, 0xf, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp((int)x, (int)x, 0x124, 0xf, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp((int)x, (int)x, 0x128, 0xf, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp((int)x, (int)x, 0x142, 0xf, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp((int)x, (int)x, 0x143, 0xf, 0xf, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
__device__ inline uint32_t wave_min_u32(uint32_t x) { return wave_reduce<false>(x); }
__device__ inline uint32_t wave_max_u32(uint32_t x) { return wave_reduce<true>(x); }

__global__ __launch_bounds__(kThreads) void plan_kernel(const Params pg) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  Smem &sm = *reinterpret_cast<Smem *>(smem_raw);
  const int tid = threadIdx.x, lane = tid & 63;

  // ---- 0. budget mode: this batch's counts, clamped to the capacities
  Params p = pg;
  if (pg.counts) {
    const DAN_GLOBAL int32_t *c = (const DAN_GLOBAL int32_t *)pg.counts;
    p.S = min(max(c[0], 0), pg.S);
    p.B = min(max(c[1], 0), pg.B);
    p.W = min(max(c[2], 0), pg.W);
    p.C = min(max(c[3], 0), pg.C);
    p.k = max(1, min(pg.kcap, p.W));
    p.max_rounds = 2 * p.W + 64;
  }
  // ---- 0. the segment table and branch starts into LDS
  for (int i = tid; i < p.S; i += kThreads) sm.seg[i] = ld(pg.segs + i);
  for (int b = tid; b < p.B; b += kThreads) sm.bst[b] = ld(pg.bstart + b);
  p.segs = sm.seg;
  p.bstart = sm.bst;

  // ---- 1. key_lo, col_seg
  for (int r = tid; r < p.N; r += kThreads) p.key_lo[r] = 0;
  __syncthreads();
  for (int b = tid; b < p.B; b += kThreads) {  // one thread per branch: its rows
    const int i = find_seg(p, b, [](const DanSegmentDesc &s) { return s.reserved[1]; });
    const DanSegmentDesc s = seg_at(p, i);
    const int end = b + 1 < branch_end_idx(p, i) ? p.bstart[b + 1] : s.start + s.n;
    const int lo = s.past_len + (max(p.bstart[b], s.start + s.trunk) - s.start);
    for (int r = max(p.bstart[b], 0); r < min(end, p.N); ++r) p.key_lo[r] = lo;
  }
  for (int c = tid; c < p.C; c += kThreads)
    p.col_seg[c] = find_seg(p, c * kTile, [](const DanSegmentDesc &s) { return s.vt_col; });

  // ---- 2. work items, sorted longest first (ties: creation order)
  int np2 = 1;
  while (np2 < p.W) np2 <<= 1;
  for (int r = tid; r < np2; r += kThreads) {
    uint64_t key = ~0ull;
    if (r < p.W) {
      int c;
      make_item(p, r, c);
      key = ((uint64_t)(0xffffffffu - (uint32_t)c) << 32) | (uint32_t)r;
    }
    sm.keys[r] = key;
  }
  __syncthreads();
  bitonic(sm.keys, np2);
  for (int q = tid; q < p.W; q += kThreads) {
    int c;
    const DanWorkItem it = make_item(p, (int)(sm.keys[q] & 0xffffffffu), c);
    p.work[q] = it;
    p.cost[q] = c;
    sm.w[q] = c + p.overhead;
  }
  __syncthreads();
  // Longest first onto empty slots: item q < k goes to slot q (every weight
  // is at least 1, so the least loaded slot, lowest first, is always the
  // next empty one).
  const int k0 = min(p.k, p.W);
  for (int j = tid; j < p.k; j += kThreads) {
    sm.load[j] = j < k0 ? sm.w[j] : 0;
    if (j < k0) sm.slot[j] = (int16_t)j;
  }
  __syncthreads();

  // ---- 3. one wave: longest-processing-time dealing, then moves and swaps
  if (tid < 64) {
    constexpr int kPer = kMaxSlots / 64;  // slots per lane: j = lane + 64 m
    int32_t lreg[kPer];
#pragma unroll
    for (int m = 0; m < kPer; ++m) lreg[m] = lane + 64 * m < p.k ? sm.load[lane + 64 * m] : 0x7fffffff;
    for (int q = k0; q < p.W; ++q) {
      uint32_t bl = 0xffffffffu, bj = 0xffffffffu;  // the lane's least loaded slot (lowest first)
#pragma unroll
      for (int m = 0; m < kPer; ++m)
        if ((uint32_t)lreg[m] < bl) {
          bl = (uint32_t)lreg[m];
          bj = (uint32_t)(lane + 64 * m);
        }
      const uint32_t gl = wave_min_u32(bl);
      const int j = (int)wave_min_u32(bl == gl ? bj : 0xffffffffu);
      const int wq = sm.w[q];
#pragma unroll
      for (int m = 0; m < kPer; ++m)
        if (lane + 64 * m == j) lreg[m] += wq;
      if (lane == 0) sm.slot[q] = (int16_t)j;
    }
#pragma unroll
    for (int m = 0; m < kPer; ++m)
      if (lane + 64 * m < p.k) sm.load[lane + 64 * m] = lreg[m];
    __builtin_amdgcn_wave_barrier();
    for (int round = 0; round < p.max_rounds; ++round) {
      uint32_t tl = 0;  // the most loaded slot (lowest first)
      for (int j = lane; j < p.k; j += 64) tl = max(tl, (uint32_t)sm.load[j]);
      tl = wave_max_u32(tl);
      uint32_t aj = 0xffffffffu;
      for (int j = lane; j < p.k; j += 64)
        if ((uint32_t)sm.load[j] == tl) aj = min(aj, (uint32_t)j);
      const int a = (int)wave_min_u32(aj);
      const int top = (int)tl;
      // ranks held by slot a, in rank order
      int ma = 0;
      for (int q0 = 0; q0 < p.W; q0 += 64) {
        const int q = q0 + lane;
        const bool in = q < p.W && sm.slot[q] == a;
        const uint64_t mask = __ballot(in);
        if (in) sm.alist[ma + __builtin_popcountll(mask & ((1ull << lane) - 1))] = (int16_t)q;
        ma += __builtin_popcountll(mask);
      }
      __builtin_amdgcn_wave_barrier();
      // best option: lowest resulting larger load, then lowest position in a's
      // list, moves before swaps, then lowest slot / rank
      uint64_t best = ~0ull;
      for (int pi = 0; pi < ma; ++pi) {
        const int ia = sm.alist[pi];
        const int wa = sm.w[ia];
        for (int b = lane; b < p.k; b += 64) {
          if (b == a) continue;
          const int nw = max(top - wa, sm.load[b] + wa);
          if (wa > 0 && nw < top) {
            const uint64_t key = ((uint64_t)(uint32_t)nw << 32) | ((uint32_t)pi << 13) | (uint32_t)b;
            best = key < best ? key : best;
          }
        }
        for (int jq = lane; jq < p.W; jq += 64) {
          const int b = sm.slot[jq];
          if (b == a) continue;
          const int d = wa - sm.w[jq];
          const int nw = max(top - d, sm.load[b] + d);
          if (d > 0 && nw < top) {
            const uint64_t key = ((uint64_t)(uint32_t)nw << 32) | ((uint32_t)pi << 13) | (1u << 12) | (uint32_t)jq;
            best = key < best ? key : best;
          }
        }
      }
      const uint32_t bhi = wave_min_u32((uint32_t)(best >> 32));
      const uint32_t blo = wave_min_u32((uint32_t)(best >> 32) == bhi ? (uint32_t)best : 0xffffffffu);
      if (bhi == 0xffffffffu && blo == 0xffffffffu) break;
      best = ((uint64_t)bhi << 32) | blo;
      const int pi = (int)((best >> 13) & 0x7ffff), kind = (int)((best >> 12) & 1), idx = (int)(best & 0xfff);
      if (lane == 0) {
        const int ia = sm.alist[pi];
        if (kind == 0) {  // move item ia to slot idx
          sm.load[a] -= sm.w[ia];
          sm.load[idx] += sm.w[ia];
          sm.slot[ia] = (int16_t)idx;
        } else {  // swap item ia with item idx
          const int b = sm.slot[idx], d = sm.w[ia] - sm.w[idx];
          sm.load[a] -= d;
          sm.load[b] += d;
          sm.slot[ia] = (int16_t)b;
          sm.slot[idx] = (int16_t)a;
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();

  // ---- 4. each slot's items in rank order; offsets and unit records
  for (int r = tid; r < np2; r += kThreads)
    sm.keys[r] = r < p.W ? ((uint64_t)(uint32_t)sm.slot[r] << 16) | (uint32_t)r : ~0ull;
  __syncthreads();
  bitonic(sm.keys, np2);
  for (int j = tid; j <= p.k; j += kThreads) {  // first position with slot >= j
    int lo = 0, hi = p.W;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((int)(sm.keys[mid] >> 16) < j) lo = mid + 1;
      else hi = mid;
    }
    sm.start[j] = lo;
  }
  __syncthreads();
  const int G = p.G;
  for (int s = tid; s <= p.kcap * G; s += kThreads) {
    if (s >= p.k * G) {  // the end, and the empty slots past this batch's (budget mode)
      p.sched_off[s] = G * p.W;
    } else {
      const int j = s / G, g = s % G;
      p.sched_off[s] = G * sm.start[j] + g * (sm.start[j + 1] - sm.start[j]);
    }
  }
  for (int x = tid; x < p.W * G; x += kThreads) {
    const int q = x / G, g = x % G;
    const int r = (int)(sm.keys[q] & 0xffff), j = (int)(sm.keys[q] >> 16);
    const int cnt = sm.start[j + 1] - sm.start[j];
    const int u = G * sm.start[j] + g * cnt + (q - sm.start[j]);
    const DanWorkItem it = ld(p.work + r);
    const DanSegmentDesc s = seg_at(p, it.seg);
    DanUnit un;
    un.item = it;
    un.start = s.start; un.n = s.n; un.trunk = s.trunk; un.past_len = s.past_len;
    un.past_idx = s.past_idx; un.vt_col = s.vt_col; un.group = g; un.reserved = 0;
    p.units[u] = un;
  }
}

}  // namespace dan_plan

extern "C" {

int dan_tree_attn_plan_abi_version(void) { return DAN_TREE_PLAN_ABI_VERSION; }

int dan_tree_attn_plan_slots(int32_t num_work, int32_t groups, int32_t num_cus) {
  if (num_work <= 0 || groups <= 0 || num_cus <= 0) return 0;
  const int k = num_cus / groups < num_work ? num_cus / groups : num_work;
  return (k < 1 ? 1 : k) * groups;
}

int dan_tree_attn_plan(const DanTreePlanArgs *a, void *stream) {
  using dan::fail;
  dan::g_err[0] = 0;
  if (!a) return fail(DAN_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != DAN_TREE_PLAN_ABI_VERSION)
    return fail(DAN_ERR_VERSION, "abi_version %d, planner speaks %d", a->abi_version, DAN_TREE_PLAN_ABI_VERSION);
  if (a->num_tokens < 0 || a->num_segments < 0 || a->num_branches < 0 || a->num_work < 0 || a->num_cols < 0)
    return fail(DAN_ERR_INVALID_ARGUMENT, "negative count");
  if (a->num_work == 0) return DAN_OK;
  if (a->num_segments == 0 || a->num_cols == 0)
    return fail(DAN_ERR_INVALID_ARGUMENT, "num_work > 0 needs segments and V^T columns");
  if (a->tile_q <= 0 || a->groups <= 0 || a->num_cus <= 0 || a->overhead < 0)
    return fail(DAN_ERR_INVALID_ARGUMENT, "tile_q, groups and num_cus must be positive, overhead >= 0");
  if (a->num_work > DAN_TREE_PLAN_MAX_WORK)
    return fail(DAN_ERR_UNSUPPORTED, "num_work %d > %d", a->num_work, DAN_TREE_PLAN_MAX_WORK);
  if (a->num_segments > DAN_TREE_PLAN_MAX_SEGMENTS || a->num_branches > DAN_TREE_PLAN_MAX_BRANCHES)
    return fail(DAN_ERR_UNSUPPORTED, "%d segments / %d branches > %d / %d", a->num_segments, a->num_branches,
                DAN_TREE_PLAN_MAX_SEGMENTS, DAN_TREE_PLAN_MAX_BRANCHES);
  const int slots = dan_tree_attn_plan_slots(a->num_work, a->groups, a->num_cus);
  const int k = slots / a->groups;
  if (k > DAN_TREE_PLAN_MAX_SLOTS) return fail(DAN_ERR_UNSUPPORTED, "%d slots per head group > %d", k, DAN_TREE_PLAN_MAX_SLOTS);
  if ((int64_t)a->num_work * a->groups > 0x7fffffff) return fail(DAN_ERR_INVALID_ARGUMENT, "too many units");
  if (!a->segments || (a->num_branches > 0 && !a->branch_starts) || !a->key_lo || !a->col_seg || !a->work ||
      !a->cost || !a->units || !a->sched_off)
    return fail(DAN_ERR_INVALID_ARGUMENT, "NULL table pointer");
  dan_plan::Params p;
  p.N = a->num_tokens; p.S = a->num_segments; p.B = a->num_branches; p.W = a->num_work; p.C = a->num_cols;
  p.tile_q = a->tile_q; p.G = a->groups; p.k = k; p.kcap = k; p.overhead = a->overhead;
  p.max_rounds = 2 * a->num_work + 64;
  p.counts = a->counts;
  p.segs = a->segments; p.bstart = a->branch_starts;
  p.key_lo = a->key_lo; p.col_seg = a->col_seg; p.cost = a->cost; p.work = a->work;
  p.units = a->units; p.sched_off = a->sched_off;
  const int lds = (int)sizeof(dan_plan::Smem);
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(dan_plan::plan_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return fail(DAN_ERR_LAUNCH, "planner LDS attribute: %s", hipGetErrorString(attr));
  hipLaunchKernelGGL(dan_plan::plan_kernel, dim3(1), dim3(dan_plan::kThreads), lds, static_cast<hipStream_t>(stream), p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(DAN_ERR_LAUNCH, "planner launch failed: %s", hipGetErrorString(err));
  return DAN_OK;
}

}  // extern "C"
