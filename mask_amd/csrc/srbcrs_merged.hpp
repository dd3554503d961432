// Merged-window SR-BCRS SpMM for gfx950: one wave walks the blocks of W
// consecutive row windows interleaved, so that it sweeps its B rows once in
// ascending order, with its column chunk pinned to one XCD.
//
// Why.  On matrices whose columns are spread evenly (the uniform workload),
// a window's B rows land anywhere in B, so a wave that walks its windows one
// after the other sweeps B once per window, and the rows it gathers are
// rarely still in its XCD's L2 when another wave on that XCD needs them.
// Interleaving the W windows' blocks (each window's blocks ascend by B-row
// index) makes every resident wave sweep B from the low rows to the high
// rows once, all of them roughly in step, and pinning each column chunk to
// one XCD (chunk = XCD % chunks) shrinks the B slice one L2 serves to
// K x chunk columns.  Rows one wave gathers are then reused from the L2 by
// the other waves of its XCD shortly after.  Measured with the gather probe
// on uniform-65536 at N = 512 (bench.py --gather-study): 0.230 ms for the
// gathers in unit order, 0.100-0.115 ms merged over 8 windows.
//
// Layout (built once per plan and W on the host, srbcrs_capi.cpp): group g
// covers windows [g*W, g*W + W); its stream holds R rounds of W units, round
// r = block r of each window in window order, R the most blocks any of the
// windows has.  A window with fewer blocks leaves null units (B-row indices
// -1, A words zero), which the kernel skips.  So unit j of a round always
// belongs to window slot j: the accumulator tile of every unit is known at
// compile time (a runtime tile choice made the compiler copy the
// accumulators through registers on every unit).
//
// Arithmetic.  Each window keeps its own accumulator tile and receives its
// blocks' MFMAs in its own block order, exactly as in spmm_stream, so the
// result is bit-identical to every other launch setting.
//
// Operands.  sidx and the compact A words are copies in the stream order;
// the packed values are the plan's own (each word carries the index of its
// first value).
#pragma once
#include "srbcrs_stream.hpp"

#ifdef SRBCRS_MERGED_SCHED_PIN
#define SRBCRS_MERGED_PIN __builtin_amdgcn_sched_barrier(0)
#else
#define SRBCRS_MERGED_PIN (void)0
#endif

namespace srbcrs {

// The B-row indices of one unit for the lane.  By default all 8 are read
// wave-uniformly (scalar loads) and the lane picks its pair; with
// SRBCRS_MERGED_VEC_IDX each lane loads its own pair (one 8-byte vector load,
// no selects), counted on vmcnt with the ring's other loads.
#ifdef SRBCRS_MERGED_VEC_IDX
struct MergedRows {
  int2 p;
  __device__ __forceinline__ void load(const int* __restrict__ sidx, int64_t unit, int k) {
    p = *reinterpret_cast<const int2*>(sidx + unit * 8 + 2 * k);
  }
  __device__ __forceinline__ bool live() const { return __builtin_amdgcn_readfirstlane(p.x) >= 0; }
  __device__ __forceinline__ int2 rows(int) const { return int2{p.x > 0 ? p.x : 0, p.y > 0 ? p.y : 0}; }
};
#else
struct MergedRows {
  UnitRows r;
  __device__ __forceinline__ void load(const int* __restrict__ sidx, int64_t unit, int) { r.load(sidx, unit); }
  __device__ __forceinline__ bool live() const { return r.lo.x >= 0; }
  __device__ __forceinline__ int2 rows(int k) const {
    const int2 q = r.pick(k);
    return int2{q.x > 0 ? q.x : 0, q.y > 0 ? q.y : 0};
  }
};
#endif

// Workgroup id -> (window group g, column chunk c) with the chunk pinned to
// the XCD the dispatcher deals the workgroup to (id % 8).  n_chunks divides
// 8 (XCD x serves chunk x % n_chunks, 8 / n_chunks groups per round of 8
// workgroups) or is a multiple of 8 (XCD x serves chunks x, x + 8, ...);
// any other count runs unpinned, the chunks of a group on consecutive
// workgroups.  Returns false for the padding workgroups of the last round.
__device__ __forceinline__ bool xcd_chunk(int64_t bid, int n_chunks, int64_t n_groups, int64_t& g, int& c) {
  const int x = (int)(bid % kNumXcd);
  const int64_t t = bid / kNumXcd;
  if (n_chunks <= kNumXcd ? kNumXcd % n_chunks != 0 : n_chunks % kNumXcd != 0) {
    c = (int)(bid % n_chunks);
    g = bid / n_chunks;
  } else if (n_chunks <= kNumXcd) {
    const int per = kNumXcd / n_chunks;
    c = x % n_chunks;
    g = t * per + x / n_chunks;
  } else {
    const int k = n_chunks / kNumXcd;
    c = x + kNumXcd * (int)(t % k);
    g = t / k;
  }
  return g < n_groups;
}

// 16x8 blocks, one wave per workgroup, 16*VEC*G columns per wave, W windows
// per group (DEPTH divides W).  The register ring is spmm_stream's: DEPTH
// units in flight, the B-row indices and A words of each slot's next unit
// fetched one ring ahead by scalar loads.  The loop body covers one round
// (W units), so ring slot (j % DEPTH) and window slot (j) are constants;
// every round but the last refills every slot unconditionally with a unit
// that exists (rounds are whole), and the last round refills only the slots
// still needed.  Null units are loaded from B row 0 and skipped by a
// wave-uniform branch.  One group per wave: the tiles are stored once, at
// the wave's end.  (Waves that streamed several groups and stored each
// group's tiles between them were slower, 0.243 against 0.215 ms on
// uniform-65536: vmcnt counts stores with loads, so the ring's next waits
// also waited for the stores.)
template <int VEC, int G, int W, int DEPTH, class AF>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void spmm_merged(
    const int* __restrict__ moff, int Mo, const int* __restrict__ sidx, AF asrc, const float* __restrict__ B,
    float* __restrict__ C, const int* __restrict__ rowmap, int M, int N, int64_t ldb, int64_t ldc, int n_chunks,
    int64_t n_groups, int relu) {
  static_assert(W % DEPTH == 0, "the ring depth divides the round");
  constexpr int BH = 16, BW = 8;
  constexpr int WCOLS = 16 * VEC * G;
  int64_t g;
  int c;
  if (!xcd_chunk(blockIdx.x, n_chunks, n_groups, g, c)) return;
  const int wcol = c * WCOLS;
  if (wcol >= N) return;
  const int lane = threadIdx.x;
  const int col0 = wcol + VEC * (lane & 15);
  const int w0 = (int)(g * W);
  const int nw = w0 + W < Mo ? W : Mo - w0;
  f4 acc[W][1][G][VEC];
#pragma unroll
  for (int w = 0; w < W; ++w)
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
      for (int s = 0; s < VEC; ++s) acc[w][0][gg][s] = f4{0.f, 0.f, 0.f, 0.f};
  const int64_t us = uniform_load(moff, g), ue = uniform_load(moff, g + 1);
  if (us < ue) {
    const int k = lane >> 4;
    int a_off[1][1];
    a_off[0][0] = swizzle_2_2_3(BW * (lane & 15) + 2 * k);
    Frag<1, VEC, G> f[DEPTH];
    MergedRows idx[DEPTH];
    typename AF::template Meta<1> am[DEPTH];
    bool live[DEPTH];
    const int64_t last = ue - 1;
    // a null unit (indices -1) reads B row 0 (MergedRows::rows) and is skipped
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {   // rounds hold W >= DEPTH units
      const int64_t u = us + d;
      MergedRows r;
      r.load(sidx, u, k);
      live[d] = r.live();
      load_frag<BH, BW, VEC, G>(f[d], B, asrc, u, r.rows(k), asrc.template meta<BH, BW>(u, lane), a_off, ldb,
                                col0, lane);
      const int64_t nu = us + DEPTH + d < last ? us + DEPTH + d : last;
      idx[d].load(sidx, nu, k);
      am[d] = asrc.template meta<BH, BW>(nu, lane);
    }
    int64_t base = us;
    for (; base + W < ue; base += W) {
#pragma unroll
      for (int j = 0; j < W; ++j) {
        const int d = j % DEPTH;
        if (live[d]) mma_frag<1, VEC, G>(f[d], acc[j]);
        SRBCRS_MERGED_PIN;
        const int64_t nu = base + j + DEPTH;   // exists: a whole round follows this one
        live[d] = idx[d].live();
        load_frag<BH, BW, VEC, G>(f[d], B, asrc, nu, idx[d].rows(k), am[d], a_off, ldb, col0, lane);
        const int64_t nn = nu + DEPTH < last ? nu + DEPTH : last;
        idx[d].load(sidx, nn, k);
        am[d] = asrc.template meta<BH, BW>(nn, lane);
        SRBCRS_MERGED_PIN;
      }
    }
    // the last round: refill only the slots whose next unit is in it
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const int d = j % DEPTH;
      if (live[d]) mma_frag<1, VEC, G>(f[d], acc[j]);
      if (j + DEPTH < W) {
        const int64_t nu = base + j + DEPTH;
        live[d] = idx[d].live();
        load_frag<BH, BW, VEC, G>(f[d], B, asrc, nu, idx[d].rows(k), am[d], a_off, ldb, col0, lane);
        if (j + 2 * DEPTH < W) {
          idx[d].load(sidx, nu + DEPTH, k);
          am[d] = asrc.template meta<BH, BW>(nu + DEPTH, lane);
        }
      }
    }
  }
#pragma unroll
  for (int w = 0; w < W; ++w)
    if (w < nw) store_tile<VEC, G>(acc[w][0], C, (int64_t)(w0 + w) * BH, M, ldc, col0, lane, rowmap, relu != 0);
}

}  // namespace srbcrs
