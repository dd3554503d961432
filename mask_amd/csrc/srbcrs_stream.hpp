// SR-BCRS SpMM device code for gfx950: the kernel templates shared by the
// library (srbcrs_kernels.hip) and by operators the HIP emitter generates
// (mask_amd/emitter.py), which include this header and instantiate them.
#pragma once
// SR-BCRS fp32 SpMM kernels for gfx950 (CDNA4, wave64).
//
// C[M x N] = A[M x K] * B[K x N], A in SR-BCRS with BH x BW blocks
// (16 x 8, or the 32 x 32 base variant):
//   soff[Mo+1]      block offsets per BH-row window
//   sidx[BW*nb]     the BW B-row (column) indices of each block
//   val[BH*BW*nb]   the block values, BH x BW row-major with CuTe
//                   Swizzle<2,2,3> applied to the offset:
//                   pos(r,c) = o ^ ((o & 0x60) >> 3), o = BW*r + c.
// This is the data the reference's sr_bcrs_spmm_kernel_tf32<16,64,8> (and
// its 32x32 sibling) consumes (examples/src_fp32/sr_bcrs/testbed/
// kernel.inc:1590-1700); the arithmetic here is native fp32 MFMA instead of
// TF32 MMA.
//
// Units.  A block is BW/8 "units" of 8 columns; unit u of block b has
// index b*(BW/8) + q and its 8 B-row indices are sidx[8u .. 8u+8), so the
// kernel walks one contiguous unit sequence for either block shape.
//
// MFMA mapping.  v_mfma_f32_16x16x4_f32 (wave64) computes D(16x16) +=
// A(16x4) * B(4x16) with lane l holding A[l%16][l/16], B[l/16][l%16] and
// D[4*(l/16)+r][l%16], r = 0..3.  A unit times one 16-row half of the
// block is two such k-steps; the unit's 8 columns split as k-step 0 =
// {0,2,4,6}, k-step 1 = {1,3,5,7}, so lane (i = l%16, k = l/16) needs
// A[i][8q+2k] and A[i][8q+2k+1].  The swizzle only touches offset bits 2..3,
// so those two values sit next to each other in memory: one 8-byte load per
// lane and row half fetches the lane's A fragment.
//
// Column mapping.  A wave owns 16*VEC*G output columns.  In column group g
// lane j = l%16 owns columns base + 16*VEC*g + VEC*j + s (s < VEC): one
// VEC-wide vector load per (B row, g) per lane, VEC MFMAs per k-step, g and
// row half.  For VEC = 4 a wave's B load covers four 256-byte row segments.
//
// B ring.  Every B element is used by exactly one wave (waves split N), so
// staging through LDS adds no reuse; by default latency is hidden by a
// register ring DEPTH units deep, with the B-row indices fetched one ring
// further ahead (by scalar loads, see UnitRows).  BSTAGE 1 stages the ring
// through LDS with direct-to-LDS loads instead (LdsB).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace srbcrs {

constexpr int kNumXcd = 8;   // MI355X: 8 XCDs, 32 CUs each

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

template <int VEC> struct VecT;
template <> struct VecT<1> { typedef float type; };
template <> struct VecT<2> { typedef f2 type; };
template <> struct VecT<4> { typedef f4 type; };

template <int VEC>
__device__ __forceinline__ float vget(const typename VecT<VEC>::type& v, int s);
template <> __device__ __forceinline__ float vget<1>(const float& v, int) { return v; }
template <> __device__ __forceinline__ float vget<2>(const f2& v, int s) { return v[s]; }
template <> __device__ __forceinline__ float vget<4>(const f4& v, int s) { return v[s]; }

__device__ __forceinline__ int swizzle_2_2_3(int o) { return o ^ ((o & 0x60) >> 3); }

// Map the hardware workgroup id to a logical one so that each XCD (the
// dispatcher deals workgroups round-robin over the 8 XCDs) receives a
// contiguous range of logical ids: neighbouring row windows, which share B
// rows in banded matrices, then share one L2.
__device__ __forceinline__ int64_t xcd_remap(int64_t id, int64_t n) {
  const int64_t q = n / kNumXcd, r = n % kNumXcd;
  const int64_t x = id % kNumXcd, t = id / kNumXcd;
  return x * q + (x < r ? x : r) + t;
}

// Block geometry: BH x BW blocks, H = BH/16 row halves, Q = BW/8 units.
template <int BH, int BW>
struct Shape {
  static constexpr int H = BH / 16;
  static constexpr int Q = BW / 8;
  static constexpr int SIZE = BH * BW;
};

// One unit in flight: the lane's A fragments (one per row half) and its B
// vectors for the two k-steps.
template <int H, int VEC, int G>
struct Frag {
  typedef typename VecT<VEC>::type V;
  f2 a[H];       // A[16h+i][8q+2k], A[16h+i][8q+2k+1]
  V b0[G];       // B[sidx[8u+2k]][cols of g]
  V b1[G];       // B[sidx[8u+2k+1]][cols of g]
};

// A-operand sources.  Both hand the MFMA the same fragments, bit for bit.
//
// DenseA reads the block values in the reference's layout (val, BH*BW
// swizzled fp32 per block): the lane's two values are adjacent, one 8-byte
// load per row half.
//
// CompactA reads them from a compact copy: for every 32 logical positions
// o = BW*r + c of a block one word {mask, base}, bit t of mask marking a
// stored value at position 32*w + t, whose index in `packed` is base plus
// the number of mask bits below t; unmarked positions are +0.0f.  At the
// low block fills of graph matrices most of the dense array is zeros, so
// this cuts the A bytes a column chunk re-reads by up to ~10x.  The word is
// fetched one ring slot ahead (Meta), so the value loads it steers issue
// with the unit's B loads.  `packed` must hold at least one readable float
// past its last stored value (srbcrs_compact.hip pads it with zeros).
struct DenseA {
  const float* __restrict__ val;
  template <int H> struct Meta {};
  template <int BH, int BW>
  __device__ __forceinline__ Meta<BH / 16> meta(int64_t, int) const { return {}; }
  template <int BH, int BW>
  __device__ __forceinline__ void load(f2 (&a)[BH / 16], int64_t unit, const Meta<BH / 16>&,
                                       const int (&a_off)[BW / 8][BH / 16], int) const {
    typedef Shape<BH, BW> S;
    const int64_t blk = unit / S::Q;
    const int q = (int)(unit % S::Q);
    const float* vb = val + blk * S::SIZE;
#pragma unroll
    for (int h = 0; h < S::H; ++h) {
      int off = a_off[0][h];
#pragma unroll
      for (int qq = 1; qq < S::Q; ++qq)
        if (q == qq) off = a_off[qq][h];
#ifdef SRBCRS_EXPERIMENT_NO_A
      a[h] = f2{1.f, (float)off};
#else
      a[h] = *reinterpret_cast<const f2*>(vb + off);
#endif
    }
  }
};

struct CompactA {
  const uint2* __restrict__ words;
  const float* __restrict__ packed;
  template <int H> struct Meta { uint2 w[H]; };
  // logical position of the lane's first value in unit q, row half h
  template <int BW>
  __device__ __forceinline__ static int pos(int h, int q, int lane) {
    return BW * (16 * h + (lane & 15)) + 8 * q + 2 * (lane >> 4);
  }
  template <int BH, int BW>
  __device__ __forceinline__ Meta<BH / 16> meta(int64_t unit, int lane) const {
    typedef Shape<BH, BW> S;
    const int64_t blk = unit / S::Q;
    const int q = (int)(unit % S::Q);
    Meta<S::H> m;
#pragma unroll
    for (int h = 0; h < S::H; ++h) {
#ifdef SRBCRS_EXPERIMENT_NO_A
      m.w[h] = uint2{(uint32_t)blk, (uint32_t)q};
#else
      m.w[h] = words[blk * (S::SIZE / 32) + (pos<BW>(h, q, lane) >> 5)];
#endif
    }
    return m;
  }
  template <int BH, int BW>
  __device__ __forceinline__ void load(f2 (&a)[BH / 16], int64_t unit, const Meta<BH / 16>& m,
                                       const int (&)[BW / 8][BH / 16], int lane) const {
    typedef Shape<BH, BW> S;
    const int q = (int)(unit % S::Q);
#pragma unroll
    for (int h = 0; h < S::H; ++h) {
      const int bit = pos<BW>(h, q, lane) & 31;   // even, so bit + 1 is in the same word
      const uint32_t mask = m.w[h].x;
      const uint32_t n = m.w[h].y + (uint32_t)__builtin_popcount(mask & ((1u << bit) - 1u));
      const uint32_t b0 = (mask >> bit) & 1u, b1 = (mask >> (bit + 1)) & 1u;
      float v0 = 0.f, v1 = 0.f;
#ifdef SRBCRS_EXPERIMENT_NO_A
      v0 = (float)n;
      v1 = (float)(b0 + b1);
#else
      // Both loads are issued on every lane and the absent values are
      // selected away: n + b0 <= the stored-value count, and the array holds
      // a few zero floats after the last one.  As loads inside lane-divergent
      // branches their number was unknown to the compiler, which then waited
      // for the next unit's B rows before issuing this refill (vmcnt counted
      // for the fewest loads on any path).
      const float p0 = packed[n], p1 = packed[n + b0];
      v0 = b0 ? p0 : 0.f;
      v1 = b1 ? p1 : 0.f;
#endif
      a[h] = f2{v0, v1};
    }
  }
};

// Issue the loads of one unit: the A fragment (through the A source) and the
// lane's B vectors of rows rows.x (k-step 0) and rows.y (k-step 1).
template <int BH, int BW, int VEC, int G, class AF>
__device__ __forceinline__ void load_frag(Frag<BH / 16, VEC, G>& f, const float* __restrict__ B,
                                          const AF& asrc, int64_t unit, int2 rows,
                                          const typename AF::template Meta<BH / 16>& am,
                                          const int (&a_off)[BW / 8][BH / 16], int64_t ldb,
                                          int col0, int lane) {
  typedef typename VecT<VEC>::type V;
  asrc.template load<BH, BW>(f.a, unit, am, a_off, lane);
#ifdef SRBCRS_EXPERIMENT_B_HIT_MASK
  if ((unit & SRBCRS_EXPERIMENT_B_HIT_MASK) == SRBCRS_EXPERIMENT_B_HIT_MASK) rows = int2{0, 0};
#endif
#ifdef SRBCRS_EXPERIMENT_B_SKIP
  // the other units keep the previous B registers: as if neighbouring row
  // windows shared those gathers
  if (unit % SRBCRS_EXPERIMENT_B_SKIP != 0) return;
#endif
  const float* r0 = B + (int64_t)rows.x * ldb + col0;
  const float* r1 = B + (int64_t)rows.y * ldb + col0;
#pragma unroll
  for (int g = 0; g < G; ++g) {
#ifdef SRBCRS_EXPERIMENT_NO_B
    f.b0[g] = V{} + (float)rows.x;
    f.b1[g] = V{} + (float)rows.y;
#else
    f.b0[g] = *reinterpret_cast<const V*>(r0 + 16 * VEC * g);
    f.b1[g] = *reinterpret_cast<const V*>(r1 + 16 * VEC * g);
#endif
  }
}

// The 8 B-row indices of one unit, loaded wave-uniformly, and the lane's
// pair.  Reading them through the constant address space lets the compiler
// use scalar loads, which are counted apart from the vector loads in flight:
// with per-lane vector loads, consuming the indices (to address the next
// unit's B rows) waited for every older vector load, the other ring slots'
// B rows included.  The pair is picked with two-level selects on the bits
// of k (v_cndmask), not an indexed array, which would go through scratch.
// Banded: 0.495 -> 0.465 ms; the other workloads unchanged or slightly
// faster.
struct UnitRows {
  int4 lo, hi;
  __device__ __forceinline__ void load(const int* __restrict__ sidx, int64_t unit) {
    const int* q = sidx + unit * 8;
#if defined(__HIP_DEVICE_COMPILE__)
    typedef const __attribute__((address_space(4))) int cint;
    cint* p = (cint*)q;
#else
    const int* p = q;
#endif
    lo = int4{p[0], p[1], p[2], p[3]};
    hi = int4{p[4], p[5], p[6], p[7]};
  }
  __device__ __forceinline__ int2 pick(int k) const {
    const bool b0 = k & 1, b1 = k & 2;
    const int x0 = b0 ? lo.z : lo.x, x1 = b0 ? hi.z : hi.x;
    const int y0 = b0 ? lo.w : lo.y, y1 = b0 ? hi.w : hi.y;
    return int2{b1 ? x1 : x0, b1 ? y1 : y0};
  }
  template <int I>
  __device__ __forceinline__ int get() const {
    static_assert(I >= 0 && I < 8, "unit row index");
    if constexpr (I == 0) return lo.x;
    else if constexpr (I == 1) return lo.y;
    else if constexpr (I == 2) return lo.z;
    else if constexpr (I == 3) return lo.w;
    else if constexpr (I == 4) return hi.x;
    else if constexpr (I == 5) return hi.y;
    else if constexpr (I == 6) return hi.z;
    else return hi.w;
  }
};

// B staged through LDS (BSTAGE = 1).  Each wave owns DEPTH private LDS
// slots of 8 rows x WCOLS floats; a unit's 8 B-row segments are copied
// into its slot by direct-to-LDS loads (global_load_lds_dwordx4: each lane
// supplies a 16-byte global address, the wave's 64 x 16 bytes land
// contiguously at the slot offset), then read back with ds_read_b128 in
// the MFMA lane layout.  No data is shared between waves, so no barrier is
// needed; ordering is by the wave's own counters:
//  - the compiler does not order LDS reads after the direct-to-LDS loads
//    that write them, so before reading slot d the wave waits until at
//    most (DEPTH-1)*IPU vector-memory operations are outstanding: every
//    slot is refilled on every ring step (at the tail with the last unit
//    again), so exactly that many direct-to-LDS loads were issued after
//    slot d's, and vmcnt retires in order;
//  - a slot is refilled only after lgkmcnt(0), i.e. after its reads have
//    returned;
//  - the wave drains vmcnt before it exits, so no load writes the LDS of a
//    workgroup that has ended.
template <int WCOLS>
struct LdsB {
  static constexpr int LPR = WCOLS / 4;    // lanes per B-row segment (16 bytes each)
  static constexpr int RPI = 64 / LPR;     // rows per load instruction
  static constexpr int IPU = 8 / RPI;      // load instructions per unit
  static constexpr int SLOT = 8 * WCOLS;   // floats per slot
  static_assert(WCOLS == 64 || WCOLS == 128, "LDS staging covers 64- and 128-column waves");

  template <int M>
  __device__ __forceinline__ static int row_of(const UnitRows& r, int sub) {
    if constexpr (RPI == 2) {
      return sub ? r.template get<2 * M + 1>() : r.template get<2 * M>();
    } else {   // RPI == 4
      const int x = (sub & 1) ? r.template get<4 * M + 1>() : r.template get<4 * M>();
      const int y = (sub & 1) ? r.template get<4 * M + 3>() : r.template get<4 * M + 2>();
      return (sub & 2) ? y : x;
    }
  }
  template <int M>
  __device__ __forceinline__ static void issue_one(float* slot, const float* __restrict__ B, const UnitRows& r,
                                                   int64_t ldb, int wcol, int lane) {
    typedef __attribute__((address_space(3))) void lds_void;
    const int row = row_of<M>(r, lane / LPR);
    const float* g = B + (int64_t)row * ldb + wcol + 4 * (lane % LPR);
    __builtin_amdgcn_global_load_lds(g, (lds_void*)(slot + M * RPI * WCOLS), 16, 0, 0);
  }
  __device__ __forceinline__ static void issue(float* slot, const float* __restrict__ B, const UnitRows& r,
                                               int64_t ldb, int wcol, int lane) {
    issue_one<0>(slot, B, r, ldb, wcol, lane);
    issue_one<1>(slot, B, r, ldb, wcol, lane);
    if constexpr (IPU == 4) {
      issue_one<2>(slot, B, r, ldb, wcol, lane);
      issue_one<3>(slot, B, r, ldb, wcol, lane);
    }
  }
  // lane (k, j): k-step 0 reads row 2k, k-step 1 row 2k+1, columns 4j.. of each group
  template <int H, int G>
  __device__ __forceinline__ static void read(Frag<H, 4, G>& f, const float* slot, int lane) {
    const int k = lane >> 4, j = lane & 15;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      f.b0[g] = *reinterpret_cast<const f4*>(slot + (2 * k) * WCOLS + 64 * g + 4 * j);
      f.b1[g] = *reinterpret_cast<const f4*>(slot + (2 * k + 1) * WCOLS + 64 * g + 4 * j);
    }
  }
};

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their
// maxima).  The empty asm statements with a memory clobber keep the
// compiler from moving memory accesses across the wait.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ void wait_lgkmcnt0() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
  asm volatile("" ::: "memory");
}

template <int H, int VEC, int G>
__device__ __forceinline__ void mma_frag(const Frag<H, VEC, G>& f, f4 (&acc)[H][G][VEC]) {
#pragma unroll
  for (int h = 0; h < H; ++h)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int s = 0; s < VEC; ++s) {
#ifdef SRBCRS_EXPERIMENT_NO_MFMA
        acc[h][g][s].x += f.a[h].x * vget<VEC>(f.b0[g], s) + f.a[h].y * vget<VEC>(f.b1[g], s);
#else
        acc[h][g][s] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[h].x, vget<VEC>(f.b0[g], s), acc[h][g][s], 0, 0, 0);
        acc[h][g][s] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[h].y, vget<VEC>(f.b1[g], s), acc[h][g][s], 0, 0, 0);
#endif
      }
}

// An int at p[i] for a wave-uniform i, read through the constant address
// space so that the compiler emits a scalar load (counted on lgkmcnt).  Task
// metadata is read this way: as a vector load it would be counted on vmcnt
// with the B ring, and the wait for it at a task boundary would drain every
// B load in flight.
__device__ __forceinline__ int uniform_load(const int* __restrict__ p, int64_t i) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef const __attribute__((address_space(4))) int cint;
  return ((cint*)p)[i];
#else
  return p[i];
#endif
}

// The relu epilogue: negative values become +0; NaN, +0 and -0 pass
// unchanged (torch.relu's results).
__device__ __forceinline__ float relu1(float x) { return x < 0.f ? 0.f : x; }
__device__ __forceinline__ f4 relu4(f4 v) { return f4{relu1(v[0]), relu1(v[1]), relu1(v[2]), relu1(v[3])}; }

// Store a 16 x (16*VEC*G) accumulator tile.  row0 is the tile's first
// (packed) row, rows >= row_limit are skipped (M % 16 != 0).  With a row map
// packed row p is written to output row rowmap[p] (reordered or sparse-row
// packings); the map is applied here, in the store, not in a separate pass.
// relu (wave-uniform) applies the relu epilogue to the stored values.
template <int VEC, int G>
__device__ __forceinline__ void store_tile(const f4 (&acc)[G][VEC], float* __restrict__ out,
                                           int64_t row0, int64_t row_limit, int64_t ldc, int col0,
                                           int lane, const int* __restrict__ rowmap = nullptr,
                                           bool relu = false) {
  typedef typename VecT<VEC>::type V;
  const int k = lane >> 4;
  // The tile's 16 map entries are read with scalar loads (clamped to the
  // last row, so a partial tile stays in bounds) and each lane picks its
  // four: a per-lane vector load here would be counted on vmcnt with the
  // B ring, and its wait would drain every B load in flight at each flush.
  // (int4 members, not an array: selects between array elements become
  // indexed scratch loads)
  int4 m0{}, m1{}, m2{}, m3{};
  if (rowmap) {
    auto at = [&](int i) { return uniform_load(rowmap, row0 + i < row_limit ? row0 + i : row_limit - 1); };
    m0 = int4{at(0), at(1), at(2), at(3)};
    m1 = int4{at(4), at(5), at(6), at(7)};
    m2 = int4{at(8), at(9), at(10), at(11)};
    m3 = int4{at(12), at(13), at(14), at(15)};
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t row = row0 + 4 * k + r;
    if (row < row_limit) {
      int64_t orow = row;
      if (rowmap) {
        auto c = [r](const int4& v) { return r == 0 ? v.x : r == 1 ? v.y : r == 2 ? v.z : v.w; };
        const int lo = (k & 1) ? c(m1) : c(m0);
        const int hi = (k & 1) ? c(m3) : c(m2);
        orow = (k & 2) ? hi : lo;
      }
      float* p = out + orow * ldc + col0;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        V v;
        if constexpr (VEC == 1) {
          v = acc[g][0][r];
        } else {
#pragma unroll
          for (int s = 0; s < VEC; ++s) v[s] = acc[g][s][r];
        }
        if (relu) {
          if constexpr (VEC == 1) {
            v = relu1(v);
          } else {
#pragma unroll
            for (int s = 0; s < VEC; ++s) v[s] = relu1(v[s]);
          }
        }
#ifdef SRBCRS_EXPERIMENT_PLAIN_C_STORE
        *reinterpret_cast<V*>(p + 16 * VEC * g) = v;
#else
        __builtin_nontemporal_store(v, reinterpret_cast<V*>(p + 16 * VEC * g));
#endif
      }
    }
  }
}

// Task sources.  A task is a block range [begin, end) of one row window
// whose BH-row result goes straight into C (slot < 0) or into partial slot
// `slot` for the segment reduction.  A group is a run of consecutive tasks
// with contiguous block ranges, processed by one wave per column chunk.

// Row schedule: task t = row window t, groups of `wpw` consecutive windows.
struct RowTasks {
  const int* __restrict__ soff;
  int Mo;
  int wpw;
  const int* __restrict__ rowmap = nullptr;   // packed row -> output row (null = identity)
  int relu = 0;                               // relu epilogue on the output rows
  __device__ __forceinline__ void group(int g, int& t0, int& t1) const {
    t0 = g * wpw;
    t1 = t0 + wpw < Mo ? t0 + wpw : Mo;
  }
  __device__ __forceinline__ int64_t begin(int t) const { return uniform_load(soff, t); }
  __device__ __forceinline__ int64_t end(int t) const { return uniform_load(soff, t + 1); }
  __device__ __forceinline__ int window(int t) const { return t; }
  __device__ __forceinline__ int slot(int) const { return -1; }
};

// Table schedule (split / strict_lb / multi_bind) built on the host.
struct TableTasks {
  const int* __restrict__ group_off;
  const int* __restrict__ task_begin;
  const int* __restrict__ task_end;
  const int* __restrict__ task_window;
  const int* __restrict__ task_slot;
  const int* __restrict__ rowmap = nullptr;   // packed row -> output row (null = identity)
  int relu = 0;                               // relu epilogue on rows written to C (not on partials)
  __device__ __forceinline__ void group(int g, int& t0, int& t1) const {
    t0 = uniform_load(group_off, g);
    t1 = uniform_load(group_off, g + 1);
  }
  __device__ __forceinline__ int64_t begin(int t) const { return uniform_load(task_begin, t); }
  __device__ __forceinline__ int64_t end(int t) const { return uniform_load(task_end, t); }
  __device__ __forceinline__ int window(int t) const { return uniform_load(task_window, t); }
  __device__ __forceinline__ int slot(int t) const { return uniform_load(task_slot, t); }
};

template <class Src, int BH, int VEC, int G>
__device__ __forceinline__ void flush_task(const Src& src, int t, f4 (&acc)[BH / 16][G][VEC],
                                           float* __restrict__ C, float* __restrict__ partial,
                                           int M, int64_t ldc, int col0, int lane) {
  const int slot = src.slot(t);
#pragma unroll
  for (int h = 0; h < BH / 16; ++h) {
    if (slot < 0)
      store_tile<VEC, G>(acc[h], C, (int64_t)src.window(t) * BH + 16 * h, M, ldc, col0, lane, src.rowmap,
                         src.relu != 0);
    else
      store_tile<VEC, G>(acc[h], partial, (int64_t)slot * BH + 16 * h, (int64_t)(slot + 1) * BH, ldc,
                         col0, lane);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int s = 0; s < VEC; ++s) acc[h][g][s] = f4{0.f, 0.f, 0.f, 0.f};
  }
}

// One workgroup = WAVES waves on one (task group, column chunk); a column
// chunk is WAVES * 16*VEC*G columns.  The grid is 1-D over n_groups *
// n_chunks, in group-major order (all chunks of a group adjacent) or
// chunk-major order (one column chunk of every group first: the B rows a
// chunk touches are narrower, so neighbouring windows' shared rows stay in
// L2), or chunk-major in plain dispatch order (below).  Each wave streams the group's units through one DEPTH-deep register
// ring without draining it at task boundaries: the accumulator tile is
// flushed and cleared when the unit index crosses a task's end.  Every
// output element has exactly one writer per launch: no atomics.
//
// Occupancy is left to the compiler: forcing 4 waves/SIMD on the default
// instantiation (amdgpu_waves_per_eu, 98 registers instead of 146) made it
// slower on the GPU (GCN N=256 1.83 -> 2.02 ms), because the tighter budget
// delays the ring's loads.  With the compact A source (129 registers, 3
// waves) forcing 4 waves is slower too (uniform 0.259 -> 0.274 ms).
//
// BSTAGE 0 keeps the B ring in registers; BSTAGE 1 stages B through LDS
// (LdsB, VEC = 4 only): the ring then holds only the A fragments and the
// B-row indices in registers.  Both feed the MFMAs the same values.
template <class Src, int BH, int BW, int VEC, int G, int WAVES, int DEPTH, class AF, int BSTAGE = 0>
__global__ __launch_bounds__(64 * WAVES) void spmm_stream(
    Src src, const float* __restrict__ B, float* __restrict__ C, float* __restrict__ partial,
    const int* __restrict__ sidx, AF asrc, int M, int N, int64_t ldb,
    int64_t ldc, int n_chunks, int chunk_major) {
  typedef Shape<BH, BW> S;
  constexpr int WCOLS = 16 * VEC * G;
  const int64_t nwg = (int64_t)gridDim.x;
  // chunk_major 2: chunk-major in dispatch order (no XCD blocking), so every
  // XCD sweeps the same column chunk at the same time and the chunk's B rows
  // are shared through the memory-side cache instead of each XCD holding a
  // different chunk.
  const int64_t lid = chunk_major == 2 ? (int64_t)blockIdx.x : xcd_remap(blockIdx.x, nwg);
#ifdef SRBCRS_EXPERIMENT_LDS_PAD
  if constexpr (BSTAGE == 0) {
    // occupancy probe: unused LDS per workgroup caps the workgroups per CU
    __shared__ float lds_pad[SRBCRS_EXPERIMENT_LDS_PAD / 4];
    if (threadIdx.x == 0 && blockIdx.x == 0x7fffffff) lds_pad[0] = 0.f;
    __syncthreads();
    if (threadIdx.x == 0 && blockIdx.x == 0x7fffffff) C[0] = lds_pad[0];
  }
#endif
  const int64_t n_units = nwg / n_chunks;
  const int grp = (int)(chunk_major ? lid % n_units : lid / n_chunks);
  const int chunk = (int)(chunk_major ? lid / n_units : lid % n_chunks);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wcol = (chunk * WAVES + wave) * WCOLS;
  if (wcol >= N) return;
  const int col0 = wcol + VEC * (lane & 15);
  int t0, t1;
  src.group(grp, t0, t1);
  if (t0 >= t1) return;
  f4 acc[S::H][G][VEC];
#pragma unroll
  for (int h = 0; h < S::H; ++h)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int s = 0; s < VEC; ++s) acc[h][g][s] = f4{0.f, 0.f, 0.f, 0.f};
  const int64_t us = src.begin(t0) * S::Q, ue = src.end(t1 - 1) * S::Q;
  int t = t0;
  int64_t tend = src.end(t0) * S::Q;
  if (us < ue) {
    const int k = lane >> 4;
    const int i = lane & 15;
    int a_off[S::Q][S::H];
#pragma unroll
    for (int q = 0; q < S::Q; ++q)
#pragma unroll
      for (int h = 0; h < S::H; ++h) a_off[q][h] = swizzle_2_2_3(BW * (16 * h + i) + 8 * q + 2 * k);
    Frag<S::H, VEC, G> f[DEPTH];
    UnitRows idx[DEPTH];
    typename AF::template Meta<S::H> am[DEPTH];
    const int64_t last = ue - 1;
    if constexpr (BSTAGE == 1) {
      static_assert(VEC == 4, "LDS staging reads 16-byte B vectors");
      static_assert(DEPTH % 2 == 0, "the B register pair alternates with the ring position");
      typedef LdsB<WCOLS> L;
      __shared__ __attribute__((aligned(16))) float lds_ring[WAVES * DEPTH * L::SLOT];
      float* my_ring = lds_ring + wave * DEPTH * L::SLOT;
      // B of the unit being multiplied and of the next one, in registers:
      // the next unit's LDS reads run under the current unit's MFMAs.
      Frag<S::H, VEC, G> fb[2];
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int64_t u = us + d < last ? us + d : last;
        UnitRows r;
        r.load(sidx, u);
        asrc.template load<BH, BW>(f[d].a, u, asrc.template meta<BH, BW>(u, lane), a_off, lane);
        L::issue(my_ring + d * L::SLOT, B, r, ldb, wcol, lane);
        const int64_t nu = us + DEPTH + d < last ? us + DEPTH + d : last;
        idx[d].load(sidx, nu);
        am[d] = asrc.template meta<BH, BW>(nu, lane);
      }
      wait_vmcnt<(DEPTH - 1) * L::IPU>();   // slot 0 has landed
      __builtin_amdgcn_sched_barrier(0);
      L::template read<S::H, G>(fb[0], my_ring, lane);
      // Steady state: unit u = base + d sits in slot d.  Its B was read into
      // fb[d & 1] one step earlier; the wait below is for slot d + 1, with
      // the DEPTH - 2 younger slots' B loads allowed in flight (every slot is
      // refilled on every step, so that count is exact for the B loads; A
      // loads in between only make the wait longer, never too short).
      int64_t base = us;
      for (; base + DEPTH < ue; base += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
          const int64_t u = base + d;
          const int c = d & 1;
          wait_lgkmcnt0();                    // fb[c] (and the scalar indices) ready
          __builtin_amdgcn_sched_barrier(0);
          while (u >= tend) {
            flush_task<Src, BH, VEC, G>(src, t, acc, C, partial, M, ldc, col0, lane);
            ++t;
            tend = src.end(t) * S::Q;
          }
#pragma unroll
          for (int h = 0; h < S::H; ++h) fb[c].a[h] = f[d].a[h];
          mma_frag<S::H, VEC, G>(fb[c], acc);
          __builtin_amdgcn_sched_barrier(0);
          wait_vmcnt<(DEPTH - 2) * L::IPU>();   // slot d + 1 has landed
          __builtin_amdgcn_sched_barrier(0);
          L::template read<S::H, G>(fb[c ^ 1], my_ring + ((d + 1) % DEPTH) * L::SLOT, lane);
          __builtin_amdgcn_sched_barrier(0);
          // refill slot d (its B was read into fb[c] a step ago)
          const int64_t nu = u + DEPTH < last ? u + DEPTH : last;
          asrc.template load<BH, BW>(f[d].a, nu, am[d], a_off, lane);
          L::issue(my_ring + d * L::SLOT, B, idx[d], ldb, wcol, lane);
          const int64_t nn = nu + DEPTH < last ? nu + DEPTH : last;
          idx[d].load(sidx, nn);
          am[d] = asrc.template meta<BH, BW>(nn, lane);
        }
      }
      // Drain: the last round's units are in the ring; nothing more to load.
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int64_t u = base + d;
        const int c = d & 1;
        if (u < ue) {
          wait_lgkmcnt0();
          __builtin_amdgcn_sched_barrier(0);
          while (u >= tend) {
            flush_task<Src, BH, VEC, G>(src, t, acc, C, partial, M, ldc, col0, lane);
            ++t;
            tend = src.end(t) * S::Q;
          }
#pragma unroll
          for (int h = 0; h < S::H; ++h) fb[c].a[h] = f[d].a[h];
          mma_frag<S::H, VEC, G>(fb[c], acc);
          __builtin_amdgcn_sched_barrier(0);
          if (u + 1 < ue) {
            wait_vmcnt<0>();
            __builtin_amdgcn_sched_barrier(0);
            L::template read<S::H, G>(fb[c ^ 1], my_ring + ((d + 1) % DEPTH) * L::SLOT, lane);
          }
        }
      }
      wait_vmcnt<0>();
    } else {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int64_t u = us + d < last ? us + d : last;
      UnitRows r;
      r.load(sidx, u);
      load_frag<BH, BW, VEC, G>(f[d], B, asrc, u, r.pick(k), asrc.template meta<BH, BW>(u, lane), a_off, ldb,
                                col0, lane);
      const int64_t nu = us + DEPTH + d < last ? us + DEPTH + d : last;
      idx[d].load(sidx, nu);
      am[d] = asrc.template meta<BH, BW>(nu, lane);
    }
    // Steady state: while a unit lies beyond this round, every slot is
    // refilled after its MFMAs, unconditionally (a refill past the last unit
    // reloads the last unit: at most DEPTH - 1 duplicate loads per wave).
    // With the same loads on every path through the loop body the compiler
    // counts the younger loads exactly and waits only for the slot it is
    // about to use; conditional refills gave it paths with fewer loads and
    // made it wait for the whole ring (vmcnt(0)) once per round.
    int64_t base = us;
    for (; base + DEPTH < ue; base += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int64_t u = base + d;
        while (u >= tend) {   // crossed into the next task (empty tasks flush zeros)
          flush_task<Src, BH, VEC, G>(src, t, acc, C, partial, M, ldc, col0, lane);
          ++t;
          tend = src.end(t) * S::Q;
        }
        mma_frag<S::H, VEC, G>(f[d], acc);
        const int64_t nu = u + DEPTH < last ? u + DEPTH : last;
        load_frag<BH, BW, VEC, G>(f[d], B, asrc, nu, idx[d].pick(k), am[d], a_off, ldb, col0, lane);
        const int64_t nn = nu + DEPTH < last ? nu + DEPTH : last;
        idx[d].load(sidx, nn);
        am[d] = asrc.template meta<BH, BW>(nn, lane);
      }
    }
    // Drain: the last round's units are in the ring; nothing more to load.
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int64_t u = base + d;
      if (u < ue) {
        while (u >= tend) {
          flush_task<Src, BH, VEC, G>(src, t, acc, C, partial, M, ldc, col0, lane);
          ++t;
          tend = src.end(t) * S::Q;
        }
        mma_frag<S::H, VEC, G>(f[d], acc);
      }
    }
    }
  }
  for (; t < t1; ++t) flush_task<Src, BH, VEC, G>(src, t, acc, C, partial, M, ldc, col0, lane);
}

// out rows of window red_window[i] = sum over slots [red_slot_off[i],
// red_slot_off[i+1]) of the partial tiles (tile_rows x N each), in slot
// order (deterministic; zero slots give zeros).  The atomic-free
// counterpart of the reference's reduce_tcf_segments
// (examples/src_fp32/acc/testbed/custom_format_e2e.cu:832-853).  One thread
// per VEC consecutive columns.  M counts packed rows; rowmap (or null) maps
// them to output rows as in store_tile; relu applies the relu epilogue to
// the sums.
template <int VEC>
__global__ __launch_bounds__(256) void segment_reduce(const float* __restrict__ partial,
                                                      float* __restrict__ C,
                                                      const int* __restrict__ red_window,
                                                      const int* __restrict__ red_slot_off,
                                                      int n_red, int tile_rows, int M, int N,
                                                      int64_t ldc, const int* __restrict__ rowmap, int relu) {
  typedef typename VecT<VEC>::type V;
  const int64_t nv = N / VEC;
  const int64_t per = tile_rows * nv;
  const int64_t total = (int64_t)n_red * per;
  for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(id / per);
    const int64_t within = id % per;
    const int r = (int)(within / nv);
    const int64_t cv = within % nv;
    const int64_t row = (int64_t)red_window[i] * tile_rows + r;
    if (row >= M) continue;
    V s;
    if constexpr (VEC == 1) s = 0.f; else { for (int q = 0; q < VEC; ++q) s[q] = 0.f; }
    for (int sl = red_slot_off[i]; sl < red_slot_off[i + 1]; ++sl)
      s += *reinterpret_cast<const V*>(partial + ((int64_t)sl * tile_rows + r) * ldc + VEC * cv);
    if (relu) {
      if constexpr (VEC == 1) s = relu1(s); else { for (int q = 0; q < VEC; ++q) s[q] = relu1(s[q]); }
    }
    const int64_t orow = rowmap ? (int64_t)rowmap[row] : row;
    *reinterpret_cast<V*>(C + orow * ldc + VEC * cv) = s;
  }
}

// Zero the listed output rows (rows a sparse-row packing leaves out).  A
// template (T = float) so that every translation unit including this header
// may instantiate it.
template <class T>
__global__ __launch_bounds__(256) void zero_rows(T* __restrict__ C, const int* __restrict__ rows,
                                                 int n_rows, int N, int64_t ldc) {
  const int64_t total = (int64_t)n_rows * N;
  for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = id / N, c = id % N;
    C[(int64_t)rows[i] * ldc + c] = T(0);
  }
}

// CSR SpMM, one wave per (row, column chunk): lane owns VEC consecutive
// columns of a 64*VEC-column chunk.  Edge-ordered fp32 accumulation, the
// arithmetic of the reference's csr_spmm_value_kernel (examples/src_fp32/
// sr_bcrs/testbed/SRBCRSSpMM_kernel.cu:66-87), laid out for wave64 vector
// loads.  The grid is chunk-major (every row's first chunk before any second
// chunk), which keeps the B columns in flight narrow: 17-22 % faster than
// looping over the chunks inside the wave on the uniform and R-MAT
// workloads.  UNROLL B rows are loaded before their FMAs.
template <int VEC, int UNROLL>
__global__ __launch_bounds__(256) void csr_spmm_rowwave(
    const int* __restrict__ rowptr, const int* __restrict__ colind,
    const float* __restrict__ values, const float* __restrict__ B, float* __restrict__ C, int M,
    int N, int64_t ldb, int64_t ldc, int n_chunks) {
  typedef typename VecT<VEC>::type V;
  const int64_t nwg = (int64_t)gridDim.x;
  const int64_t lid = xcd_remap(blockIdx.x, nwg);
  const int64_t row_groups = nwg / n_chunks;
  const int chunk = (int)(lid / row_groups);
  const int64_t row = (lid % row_groups) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = chunk * 64 * VEC + VEC * lane;
  if (row >= M || c >= N) return;
  const int e0 = rowptr[row], e1 = rowptr[row + 1];
  V acc;
  if constexpr (VEC == 1) acc = 0.f; else { for (int s = 0; s < VEC; ++s) acc[s] = 0.f; }
  int e = e0;
  for (; e + UNROLL <= e1; e += UNROLL) {
    V bv[UNROLL];
    float av[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int col = colind[e + u];
      av[u] = values[e + u];
      bv[u] = *reinterpret_cast<const V*>(B + (int64_t)col * ldb + c);
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc += av[u] * bv[u];
  }
  for (; e < e1; ++e) {
    const int col = colind[e];
    acc += values[e] * *reinterpret_cast<const V*>(B + (int64_t)col * ldb + c);
  }
  *reinterpret_cast<V*>(C + row * ldc + c) = acc;
}

}  // namespace srbcrs
