// Nonzero sweep: the vector kernel for low block density.  One wave walks
// the stored values of W consecutive row windows in the merged-window order
// (one B-row gather per value, no padded block arithmetic) and accumulates
// into an LDS tile of 16*W rows x 64 columns.
//
// Why.  At a few values per 16x8 block (6 % fill on uniform-65536) the
// MFMA kernels spend 16x the useful arithmetic: the padded MFMA work alone
// takes about as long as the B gathers, and the two overlap only in part.
// Here the work per value is one 256-byte gather and a 256-byte LDS
// read-add-write, so the gathers, in the merged-window sweep order that
// lets an XCD's waves reuse each other's B rows from the L2, share the
// time with the LDS traffic only.  This is the "CSR scalar/vector fallback"
// of the reference (SRBCRSSpMM_kernel.cu:66-105, csr_spmm_value_kernel),
// fed from the SR-BCRS plan instead of a CSR copy.
//
// Stream (built on the host per plan and setting, srbcrs_capi.cpp): group
// g's entries [eoff[g], eoff[g+1]), each an (entry, value) pair, entry =
// (tile row << 24) | B row, tile row = 16 * (window - g*W) + row in the
// window.  Within a group the values follow the merged unit order (block r
// of every window, in window order, then block r + 1), within a block
// column by column, cut into sub-batches of distinct tile rows; padding
// entries point at tile row 16*W, an LDS row that is never stored.
//
// Arithmetic.  C[row, col] is the sum of fl(value * B[col', col]) over the
// row's stored values in ascending column order (a window's columns ascend
// through its blocks and a row's values keep their order in the stream),
// each product rounded, then added to the running sum in fp32 (the
// multiply and the add are not fused).  That is the fp32 CSR SpMM of the
// CPU oracle, bit for bit, on rows whose values are distinct (row, column)
// pairs; it differs from the MFMA kernels' bits.  One wave owns its LDS
// tile and its adds apply in program order, so two runs are bit-identical.
#pragma once
#include "srbcrs_merged.hpp"

namespace srbcrs {

constexpr int kNzRowShift = 24;   // entry = (tile row << 24) | B row: 16*W + 1 <= 256, B rows < 2^24

// Each step's loads are pinned ahead of its adds (sched_barrier): left to
// itself the compiler hoisted the multiplies above the next sub-batch's
// gathers, and every step then waited for all its loads before issuing any.
#ifdef SRBCRS_NZ_NO_PIN
#define SRBCRS_NZ_PIN (void)0
#else
#define SRBCRS_NZ_PIN __builtin_amdgcn_sched_barrier(0)
#endif

// Lane l of a wave64 broadcast to the 16 lanes of its row (DPP
// row_newbcast), l = 16 * row + q.  Every lane of a row reads a valid
// source lane, so no old value is needed (mov_dpp, bound_ctrl).
#define SRBCRS_ROW_BCAST(q) return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x150 + (q), 0xf, 0xf, true)
__device__ __forceinline__ uint32_t row_bcast(uint32_t v, int q) {
  const int x = (int)v;
  switch (q) {
    case 0: SRBCRS_ROW_BCAST(0);
    case 1: SRBCRS_ROW_BCAST(1);
    case 2: SRBCRS_ROW_BCAST(2);
    case 3: SRBCRS_ROW_BCAST(3);
    case 4: SRBCRS_ROW_BCAST(4);
    case 5: SRBCRS_ROW_BCAST(5);
    case 6: SRBCRS_ROW_BCAST(6);
    case 7: SRBCRS_ROW_BCAST(7);
    case 8: SRBCRS_ROW_BCAST(8);
    case 9: SRBCRS_ROW_BCAST(9);
    case 10: SRBCRS_ROW_BCAST(10);
    case 11: SRBCRS_ROW_BCAST(11);
    case 12: SRBCRS_ROW_BCAST(12);
    case 13: SRBCRS_ROW_BCAST(13);
    case 14: SRBCRS_ROW_BCAST(14);
    default: SRBCRS_ROW_BCAST(15);
  }
}
#undef SRBCRS_ROW_BCAST

// 64 columns per wave, W windows per group, sub-batches of U entries.  One
// gather instruction serves 4 entries: lane (g, i) = (lane / 16, lane % 16)
// takes entry 4q + g of instruction q and loads columns 4i..4i+3 of its B
// row (16 bytes; 4 rows x 256 bytes in one buffer_load_dwordx4).  A
// sub-batch's (entry, value) pairs are stored transposed, pair g * Q + q
// holding entry 4q + g (Q = U / 4 instructions): lane (g, i) loads pair
// g * Q + i % Q (one 8-byte load per lane per sub-batch) and instruction q
// takes lane q of each row by DPP broadcast.
//
// Pipeline, at step s: the pairs of sub-batch s + D are loaded, the gathers
// of sub-batch s + D - 1 issued, and sub-batch s added into the tile.  Pairs
// live in a ring of 2D slots, gathered rows in a ring of D; the loop body
// covers 2D steps so that every slot index is a constant.  Group streams are
// padded to whole loop bodies, and sub-batches past a group's end repeat its
// last (their loads are never added), so every step issues the same loads
// and the compiler's vmcnt waits count them exactly.  B + col0 is addressed
// through a buffer resource with 32-bit offsets: K * ldb * 4 < 2^32, and B
// rows and ldb * 4 below 2^24 (24-bit multiplies).  Per gather instruction
// the lane needs two addresses from its entry: the B offset, one 24-bit
// multiply-add of the entry's low 24 bits, and the LDS byte offset (tile row
// << 8) | (16 * i), one byte permute of the entry's high byte.
template <int W, int U, int D>
__global__ __launch_bounds__(64) void spmm_nzsweep(const int* __restrict__ eoff, const uint2* __restrict__ pairs,
                                                   const float* __restrict__ B, float* __restrict__ C,
                                                   const int* __restrict__ rowmap, int M, int N, int64_t ldb,
                                                   int64_t ldc, int n_chunks, int64_t n_groups, int relu) {
  constexpr int ROWS = 16 * W;
  constexpr int Q = U / 4;   // gather instructions per sub-batch
  constexpr int P = 2 * D;   // steps per loop body
  static_assert(ROWS + 1 <= (1 << (32 - kNzRowShift)), "tile rows fit the entry's row byte");
  static_assert(U % 4 == 0 && Q <= 16 && D >= 2, "a sub-batch's pairs fit one load per lane");
  __shared__ __attribute__((aligned(16))) float tile[(ROWS + 1) * 64];
  int64_t g;
  int c;
  if (!xcd_chunk(blockIdx.x, n_chunks, n_groups, g, c)) return;
  const int col0 = c * 64;
  if (col0 >= N) return;
  const int lane = threadIdx.x;
  const int grp = lane >> 4, sub = lane & 15;
  f4* tile4 = reinterpret_cast<f4*>(tile);
  constexpr int T4 = (ROWS + 1) * 16;   // f4 slots of the tile
#pragma unroll
  for (int i = 0; i < (T4 + 63) / 64; ++i)
    if (i * 64 + lane < T4) tile4[i * 64 + lane] = f4{0.f, 0.f, 0.f, 0.f};
  const int64_t e0 = uniform_load(eoff, g), e1 = uniform_load(eoff, g + 1);
  if (e0 < e1) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(B + col0), 0, (int)0xffffffffu, 0x00020000);   // 4 GiB
    const uint32_t ldb4 = (uint32_t)(ldb * 4);
    const uint32_t boff = (uint32_t)sub * 16u;
    const int64_t n_sb = (e1 - e0) / U;
    const uint2* gp = pairs + e0 + grp * Q + (sub % Q);
    char* tileb = reinterpret_cast<char*>(tile);
    uint2 m[P];
    f4 b[D][Q];
    uint32_t la[D][Q];   // LDS byte offsets of the gathered rows' tile rows
    // (nontemporal pair loads ran 35 % slower: 0.181 against 0.134 ms)
    auto fetch = [&](int ms, int64_t j) { m[ms] = gp[(j < n_sb ? j : n_sb - 1) * U]; };
    auto issue = [&](int bs, int ms) {
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const uint32_t w = row_bcast(m[ms].x, q);
        // byte 0 = 16 i, byte 1 = the entry's top byte (the tile row)
        la[bs][q] = __builtin_amdgcn_perm(w, boff, 0x0c0c0700u);
#ifdef SRBCRS_EXPERIMENT_NZ_NO_B
        b[bs][q] = f4{__builtin_bit_cast(float, w), 1.f, 2.f, 3.f};
#else
        b[bs][q] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rs, __umul24(w, ldb4) + boff, 0, 0));   // the low 24 bits: the B row
#endif
      }
    };
    // tile rows of one sub-batch are distinct (the dummy row aside), so its
    // read-add-writes are independent: all reads, then all writes.  A
    // sub-batch's reads are issued right after the previous sub-batch's
    // writes (the wave's LDS operations execute in order, so they see them)
    // and complete while the step issues its loads and waits for its
    // gathers.  (LDS float atomics, ds_add_f32, ran the same work about ten
    // times slower.)
    f4 o[Q];
#ifdef SRBCRS_EXPERIMENT_NZ_NO_LDS
    f4 racc = f4{0.f, 0.f, 0.f, 0.f};
    auto read = [&](int) {};
    auto add = [&](int bs, int ms) {
#pragma unroll
      for (int q = 0; q < Q; ++q) racc += __builtin_bit_cast(float, row_bcast(m[ms].y, q)) * b[bs][q];
    };
#else
    auto read = [&](int bs) {
#pragma unroll
      for (int q = 0; q < Q; ++q) o[q] = *reinterpret_cast<const f4*>(tileb + la[bs][q]);
    };
    auto add = [&](int bs, int ms) {
#pragma clang fp contract(off)
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const f4 p = __builtin_bit_cast(float, row_bcast(m[ms].y, q)) * b[bs][q];
        *reinterpret_cast<f4*>(tileb + la[bs][q]) = o[q] + p;
      }
    };
#endif
    // the prologue in steady-state order (pairs, then gathers), pinned: the
    // loop's first wait then counts the same loads on both incoming paths
#pragma unroll
    for (int j = 0; j < D; ++j) fetch(j, j);
    SRBCRS_NZ_PIN;
#pragma unroll
    for (int j = 0; j + 1 < D; ++j) issue(j, j);
    SRBCRS_NZ_PIN;
    read(0);
    for (int64_t base = 0; base < n_sb; base += P) {
#pragma unroll
      for (int k = 0; k < P; ++k) {
        fetch((k + D) % P, base + k + D);
        issue((k + D - 1) % D, (k + D - 1) % P);
        SRBCRS_NZ_PIN;
        add(k % D, k % P);
        read((k + 1) % D);
        SRBCRS_NZ_PIN;
      }
    }
#ifdef SRBCRS_EXPERIMENT_NZ_NO_LDS
    tile4[lane] = racc;
#endif
  }
  // the wave's own LDS writes are complete before its reads (LDS operations
  // of one wave execute in order)
  const int64_t row0 = g * ROWS;
#pragma unroll 4
  for (int r = grp; r < ROWS; r += 4) {
    const int64_t row = row0 + r;
    if (row < M) {
      const int64_t orow = rowmap ? rowmap[row] : row;
      const f4 v = relu ? relu4(tile4[r * 16 + sub]) : tile4[r * 16 + sub];
#ifdef SRBCRS_NZ_PLAIN_C_STORE
      *reinterpret_cast<f4*>(C + orow * ldc + col0 + 4 * sub) = v;
#else
      // C is written once: nontemporal, so that it does not push B's rows out of the L2
      __builtin_nontemporal_store(v, reinterpret_cast<f4*>(C + orow * ldc + col0 + 4 * sub));
#endif
    }
  }
}

}  // namespace srbcrs
