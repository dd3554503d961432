// Compact copy of the SR-BCRS block values (the A operand the SpMM kernel
// reads by default).
//
// The reference's block-value array stores every block densely (BH*BW fp32,
// swizzled), so at low block fill most of its bytes are zeros, and the SpMM
// re-reads it once per column chunk.  The compact copy keeps, for every 32
// consecutive logical positions o = BW*r + c of a block (unswizzled,
// row-major), one word {mask, base}: bit t of mask is set when position
// 32*w + t holds a value whose bits are not all zero, and base is the index
// in `packed` of the first such value; `packed` lists those values in
// logical order.  Zeros (+0.0f) are rebuilt in registers, any other bit
// pattern (-0.0f included) is stored, so the kernel's MFMA fragments are
// bit-identical to the ones read from the dense array.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>
#include <stdint.h>

#include "srbcrs_convert.h"

namespace srbcrs {

namespace {

__device__ __forceinline__ int swz(int o) { return o ^ ((o & 0x60) >> 3); }

int grid_for(int64_t n) {
  const int64_t g = (n + 255) / 256;
  return (int)(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

// One thread per logical block position.  The swizzle only permutes offset
// bits 2..3, so the 32 positions of a word lie in one 128-byte span of val
// and a wave's reads coalesce; a wave ballot gives the masks of its two
// words.  Grid-stride steps are multiples of 64 positions, so every wave
// stays whole for the ballot (the position count is a multiple of 64).
__global__ void k_word_masks(const float* __restrict__ val, int64_t n_pos, int block_size,
                             uint2* __restrict__ words, uint32_t* __restrict__ counts) {
  const int lane = threadIdx.x & 63;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < n_pos;
       g += (int64_t)gridDim.x * blockDim.x) {
    const int64_t blk = g / block_size;
    const int p = (int)(g % block_size);
    const bool stored = __float_as_uint(val[blk * block_size + swz(p)]) != 0u;
    const uint64_t bal = __ballot(stored);
    if ((lane & 31) == 0) {
      const uint32_t m = (uint32_t)(bal >> (lane & 32));
      const int64_t w = g >> 5;
      words[w] = make_uint2(m, 0u);
      counts[w] = (uint32_t)__builtin_popcount(m);
    }
  }
}

// One thread per logical block position: the word's base offset and the
// packed value of every stored position.
__global__ void k_word_fill(const float* __restrict__ val, int64_t n_pos, int block_size,
                            const uint32_t* __restrict__ bases, uint2* __restrict__ words,
                            float* __restrict__ packed) {
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < n_pos;
       g += (int64_t)gridDim.x * blockDim.x) {
    const int64_t w = g >> 5;
    const int t = (int)(g & 31);
    uint32_t* wd = reinterpret_cast<uint32_t*>(words);   // [2w] = mask (read), [2w+1] = base (written)
    const uint32_t m = wd[2 * w], base = bases[w];
    if ((m >> t) & 1u) {
      const int64_t blk = g / block_size;
      packed[base + __builtin_popcount(m & ((1u << t) - 1u))] = val[blk * block_size + swz((int)(g % block_size))];
    }
    if (t == 0) wd[2 * w + 1] = base;
  }
}

}  // namespace

hipError_t device_compact(const float* val, int64_t n_blocks, int blk_h, int blk_w, DeviceAlloc alloc,
                          DeviceFree dfree, void* ctx, hipStream_t st, CompactOut& out) {
  out = CompactOut{};
  const int block_size = blk_h * blk_w;
  const int wpb = block_size / 32;
  const int64_t n_words = n_blocks * wpb;
  if (n_words <= 0) return hipSuccess;
  if (n_words >= INT32_MAX) return hipErrorInvalidValue;   // hipCUB scans take int item counts
  uint32_t* counts = nullptr;
  uint32_t* bases = nullptr;
  void* tmp = nullptr;
  uint32_t* tail = nullptr;
  auto cleanup = [&] {
    if (counts) dfree(ctx, counts);
    if (bases) dfree(ctx, bases);
    if (tmp) dfree(ctx, tmp);
    if (tail) dfree(ctx, tail);
  };
  auto fail = [&](hipError_t e) {
    cleanup();
    if (out.words) dfree(ctx, out.words);
    if (out.packed) dfree(ctx, out.packed);
    out = CompactOut{};
    return e;
  };
#define SRBCRS_STEP(x)                       \
  do {                                       \
    const hipError_t e_ = (x);               \
    if (e_ != hipSuccess) return fail(e_);   \
  } while (0)
  out.words = (uint2*)alloc(ctx, (size_t)n_words * sizeof(uint2));
  counts = (uint32_t*)alloc(ctx, (size_t)n_words * 4);
  bases = (uint32_t*)alloc(ctx, (size_t)n_words * 4);
  tail = (uint32_t*)alloc(ctx, 8);
  if (!out.words || !counts || !bases || !tail) return fail(hipErrorOutOfMemory);
  const int64_t n_pos = n_words * 32;
  hipLaunchKernelGGL(k_word_masks, dim3(grid_for(n_pos)), dim3(256), 0, st, val, n_pos, block_size, out.words,
                     counts);
  SRBCRS_STEP(hipGetLastError());
  size_t bytes = 0;
  SRBCRS_STEP(hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, counts, bases, (int)n_words, st));
  tmp = alloc(ctx, bytes ? bytes : 1);
  if (!tmp) return fail(hipErrorOutOfMemory);
  SRBCRS_STEP(hipcub::DeviceScan::ExclusiveSum(tmp, bytes, counts, bases, (int)n_words, st));
  SRBCRS_STEP(hipMemcpyAsync(tail, bases + n_words - 1, 4, hipMemcpyDeviceToDevice, st));
  SRBCRS_STEP(hipMemcpyAsync(tail + 1, counts + n_words - 1, 4, hipMemcpyDeviceToDevice, st));
  uint32_t h_tail[2] = {0, 0};
  SRBCRS_STEP(hipMemcpyAsync(h_tail, tail, 8, hipMemcpyDeviceToHost, st));
  SRBCRS_STEP(hipStreamSynchronize(st));
  out.n_packed = (int64_t)h_tail[0] + h_tail[1];
  // kPackedPad zero floats after the stored values: the SpMM reads packed[n]
  // and packed[n + 1] unconditionally (n <= n_packed) and selects, so that
  // its loads do not sit in lane-divergent branches
  out.packed = (float*)alloc(ctx, (size_t)(out.n_packed + kPackedPad) * 4);
  if (!out.packed) return fail(hipErrorOutOfMemory);
  SRBCRS_STEP(hipMemsetAsync(out.packed + out.n_packed, 0, kPackedPad * 4, st));
  hipLaunchKernelGGL(k_word_fill, dim3(grid_for(n_pos)), dim3(256), 0, st, val, n_pos, block_size, bases,
                     out.words, out.packed);
  SRBCRS_STEP(hipGetLastError());
  SRBCRS_STEP(hipStreamSynchronize(st));
#undef SRBCRS_STEP
  cleanup();
  return hipSuccess;
}

}  // namespace srbcrs
