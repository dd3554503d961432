// Device-side CSR -> SR-BCRS conversion (see srbcrs_convert.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace srbcrs {

struct DeviceConvertIn {
  const int* rowptr;       // device, num_nodes + 1
  const int* colind;       // device, nnz
  const float* values;     // device, nnz
  int num_nodes;
  int64_t nnz;
  int blk_h, blk_w;
  int* edge_to_row;        // device, nnz (required; caller zero-fills it)
  int* edge_to_col;        // device, nnz or null (caller zero-fills it)
  int* block_partition;    // device, Mo or null
};

struct DeviceConvertOut {
  int* soff;               // device, Mo + 1, allocated by the caller
  int* sidx = nullptr;     // allocated through the callback
  float* val = nullptr;    // allocated through the callback
  int Mo = 0;
  int64_t total = 0;
  int max_col = -1;
  int bad = 0;             // 1: malformed rowptr, 2: negative column (nothing else produced)
};

typedef void* (*DeviceAlloc)(void* ctx, size_t bytes);
typedef void (*DeviceFree)(void* ctx, void* p);

hipError_t device_convert(const DeviceConvertIn& in, DeviceConvertOut& out, DeviceAlloc alloc,
                          DeviceFree dfree, void* ctx, hipStream_t st);

// Compact copy of the block values (srbcrs_compact.hip): per 32 logical
// positions of a block one {mask, base} word, and the stored values.
// Zero floats allocated after the stored values (CompactA reads packed[n]
// and packed[n + 1] for n <= n_packed without a branch).
constexpr int64_t kPackedPad = 16;

struct CompactOut {
  uint2* words = nullptr;   // n_blocks * BH*BW/32
  float* packed = nullptr;  // n_packed stored values, then kPackedPad zeros
  int64_t n_packed = 0;
};

hipError_t device_compact(const float* val, int64_t n_blocks, int blk_h, int blk_w, DeviceAlloc alloc,
                          DeviceFree dfree, void* ctx, hipStream_t st, CompactOut& out);

}  // namespace srbcrs
