// Row orders and the general SR-BCRS packer (host).  See srbcrs_pack.cpp.
#pragma once
#include <cstdint>
#include <vector>

namespace srbcrs {

enum RowOrder { kOrderIdentity = 0, kOrderRcm = 1, kOrderFirstCol = 2, kOrderJaccard = 3, kOrderSparseRows = 4 };
enum Packing { kPackCondensed = 0, kPackFixedBlocks = 1 };

struct PackSpec {
  int blk_h = 16, blk_w = 8;
  int packing = kPackCondensed;
  bool dup_sum = false;            // false: last write wins; true: summed in edge order
  const int32_t* order = nullptr;  // new row -> original row (nullptr = identity)
  int64_t rows = 0;                // packed rows (length of order, or num_nodes)
  int32_t K = -1;                  // column bound (< 0 = unchecked; required for fixed blocks)
};

std::vector<int32_t> row_order(const int32_t* rowptr, const int32_t* colind, int32_t m, int32_t k,
                               int method);
int64_t pack_count(const int32_t* rowptr, const int32_t* colind, const PackSpec& s, int32_t* soff);
void pack_fill(const int32_t* rowptr, const int32_t* colind, const float* values, const PackSpec& s,
               const int32_t* soff, int32_t* sidx, float* val);

}  // namespace srbcrs
