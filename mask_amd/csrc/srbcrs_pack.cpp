// Row orders and the general SR-BCRS packer (host, multithreaded).
//
// Row orders (new row -> original row), the reorders of the reference's
// generated-operator bridge (examples/src_fp32/acc/testbed/
// custom_format_e2e.cu:157-349, sparse rows :483-488):
//   rcm       reverse Cuthill-McKee on the symmetrised structure
//   first_col rows by their first structural column
//   jaccard   minhash buckets of 64 rows, greedy nearest-Jaccard inside
//   sparse    the non-empty rows only (omitted rows are zero in C)
// Their tie-break rules fix the result uniquely and are kept as in the
// reference so that a plan's row order equals the reference's.
//
// Packing: BH-row windows over the reordered rows; per window either the
// sorted distinct columns cut into BW-column tiles (column-condensed,
// SR-BCRS) or the distinct BW-aligned column blocks (active fixed blocks,
// custom_format_e2e.cu:596-625, tile columns clamped to K-1).  Duplicate
// (row, column) entries keep the last value or are summed in edge order.
#include "srbcrs_pack.h"

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <limits>
#include <numeric>
#include <stdexcept>
#include <thread>
#include <vector>

namespace srbcrs {

namespace {

template <class F>
void for_chunks(int64_t n, int64_t chunk, F&& body) {
  unsigned hw = std::thread::hardware_concurrency();
  int64_t nt = hw ? std::min<unsigned>(hw, 64) : 1;
  if (n <= chunk || nt == 1) {
    body((int64_t)0, n);
    return;
  }
  std::atomic<int64_t> next{0};
  std::vector<std::thread> th;
  std::exception_ptr err;
  std::atomic<bool> failed{false};
  for (int64_t t = 0; t < nt; ++t)
    th.emplace_back([&] {
      try {
        for (;;) {
          const int64_t lo = next.fetch_add(chunk);
          if (lo >= n) break;
          body(lo, std::min(n, lo + chunk));
        }
      } catch (...) {
        bool f = false;
        if (failed.compare_exchange_strong(f, true)) err = std::current_exception();
      }
    });
  for (auto& t : th) t.join();
  if (err) std::rethrow_exception(err);
}

int first_structural(const int32_t* rowptr, const int32_t* colind, int32_t r, int32_t k) {
  int32_t f = k;
  for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e)
    if (colind[e] >= 0 && colind[e] < k && colind[e] < f) f = colind[e];
  return f;
}

uint64_t splitmix64(uint64_t v) {   // SplitMix64 finaliser (Steele, Lea, Flood 2014)
  v += 0x9e3779b97f4a7c15ULL;
  v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ULL;
  v = (v ^ (v >> 27)) * 0x94d049bb133111ebULL;
  return v ^ (v >> 31);
}

// Distinct-run merge of two rows' column lists in storage order.
double run_jaccard(const int32_t* rowptr, const int32_t* colind, int32_t a, int32_t b) {
  const int32_t* x = colind + rowptr[a];
  const int32_t* xe = colind + rowptr[a + 1];
  const int32_t* y = colind + rowptr[b];
  const int32_t* ye = colind + rowptr[b + 1];
  int64_t both = 0, na = 0, nb = 0;
  constexpr int32_t kEnd = std::numeric_limits<int32_t>::max();
  while (x < xe || y < ye) {
    const int32_t cx = x < xe ? *x : kEnd, cy = y < ye ? *y : kEnd;
    const int32_t c = std::min(cx, cy);
    if (cx == c) {
      ++na;
      while (x < xe && *x == c) ++x;
    }
    if (cy == c) {
      ++nb;
      while (y < ye && *y == c) ++y;
    }
    if (cx == c && cy == c) ++both;
  }
  const int64_t uni = na + nb - both;
  return uni ? (double)both / (double)uni : 1.0;
}

std::vector<int32_t> order_rcm(const int32_t* rowptr, const int32_t* colind, int32_t m, int32_t k) {
  if (m != k) throw std::invalid_argument("row_rcm currently requires a square matrix");
  // symmetrised adjacency (no self loops) by counting sort, then per-node unique
  std::vector<int64_t> cnt((size_t)m + 1, 0);
  for (int32_t r = 0; r < m; ++r)
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
      const int32_t c = colind[e];
      if (c < 0 || c >= m || c == r) continue;
      ++cnt[r + 1];
      ++cnt[c + 1];
    }
  for (int32_t r = 0; r < m; ++r) cnt[r + 1] += cnt[r];
  std::vector<int32_t> adj((size_t)cnt[m]);
  std::vector<int64_t> fill(cnt.begin(), cnt.end() - 1);
  for (int32_t r = 0; r < m; ++r)
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
      const int32_t c = colind[e];
      if (c < 0 || c >= m || c == r) continue;
      adj[fill[r]++] = c;
      adj[fill[c]++] = r;
    }
  std::vector<int32_t> deg((size_t)m);
  std::vector<int64_t> uend((size_t)m);
  for_chunks(m, 4096, [&](int64_t lo, int64_t hi) {
    for (int64_t r = lo; r < hi; ++r) {
      int32_t* b = adj.data() + cnt[r];
      int32_t* e = adj.data() + cnt[r + 1];
      std::sort(b, e);
      e = std::unique(b, e);
      uend[r] = e - adj.data();
      deg[r] = (int32_t)(e - b);
    }
  });
  auto by_deg = [&](int32_t a, int32_t b) { return deg[a] != deg[b] ? deg[a] < deg[b] : a < b; };
  std::vector<int32_t> starts((size_t)m);
  std::iota(starts.begin(), starts.end(), 0);
  std::sort(starts.begin(), starts.end(), by_deg);
  std::vector<uint8_t> seen((size_t)m, 0);
  std::vector<int32_t> out;
  out.reserve((size_t)m);
  std::vector<int32_t> cand;
  for (int32_t s : starts) {
    if (seen[s]) continue;
    const size_t comp0 = out.size();
    seen[s] = 1;
    out.push_back(s);   // `out` doubles as the BFS queue of this component
    for (size_t head = comp0; head < out.size(); ++head) {
      const int32_t v = out[head];
      cand.clear();
      for (int64_t p = cnt[v]; p < uend[v]; ++p)
        if (!seen[adj[p]]) cand.push_back(adj[p]);
      std::sort(cand.begin(), cand.end(), by_deg);
      for (int32_t w : cand) {
        seen[w] = 1;
        out.push_back(w);
      }
    }
    std::reverse(out.begin() + (int64_t)comp0, out.end());
  }
  return out;
}

std::vector<int32_t> order_first_col(const int32_t* rowptr, const int32_t* colind, int32_t m, int32_t k) {
  std::vector<int32_t> first((size_t)m);
  for_chunks(m, 65536, [&](int64_t lo, int64_t hi) {
    for (int64_t r = lo; r < hi; ++r) first[r] = first_structural(rowptr, colind, (int32_t)r, k);
  });
  std::vector<int32_t> order((size_t)m);
  std::iota(order.begin(), order.end(), 0);
  std::sort(order.begin(), order.end(),
            [&](int32_t a, int32_t b) { return first[a] != first[b] ? first[a] < first[b] : a < b; });
  return order;
}

std::vector<int32_t> order_jaccard(const int32_t* rowptr, const int32_t* colind, int32_t m, int32_t k) {
  constexpr int kBucket = 64;
  std::vector<uint64_t> sig((size_t)m);
  std::vector<int32_t> first((size_t)m);
  for_chunks(m, 16384, [&](int64_t lo, int64_t hi) {
    for (int64_t r = lo; r < hi; ++r) {
      uint64_t s = std::numeric_limits<uint64_t>::max();
      for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e)
        s = std::min(s, splitmix64((uint64_t)(uint32_t)colind[e]));
      sig[r] = s;
      first[r] = first_structural(rowptr, colind, (int32_t)r, k);
    }
  });
  std::vector<int32_t> ranked((size_t)m);
  std::iota(ranked.begin(), ranked.end(), 0);
  std::sort(ranked.begin(), ranked.end(), [&](int32_t a, int32_t b) {
    if (sig[a] != sig[b]) return sig[a] < sig[b];
    if (first[a] != first[b]) return first[a] < first[b];
    return a < b;
  });
  std::vector<int32_t> out((size_t)m);
  const int64_t nb = ((int64_t)m + kBucket - 1) / kBucket;
  for_chunks(nb, 64, [&](int64_t lo, int64_t hi) {
    std::vector<int32_t> rest;
    for (int64_t b = lo; b < hi; ++b) {
      const int64_t base = b * kBucket, end = std::min<int64_t>(base + kBucket, m);
      rest.assign(ranked.begin() + base + 1, ranked.begin() + end);
      int32_t cur = ranked[base];
      out[base] = cur;
      for (int64_t pos = base + 1; pos < end; ++pos) {
        size_t best = 0;
        double best_s = -1.0;
        for (size_t c = 0; c < rest.size(); ++c) {
          const double s = run_jaccard(rowptr, colind, cur, rest[c]);
          if (s > best_s || (s == best_s && rest[c] < rest[best])) {
            best_s = s;
            best = c;
          }
        }
        cur = rest[best];
        rest.erase(rest.begin() + (int64_t)best);
        out[pos] = cur;
      }
    }
  });
  return out;
}

}  // namespace

std::vector<int32_t> row_order(const int32_t* rowptr, const int32_t* colind, int32_t m, int32_t k,
                               int method) {
  switch (method) {
    case kOrderIdentity: {
      std::vector<int32_t> o((size_t)m);
      std::iota(o.begin(), o.end(), 0);
      return o;
    }
    case kOrderRcm: return order_rcm(rowptr, colind, m, k);
    case kOrderFirstCol: return order_first_col(rowptr, colind, m, k);
    case kOrderJaccard: return order_jaccard(rowptr, colind, m, k);
    case kOrderSparseRows: {
      std::vector<int32_t> o;
      for (int32_t r = 0; r < m; ++r)
        if (rowptr[r] != rowptr[r + 1]) o.push_back(r);
      return o;
    }
    default: throw std::invalid_argument("unknown row order method");
  }
}

namespace {

struct Entry {
  int64_t key;     // column (condensed) or column block (fixed blocks)
  int32_t lrow;    // row inside the window
  int32_t edge;
};

void window_entries(const int32_t* rowptr, const int32_t* colind, const PackSpec& s, int64_t w,
                    std::vector<Entry>& ent) {
  ent.clear();
  const int64_t r0 = w * s.blk_h, r1 = std::min<int64_t>(r0 + s.blk_h, s.rows);
  for (int64_t nr = r0; nr < r1; ++nr) {
    const int32_t orow = s.order ? s.order[nr] : (int32_t)nr;
    for (int64_t e = rowptr[orow]; e < rowptr[orow + 1]; ++e) {
      const int32_t c = colind[e];
      if (c < 0 || (s.K >= 0 && c >= s.K)) throw std::out_of_range("CSR column index out of range");
      ent.push_back(Entry{s.packing == kPackFixedBlocks ? (int64_t)(c / s.blk_w) : (int64_t)c,
                          (int32_t)(nr - r0), (int32_t)e});
    }
  }
  std::sort(ent.begin(), ent.end(), [](const Entry& a, const Entry& b) {
    if (a.key != b.key) return a.key < b.key;
    if (a.lrow != b.lrow) return a.lrow < b.lrow;
    return a.edge < b.edge;
  });
}

int64_t distinct_keys(const std::vector<Entry>& ent) {
  int64_t n = 0;
  for (size_t i = 0; i < ent.size(); ++i)
    if (i == 0 || ent[i].key != ent[i - 1].key) ++n;
  return n;
}

inline int swizzle_2_2_3(int o) { return o ^ ((o & 0x60) >> 3); }

}  // namespace

int64_t pack_count(const int32_t* rowptr, const int32_t* colind, const PackSpec& s, int32_t* soff) {
  const int64_t W = (s.rows + s.blk_h - 1) / s.blk_h;
  std::vector<int64_t> tiles((size_t)W, 0);
  for_chunks(W, 1024, [&](int64_t lo, int64_t hi) {
    std::vector<Entry> ent;
    for (int64_t w = lo; w < hi; ++w) {
      window_entries(rowptr, colind, s, w, ent);
      const int64_t nk = distinct_keys(ent);
      tiles[w] = s.packing == kPackFixedBlocks ? nk : (nk + s.blk_w - 1) / s.blk_w;
    }
  });
  int64_t total = 0;
  for (int64_t w = 0; w < W; ++w) {
    if (total > std::numeric_limits<int32_t>::max()) throw std::overflow_error("tile count exceeds int32 offsets");
    soff[w] = (int32_t)total;
    total += tiles[w];
  }
  if (total > std::numeric_limits<int32_t>::max()) throw std::overflow_error("tile count exceeds int32 offsets");
  soff[W] = (int32_t)total;
  return total;
}

void pack_fill(const int32_t* rowptr, const int32_t* colind, const float* values, const PackSpec& s,
               const int32_t* soff, int32_t* sidx, float* val) {
  const int64_t W = (s.rows + s.blk_h - 1) / s.blk_h;
  const int64_t bsz = (int64_t)s.blk_h * s.blk_w;
  for_chunks(W, 1024, [&](int64_t lo, int64_t hi) {
    std::vector<Entry> ent;
    for (int64_t w = lo; w < hi; ++w) {
      window_entries(rowptr, colind, s, w, ent);
      int32_t* sw = sidx + (int64_t)soff[w] * s.blk_w;
      float* vw = val + (int64_t)soff[w] * bsz;
      const int64_t ntile = soff[w + 1] - soff[w];
      std::fill(vw, vw + ntile * bsz, 0.0f);
      int64_t kidx = -1;
      for (size_t i = 0; i < ent.size(); ++i) {
        const Entry& x = ent[i];
        const bool new_key = i == 0 || x.key != ent[i - 1].key;
        if (new_key) {
          ++kidx;
          if (s.packing == kPackFixedBlocks) {
            for (int c = 0; c < s.blk_w; ++c) {
              const int64_t col = x.key * s.blk_w + c;
              sw[kidx * s.blk_w + c] = (int32_t)(s.K > 0 ? std::min<int64_t>(col, s.K - 1) : col);
            }
          } else {
            sw[kidx] = (int32_t)x.key;
          }
        }
        const int64_t tile = s.packing == kPackFixedBlocks ? kidx : kidx / s.blk_w;
        const int lcol = s.packing == kPackFixedBlocks ? colind[x.edge] % s.blk_w : (int)(kidx % s.blk_w);
        float& dst = vw[tile * bsz + swizzle_2_2_3(x.lrow * s.blk_w + lcol)];
        if (s.dup_sum)
          dst += values[x.edge];
        else
          dst = values[x.edge];   // entries are in edge order: the last write wins
      }
      if (s.packing != kPackFixedBlocks) {
        const int64_t nk = kidx + 1;
        for (int64_t i = nk; i < ntile * s.blk_w; ++i) sw[i] = sw[nk - 1];
      }
    }
  });
}

}  // namespace srbcrs
