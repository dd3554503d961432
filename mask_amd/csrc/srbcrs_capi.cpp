// C ABI of the SR-BCRS backend: host conversion, schedules, plans, launch.
// Declarations and the reference interfaces they replace: include/srbcrs.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <exception>
#include <new>
#include <string>
#include <thread>
#include <map>
#include <mutex>
#include <vector>

#include "../../include/srbcrs.h"
#include "srbcrs_kernels.h"
#include "srbcrs_convert.h"
#include "srbcrs_pack.h"
#include "srbcrs_probe.h"

namespace {

thread_local std::string g_last_error;

struct Error {
  int code;
  std::string msg;
};

[[noreturn]] void fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw Error{code, buf};
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(SRBCRS_EHIP, "%s: %s", what, hipGetErrorString(e));
}

template <class F>
int guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return SRBCRS_OK;
  } catch (const Error& e) {
    g_last_error = e.msg;
    return e.code;
  } catch (const std::bad_alloc&) {
    g_last_error = "host allocation failed";
    return SRBCRS_ENOMEM;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return SRBCRS_EINVAL;
  }
}

// Run body(lo, hi) over [0, n) on up to hardware_concurrency threads.
template <class F>
void parallel_for(int64_t n, F&& body) {
  unsigned hw = std::thread::hardware_concurrency();
  int64_t nt = hw ? hw : 1;
  if (nt > 64) nt = 64;
  if (n < 4096 || nt == 1) {
    body((int64_t)0, n);
    return;
  }
  // dynamic chunks so skewed windows (power-law rows) balance
  const int64_t chunk = std::max<int64_t>(256, n / (nt * 16));
  std::atomic<int64_t> next{0};
  std::vector<std::thread> th;
  std::exception_ptr err;
  std::atomic<bool> has_err{false};
  for (int64_t t = 0; t < nt; ++t) {
    th.emplace_back([&] {
      try {
        for (;;) {
          int64_t lo = next.fetch_add(chunk);
          if (lo >= n) break;
          body(lo, std::min(n, lo + chunk));
        }
      } catch (...) {
        bool expected = false;
        if (has_err.compare_exchange_strong(expected, true)) err = std::current_exception();
      }
    });
  }
  for (auto& t : th) t.join();
  if (err) std::rethrow_exception(err);
}

inline int swizzle_2_2_3(int o) { return o ^ ((o & 0x60) >> 3); }

void check_block_shape(int blk_h, int blk_w) {
  if (!((blk_h == 16 && blk_w == 8) || (blk_h == 32 && blk_w == 32)))
    fail(SRBCRS_EINVAL, "unsupported SR-BCRS block %dx%d: expected 16x8 or 32x32", blk_h, blk_w);
}

void check_csr(const int32_t* rowptr, const int32_t* colind, int32_t num_nodes, int64_t nnz) {
  if (num_nodes < 1) fail(SRBCRS_EINVAL, "num_nodes must be positive");
  if (nnz < 0 || nnz > INT32_MAX) fail(SRBCRS_EINVAL, "nnz out of range: %lld", (long long)nnz);
  if (!rowptr) fail(SRBCRS_EINVAL, "rowptr is NULL");
  if (nnz > 0 && !colind) fail(SRBCRS_EINVAL, "colind is NULL");
  if (rowptr[0] < 0) fail(SRBCRS_EINVAL, "rowptr[0] must be >= 0");
  for (int64_t r = 0; r < num_nodes; ++r)
    if (rowptr[r + 1] < rowptr[r])
      fail(SRBCRS_EINVAL, "rowptr must be non-decreasing (row %lld)", (long long)r);
  if ((int64_t)rowptr[num_nodes] > nnz)
    fail(SRBCRS_EINVAL, "rowptr[num_nodes]=%d exceeds colind length %lld", rowptr[num_nodes],
         (long long)nnz);
}

// Per-window sorted unique columns, stored in a scratch array at the
// window's edge offset (a window never has more unique columns than edges).
struct Uniq {
  std::vector<int32_t> cols;   // size = edges covered
  std::vector<int32_t> count;  // per window
  int32_t max_col = -1;
  int64_t base = 0;            // rowptr[0]
};

void build_uniq(const int32_t* rowptr, const int32_t* colind, int32_t num_nodes, int blk_h,
                Uniq& u) {
  const int32_t Mo = (num_nodes + blk_h - 1) / blk_h;
  u.base = rowptr[0];
  u.cols.assign((size_t)(rowptr[num_nodes] - rowptr[0]), 0);
  u.count.assign((size_t)Mo, 0);
  std::atomic<int32_t> gmax{-1};
  std::atomic<bool> neg{false};
  parallel_for(Mo, [&](int64_t lo, int64_t hi) {
    int32_t lmax = -1;
    for (int64_t w = lo; w < hi; ++w) {
      const int64_t r0 = w * blk_h;
      const int64_t r1 = std::min<int64_t>(r0 + blk_h, num_nodes);
      const int64_t e0 = rowptr[r0], e1 = rowptr[r1];
      int32_t* out = u.cols.data() + (e0 - u.base);
      std::copy(colind + e0, colind + e1, out);
      std::sort(out, out + (e1 - e0));
      int32_t* end = std::unique(out, out + (e1 - e0));
      u.count[w] = (int32_t)(end - out);
      if (end != out) {
        if (out[0] < 0) neg = true;
        lmax = std::max(lmax, end[-1]);
      }
    }
    int32_t cur = gmax.load();
    while (lmax > cur && !gmax.compare_exchange_weak(cur, lmax)) {
    }
  });
  if (neg) fail(SRBCRS_EINVAL, "colind holds a negative column index");
  u.max_col = gmax.load();
}

int64_t soff_from_uniq(const Uniq& u, int blk_w, int32_t* soff) {
  int64_t total = 0;
  const int64_t Mo = (int64_t)u.count.size();
  for (int64_t w = 0; w < Mo; ++w) {
    if (total > INT32_MAX) fail(SRBCRS_EINVAL, "block count exceeds int32 offsets");
    soff[w] = (int32_t)total;
    total += (u.count[w] + blk_w - 1) / blk_w;
  }
  if (total > INT32_MAX) fail(SRBCRS_EINVAL, "block count exceeds int32 offsets");
  soff[Mo] = (int32_t)total;
  return total;
}

void fill_from_uniq(const int32_t* rowptr, const int32_t* colind, const float* values,
                    int32_t num_nodes, int blk_h, int blk_w, const Uniq& u, const int32_t* soff,
                    int32_t* sidx, float* val, int32_t* block_partition, int32_t* edge_to_row,
                    int32_t* edge_to_col) {
  const int32_t Mo = (num_nodes + blk_h - 1) / blk_h;
  const int64_t bsz = (int64_t)blk_h * blk_w;
  parallel_for(Mo, [&](int64_t lo, int64_t hi) {
    for (int64_t w = lo; w < hi; ++w) {
      const int32_t cnt = u.count[w];
      const int32_t nb = (cnt + blk_w - 1) / blk_w;
      if (soff[w + 1] - soff[w] != nb) fail(SRBCRS_EINVAL, "soff does not match the CSR (window %lld)", (long long)w);
      if (block_partition) block_partition[w] = nb;
      const int64_t r0 = w * blk_h;
      const int64_t r1 = std::min<int64_t>(r0 + blk_h, num_nodes);
      const int32_t* cols = u.cols.data() + (rowptr[r0] - u.base);
      int32_t* sw = sidx + (int64_t)soff[w] * blk_w;
      for (int64_t i = 0; i < (int64_t)nb * blk_w; ++i) sw[i] = i < cnt ? cols[i] : cols[cnt - 1];
      float* vw = val + (int64_t)soff[w] * bsz;
      std::fill(vw, vw + nb * bsz, 0.0f);
      for (int64_t r = r0; r < r1; ++r) {
        const int ir = (int)(r - r0);
        for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
          const int32_t c = colind[e];
          const int32_t pos = (int32_t)(std::lower_bound(cols, cols + cnt, c) - cols);
          if (edge_to_row) edge_to_row[e] = (int32_t)r;
          if (edge_to_col) edge_to_col[e] = pos;
          const int o = ir * blk_w + pos % blk_w;
          vw[(int64_t)(pos / blk_w) * bsz + swizzle_2_2_3(o)] = values[e];
        }
      }
    }
  });
}

// ---- schedules ------------------------------------------------------------

struct Schedule {
  std::string policy;
  int32_t param = 0;
  std::vector<int32_t> group_off{0};
  std::vector<int32_t> task_begin, task_end, task_window, task_slot;
  std::vector<int32_t> red_window, red_slot_off{0};
  int32_t n_slots = 0;
};

// Give every task of a window with several tasks its own partial slot (in
// task order) and list those windows, plus windows without any task, for
// the reduction.  Windows with one task store directly.
void assign_slots(Schedule& s, int32_t Mo) {
  std::vector<int32_t> ntask(Mo, 0);
  for (int32_t w : s.task_window) ntask[w]++;
  std::vector<int32_t> first_slot(Mo, -1);
  // slots of one window must be contiguous: allocate in window order
  int32_t next = 0;
  for (int32_t w = 0; w < Mo; ++w) {
    if (ntask[w] >= 2) {
      first_slot[w] = next;
      next += ntask[w];
    }
  }
  std::vector<int32_t> seen(Mo, 0);
  for (size_t t = 0; t < s.task_window.size(); ++t) {
    const int32_t w = s.task_window[t];
    s.task_slot[t] = ntask[w] >= 2 ? first_slot[w] + seen[w]++ : -1;
  }
  for (int32_t w = 0; w < Mo; ++w) {
    if (ntask[w] == 0 || ntask[w] >= 2) {
      s.red_window.push_back(w);
      s.red_slot_off.push_back(s.red_slot_off.back() + (ntask[w] >= 2 ? ntask[w] : 0));
    }
  }
  s.n_slots = next;
}

void push_task(Schedule& s, int32_t b, int32_t e, int32_t w) {
  s.task_begin.push_back(b);
  s.task_end.push_back(e);
  s.task_window.push_back(w);
  s.task_slot.push_back(-1);
}

// Longest window and the 95th-percentile window length, in blocks.
void window_stats(const int32_t* soff, int32_t Mo, int32_t& mx, int32_t& p95) {
  std::vector<int32_t> len(Mo);
  mx = 0;
  for (int32_t w = 0; w < Mo; ++w) {
    len[w] = soff[w + 1] - soff[w];
    mx = std::max(mx, len[w]);
  }
  p95 = 0;
  if (Mo > 0) {
    std::sort(len.begin(), len.end());
    int64_t i = (int64_t)std::ceil(Mo * 0.95) - 1;
    i = std::min<int64_t>(std::max<int64_t>(i, 0), Mo - 1);
    p95 = len[i];
  }
}

Schedule* build_schedule(const int32_t* soff, int32_t Mo, const char* policy_c, int32_t param) {
  if (!soff) fail(SRBCRS_EINVAL, "soff is NULL");
  if (Mo < 0) fail(SRBCRS_EINVAL, "row_windows must be >= 0");
  for (int32_t w = 0; w < Mo; ++w)
    if (soff[w + 1] < soff[w]) fail(SRBCRS_EINVAL, "soff must be non-decreasing");
  std::string policy = policy_c ? policy_c : "row";
  if (policy.empty()) policy = "row";
  if (param < 0) fail(SRBCRS_EINVAL, "schedule parameter must be >= 0");
  if (policy == "auto") {
    // split when the block counts have a heavy tail (the split policy's own
    // test: longest window > max(64, 4 * p95)), else one task per window
    int32_t mx, p95;
    window_stats(soff, Mo, mx, p95);
    policy = mx > std::max(64, 4 * std::max(p95, 1)) ? "split" : "row";
    param = 0;
  }
  auto* s = new Schedule();
  s->policy = policy;
  s->param = param;
  try {
    if (policy == "row") {
      for (int32_t w = 0; w < Mo; ++w) {
        push_task(*s, soff[w], soff[w + 1], w);
        s->group_off.push_back((int32_t)s->task_begin.size());
      }
    } else if (policy == "split") {
      // custom_format_e2e.cu:640-699: p95 / heavy-tail cap, then segments
      int32_t cap;
      if (param > 0) {
        cap = param;
      } else {
        int32_t mx, p95;
        window_stats(soff, Mo, mx, p95);
        const int32_t p = std::max(p95, 1);
        const bool heavy = mx > std::max(64, 4 * p);
        cap = heavy ? std::max(32, std::min(128, 2 * p95)) : std::max(mx, 1);
      }
      s->param = cap;
      for (int32_t w = 0; w < Mo; ++w) {
        const int32_t b = soff[w], e = soff[w + 1];
        if (b == e) {
          push_task(*s, b, e, w);
          s->group_off.push_back((int32_t)s->task_begin.size());
        }
        for (int64_t t = b; t < e; t += cap) {
          push_task(*s, (int32_t)t, (int32_t)std::min<int64_t>(t + cap, e), w);
          s->group_off.push_back((int32_t)s->task_begin.size());
        }
      }
    } else if (policy == "strict_lb") {
      // main_strict_lb_16x8.cu:208-256: fixed `workload` blocks per group
      const int32_t workload = param > 0 ? param : 64;
      s->param = workload;
      int32_t cur = 0;
      for (int32_t w = 0; w < Mo; ++w) {
        int32_t b = soff[w];
        const int32_t e = soff[w + 1];
        while (b < e) {
          const int32_t take = std::min(workload - cur, e - b);
          push_task(*s, b, b + take, w);
          b += take;
          cur += take;
          if (cur == workload) {
            s->group_off.push_back((int32_t)s->task_begin.size());
            cur = 0;
          }
        }
      }
      if (cur != 0 || s->group_off.size() == 1) s->group_off.push_back((int32_t)s->task_begin.size());
    } else if (policy == "multi_bind") {
      // main_multi_bind_16x8.cu:211-270: alpha = 2, parts = ceil(x / mean)
      double avg = 0.0;
      for (int32_t w = 0; w < Mo; ++w) avg += (double)(soff[w + 1] - soff[w]);
      if (Mo > 0) avg /= (double)Mo;
      for (int32_t w = 0; w < Mo; ++w) {
        const int32_t x = soff[w + 1] - soff[w];
        if (x == 0) continue;
        int32_t parts = 1;
        if (avg > 0.0 && x > 2.0 * avg) {
          const double p = std::ceil((double)x / avg);
          parts = p > 9999.0 ? 9999 : std::max(1, (int32_t)p);
        }
        const int32_t base = x / parts, rem = x % parts;
        int32_t b = soff[w];
        for (int32_t i = 0; i < parts; ++i) {
          const int32_t take = base + (i < rem ? 1 : 0);
          push_task(*s, b, b + take, w);
          s->group_off.push_back((int32_t)s->task_begin.size());
          b += take;
        }
      }
    } else {
      fail(SRBCRS_EINVAL, "unknown schedule policy '%s' (row, split, strict_lb, multi_bind, auto)",
           policy.c_str());
    }
    assign_slots(*s, Mo);
  } catch (...) {
    delete s;
    throw;
  }
  return s;
}

// ---- device memory helpers ------------------------------------------------

template <class T>
T* dev_alloc(size_t n) {
  void* p = nullptr;
  if (n == 0) n = 1;
  hipError_t e = hipMalloc(&p, n * sizeof(T));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    fail(SRBCRS_ENOMEM, "hipMalloc(%zu bytes) failed: %s", n * sizeof(T), hipGetErrorString(e));
  }
  return static_cast<T*>(p);
}

template <class T>
void dev_free(T*& p) {
  if (p) (void)hipFree(p);
  p = nullptr;
}

template <class T>
T* upload(const std::vector<T>& v) {
  T* d = dev_alloc<T>(v.size());
  if (!v.empty()) hip_check(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
  return d;
}

}  // namespace

struct srbcrs_schedule {
  Schedule s;
};

struct srbcrs_plan {
  int device = 0;
  int32_t num_nodes = 0, blk_h = 16, blk_w = 8, Mo = 0, max_col = -1;
  int64_t nnz = 0, total = 0;
  int32_t* d_soff = nullptr;
  int32_t* d_sidx = nullptr;
  float* d_val = nullptr;
  std::vector<int32_t> h_soff;
  // edge maps kept on the host until requested
  std::vector<int32_t> h_block_partition, h_edge_to_row, h_edge_to_col;
  // schedule
  Schedule sched;
  int32_t *d_group_off = nullptr, *d_task_begin = nullptr, *d_task_end = nullptr,
          *d_task_window = nullptr, *d_task_slot = nullptr, *d_red_window = nullptr,
          *d_red_slot_off = nullptr;
  float* d_partial = nullptr;
  size_t partial_cap = 0;  // floats
  // Device buffers a plan replaced (older partial buffers and task tables).
  // They are freed only with the plan: a HIP graph captured on an earlier
  // run may still hold their addresses, and a replay must not write freed
  // memory.
  std::vector<void*> retired;
  // packing (generated-operator bridge): packed rows, row map, omitted rows
  bool canonical = true;   // the preprocess_gpu conversion (edge maps available)
  int32_t packing = 0, dup_policy = 0;
  int64_t packed_rows = 0;
  std::vector<int32_t> h_order;          // empty = identity
  int32_t* d_rowmap = nullptr;
  int32_t* d_zero_rows = nullptr;
  int32_t n_zero_rows = 0;
  // edge maps of a plan converted on the device (host vectors above are empty then)
  int32_t *d_e2r = nullptr, *d_e2c = nullptr, *d_bp = nullptr;
  // compact copy of val that the SpMM reads by default (null: read val)
  uint2* d_awords = nullptr;
  float* d_apacked = nullptr;
  int64_t n_apacked = 0;
  // launch settings chosen by srbcrs_plan_tune, per dense width N, for the
  // current schedule (cleared when it changes)
  std::map<int64_t, srbcrs_run_opts> tuned;
  // interleaved unit streams of the merged-window grid, per windows-per-group
  // W (built on first use, kept until the plan is destroyed)
  struct Merged {
    int32_t* d_moff = nullptr;   // group g's units: [moff[g], moff[g+1])
    int32_t* d_sidx = nullptr;   // 8 B-row indices per unit, -1 for null units
    uint2* d_words = nullptr;    // compact A words per unit, zero for null units
    int64_t units = 0;
  };
  std::map<int, Merged> merged;
  // nonzero-sweep streams (spmm_nzsweep), per windows per group W,
  // sub-batch size U and chunk size (key nz_key)
  struct Nz {
    int32_t* d_eoff = nullptr;   // group g's pairs: [eoff[g], eoff[g+1])
    uint2* d_pairs = nullptr;    // ((tile row << 24) | B row, value bits)
    int64_t entries = 0;
  };
  std::map<int64_t, Nz> nz;

  template <class T>
  void retire(T*& p) {
    if (p) retired.push_back(static_cast<void*>(p));
    p = nullptr;
  }
  void retire_schedule() {
    retire(d_group_off);
    retire(d_task_begin);
    retire(d_task_end);
    retire(d_task_window);
    retire(d_task_slot);
    retire(d_red_window);
    retire(d_red_slot_off);
  }
  ~srbcrs_plan() {
    int cur = 0;
    bool switched = false;
    if (hipGetDevice(&cur) == hipSuccess && cur != device) switched = hipSetDevice(device) == hipSuccess;
    retire_schedule();
    retire(d_partial);
    for (void* p : retired) (void)hipFree(p);
    dev_free(d_soff);
    dev_free(d_sidx);
    dev_free(d_val);
    dev_free(d_rowmap);
    dev_free(d_zero_rows);
    dev_free(d_e2r);
    dev_free(d_e2c);
    dev_free(d_bp);
    dev_free(d_awords);
    dev_free(d_apacked);
    for (auto& kv : merged) {
      dev_free(kv.second.d_moff);
      dev_free(kv.second.d_sidx);
      dev_free(kv.second.d_words);
    }
    for (auto& kv : nz) {
      dev_free(kv.second.d_eoff);
      dev_free(kv.second.d_pairs);
    }
    if (switched) (void)hipSetDevice(cur);
  }
};

namespace {

void check_pack_opts(const srbcrs_pack_opts& o, int32_t num_nodes) {
  if (o.packing != SRBCRS_PACK_CONDENSED && o.packing != SRBCRS_PACK_FIXED_BLOCKS)
    fail(SRBCRS_EINVAL, "unknown packing %d", o.packing);
  if (o.dup_policy != SRBCRS_DUP_LAST && o.dup_policy != SRBCRS_DUP_SUM)
    fail(SRBCRS_EINVAL, "unknown duplicate policy %d", o.dup_policy);
  if (o.row_order < SRBCRS_ORDER_IDENTITY || o.row_order > SRBCRS_ORDER_EXPLICIT)
    fail(SRBCRS_EINVAL, "unknown row order %d", o.row_order);
  if (o.packing == SRBCRS_PACK_FIXED_BLOCKS && o.K <= 0)
    fail(SRBCRS_EINVAL, "fixed-block packing needs the column count K");
  if (o.row_order == SRBCRS_ORDER_EXPLICIT) {
    if (!o.order && o.order_len > 0) fail(SRBCRS_EINVAL, "explicit order is NULL");
    if (o.order_len < 0 || o.order_len > num_nodes) fail(SRBCRS_EINVAL, "explicit order length out of range");
    std::vector<uint8_t> seen((size_t)num_nodes, 0);
    for (int32_t i = 0; i < o.order_len; ++i) {
      const int32_t r = o.order[i];
      if (r < 0 || r >= num_nodes || seen[r]) fail(SRBCRS_EINVAL, "explicit order must hold distinct rows in [0, num_nodes)");
      seen[r] = 1;
    }
  }
}

srbcrs::PackSpec pack_spec(const srbcrs_pack_opts& o, int32_t num_nodes, const int32_t* order) {
  srbcrs::PackSpec s;
  s.blk_h = o.blk_h;
  s.blk_w = o.blk_w;
  s.packing = o.packing == SRBCRS_PACK_FIXED_BLOCKS ? srbcrs::kPackFixedBlocks : srbcrs::kPackCondensed;
  s.dup_sum = o.dup_policy == SRBCRS_DUP_SUM;
  s.order = (o.row_order == SRBCRS_ORDER_IDENTITY) ? nullptr : order;
  s.rows = (o.row_order == SRBCRS_ORDER_IDENTITY) ? num_nodes : o.order_len;
  s.K = o.K;
  return s;
}

template <class F>
auto guard_pack(F&& f) -> decltype(f()) {
  try {
    return f();
  } catch (const std::out_of_range& e) {
    fail(SRBCRS_EINVAL, "%s", e.what());
  } catch (const std::overflow_error& e) {
    fail(SRBCRS_EINVAL, "%s", e.what());
  } catch (const std::invalid_argument& e) {
    fail(SRBCRS_EINVAL, "%s", e.what());
  }
}

std::vector<int32_t> compute_order(const int32_t* rowptr, const int32_t* colind, int32_t m, int32_t K,
                                   int32_t method) {
  int32_t k = K;
  if (k < 0) {   // unknown column count: one past the largest column
    k = 0;
    for (int64_t e = rowptr[0]; e < rowptr[m]; ++e) k = std::max(k, colind[e] + 1);
  }
  return guard_pack([&] { return srbcrs::row_order(rowptr, colind, m, k, method); });
}

// A packed plan: resolve the order, pack on the host, upload arrays and the
// row map, and list the output rows the order leaves out (zeroed per run).
void create_packed(srbcrs_plan& plan, const int32_t* rp, const int32_t* ci, const float* vv,
                   const srbcrs_pack_opts& o) {
  const int32_t n = plan.num_nodes;
  std::vector<int32_t> order;
  if (o.row_order == SRBCRS_ORDER_EXPLICIT)
    order.assign(o.order, o.order + o.order_len);
  else
    order = compute_order(rp, ci, n, o.K, o.row_order);
  srbcrs_pack_opts eo = o;
  eo.row_order = SRBCRS_ORDER_EXPLICIT;
  eo.order = order.data();
  eo.order_len = (int32_t)order.size();
  srbcrs::PackSpec s = pack_spec(eo, n, order.data());
  plan.packed_rows = (int64_t)order.size();
  plan.Mo = (int32_t)((plan.packed_rows + plan.blk_h - 1) / plan.blk_h);
  plan.h_soff.assign((size_t)plan.Mo + 1, 0);
  plan.total = guard_pack([&] { return srbcrs::pack_count(rp, ci, s, plan.h_soff.data()); });
  std::vector<int32_t> sidx((size_t)(plan.total * plan.blk_w));
  std::vector<float> val((size_t)(plan.total * plan.blk_h * plan.blk_w));
  guard_pack([&] {
    srbcrs::pack_fill(rp, ci, vv, s, plan.h_soff.data(), sidx.data(), val.data());
    return 0;
  });
  plan.max_col = -1;
  for (int32_t c : sidx) plan.max_col = std::max(plan.max_col, c);
  bool identity = (int64_t)order.size() == n;
  for (int64_t i = 0; identity && i < (int64_t)order.size(); ++i) identity = order[i] == i;
  if (!identity) {
    plan.h_order = order;
    plan.d_rowmap = upload(order);
    std::vector<uint8_t> used((size_t)n, 0);
    for (int32_t r : order) used[r] = 1;
    std::vector<int32_t> zero;
    for (int32_t r = 0; r < n; ++r)
      if (!used[r]) zero.push_back(r);
    plan.n_zero_rows = (int32_t)zero.size();
    if (!zero.empty()) plan.d_zero_rows = upload(zero);
  }
  plan.d_soff = upload(plan.h_soff);
  plan.d_sidx = upload(sidx);
  plan.d_val = upload(val);
  plan.sched.policy = "row";
}

void* conv_alloc(void*, size_t bytes) {
  void* p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return p;
}

void conv_free(void*, void* p) { (void)hipFree(p); }

// Canonical conversion of a device CSR on the device (srbcrs_convert.hip).
void create_on_device(srbcrs_plan& plan, const int32_t* rowptr, const int32_t* colind,
                      const float* values, hipStream_t st) {
  const int32_t Mo = (plan.num_nodes + plan.blk_h - 1) / plan.blk_h;
  plan.Mo = Mo;
  plan.d_soff = dev_alloc<int32_t>((size_t)Mo + 1);
  plan.d_e2r = dev_alloc<int32_t>((size_t)plan.nnz);
  plan.d_e2c = dev_alloc<int32_t>((size_t)plan.nnz);
  plan.d_bp = dev_alloc<int32_t>((size_t)Mo);
  if (plan.nnz) {
    hip_check(hipMemsetAsync(plan.d_e2r, 0, (size_t)plan.nnz * 4, st), "hipMemsetAsync");
    hip_check(hipMemsetAsync(plan.d_e2c, 0, (size_t)plan.nnz * 4, st), "hipMemsetAsync");
  }
  srbcrs::DeviceConvertIn in{rowptr, colind, values, plan.num_nodes, plan.nnz, plan.blk_h, plan.blk_w,
                             plan.d_e2r, plan.d_e2c, plan.d_bp};
  srbcrs::DeviceConvertOut out;
  out.soff = plan.d_soff;
  const hipError_t e = srbcrs::device_convert(in, out, conv_alloc, conv_free, nullptr, st);
  plan.d_sidx = out.sidx;   // owned by the plan from here on, even on failure
  plan.d_val = out.val;
  hip_check(e, "device conversion");
  if (out.bad == 1) fail(SRBCRS_EINVAL, "rowptr must be non-decreasing and within [0, nnz]");
  if (out.bad == 2) fail(SRBCRS_EINVAL, "colind holds a negative column index");
  plan.total = out.total;
  plan.max_col = out.max_col;
  plan.h_soff.resize((size_t)Mo + 1);
  hip_check(hipMemcpyAsync(plan.h_soff.data(), plan.d_soff, plan.h_soff.size() * 4, hipMemcpyDeviceToHost, st),
            "copy soff");
  hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
  plan.sched.policy = "row";
}

// no launch knob set (the epilogue is not a launch knob: a tuned setting
// runs with the caller's epilogue)
bool all_default(const srbcrs_run_opts& o) {
  return !o.depth && !o.tile_b && !o.wg_cols && !o.grid_order && !o.windows_per_wave && !o.a_operand &&
         !o.b_stage;
}

// Compact copy of the block values (srbcrs_compact.hip).  A plan too large
// for it, or a device without the memory, keeps reading val.
void build_compact(srbcrs_plan& plan, hipStream_t st) {
  if (plan.total == 0) return;
  srbcrs::CompactOut c;
  const hipError_t e = srbcrs::device_compact(plan.d_val, plan.total, plan.blk_h, plan.blk_w, conv_alloc,
                                              conv_free, nullptr, st, c);
  if (e == hipErrorOutOfMemory || e == hipErrorInvalidValue) {
    (void)hipGetLastError();
    return;
  }
  hip_check(e, "compact block values");
  plan.d_awords = c.words;
  plan.d_apacked = c.packed;
  plan.n_apacked = c.n_packed;
}

// The interleaved unit stream of the merged-window grid for groups of W row
// windows (spmm_merged, srbcrs_merged.hpp): group g = windows [gW, gW + W);
// its stream is R rounds of W units, round r holding block r of each window
// (null units where a window has fewer than R blocks, and for the slots past
// the last window).  Built on the host from the plan's sidx and compact A
// words (copied down once), uploaded once per W.
const srbcrs_plan::Merged& merged_stream(srbcrs_plan& plan, int W, hipStream_t st) {
  auto it = plan.merged.find(W);
  if (it != plan.merged.end()) return it->second;
  const int64_t nb = plan.total;
  const int Mo = plan.Mo;
  constexpr int kWords = 16 * 8 / 32;   // compact A words per 16x8 block
  std::vector<int32_t> sidx((size_t)nb * 8);
  std::vector<uint2> words((size_t)nb * kWords);
  if (nb) {
    hip_check(hipMemcpyAsync(sidx.data(), plan.d_sidx, sidx.size() * sizeof(int32_t), hipMemcpyDeviceToHost, st),
              "hipMemcpyAsync sidx D2H");
    hip_check(hipMemcpyAsync(words.data(), plan.d_awords, words.size() * sizeof(uint2), hipMemcpyDeviceToHost, st),
              "hipMemcpyAsync A words D2H");
    hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
  }
  const int64_t n_groups = (Mo + W - 1) / W;
  std::vector<int32_t> moff((size_t)n_groups + 1, 0);
  for (int64_t g = 0; g < n_groups; ++g) {
    int32_t rounds = 0;
    for (int w = (int)(g * W); w < Mo && w < (g + 1) * W; ++w)
      rounds = std::max(rounds, plan.h_soff[w + 1] - plan.h_soff[w]);
    const int64_t next = (int64_t)moff[g] + (int64_t)rounds * W;
    if (next > INT32_MAX) fail(SRBCRS_EINVAL, "the merged-window stream exceeds 2^31 units");
    moff[g + 1] = (int32_t)next;
  }
  const int64_t units = moff[n_groups];
  std::vector<int32_t> msidx((size_t)units * 8, -1);
  std::vector<uint2> mwords((size_t)units * kWords, uint2{0u, 0u});
  parallel_for(n_groups, [&](int64_t lo, int64_t hi) {
    for (int64_t g = lo; g < hi; ++g)
      for (int w = 0; w < W; ++w) {
        const int64_t win = g * W + w;
        if (win >= Mo) break;
        const int32_t b0 = plan.h_soff[win], b1 = plan.h_soff[win + 1];
        for (int32_t b = b0; b < b1; ++b) {
          const int64_t u = moff[g] + (int64_t)(b - b0) * W + w;
          std::copy_n(&sidx[(size_t)b * 8], 8, &msidx[(size_t)u * 8]);
          std::copy_n(&words[(size_t)b * kWords], kWords, &mwords[(size_t)u * kWords]);
        }
      }
  });
  srbcrs_plan::Merged m;
  try {
    m.d_moff = upload(moff);
    m.d_sidx = upload(msidx);
    m.d_words = upload(mwords);
  } catch (...) {
    dev_free(m.d_moff);
    dev_free(m.d_sidx);
    dev_free(m.d_words);
    throw;
  }
  m.units = units;
  return plan.merged.emplace(W, m).first->second;
}

int64_t nz_key(int W, int U, int D) { return ((int64_t)W << 16) | ((int64_t)U << 8) | (int64_t)D; }

// The entry stream of the nonzero sweep for groups of W row windows and
// sub-batches of U entries (spmm_nzsweep, srbcrs_nzsweep.hpp).  A group's
// stored values are listed in the merged unit order (block r of each window
// in window order, then r + 1), within a block column by column and, in a
// column, row by row; each is the entry ((16 * window slot + row) << 24) |
// B row with its value.  The list is then cut into sub-batches of U entries
// with distinct tile rows: each sub-batch takes, in list order, the entries
// among the next 4U not yet taken whose row is neither in the sub-batch nor
// held by an earlier entry left behind, so every row keeps its values in
// list order (ascending columns); a sub-batch short of U is filled with
// entries for tile row 16 * W (never stored) that repeat the previous B row
// (a cache hit).  Groups are padded the same way to whole loop bodies of
// the kernel (2D sub-batches).  Each sub-batch is stored transposed for the
// kernel's gather instructions (pair g * U/4 + q = entry 4q + g).  Built on
// the host from the plan's sidx, compact A words and packed values.
const srbcrs_plan::Nz& nz_stream(srbcrs_plan& plan, int W, int U, int D, hipStream_t st) {
  const int64_t key = nz_key(W, U, D);
  auto it = plan.nz.find(key);
  if (it != plan.nz.end()) return it->second;
  const int kChunk = 2 * D * U;      // the kernel's loop body
  const int E = 4, Q = U / E;   // entries per gather instruction, instructions per sub-batch
  constexpr int kRowShift = 24;   // entry = (tile row << 24) | B row
  constexpr int kWords = 16 * 8 / 32;
  const int64_t nb = plan.total;
  const int Mo = plan.Mo;
  if (plan.max_col >= (1 << kRowShift))
    fail(SRBCRS_EINVAL, "the nonzero sweep takes B-row indices below 2^%d (the matrix references column %d)",
         kRowShift, plan.max_col);
  std::vector<int32_t> sidx((size_t)nb * 8);
  std::vector<uint2> words((size_t)nb * kWords);
  std::vector<float> packed((size_t)plan.n_apacked);
  if (nb) {
    hip_check(hipMemcpyAsync(sidx.data(), plan.d_sidx, sidx.size() * sizeof(int32_t), hipMemcpyDeviceToHost, st),
              "hipMemcpyAsync sidx D2H");
    hip_check(hipMemcpyAsync(words.data(), plan.d_awords, words.size() * sizeof(uint2), hipMemcpyDeviceToHost, st),
              "hipMemcpyAsync A words D2H");
    if (!packed.empty())
      hip_check(hipMemcpyAsync(packed.data(), plan.d_apacked, packed.size() * sizeof(float), hipMemcpyDeviceToHost,
                               st),
                "hipMemcpyAsync packed values D2H");
    hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
  }
  const uint32_t dummy = (uint32_t)(16 * W);
  const int64_t n_groups = (Mo + W - 1) / W;
  // a row with many more values than its group's other rows puts one value
  // per sub-batch and fills the rest with padding (up to U entries per
  // value): a stream that would be mostly padding and large is refused (the
  // MFMA grids serve such matrices), before it is built when the groups'
  // lower bounds (U entries per sub-batch, at least as many sub-batches as
  // the longest row has values) already exceed the limit
  const int64_t limit = std::max<int64_t>(8 * plan.n_apacked, (int64_t)1 << 22) + (int64_t)kChunk * n_groups;
  std::atomic<int64_t> bound{0};
  std::atomic<bool> over{false};
  std::vector<std::vector<uint2>> g_pairs((size_t)n_groups);
  parallel_for(n_groups, [&](int64_t lo, int64_t hi) {
    std::vector<uint32_t> le;
    std::vector<float> lv;
    std::vector<char> taken;
    for (int64_t g = lo; g < hi; ++g) {
      if (over.load(std::memory_order_relaxed)) return;
      // the group's values in list order
      le.clear();
      lv.clear();
      int32_t rounds = 0;
      for (int64_t win = g * W; win < Mo && win < (g + 1) * W; ++win)
        rounds = std::max(rounds, plan.h_soff[win + 1] - plan.h_soff[win]);
      for (int32_t r = 0; r < rounds; ++r)
        for (int w = 0; w < W; ++w) {
          const int64_t win = g * W + w;
          if (win >= Mo) break;
          const int64_t b = (int64_t)plan.h_soff[win] + r;
          if (b >= plan.h_soff[win + 1]) continue;
          for (int k = 0; k < 8; ++k)
            for (int row = 0; row < 16; ++row) {
              const int pos = 8 * row + k;
              const uint2 wd = words[(size_t)b * kWords + (pos >> 5)];
              const int bit = pos & 31;
              if (!((wd.x >> bit) & 1u)) continue;
              le.push_back(((uint32_t)(16 * w + row) << kRowShift) | (uint32_t)sidx[(size_t)b * 8 + k]);
              lv.push_back(packed[(size_t)wd.y + __builtin_popcount(wd.x & ((1u << bit) - 1u))]);
            }
        }
      {
        int count[256] = {0}, longest = 0;
        for (const uint32_t e : le) longest = std::max(longest, ++count[e >> kRowShift]);
        const int64_t batches = std::max<int64_t>(((int64_t)le.size() + U - 1) / U, longest);
        if (bound.fetch_add(batches * U, std::memory_order_relaxed) + batches * U > limit) {
          over.store(true, std::memory_order_relaxed);
          return;
        }
      }
      // sub-batches of U distinct tile rows, each stored transposed: pair
      // gg * Q + q = entry E * q + gg
      std::vector<uint2>& op = g_pairs[(size_t)g];
      std::vector<uint2> batch((size_t)U);
      const size_t n = le.size();
      taken.assign(n, 0);
      size_t head = 0;
      const uint32_t kBRow = (1u << kRowShift) - 1u;
      uint32_t prev = le.empty() ? 0u : le[0] & kBRow;
      auto put = [&](int u, uint32_t e, float v) {
        batch[(size_t)((u % E) * Q + u / E)] = uint2{e, __builtin_bit_cast(uint32_t, v)};
      };
      while (head < n) {
        uint64_t used[4] = {0, 0, 0, 0}, held[4] = {0, 0, 0, 0};
        int got = 0;
        for (size_t i = head; i < n && i < head + 4 * (size_t)U && got < U; ++i) {
          if (taken[i]) continue;
          const uint32_t t = le[i] >> kRowShift;
          const uint64_t bit = 1ull << (t & 63);
          if ((used[t >> 6] | held[t >> 6]) & bit) {
            held[t >> 6] |= bit;
            continue;
          }
          used[t >> 6] |= bit;
          taken[i] = 1;
          put(got, le[i], lv[i]);
          prev = le[i] & kBRow;
          ++got;
        }
        for (; got < U; ++got) put(got, (dummy << kRowShift) | prev, 0.f);
        op.insert(op.end(), batch.begin(), batch.end());
        while (head < n && taken[head]) ++head;
      }
      while (op.size() % kChunk) op.push_back(uint2{(dummy << kRowShift) | prev, 0u});
    }
  });
#define SRBCRS_NZ_PADDED(what)                                                                              \
  "the nonzero sweep would pad this matrix to " what " entries for %lld values (rows much longer than their " \
  "group's others): use another grid order"
  if (over.load())
    fail(SRBCRS_EINVAL, SRBCRS_NZ_PADDED("over %lld"), (long long)limit, (long long)plan.n_apacked);
  std::vector<int32_t> eoff((size_t)n_groups + 1, 0);
  int64_t entries = 0;
  for (int64_t g = 0; g < n_groups; ++g) {
    entries += (int64_t)g_pairs[(size_t)g].size();
    if (entries > INT32_MAX) fail(SRBCRS_EINVAL, "the nonzero-sweep stream exceeds 2^31 entries");
    eoff[(size_t)g + 1] = (int32_t)entries;
  }
  if (entries > limit) fail(SRBCRS_EINVAL, SRBCRS_NZ_PADDED("%lld"), (long long)entries, (long long)plan.n_apacked);
#undef SRBCRS_NZ_PADDED
  std::vector<uint2> pairs((size_t)entries);
  parallel_for(n_groups, [&](int64_t lo, int64_t hi) {
    for (int64_t g = lo; g < hi; ++g)
      std::copy(g_pairs[(size_t)g].begin(), g_pairs[(size_t)g].end(), pairs.begin() + eoff[(size_t)g]);
  });
  srbcrs_plan::Nz z;
  try {
    z.d_eoff = upload(eoff);
    z.d_pairs = upload(pairs);
  } catch (...) {
    dev_free(z.d_eoff);
    dev_free(z.d_pairs);
    throw;
  }
  z.entries = entries;
  return plan.nz.emplace(key, z).first->second;
}

}  // namespace

extern "C" {

const char* srbcrs_last_error(void) { return g_last_error.c_str(); }

// A decomposition build (mask_amd/build.py --experiment) carries its name in
// the version string, so that loaders can refuse it.
#define SRBCRS_STR2(x) #x
#define SRBCRS_STR(x) SRBCRS_STR2(x)
#ifdef SRBCRS_EXPERIMENT_TAG
const char* srbcrs_version(void) { return "mask_amd-srbcrs 0.2 gfx950+experiment:" SRBCRS_STR(SRBCRS_EXPERIMENT_TAG); }
#else
const char* srbcrs_version(void) { return "mask_amd-srbcrs 0.2 gfx950"; }
#endif

int srbcrs_convert_count(const int32_t* rowptr, const int32_t* colind, int32_t num_nodes,
                         int64_t nnz, int32_t blk_h, int32_t blk_w, int32_t* soff,
                         int64_t* total_blocks) {
  return guarded([&] {
    check_block_shape(blk_h, blk_w);
    check_csr(rowptr, colind, num_nodes, nnz);
    if (!soff || !total_blocks) fail(SRBCRS_EINVAL, "soff / total_blocks is NULL");
    Uniq u;
    build_uniq(rowptr, colind, num_nodes, blk_h, u);
    *total_blocks = soff_from_uniq(u, blk_w, soff);
  });
}

int srbcrs_convert_fill(const int32_t* rowptr, const int32_t* colind, const float* values,
                        int32_t num_nodes, int64_t nnz, int32_t blk_h, int32_t blk_w,
                        const int32_t* soff, int32_t* sidx, float* val, int32_t* block_partition,
                        int32_t* edge_to_row, int32_t* edge_to_col) {
  return guarded([&] {
    check_block_shape(blk_h, blk_w);
    check_csr(rowptr, colind, num_nodes, nnz);
    if (!soff || !sidx || !val) fail(SRBCRS_EINVAL, "soff / sidx / val is NULL");
    if (nnz > 0 && !values) fail(SRBCRS_EINVAL, "values is NULL");
    Uniq u;
    build_uniq(rowptr, colind, num_nodes, blk_h, u);
    fill_from_uniq(rowptr, colind, values, num_nodes, blk_h, blk_w, u, soff, sidx, val,
                   block_partition, edge_to_row, edge_to_col);
  });
}

int srbcrs_plan_create(const int32_t* rowptr, const int32_t* colind, const float* values,
                       int32_t num_nodes, int64_t nnz, int32_t blk_h, int32_t blk_w,
                       int32_t is_device, void* stream, srbcrs_plan** out) {
  srbcrs_pack_opts o{};
  o.blk_h = blk_h;
  o.blk_w = blk_w;
  o.packing = SRBCRS_PACK_CONDENSED;
  o.dup_policy = SRBCRS_DUP_LAST;
  o.row_order = SRBCRS_ORDER_IDENTITY;
  o.K = -1;
  return srbcrs_plan_create_ex(rowptr, colind, values, num_nodes, nnz, &o, is_device, stream, out);
}

int srbcrs_plan_create_ex(const int32_t* rowptr, const int32_t* colind, const float* values,
                          int32_t num_nodes, int64_t nnz, const srbcrs_pack_opts* opts,
                          int32_t is_device, void* stream, srbcrs_plan** out) {
  return guarded([&] {
    if (!out) fail(SRBCRS_EINVAL, "out is NULL");
    *out = nullptr;
    srbcrs_pack_opts o{};
    if (opts) {
      o = *opts;
    } else {
      o.blk_h = 16;
      o.blk_w = 8;
      o.K = -1;
    }
    const int32_t blk_h = o.blk_h, blk_w = o.blk_w;
    check_block_shape(blk_h, blk_w);
    check_pack_opts(o, num_nodes);
    const bool canonical = o.packing == SRBCRS_PACK_CONDENSED && o.dup_policy == SRBCRS_DUP_LAST &&
                           o.row_order == SRBCRS_ORDER_IDENTITY;
    if (num_nodes < 1) fail(SRBCRS_EINVAL, "num_nodes must be positive");
    if (nnz < 0 || nnz > INT32_MAX) fail(SRBCRS_EINVAL, "nnz out of range");
    if (is_device < 0 || is_device > 2) fail(SRBCRS_EINVAL, "is_device must be 0, 1 or 2");
    std::vector<int32_t> h_rowptr, h_colind;
    std::vector<float> h_values;
    const int32_t *rp = rowptr, *ci = colind;
    const float* vv = values;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (canonical && is_device == 1) {
      // device CSR converted in HBM (no host round trip)
      if (!rowptr || (nnz > 0 && (!colind || !values))) fail(SRBCRS_EINVAL, "NULL CSR array");
      auto plan = std::make_unique<srbcrs_plan>();
      hip_check(hipGetDevice(&plan->device), "hipGetDevice");
      plan->num_nodes = num_nodes;
      plan->blk_h = blk_h;
      plan->blk_w = blk_w;
      plan->nnz = nnz;
      plan->canonical = true;
      plan->packed_rows = num_nodes;
      create_on_device(*plan, rowptr, colind, values, st);
      build_compact(*plan, st);
      *out = plan.release();
      return;
    }
    if (is_device) {
      // the reference copies the device CSR to the host for conversion
      // (SRBCRSSpMM_kernel.cu:203-205)
      h_rowptr.resize((size_t)num_nodes + 1);
      h_colind.resize((size_t)nnz);
      h_values.resize((size_t)nnz);
      hip_check(hipMemcpyAsync(h_rowptr.data(), rowptr, h_rowptr.size() * 4, hipMemcpyDeviceToHost, st), "copy rowptr");
      if (nnz) {
        hip_check(hipMemcpyAsync(h_colind.data(), colind, (size_t)nnz * 4, hipMemcpyDeviceToHost, st), "copy colind");
        hip_check(hipMemcpyAsync(h_values.data(), values, (size_t)nnz * 4, hipMemcpyDeviceToHost, st), "copy values");
      }
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
      rp = h_rowptr.data();
      ci = h_colind.data();
      vv = h_values.data();
    }
    check_csr(rp, ci, num_nodes, nnz);
    if (nnz > 0 && !vv) fail(SRBCRS_EINVAL, "values is NULL");
    auto plan = std::make_unique<srbcrs_plan>();
    hip_check(hipGetDevice(&plan->device), "hipGetDevice");
    plan->num_nodes = num_nodes;
    plan->blk_h = blk_h;
    plan->blk_w = blk_w;
    plan->nnz = nnz;
    plan->packing = o.packing;
    plan->dup_policy = o.dup_policy;
    plan->canonical = canonical;
    if (!canonical) {
      create_packed(*plan, rp, ci, vv, o);
      build_compact(*plan, st);
      *out = plan.release();
      return;
    }
    plan->packed_rows = num_nodes;
    plan->Mo = (num_nodes + blk_h - 1) / blk_h;
    Uniq u;
    build_uniq(rp, ci, num_nodes, blk_h, u);
    plan->max_col = u.max_col;
    plan->h_soff.resize((size_t)plan->Mo + 1);
    plan->total = soff_from_uniq(u, blk_w, plan->h_soff.data());
    std::vector<int32_t> sidx((size_t)(plan->total * blk_w));
    std::vector<float> val((size_t)(plan->total * blk_h * blk_w));
    plan->h_block_partition.assign((size_t)plan->Mo, 0);
    plan->h_edge_to_row.assign((size_t)nnz, 0);
    plan->h_edge_to_col.assign((size_t)nnz, 0);
    fill_from_uniq(rp, ci, vv, num_nodes, blk_h, blk_w, u, plan->h_soff.data(), sidx.data(),
                   val.data(), plan->h_block_partition.data(), plan->h_edge_to_row.data(),
                   plan->h_edge_to_col.data());
    plan->d_soff = upload(plan->h_soff);
    plan->d_sidx = upload(sidx);
    plan->d_val = upload(val);
    plan->sched.policy = "row";
    build_compact(*plan, st);
    *out = plan.release();
  });
}

void srbcrs_plan_destroy(srbcrs_plan* plan) { delete plan; }

int srbcrs_plan_get(const srbcrs_plan* plan, srbcrs_plan_desc* out) {
  return guarded([&] {
    if (!plan || !out) fail(SRBCRS_EINVAL, "plan / out is NULL");
    out->num_nodes = plan->num_nodes;
    out->blk_h = plan->blk_h;
    out->blk_w = plan->blk_w;
    out->row_windows = plan->Mo;
    out->max_col = plan->max_col;
    out->device = plan->device;
    out->nnz = plan->nnz;
    out->total_blocks = plan->total;
    out->d_soff = plan->d_soff;
    out->d_sidx = plan->d_sidx;
    out->d_val = plan->d_val;
    out->packed_rows = plan->packed_rows;
    out->d_row_map = plan->d_rowmap;
    out->packing = plan->packing;
    out->dup_policy = plan->dup_policy;
    out->stored_values = plan->d_awords || plan->total == 0 ? plan->n_apacked : -1;
    out->d_a_words = plan->d_awords;
    out->d_a_packed = plan->d_apacked;
  });
}

int srbcrs_plan_row_order(const srbcrs_plan* plan, int32_t* order, int32_t capacity, int32_t* len) {
  return guarded([&] {
    if (!plan || !len) fail(SRBCRS_EINVAL, "plan / len is NULL");
    *len = (int32_t)plan->packed_rows;
    if (!order) return;
    if (capacity < plan->packed_rows) fail(SRBCRS_EINVAL, "order buffer too short");
    if (plan->h_order.empty())
      for (int64_t i = 0; i < plan->packed_rows; ++i) order[i] = (int32_t)i;
    else
      std::memcpy(order, plan->h_order.data(), plan->h_order.size() * 4);
  });
}

int srbcrs_row_order(const int32_t* rowptr, const int32_t* colind, int32_t num_nodes, int64_t nnz,
                     int32_t K, int32_t method, int32_t* order, int32_t* order_len) {
  return guarded([&] {
    check_csr(rowptr, colind, num_nodes, nnz);
    if (!order || !order_len) fail(SRBCRS_EINVAL, "order / order_len is NULL");
    if (method < SRBCRS_ORDER_IDENTITY || method > SRBCRS_ORDER_SPARSE_ROWS)
      fail(SRBCRS_EINVAL, "unknown row order method %d", method);
    std::vector<int32_t> o = compute_order(rowptr, colind, num_nodes, K, method);
    std::memcpy(order, o.data(), o.size() * 4);
    *order_len = (int32_t)o.size();
  });
}

int srbcrs_pack_count(const int32_t* rowptr, const int32_t* colind, int32_t num_nodes, int64_t nnz,
                      const srbcrs_pack_opts* opts, int32_t* soff, int64_t* total_tiles) {
  return guarded([&] {
    check_csr(rowptr, colind, num_nodes, nnz);
    if (!opts || !soff || !total_tiles) fail(SRBCRS_EINVAL, "NULL argument");
    check_block_shape(opts->blk_h, opts->blk_w);
    check_pack_opts(*opts, num_nodes);
    if (opts->row_order != SRBCRS_ORDER_IDENTITY && opts->row_order != SRBCRS_ORDER_EXPLICIT)
      fail(SRBCRS_EINVAL, "pack_count takes an identity or explicit order (use srbcrs_row_order)");
    srbcrs::PackSpec s = pack_spec(*opts, num_nodes, opts->order);
    *total_tiles = guard_pack([&] { return srbcrs::pack_count(rowptr, colind, s, soff); });
  });
}

int srbcrs_pack_fill(const int32_t* rowptr, const int32_t* colind, const float* values,
                     int32_t num_nodes, int64_t nnz, const srbcrs_pack_opts* opts,
                     const int32_t* soff, int32_t* sidx, float* val) {
  return guarded([&] {
    check_csr(rowptr, colind, num_nodes, nnz);
    if (!opts || !soff || !sidx || !val) fail(SRBCRS_EINVAL, "NULL argument");
    if (nnz > 0 && !values) fail(SRBCRS_EINVAL, "values is NULL");
    check_block_shape(opts->blk_h, opts->blk_w);
    check_pack_opts(*opts, num_nodes);
    if (opts->row_order != SRBCRS_ORDER_IDENTITY && opts->row_order != SRBCRS_ORDER_EXPLICIT)
      fail(SRBCRS_EINVAL, "pack_fill takes an identity or explicit order (use srbcrs_row_order)");
    srbcrs::PackSpec s = pack_spec(*opts, num_nodes, opts->order);
    guard_pack([&] {
      srbcrs::pack_fill(rowptr, colind, values, s, soff, sidx, val);
      return 0;
    });
  });
}

int srbcrs_plan_write_edges(const srbcrs_plan* plan, int32_t* d_block_partition,
                            int64_t block_partition_len, int32_t* d_edge_to_col,
                            int64_t edge_to_col_len, int32_t* d_edge_to_row,
                            int64_t edge_to_row_len, void* stream) {
  return guarded([&] {
    if (!plan) fail(SRBCRS_EINVAL, "plan is NULL");
    if (!plan->canonical) fail(SRBCRS_EINVAL, "edge maps exist only for canonical (preprocess_gpu) plans");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (plan->d_e2r) {   // converted on the device: device-to-device copies
      if (d_block_partition && block_partition_len >= plan->Mo && plan->Mo > 0)
        hip_check(hipMemcpyAsync(d_block_partition, plan->d_bp, (size_t)plan->Mo * 4, hipMemcpyDeviceToDevice, st),
                  "copy block_partition");
      if (d_edge_to_col && edge_to_col_len >= plan->nnz && plan->nnz > 0)
        hip_check(hipMemcpyAsync(d_edge_to_col, plan->d_e2c, (size_t)plan->nnz * 4, hipMemcpyDeviceToDevice, st),
                  "copy edge_to_col");
      if (d_edge_to_row && edge_to_row_len >= plan->nnz && plan->nnz > 0)
        hip_check(hipMemcpyAsync(d_edge_to_row, plan->d_e2r, (size_t)plan->nnz * 4, hipMemcpyDeviceToDevice, st),
                  "copy edge_to_row");
      hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
      return;
    }
    if (d_block_partition && block_partition_len >= plan->Mo && plan->Mo > 0)
      hip_check(hipMemcpyAsync(d_block_partition, plan->h_block_partition.data(), (size_t)plan->Mo * 4,
                               hipMemcpyHostToDevice, st), "copy block_partition");
    if (d_edge_to_col && edge_to_col_len >= plan->nnz && plan->nnz > 0)
      hip_check(hipMemcpyAsync(d_edge_to_col, plan->h_edge_to_col.data(), (size_t)plan->nnz * 4,
                               hipMemcpyHostToDevice, st), "copy edge_to_col");
    if (d_edge_to_row && edge_to_row_len >= plan->nnz && plan->nnz > 0)
      hip_check(hipMemcpyAsync(d_edge_to_row, plan->h_edge_to_row.data(), (size_t)plan->nnz * 4,
                               hipMemcpyHostToDevice, st), "copy edge_to_row");
    hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
  });
}

int srbcrs_plan_export_index(const srbcrs_plan* plan, int32_t* d_row_window_offset,
                             int64_t row_window_offset_len, int32_t* d_tcblocktile_id,
                             int64_t tcblocktile_id_len, void* stream) {
  return guarded([&] {
    if (!plan) fail(SRBCRS_EINVAL, "plan is NULL");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t ns = (int64_t)plan->Mo + 1, nx = plan->total * plan->blk_w;
    if (d_row_window_offset) {
      if (row_window_offset_len < ns) fail(SRBCRS_EINVAL, "row_window_offset buffer too short (%lld < %lld)", (long long)row_window_offset_len, (long long)ns);
      hip_check(hipMemcpyAsync(d_row_window_offset, plan->d_soff, (size_t)ns * 4, hipMemcpyDeviceToDevice, st), "copy soff");
    }
    if (d_tcblocktile_id && nx > 0) {
      if (tcblocktile_id_len < nx) fail(SRBCRS_EINVAL, "tcblocktile_id buffer too short (%lld < %lld)", (long long)tcblocktile_id_len, (long long)nx);
      hip_check(hipMemcpyAsync(d_tcblocktile_id, plan->d_sidx, (size_t)nx * 4, hipMemcpyDeviceToDevice, st), "copy sidx");
    }
  });
}

int srbcrs_plan_export_values(const srbcrs_plan* plan, float* d_val, int64_t val_len, void* stream) {
  return guarded([&] {
    if (!plan) fail(SRBCRS_EINVAL, "plan is NULL");
    const int64_t n = plan->total * plan->blk_h * plan->blk_w;
    if (n == 0) return;
    if (!d_val || val_len < n) fail(SRBCRS_EINVAL, "value buffer too short (%lld < %lld)", (long long)val_len, (long long)n);
    hip_check(hipMemcpyAsync(d_val, plan->d_val, (size_t)n * 4, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)),
              "copy values");
  });
}

int srbcrs_schedule_build(const int32_t* soff, int32_t row_windows, const char* policy,
                          int32_t param, srbcrs_schedule** out) {
  return guarded([&] {
    if (!out) fail(SRBCRS_EINVAL, "out is NULL");
    *out = nullptr;
    Schedule* s = build_schedule(soff, row_windows, policy, param);
    auto* h = new srbcrs_schedule{std::move(*s)};
    delete s;
    *out = h;
  });
}

int srbcrs_schedule_info(const srbcrs_schedule* s, int32_t* n_groups, int32_t* n_tasks,
                         int32_t* n_slots, int32_t* n_red) {
  return guarded([&] {
    if (!s) fail(SRBCRS_EINVAL, "schedule is NULL");
    if (n_groups) *n_groups = (int32_t)s->s.group_off.size() - 1;
    if (n_tasks) *n_tasks = (int32_t)s->s.task_begin.size();
    if (n_slots) *n_slots = s->s.n_slots;
    if (n_red) *n_red = (int32_t)s->s.red_window.size();
  });
}

int srbcrs_schedule_export(const srbcrs_schedule* s, int32_t* group_off, int32_t* task_begin,
                           int32_t* task_end, int32_t* task_window, int32_t* task_slot,
                           int32_t* red_window, int32_t* red_slot_off) {
  return guarded([&] {
    if (!s) fail(SRBCRS_EINVAL, "schedule is NULL");
    auto cp = [](const std::vector<int32_t>& v, int32_t* dst) {
      if (dst && !v.empty()) std::memcpy(dst, v.data(), v.size() * 4);
    };
    cp(s->s.group_off, group_off);
    cp(s->s.task_begin, task_begin);
    cp(s->s.task_end, task_end);
    cp(s->s.task_window, task_window);
    cp(s->s.task_slot, task_slot);
    cp(s->s.red_window, red_window);
    cp(s->s.red_slot_off, red_slot_off);
  });
}

void srbcrs_schedule_destroy(srbcrs_schedule* s) { delete s; }

int srbcrs_plan_set_schedule(srbcrs_plan* plan, const char* policy, int32_t param) {
  return guarded([&] {
    if (!plan) fail(SRBCRS_EINVAL, "plan is NULL");
    int cur = 0;
    hip_check(hipGetDevice(&cur), "hipGetDevice");
    if (cur != plan->device) fail(SRBCRS_ESTATE, "plan lives on device %d, current device is %d", plan->device, cur);
    Schedule* s = build_schedule(plan->h_soff.data(), plan->Mo, policy, param);
    std::unique_ptr<Schedule> hold(s);
    plan->retire_schedule();
    plan->tuned.clear();
    plan->sched = std::move(*s);
    if (plan->sched.policy != "row") {
      plan->d_group_off = upload(plan->sched.group_off);
      plan->d_task_begin = upload(plan->sched.task_begin);
      plan->d_task_end = upload(plan->sched.task_end);
      plan->d_task_window = upload(plan->sched.task_window);
      plan->d_task_slot = upload(plan->sched.task_slot);
      plan->d_red_window = upload(plan->sched.red_window);
      plan->d_red_slot_off = upload(plan->sched.red_slot_off);
    }
  });
}

int srbcrs_run(srbcrs_plan* plan, const float* d_B, int64_t K, int64_t N, int64_t ldb, float* d_C,
               int64_t ldc, int64_t c_rows, void* stream) {
  return srbcrs_run_ex(plan, d_B, K, N, ldb, d_C, ldc, c_rows, nullptr, stream);
}

// The body of srbcrs_run_ex / srbcrs_run_noalloc.  fixed_partial (with room
// for fixed_cap floats) replaces the plan's grown partial buffer; with it the
// run allocates nothing.
static void run_impl(srbcrs_plan* plan, const float* d_B, int64_t K, int64_t N, int64_t ldb, float* d_C,
                     int64_t ldc, int64_t c_rows, const srbcrs_run_opts* opts, void* stream,
                     float* fixed_partial, size_t fixed_cap) {
    srbcrs_run_opts tuned_opts;
    if (plan && (!opts || all_default(*opts))) {
      const auto it = plan->tuned.find(N);
      if (it != plan->tuned.end()) {
        tuned_opts = it->second;
        tuned_opts.epilogue = opts ? opts->epilogue : SRBCRS_EPILOGUE_NONE;
        opts = &tuned_opts;
      }
    }
    srbcrs::RunOpts ro;
    int max_vec = 4;
    if (opts) {
      if (opts->depth != 0 && opts->depth != 2 && opts->depth != 4 && opts->depth != 8)
        fail(SRBCRS_EINVAL, "depth must be 0, 2, 4 or 8 (got %d)", opts->depth);
      if (opts->tile_b != 0 && opts->tile_b != 16 && opts->tile_b != 32 && opts->tile_b != 64)
        fail(SRBCRS_EINVAL, "tile_b must be 0, 16, 32 or 64 (got %d)", opts->tile_b);
      if (opts->wg_cols != 0 && (opts->wg_cols < 64 || opts->wg_cols > 512 || (opts->wg_cols & (opts->wg_cols - 1))))
        fail(SRBCRS_EINVAL, "wg_cols must be 0 or a power of two in [64, 512] (got %d)", opts->wg_cols);
      if (opts->grid_order < 0 || opts->grid_order > 5)
        fail(SRBCRS_EINVAL, "grid_order must be 0, 1, 2, 3, 4 or 5 (got %d)", opts->grid_order);
      if (opts->depth) ro.depth = opts->depth;
      if (opts->wg_cols) ro.wg_cols = opts->wg_cols;
      if (opts->grid_order)
        ro.chunk_major = opts->grid_order == SRBCRS_GRID_CHUNK_MAJOR ? 1
                         : opts->grid_order == SRBCRS_GRID_CHUNK_SWEEP ? 2 : 0;
      if (opts->windows_per_wave < 0 || opts->windows_per_wave > 4096)
        fail(SRBCRS_EINVAL, "windows_per_wave must be in [0, 4096] (got %d)", opts->windows_per_wave);
      ro.windows_per_wave = opts->windows_per_wave ? opts->windows_per_wave : 1;
      if (opts->tile_b) max_vec = opts->tile_b / 16;
      if (opts->a_operand < 0 || opts->a_operand > 2)
        fail(SRBCRS_EINVAL, "a_operand must be 0, 1 or 2 (got %d)", opts->a_operand);
      if (opts->b_stage < 0 || opts->b_stage > 2)
        fail(SRBCRS_EINVAL, "b_stage must be 0, 1 or 2 (got %d)", opts->b_stage);
      ro.b_lds = opts->b_stage == SRBCRS_B_LDS;
      if (opts->epilogue != SRBCRS_EPILOGUE_NONE && opts->epilogue != SRBCRS_EPILOGUE_RELU)
        fail(SRBCRS_EINVAL, "epilogue must be 0 (none) or 1 (relu) (got %d)", opts->epilogue);
    }
    if (!plan) fail(SRBCRS_EINVAL, "plan is NULL");
    if (opts && opts->a_operand == SRBCRS_A_COMPACT && !plan->d_awords && plan->total > 0)
      fail(SRBCRS_ESTATE, "the plan has no compact copy of its block values");
    {
      // default: for 16x8 blocks, the compact copy when at most half of the
      // block positions hold values (it skips the zeros; at full blocks it
      // only adds the mask words and the decode: banded, fill 1.0, runs 13 %
      // slower on it).  32x32 blocks read the dense array: their two 16-row
      // halves decode separate words for one B fragment, and compact lost on
      // every workload measured (uniform 0.42 vs 0.38 ms at 3 % fill)
      const int a_op = opts ? opts->a_operand : SRBCRS_A_DEFAULT;
      const bool sparse_blocks = 2 * plan->n_apacked <= plan->total * (int64_t)plan->blk_h * plan->blk_w;
      ro.a_compact = a_op == SRBCRS_A_COMPACT || (a_op == SRBCRS_A_DEFAULT && sparse_blocks && plan->blk_h == 16);
    }
    int cur = 0;
    hip_check(hipGetDevice(&cur), "hipGetDevice");
    if (cur != plan->device) fail(SRBCRS_ESTATE, "plan lives on device %d, current device is %d", plan->device, cur);
    if (N < 0 || N > INT32_MAX) fail(SRBCRS_EINVAL, "N out of range");
    if (N == 0) return;
    if (N % 16 != 0)
      fail(SRBCRS_EINVAL, "SR-BCRS requires dense feature dim divisible by 16/32/64, got %lld. Please pad feature dim before run.", (long long)N);
    if (!d_B || !d_C) fail(SRBCRS_EINVAL, "B / C is NULL");
    if (K <= plan->max_col)
      fail(SRBCRS_EINVAL, "dense has %lld rows but the matrix references column %d", (long long)K, plan->max_col);
    if (ldb < N || ldc < N) fail(SRBCRS_EINVAL, "ldb / ldc must be >= N");
    if (c_rows < plan->num_nodes) fail(SRBCRS_EINVAL, "C has %lld rows, need %d", (long long)c_rows, plan->num_nodes);
    if ((reinterpret_cast<uintptr_t>(d_B) | reinterpret_cast<uintptr_t>(d_C)) % 4)
      fail(SRBCRS_EINVAL, "B / C must be 4-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // vector width: the widest of 4/2/1 that N, ldb, ldc and the pointers allow
    int vec = max_vec;
    while (vec > 1 && ((N % (16 * vec)) || (ldb % vec) || (ldc % vec) ||
                       (reinterpret_cast<uintptr_t>(d_B) % (4 * vec)) ||
                       (reinterpret_cast<uintptr_t>(d_C) % (4 * vec))))
      vec /= 2;
    srbcrs::StreamArgs a{d_B, d_C, nullptr, plan->d_sidx, plan->d_val, (int)plan->packed_rows, (int)N, ldb, ldc,
                         plan->blk_h, plan->d_rowmap, plan->d_awords, plan->d_apacked,
                         opts && opts->epilogue == SRBCRS_EPILOGUE_RELU ? 1 : 0};
    // Everything that can refuse the call, and every allocation, comes before
    // the first launch: a refused call leaves C untouched.
    const bool merged = opts && opts->grid_order == SRBCRS_GRID_MERGED;
    if (merged) {
      // merged defaults (knobs left 0): 64-column waves with 8 windows, or 4
      // windows at 128 columns; depth 2
      const int cols = opts->wg_cols ? opts->wg_cols : 64;
      const int W = opts->windows_per_wave ? opts->windows_per_wave : (cols == 64 ? 8 : 4);
      if (plan->sched.policy != "row") fail(SRBCRS_EINVAL, "the merged-window grid runs the \"row\" schedule only");
      if (plan->blk_h != 16 || (!plan->d_awords && plan->total > 0))
        fail(SRBCRS_EINVAL, "the merged-window grid needs 16x8 blocks with the compact copy of the block values");
      if (opts->a_operand == SRBCRS_A_DENSE || opts->b_stage == SRBCRS_B_LDS)
        fail(SRBCRS_EINVAL, "the merged-window grid reads the compact A copy and keeps B in registers");
      if (cols != 64 && cols != 128) fail(SRBCRS_EINVAL, "the merged-window grid takes wg_cols 64 or 128");
      if (ro.depth != 2 && ro.depth != 4) fail(SRBCRS_EINVAL, "the merged-window grid takes depth 2 or 4");
      if (W != 4 && W != 8) fail(SRBCRS_EINVAL, "the merged-window grid takes windows_per_wave 4 or 8");
      if (!srbcrs::merged_setting_ok(cols, W, ro.depth))
        fail(SRBCRS_EINVAL, "the merged-window grid runs 8 windows per wave only at wg_cols 64 and depth 2");
      if (vec != 4) fail(SRBCRS_EINVAL, "the merged-window grid needs N, ldb, ldc multiples of 64 / 4 / 4 and "
                                        "16-byte aligned B and C");
      if (!srbcrs::merged_chunks_ok((int)(N / cols)))
        fail(SRBCRS_EINVAL, "the merged-window grid needs N / %d column chunks to divide 8 or be a multiple of 8", cols);
      if (fixed_partial && !plan->merged.count(W))
        fail(SRBCRS_EINVAL, "the merged-window stream for %d windows is not built yet: call srbcrs_run_ex once with "
                            "these knobs first (it allocates)", W);
      const srbcrs_plan::Merged& m = merged_stream(*plan, W, st);
      if (plan->n_zero_rows)
        hip_check(srbcrs::launch_zero_rows(d_C, plan->d_zero_rows, plan->n_zero_rows, (int)N, ldc, st),
                  "launch zero_rows");
      srbcrs::MergedArgs ma{m.d_moff, plan->Mo, W, m.d_sidx, m.d_words};
      hip_check(srbcrs::launch_merged(ma, a, cols, ro.depth, st), "launch spmm_merged");
      return;
    }
    if (opts && opts->grid_order == SRBCRS_GRID_NZSWEEP) {
      // defaults (knobs left 0): 8 windows per group, sub-batches of 32
      // entries, 2 in flight
      const int W = opts->windows_per_wave ? opts->windows_per_wave : 8;
      const int U = opts->tile_b ? opts->tile_b : 32;
      const int D = opts->depth ? opts->depth : 2;
      if (plan->sched.policy != "row") fail(SRBCRS_EINVAL, "the nonzero sweep runs the \"row\" schedule only");
      if (plan->blk_h != 16 || (!plan->d_awords && plan->total > 0))
        fail(SRBCRS_EINVAL, "the nonzero sweep needs 16x8 blocks with the compact copy of the block values");
      if (opts->a_operand == SRBCRS_A_DENSE || opts->b_stage == SRBCRS_B_LDS)
        fail(SRBCRS_EINVAL, "the nonzero sweep reads the compact A copy and keeps B in registers");
      if (opts->wg_cols && opts->wg_cols != 64)
        fail(SRBCRS_EINVAL, "the nonzero sweep runs 64 columns per wave (got wg_cols %d)", opts->wg_cols);
      if (!srbcrs::nz_setting_ok(W, U, D))
        fail(SRBCRS_EINVAL, "the nonzero sweep takes windows_per_wave 4 or 8 and (tile_b, depth) (16, 2), (16, 4), "
                            "(32, 2), (32, 4) or (64, 2) (got %d, %d, %d)", W, U, D);
      if (N % 64) fail(SRBCRS_EINVAL, "the nonzero sweep needs N a multiple of 64 (got %lld)", (long long)N);
      if (N % 4 || ldb % 4 || ldc % 4 || (reinterpret_cast<uintptr_t>(d_B) | reinterpret_cast<uintptr_t>(d_C)) % 16)
        fail(SRBCRS_EINVAL, "the nonzero sweep needs ldb, ldc multiples of 4 and 16-byte aligned B and C");
      if ((uint64_t)K * (uint64_t)ldb * 4u >= (1ull << 32) || (uint64_t)ldb * 4u >= (1ull << 24))
        fail(SRBCRS_EINVAL, "the nonzero sweep addresses B with 32-bit offsets: K * ldb * 4 must stay below 2^32 "
                            "and ldb * 4 below 2^24");
      if (fixed_partial && !plan->nz.count(nz_key(W, U, D)))
        fail(SRBCRS_EINVAL, "the nonzero-sweep stream for %d windows and sub-batches of %d is not built yet: call "
                            "srbcrs_run_ex once with these knobs first (it allocates)", W, U);
      const srbcrs_plan::Nz& z = nz_stream(*plan, W, U, D, st);
      if (plan->n_zero_rows)
        hip_check(srbcrs::launch_zero_rows(d_C, plan->d_zero_rows, plan->n_zero_rows, (int)N, ldc, st),
                  "launch zero_rows");
      srbcrs::NzArgs za{z.d_eoff, plan->Mo, W, z.d_pairs};
      hip_check(srbcrs::launch_nzsweep(za, a, U, D, st), "launch spmm_nzsweep");
      return;
    }
    if (plan->sched.policy == "row") {
      if (plan->n_zero_rows)
        hip_check(srbcrs::launch_zero_rows(d_C, plan->d_zero_rows, plan->n_zero_rows, (int)N, ldc, st),
                  "launch zero_rows");
      hip_check(srbcrs::launch_row(a, plan->d_soff, plan->Mo, vec, ro, st), "launch spmm_stream(row)");
      return;
    }
    const Schedule& s = plan->sched;
    const size_t need = (size_t)s.n_slots * plan->blk_h * (size_t)ldc;
    float* partial = fixed_partial;
    if (fixed_partial) {
      if (need > fixed_cap)
        fail(SRBCRS_EINVAL,
             "the schedule's partial tiles need %zu floats (%d slots x %d rows x ldc %lld), above the "
             "%zu-float scratch of srbcrs_run_noalloc; use srbcrs_run_ex or a schedule with fewer slots",
             need, s.n_slots, plan->blk_h, (long long)ldc, fixed_cap);
    } else {
      if (need > plan->partial_cap) {
        // grow-only, geometrically (a plan whose N or ldc rises step by step
        // reallocates O(log) times); the old buffer is retired, not freed
        // (launches in flight and captured graphs keep a valid address), so
        // no stream sync here.  srbcrs_plan_trim frees retired buffers.
        const size_t cap = std::max(need, 2 * plan->partial_cap);
        float* grown = dev_alloc<float>(cap);
        plan->retire(plan->d_partial);
        plan->d_partial = grown;
        plan->partial_cap = cap;
      }
      partial = plan->d_partial;
    }
    a.partial = partial;
    if (plan->n_zero_rows)
      hip_check(srbcrs::launch_zero_rows(d_C, plan->d_zero_rows, plan->n_zero_rows, (int)N, ldc, st),
                "launch zero_rows");
    srbcrs::TaskTable tt{plan->d_group_off, plan->d_task_begin, plan->d_task_end, plan->d_task_window,
                         plan->d_task_slot, (int)s.group_off.size() - 1};
    hip_check(srbcrs::launch_tasks(a, tt, vec, ro, st), "launch spmm_stream(tasks)");
    srbcrs::ReduceArgs ra{partial, d_C, plan->d_red_window, plan->d_red_slot_off,
                          (int)s.red_window.size(), plan->blk_h, (int)plan->packed_rows, (int)N, ldc,
                          plan->d_rowmap, a.relu};
    hip_check(srbcrs::launch_reduce(ra, vec, st), "launch segment_reduce");
}

int srbcrs_run_ex(srbcrs_plan* plan, const float* d_B, int64_t K, int64_t N, int64_t ldb,
                  float* d_C, int64_t ldc, int64_t c_rows, const srbcrs_run_opts* opts,
                  void* stream) {
  return guarded([&] { run_impl(plan, d_B, K, N, ldb, d_C, ldc, c_rows, opts, stream, nullptr, 0); });
}

// ---- srbcrs_run_noalloc: partial tiles in a fixed device array ------------
//
// For callers that cannot allocate.  The split schedules' partial tiles go to
// `scratch`, a file-scope device array every GPU holds from the library's
// load until the process ends; nothing is allocated per call.  In host code
// `scratch` names a host-side stand-in, not device memory: its device address
// comes from hipGetSymbolAddress, once per device with that device current,
// and only that address is handed to kernels.  Calls on one GPU share the
// array (the last call's partial tiles stay in it); calls that overlap on one
// GPU race.  No clearing is needed: each partial slot is written whole by its
// task before the reduction reads it.
namespace {
constexpr size_t kNoallocScratchFloats = size_t(16) << 20;   // 64 MiB
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) float scratch[kNoallocScratchFloats];

namespace {
std::mutex g_scratch_mu;
float* g_scratch_addr[kMaxDevices] = {};

// The device address of `scratch` on the current device (looked up once per device).
static float* noalloc_scratch() {
  int dev = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) fail(SRBCRS_ESTATE, "device %d beyond the %d the library tracks", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* addr = nullptr;
    hip_check(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!addr) fail(SRBCRS_EHIP, "hipGetSymbolAddress returned no address for the scratch array");
    g_scratch_addr[dev] = static_cast<float*>(addr);
  }
  return g_scratch_addr[dev];
}
}  // namespace

int srbcrs_run_noalloc(srbcrs_plan* plan, const float* d_B, int64_t K, int64_t N, int64_t ldb, float* d_C,
                       int64_t ldc, int64_t c_rows, const srbcrs_run_opts* opts, void* stream) {
  return guarded([&] {
    float* partial = noalloc_scratch();
    run_impl(plan, d_B, K, N, ldb, d_C, ldc, c_rows, opts, stream, partial, kNoallocScratchFloats);
  });
}

size_t srbcrs_noalloc_scratch_floats(void) { return kNoallocScratchFloats; }

int srbcrs_plan_trim(srbcrs_plan* plan, void* stream) {
  return guarded([&] {
    if (!plan) fail(SRBCRS_EINVAL, "plan is NULL");
    int cur = 0;
    hip_check(hipGetDevice(&cur), "hipGetDevice");
    if (cur != plan->device) fail(SRBCRS_ESTATE, "plan lives on device %d, current device is %d", plan->device, cur);
    // every launch that could still read a retired buffer was queued on this
    // stream (or on work the caller has already waited for)
    hip_check(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
    for (void* p : plan->retired) (void)hipFree(p);
    plan->retired.clear();
  });
}

int srbcrs_stream_probe(int32_t kind, const float* d_a, float* d_b, int64_t n_floats, int32_t blocks,
                        void* stream) {
  return guarded([&] {
    if (kind < 0 || kind > 2) fail(SRBCRS_EINVAL, "kind must be 0 (copy), 1 (read) or 2 (write)");
    if (n_floats < 0 || n_floats % 4) fail(SRBCRS_EINVAL, "n_floats must be a non-negative multiple of 4");
    if (blocks < 1 || blocks > (1 << 20)) fail(SRBCRS_EINVAL, "blocks must be in [1, 2^20]");
    if ((kind != 2 && !d_a) || !d_b) fail(SRBCRS_EINVAL, "buffer is NULL");
    if ((reinterpret_cast<uintptr_t>(d_a) | reinterpret_cast<uintptr_t>(d_b)) % 16)
      fail(SRBCRS_EINVAL, "buffers must be 16-byte aligned");
    hip_check(srbcrs::launch_stream_probe(kind, d_a, d_b, n_floats / 4, blocks, static_cast<hipStream_t>(stream)),
              "launch stream probe");
  });
}

int srbcrs_gather_probe(const int32_t* d_rows, const int64_t* d_row_off, int32_t n_groups, int32_t rows_per_instr,
                        const float* d_B, int64_t ldb, int32_t n_chunks, int32_t mapping, float* d_out,
                        void* stream) {
  return guarded([&] {
    if (rows_per_instr != 1 && rows_per_instr != 2 && rows_per_instr != 4 && rows_per_instr != 8)
      fail(SRBCRS_EINVAL, "rows_per_instr must be 1, 2, 4 or 8");
    if (n_groups < 0 || n_chunks < 1) fail(SRBCRS_EINVAL, "n_groups must be >= 0 and n_chunks >= 1");
    if (mapping < 0 || mapping > 2) fail(SRBCRS_EINVAL, "mapping must be 0, 1 or 2");
    if (mapping == 2 && 8 % n_chunks) fail(SRBCRS_EINVAL, "XCD-affine chunks need n_chunks to divide 8");
    if (ldb < (int64_t)n_chunks * (256 / rows_per_instr) || ldb % 4)
      fail(SRBCRS_EINVAL, "ldb must be a multiple of 4 covering n_chunks row segments");
    if (!d_rows || !d_row_off || !d_B || !d_out) fail(SRBCRS_EINVAL, "buffer is NULL");
    if (reinterpret_cast<uintptr_t>(d_B) % 16) fail(SRBCRS_EINVAL, "B must be 16-byte aligned");
    hip_check(srbcrs::launch_gather_probe(d_rows, d_row_off, n_groups, rows_per_instr, d_B, ldb, n_chunks, mapping,
                                          d_out, static_cast<hipStream_t>(stream)),
              "launch gather probe");
  });
}

int srbcrs_plan_tune(srbcrs_plan* plan, const float* d_B, int64_t K, int64_t N, int64_t ldb, float* d_C,
                     int64_t ldc, int64_t c_rows, int32_t reps, srbcrs_run_opts* best, void* stream) {
  return srbcrs_plan_tune_ex(plan, d_B, K, N, ldb, d_C, ldc, c_rows, reps, 0, best, stream);
}

int srbcrs_plan_tune_ex(srbcrs_plan* plan, const float* d_B, int64_t K, int64_t N, int64_t ldb, float* d_C,
                        int64_t ldc, int64_t c_rows, int32_t reps, int32_t flags, srbcrs_run_opts* best,
                        void* stream) {
  if (!plan) return guarded([] { fail(SRBCRS_EINVAL, "plan is NULL"); });
  if (reps < 1 || reps > 100) return guarded([&] { fail(SRBCRS_EINVAL, "reps must be in [1, 100] (got %d)", reps); });
  if (flags & ~SRBCRS_TUNE_NONZERO_SWEEP)
    return guarded([&] { fail(SRBCRS_EINVAL, "unknown tune flags 0x%x", (unsigned)flags); });
  hipStream_t st = static_cast<hipStream_t>(stream);
  plan->tuned.erase(N);
  std::vector<srbcrs_run_opts> cand, merged_cand;
  // block fill decides the A source outright at the extremes (measured: compact wins by 14-20 %
  // at 6 % fill, dense by 13 % at 100 %), so only the middle band times both
  const int64_t positions = plan->total * (int64_t)plan->blk_h * plan->blk_w;
  // (16x8; 32x32 blocks time only the dense source, see srbcrs_run_ex)
  const bool wide = plan->blk_h == 32;
  const bool mostly_empty = !wide && plan->d_awords && 4 * plan->n_apacked < positions;
  const bool mostly_full = 4 * plan->n_apacked > 3 * positions;
  for (int32_t a : {SRBCRS_A_COMPACT, SRBCRS_A_DENSE}) {
    if (a == SRBCRS_A_COMPACT && (!plan->d_awords || mostly_full || wide)) continue;
    if (a == SRBCRS_A_DENSE && mostly_empty) continue;
    for (int32_t order : {SRBCRS_GRID_CHUNK_MAJOR, SRBCRS_GRID_CHUNK_SWEEP})
      for (int32_t wg : {128, 64, 256})
        for (int32_t depth : {2, 4}) {
          // 256: for 32x32 two 128-column waves, for 16x8 one 256-column wave
          srbcrs_run_opts o{};
          o.depth = depth;
          o.wg_cols = wg;
          o.grid_order = order;
          o.a_operand = a;
          cand.push_back(o);
        }
    if (!wide)
      // B staged through LDS by direct-to-LDS loads, 64-column waves in the
      // chunk sweep: its registers stay few enough for 5 waves per SIMD
      // (measured 1.5-3 % ahead of the register ring on R-MAT)
      for (int32_t depth : {2, 4}) {
        srbcrs_run_opts o{};
        o.depth = depth;
        o.wg_cols = 64;
        o.grid_order = SRBCRS_GRID_CHUNK_SWEEP;
        o.a_operand = a;
        o.b_stage = SRBCRS_B_LDS;
        cand.push_back(o);
      }
    if (plan->sched.policy == "row" && a == SRBCRS_A_COMPACT && plan->blk_h == 16)
      // merged windows: each wave walks 4 or 8 windows' blocks interleaved,
      // its column chunk pinned to one XCD (runs only where N, the leading
      // dimensions and alignment allow it; others are skipped below)
      for (const auto& mw : {std::array<int32_t, 3>{128, 4, 4}, std::array<int32_t, 3>{128, 4, 2},
                             std::array<int32_t, 3>{64, 8, 2}, std::array<int32_t, 3>{64, 4, 4}})
        if (N % mw[0] == 0 && srbcrs::merged_chunks_ok((int)(N / mw[0]))) {
          srbcrs_run_opts o{};
          o.wg_cols = mw[0];
          o.windows_per_wave = mw[1];
          o.depth = mw[2];
          o.grid_order = SRBCRS_GRID_MERGED;
          o.a_operand = a;
          merged_cand.push_back(o);
        }
    if (plan->sched.policy == "row")
      // several consecutive windows per wave: fewer waves than resident
      // slots, all sweeping their windows' columns in step
      for (int32_t wg : {128, 256})
        for (int32_t wpw : {4, 8})
          for (int32_t depth : {2, 4, 8}) {
            srbcrs_run_opts o{};
            o.depth = depth;
            o.wg_cols = wg;
            o.grid_order = SRBCRS_GRID_CHUNK_MAJOR;
            o.windows_per_wave = wpw;
            o.a_operand = a;
            cand.push_back(o);
          }
  }
  if ((flags & SRBCRS_TUNE_NONZERO_SWEEP) && plan->sched.policy == "row" && plan->blk_h == 16 && plan->d_awords)
    // the nonzero sweep (its bits are the fp32 CSR product's): (windows, values
    // per sub-batch, sub-batches in flight)
    for (const auto& nz : {std::array<int32_t, 3>{8, 32, 2}, std::array<int32_t, 3>{4, 16, 2},
                           std::array<int32_t, 3>{4, 16, 4}, std::array<int32_t, 3>{8, 32, 4}}) {
      srbcrs_run_opts o{};
      o.windows_per_wave = nz[0];
      o.wg_cols = 64;
      o.tile_b = nz[1];
      o.depth = nz[2];
      o.grid_order = SRBCRS_GRID_NZSWEEP;
      o.a_operand = SRBCRS_A_COMPACT;
      merged_cand.push_back(o);
    }
  // merged-window and nonzero-sweep candidates last (a near-tie keeps the
  // plainer setting); one the operands cannot run (N, B / C alignment, ldb /
  // ldc, B's extent) is dropped here
  const size_t n_plain = cand.size();
  cand.insert(cand.end(), merged_cand.begin(), merged_cand.end());
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = guarded([&] {
    hip_check(hipEventCreate(&e0), "hipEventCreate");
    hip_check(hipEventCreate(&e1), "hipEventCreate");
  });
  std::vector<float> ms_of(cand.size(), -1.f);
  for (size_t i = 0; rc == SRBCRS_OK && i < cand.size(); ++i) {
    rc = srbcrs_run_ex(plan, d_B, K, N, ldb, d_C, ldc, c_rows, &cand[i], stream);   // warm-up, validates
    if (rc == SRBCRS_EINVAL && i >= n_plain) {   // a merged / sweep setting these operands cannot run
      rc = SRBCRS_OK;
      continue;
    }
    if (rc != SRBCRS_OK) break;
    rc = guarded([&] { hip_check(hipEventRecord(e0, st), "hipEventRecord"); });
    for (int r = 0; rc == SRBCRS_OK && r < reps; ++r)
      rc = srbcrs_run_ex(plan, d_B, K, N, ldb, d_C, ldc, c_rows, &cand[i], stream);
    if (rc != SRBCRS_OK) break;
    float ms = 0.f;
    rc = guarded([&] {
      hip_check(hipEventRecord(e1, st), "hipEventRecord");
      hip_check(hipEventSynchronize(e1), "hipEventSynchronize");
      hip_check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    });
    if (rc == SRBCRS_OK) ms_of[i] = ms;
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (rc != SRBCRS_OK) return rc;
  // the first candidate (the list runs from the plainest setting up) within
  // 3 % of the fastest: near-ties resolve the same way on every run and box
  float best_ms = -1.f;
  for (float ms : ms_of)
    if (ms >= 0.f && (best_ms < 0.f || ms < best_ms)) best_ms = ms;
  srbcrs_run_opts best_o{};
  for (size_t i = 0; i < cand.size(); ++i)
    if (ms_of[i] >= 0.f && ms_of[i] <= best_ms * 1.03f) {
      best_o = cand[i];
      break;
    }
  if (best_ms >= 0.f) plan->tuned[N] = best_o;
  if (best) *best = best_o;
  return SRBCRS_OK;
}

int srbcrs_shard_windows(const int32_t* soff, int32_t row_windows, int32_t n_shards, int32_t* bounds) {
  return guarded([&] {
    if (!soff || !bounds) fail(SRBCRS_EINVAL, "soff / bounds is NULL");
    if (row_windows < 0) fail(SRBCRS_EINVAL, "row_windows must be >= 0");
    if (n_shards < 1) fail(SRBCRS_EINVAL, "n_shards must be >= 1");
    for (int32_t w = 0; w < row_windows; ++w)
      if (soff[w + 1] < soff[w]) fail(SRBCRS_EINVAL, "soff must be non-decreasing");
    // cost of a window = its blocks + 1 (the output tile it writes): shard s
    // ends at the first window boundary whose prefix cost reaches
    // (s+1)/n_shards of the total
    const int64_t total = (int64_t)(soff[row_windows] - soff[0]) + row_windows;
    bounds[0] = 0;
    int32_t w = 0;
    for (int32_t sh = 1; sh < n_shards; ++sh) {
      const int64_t target = (total * sh + n_shards - 1) / n_shards;
      while (w < row_windows && (int64_t)(soff[w] - soff[0]) + w < target) ++w;
      bounds[sh] = w;
    }
    bounds[n_shards] = row_windows;
  });
}

int srbcrs_csr_spmm(const int32_t* d_rowptr, const int32_t* d_colind, const float* d_values,
                    int32_t M, int64_t nnz, int32_t max_col, const float* d_B, int64_t K, int64_t N,
                    int64_t ldb, float* d_C, int64_t ldc, void* stream) {
  return guarded([&] {
    if (M < 0) fail(SRBCRS_EINVAL, "M must be >= 0");
    if (N < 0 || N > INT32_MAX) fail(SRBCRS_EINVAL, "N out of range");
    if (M == 0 || N == 0) return;
    if (!d_rowptr || !d_B || !d_C) fail(SRBCRS_EINVAL, "NULL pointer");
    if (nnz > 0 && (!d_colind || !d_values)) fail(SRBCRS_EINVAL, "NULL colind / values");
    if (nnz > 0 && (max_col < 0 || max_col >= K))
      fail(SRBCRS_EINVAL, "max_col %d out of range for dense with %lld rows", max_col, (long long)K);
    if (ldb < N || ldc < N) fail(SRBCRS_EINVAL, "ldb / ldc must be >= N");
    int vec = 4;
    while (vec > 1 && ((N % (64 * vec)) || (ldb % vec) || (ldc % vec) ||
                       (reinterpret_cast<uintptr_t>(d_B) % (4 * vec)) ||
                       (reinterpret_cast<uintptr_t>(d_C) % (4 * vec))))
      vec /= 2;
    srbcrs::CsrArgs a{d_rowptr, d_colind, d_values, d_B, d_C, M, (int)N, ldb, ldc};
    hip_check(srbcrs::launch_csr(a, vec, static_cast<hipStream_t>(stream)), "launch csr_spmm_rowwave");
  });
}

}  // extern "C"
