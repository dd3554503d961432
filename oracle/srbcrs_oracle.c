/*
 * srbcrs_oracle.c -- CPU restatement of the reference's SR-BCRS path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the parity tests,
 * `__graft_entry__.smoke()` and bench.py's `cpu_baseline` leg compare the
 * product against.  The product library (mask_amd/csrc) never links, loads or
 * calls it, and nothing here is ever the thing that is measured as the
 * product.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the reference repository root:
 *   SRK = examples/src_fp32/sr_bcrs/testbed/SRBCRSSpMM_kernel.cu
 *   SLB = examples/src_fp32/sr_bcrs/testbed/main_strict_lb_16x8.cu
 *   MBD = examples/src_fp32/sr_bcrs/testbed/main_multi_bind_16x8.cu
 *   CFE = examples/src_fp32/acc/testbed/custom_format_e2e.cu
 *   SWZ = examples/src_fp32/csr_tcf/testbed/cutlass/include/cute/swizzle.hpp
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   oracle_swizzle         generic Swizzle<B,M,S> bit definition re-derived in
 *                          the test, bijection, hand values
 *   oracle_convert_*       hand-computed known answers, dense re-assembly,
 *                          structural invariants, brute force on tiny inputs
 *   oracle_csr_spmm_f64    numpy dense matmul on tiny inputs, identity / ones
 *                          special cases
 *   oracle_csr_spmm_f32    fp64 result within the fp32 accumulation bound
 *   oracle_strict_lb       hand-computed partitions + invariants
 *   oracle_multi_bind      hand-computed partitions + invariants
 *   oracle_segment_auto    hand-computed thresholds (p95, heavy-tail rule)
 *   oracle_segment_reduce  numpy sum over segments
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* CuTe Swizzle<2,2,3> (SWZ:55-79): yyy_msk = 0b11 << (2+3) = 0x60, shift 3,
 * offset ^ ((offset & yyy_msk) >> 3).  Applied to the row-major 16x8 (or
 * 32x32) block offset r*blk_w + c, as composed in SRK:227-229 / SRK:286-288. */
int oracle_swizzle(int offset) { return offset ^ ((offset & 0x60) >> 3); }

static int cmp_int(const void *a, const void *b) {
  int x = *(const int *)a, y = *(const int *)b;
  return (x > y) - (x < y);
}

/* lower_bound + equality, as find_condensed (SRK:107-113). */
static int find_condensed(const int *cols, int n, int target) {
  int lo = 0, hi = n;
  while (lo < hi) {
    int mid = lo + (hi - lo) / 2;
    if (cols[mid] < target) lo = mid + 1; else hi = mid;
  }
  if (lo == n || cols[lo] != target) return -1;
  return lo;
}

/* Collect the sorted unique columns of window w (SRK:236-250).  Returns the
 * count; *buf is grown as needed. */
static int window_unique_cols(const int *rowptr, const int *colind, int num_nodes,
                              int blk_h, int w, int **buf, int64_t *cap) {
  int64_t n = 0;
  for (int ir = 0; ir < blk_h; ++ir) {
    int64_t row = (int64_t)w * blk_h + ir;
    if (row >= num_nodes) continue;
    for (int e = rowptr[row]; e < rowptr[row + 1]; ++e) {
      if (n >= *cap) {
        *cap = (*cap < 256 ? 256 : *cap * 2);
        *buf = (int *)realloc(*buf, (size_t)(*cap) * sizeof(int));
      }
      (*buf)[n++] = colind[e];
    }
  }
  if (n == 0) return 0;
  qsort(*buf, (size_t)n, sizeof(int), cmp_int);
  int64_t u = 1;
  for (int64_t i = 1; i < n; ++i)
    if ((*buf)[i] != (*buf)[u - 1]) (*buf)[u++] = (*buf)[i];
  return (int)u;
}

/* Pass 1 of the conversion: per-window block counts and their prefix sum
 * (SRK:234-254 `tcblock_num`, `val_soff`).  soff has Mo+1 entries.
 * Returns the total block count. */
int64_t oracle_convert_count(const int *rowptr, const int *colind, int num_nodes,
                             int blk_h, int blk_w, int *soff) {
  int Mo = (num_nodes + blk_h - 1) / blk_h;
  int *buf = NULL;
  int64_t cap = 0, total = 0;
  for (int w = 0; w < Mo; ++w) {
    soff[w] = (int)total;
    int u = window_unique_cols(rowptr, colind, num_nodes, blk_h, w, &buf, &cap);
    total += (u + blk_w - 1) / blk_w;
  }
  soff[Mo] = (int)total;
  free(buf);
  return total;
}

/* Pass 2: sidx (padded with the window's last column, SRK:256-260), values
 * scattered into the swizzled block layout with the last write winning for
 * duplicate (row, col) pairs (SRK:265-279), block_partition (SRK:253),
 * edge_to_row (SRK:243) and edge_to_col = condensed position (SRK:271).
 * sidx has blk_w*total entries, val blk_h*blk_w*total (zero-filled here). */
void oracle_convert_fill(const int *rowptr, const int *colind, const float *values,
                         int num_nodes, int blk_h, int blk_w, const int *soff,
                         int *sidx, float *val, int *block_partition,
                         int *edge_to_row, int *edge_to_col) {
  int Mo = (num_nodes + blk_h - 1) / blk_h;
  int *buf = NULL;
  int64_t cap = 0;
  const int64_t bsz = (int64_t)blk_h * blk_w;
  memset(val, 0, sizeof(float) * (size_t)(bsz * soff[Mo]));
  for (int w = 0; w < Mo; ++w) {
    int u = window_unique_cols(rowptr, colind, num_nodes, blk_h, w, &buf, &cap);
    int nb = (u + blk_w - 1) / blk_w;
    if (block_partition) block_partition[w] = nb;
    int64_t sbase = (int64_t)soff[w] * blk_w;
    for (int64_t i = 0; i < (int64_t)nb * blk_w; ++i)
      sidx[sbase + i] = (i < u) ? buf[i] : buf[u - 1];
    int64_t vbase = (int64_t)soff[w] * bsz;
    for (int ir = 0; ir < blk_h; ++ir) {
      int64_t row = (int64_t)w * blk_h + ir;
      if (row >= num_nodes) continue;
      for (int e = rowptr[row]; e < rowptr[row + 1]; ++e) {
        int cpos = find_condensed(buf, u, colind[e]);
        if (edge_to_row) edge_to_row[e] = (int)row;
        if (edge_to_col) edge_to_col[e] = cpos;
        int blk = cpos / blk_w;
        int o = ir * blk_w + (cpos % blk_w);
        val[vbase + (int64_t)blk * bsz + oracle_swizzle(o)] = values[e];
      }
    }
  }
  free(buf);
}

/* Textbook CSR SpMM in fp64: C64[r, :] = sum_e val[e] * B[col[e], :].  The
 * oracle the north star's error bound is stated against.  If absC is non-NULL
 * it also receives (|A| |B|)[r, :], the scale of the elementwise bound. */
void oracle_csr_spmm_f64(const int *rowptr, const int *colind, const float *values,
                         const float *B, int M, int N, double *C, double *absC) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int r = 0; r < M; ++r) {
    double *c = C + (int64_t)r * N;
    double *a = absC ? absC + (int64_t)r * N : NULL;
    for (int j = 0; j < N; ++j) c[j] = 0.0;
    if (a) for (int j = 0; j < N; ++j) a[j] = 0.0;
    for (int e = rowptr[r]; e < rowptr[r + 1]; ++e) {
      const float *b = B + (int64_t)colind[e] * N;
      double v = values[e];
      for (int j = 0; j < N; ++j) c[j] += v * (double)b[j];
      if (a) for (int j = 0; j < N; ++j) a[j] += fabs(v) * fabs((double)b[j]);
    }
  }
}

/* CPU CSR SpMM in fp32, edge-ordered accumulation: the math of
 * csr_spmm_value_kernel (SRK:66-87) as a row-parallel CPU loop.  This is the
 * timed CPU baseline.  nthreads <= 0 uses the OpenMP default. */
void oracle_csr_spmm_f32(const int *rowptr, const int *colind, const float *values,
                         const float *B, int M, int N, float *C, int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
#pragma omp parallel for schedule(dynamic, 64)
  for (int r = 0; r < M; ++r) {
    float *c = C + (int64_t)r * N;
    for (int j = 0; j < N; ++j) c[j] = 0.0f;
    for (int e = rowptr[r]; e < rowptr[r + 1]; ++e) {
      const float *b = B + (int64_t)colind[e] * N;
      float v = values[e];
      for (int j = 0; j < N; ++j) c[j] += v * b[j];
    }
  }
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* strict_load_balance (SLB:208-256): walk the windows in order and cut their
 * block lists into fragments so that every thread block gets exactly
 * `workload` blocks (the last may get fewer).  Outputs:
 *   frag_begin[nf+1]  first block of each fragment (+ total at the end)
 *   frag_window[nf]   owning window of each fragment
 *   group_off[ng+1]   fragment offsets of each thread-block group
 * Capacities: frag arrays >= Mo + total/workload + 2, group_off likewise.
 * Returns nf; *ng receives the group count. */
int oracle_strict_lb(int Mo, int total, const int *soff, int workload,
                     int *frag_begin, int *frag_window, int *group_off, int *ng) {
  int nf = 0, g = 0, cur = 0;
  group_off[g++] = 0;
  for (int w = 0; w < Mo; ++w) {
    int start = soff[w], end = soff[w + 1];
    while (start < end) {
      int cap = workload - cur;
      int take = (cap < end - start) ? cap : end - start;
      frag_begin[nf] = start;
      frag_window[nf] = w;
      ++nf;
      start += take;
      cur += take;
      if (cur == workload) { group_off[g++] = nf; cur = 0; }
    }
  }
  frag_begin[nf] = total;
  if (cur != 0 || g == 1) group_off[g++] = nf;
  *ng = g - 1;
  return nf;
}

/* multi_binding_load_balance (MBD:211-270), alpha = 2, max_splits = 9999:
 * windows with x > 2*avg blocks are split into ceil(x/avg) near-equal parts
 * (first x%parts parts one larger); empty windows are dropped.  Outputs:
 *   part_window[np]   owning window of each part
 *   part_off[np+1]    prefix sum of part sizes (ends at total)
 *   window_split[Mo]  1 where the window was split
 * Returns np. */
int oracle_multi_bind(int Mo, const int *soff, int *part_window, int *part_off,
                      int *window_split) {
  double avg = 0.0;
  for (int w = 0; w < Mo; ++w) avg += (double)(soff[w + 1] - soff[w]);
  if (Mo > 0) avg /= (double)Mo;
  int np = 0;
  part_off[0] = 0;
  for (int w = 0; w < Mo; ++w) {
    window_split[w] = 0;
    int x = soff[w + 1] - soff[w];
    if (x == 0) continue;
    int parts = 1;
    if (avg > 0.0 && x > 2.0 * avg) {
      double p = ceil((double)x / avg);
      parts = p > 9999.0 ? 9999 : (int)p;
      if (parts < 1) parts = 1;
      if (parts > 1) window_split[w] = 1;
    }
    int base = x / parts, rem = x % parts;
    for (int i = 0; i < parts; ++i) {
      part_window[np] = w;
      part_off[np + 1] = part_off[np] + base + (i < rem ? 1 : 0);
      ++np;
    }
  }
  return np;
}

/* Automatic execution segmentation (CFE:640-699): p95 of the window lengths
 * (sorted, index min(n-1, ceil(0.95 n) - 1)), heavy tail when
 * max > max(64, 4*max(p95,1)); the cap is then max(32, min(128, 2*p95)),
 * else max(max_len, 1).  requested > 0 overrides the cap.  Each non-empty
 * window is cut into ceil(len/cap) segments of at most cap blocks; an empty
 * window keeps one empty segment.  Outputs seg_end[nseg] (absolute block end
 * of each segment; its begin is the previous end) and win_seg_off[Mo+1].
 * Returns nseg; *cap_out and *heavy_out receive the cap and the heavy flag. */
int oracle_segment_auto(int Mo, const int *soff, int requested, int *seg_end,
                        int *win_seg_off, int *cap_out, int *heavy_out) {
  int maxlen = 0;
  int *lens = (int *)malloc(sizeof(int) * (size_t)(Mo > 0 ? Mo : 1));
  for (int w = 0; w < Mo; ++w) {
    lens[w] = soff[w + 1] - soff[w];
    if (lens[w] > maxlen) maxlen = lens[w];
  }
  int p95 = 0;
  if (Mo > 0) {
    qsort(lens, (size_t)Mo, sizeof(int), cmp_int);
    int64_t idx = (int64_t)ceil(Mo * 0.95) - 1;
    if (idx > Mo - 1) idx = Mo - 1;
    if (idx < 0) idx = 0;
    p95 = lens[idx];
  }
  free(lens);
  int heavy = 0, cap;
  if (requested == 0) {
    int p = p95 > 1 ? p95 : 1;
    int thr = 4 * p > 64 ? 4 * p : 64;
    heavy = maxlen > thr;
    if (heavy) {
      int c = 2 * p95 < 128 ? 2 * p95 : 128;
      cap = c > 32 ? c : 32;
    } else {
      cap = maxlen > 1 ? maxlen : 1;
    }
  } else {
    cap = requested;
  }
  int nseg = 0;
  win_seg_off[0] = 0;
  for (int w = 0; w < Mo; ++w) {
    int b = soff[w], e = soff[w + 1];
    if (b == e) {
      seg_end[nseg++] = e;
    } else {
      for (int t = b; t < e; t += cap) seg_end[nseg++] = (t + cap < e) ? t + cap : e;
    }
    win_seg_off[w + 1] = nseg;
  }
  *cap_out = cap;
  *heavy_out = heavy;
  return nseg;
}

/* reduce_tcf_segments (CFE:832-853): out[w] = sum over the window's segments
 * (in segment order) of their 16 x N partial tiles.  fp32, fixed order. */
void oracle_segment_reduce(const float *partial, float *out, const int *win_seg_off,
                           int Mo, int tile_rows, int N) {
  int64_t te = (int64_t)tile_rows * N;
  for (int w = 0; w < Mo; ++w)
    for (int64_t i = 0; i < te; ++i) {
      float s = 0.0f;
      for (int sg = win_seg_off[w]; sg < win_seg_off[w + 1]; ++sg)
        s += partial[(int64_t)sg * te + i];
      out[(int64_t)w * te + i] = s;
    }
}

/* ===== generated-operator packing (CFE = custom_format_e2e.cu) ============ */

static int cmp_key2(const void *a, const void *b) {
  const int64_t *x = (const int64_t *)a, *y = (const int64_t *)b;
  if (x[0] != y[0]) return (x[0] > y[0]) - (x[0] < y[0]);
  return (x[1] > y[1]) - (x[1] < y[1]);
}

/* first_structural_column (CFE:228-234): min column in [0,k), k if none. */
static int first_col(int row, int k, const int *rowptr, const int *colind) {
  int f = k;
  for (int p = rowptr[row]; p < rowptr[row + 1]; ++p)
    if (colind[p] >= 0 && colind[p] < k && colind[p] < f) f = colind[p];
  return f;
}

/* first_column_order (CFE:236-249): stable sort by (first column, row). */
void oracle_order_first_col(int m, int k, const int *rowptr, const int *colind, int *order) {
  int64_t *key = (int64_t *)malloc(sizeof(int64_t) * 2 * (size_t)(m > 0 ? m : 1));
  for (int r = 0; r < m; ++r) { key[2 * r] = first_col(r, k, rowptr, colind); key[2 * r + 1] = r; }
  qsort(key, (size_t)m, 2 * sizeof(int64_t), cmp_key2);
  for (int r = 0; r < m; ++r) order[r] = (int)key[2 * r + 1];
  free(key);
}

/* reverse_cuthill_mckee (CFE:163-226), square matrices: symmetrised
 * adjacency without self loops, degree = unique neighbours; components are
 * started from nodes in (degree, id) order; BFS appends each popped node's
 * unvisited neighbours in (degree, id) order; each component is reversed.
 * Returns 0, or -1 if m != k. */
int oracle_order_rcm(int m, int k, const int *rowptr, const int *colind, int *order) {
  if (m != k) return -1;
  int64_t ne = 0;
  for (int r = 0; r < m; ++r)
    for (int p = rowptr[r]; p < rowptr[r + 1]; ++p)
      if (colind[p] >= 0 && colind[p] < m && colind[p] != r) ne += 2;
  int64_t *pairs = (int64_t *)malloc(sizeof(int64_t) * 2 * (size_t)(ne > 0 ? ne : 1));
  int64_t q = 0;
  for (int r = 0; r < m; ++r)
    for (int p = rowptr[r]; p < rowptr[r + 1]; ++p) {
      int c = colind[p];
      if (c < 0 || c >= m || c == r) continue;
      pairs[2 * q] = r; pairs[2 * q + 1] = c; ++q;
      pairs[2 * q] = c; pairs[2 * q + 1] = r; ++q;
    }
  qsort(pairs, (size_t)ne, 2 * sizeof(int64_t), cmp_key2);
  int64_t *adj_off = (int64_t *)calloc((size_t)m + 1, sizeof(int64_t));
  int *adj = (int *)malloc(sizeof(int) * (size_t)(ne > 0 ? ne : 1));
  int64_t na = 0;
  for (int64_t i = 0; i < ne; ++i) {
    if (i > 0 && pairs[2 * i] == pairs[2 * i - 2] && pairs[2 * i + 1] == pairs[2 * i - 1]) continue;
    adj[na++] = (int)pairs[2 * i + 1];
    adj_off[pairs[2 * i] + 1]++;
  }
  for (int r = 0; r < m; ++r) adj_off[r + 1] += adj_off[r];
  int *deg = (int *)malloc(sizeof(int) * (size_t)(m > 0 ? m : 1));
  for (int r = 0; r < m; ++r) deg[r] = (int)(adj_off[r + 1] - adj_off[r]);
  int64_t *key = (int64_t *)malloc(sizeof(int64_t) * 2 * (size_t)(m > 0 ? m : 1));
  for (int r = 0; r < m; ++r) { key[2 * r] = deg[r]; key[2 * r + 1] = r; }
  qsort(key, (size_t)m, 2 * sizeof(int64_t), cmp_key2);
  unsigned char *vis = (unsigned char *)calloc((size_t)(m > 0 ? m : 1), 1);
  int *queue = (int *)malloc(sizeof(int) * (size_t)(m > 0 ? m : 1));
  int64_t *nk = (int64_t *)malloc(sizeof(int64_t) * 2 * (size_t)(m > 0 ? m : 1));
  int out = 0;
  for (int s = 0; s < m; ++s) {
    int start = (int)key[2 * s + 1];
    if (vis[start]) continue;
    int head = 0, tail = 0;
    vis[start] = 1;
    queue[tail++] = start;
    while (head < tail) {
      int row = queue[head++];
      int nn = 0;
      for (int64_t p = adj_off[row]; p < adj_off[row + 1]; ++p)
        if (!vis[adj[p]]) { nk[2 * nn] = deg[adj[p]]; nk[2 * nn + 1] = adj[p]; ++nn; }
      qsort(nk, (size_t)nn, 2 * sizeof(int64_t), cmp_key2);
      for (int i = 0; i < nn; ++i) {
        int v = (int)nk[2 * i + 1];
        if (!vis[v]) { vis[v] = 1; queue[tail++] = v; }
      }
    }
    for (int i = tail - 1; i >= 0; --i) order[out++] = queue[i];   /* reversed component */
  }
  free(pairs); free(adj_off); free(adj); free(deg); free(key); free(vis); free(queue); free(nk);
  return 0;
}

/* SplitMix64 finaliser (Steele, Lea & Flood 2014 / Vigna), the column hash
 * of mix_column (CFE:251-256). */
static uint64_t splitmix64(uint64_t v) {
  v += 0x9e3779b97f4a7c15ULL;
  v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ULL;
  v = (v ^ (v >> 27)) * 0x94d049bb133111ebULL;
  return v ^ (v >> 31);
}

/* row_jaccard (CFE:266-294): run-merge of the two rows' column lists in
 * storage order, counting distinct runs; 1.0 when both are empty. */
static double jaccard(int a, int b, const int *rowptr, const int *colind) {
  int l = rowptr[a], r = rowptr[b];
  const int le = rowptr[a + 1], re = rowptr[b + 1];
  int inter = 0, lu = 0, ru = 0;
  while (l < le || r < re) {
    int lc = l < le ? colind[l] : 0x7fffffff;
    int rc = r < re ? colind[r] : 0x7fffffff;
    if (lc == rc) {
      ++inter; ++lu; ++ru;
      while (l < le && colind[l] == lc) ++l;
      while (r < re && colind[r] == rc) ++r;
    } else if (lc < rc) {
      ++lu;
      while (l < le && colind[l] == lc) ++l;
    } else {
      ++ru;
      while (r < re && colind[r] == rc) ++r;
    }
  }
  int un = lu + ru - inter;
  return un ? (double)inter / un : 1.0;
}

typedef struct { uint64_t sig; int first; int row; } rank_t;
static int cmp_rank(const void *a, const void *b) {
  const rank_t *x = (const rank_t *)a, *y = (const rank_t *)b;
  if (x->sig != y->sig) return x->sig < y->sig ? -1 : 1;
  if (x->first != y->first) return x->first < y->first ? -1 : 1;
  return (x->row > y->row) - (x->row < y->row);
}

/* jaccard_greedy_order (CFE:300-340): rows ranked by (minhash of columns,
 * first column, row); buckets of 64 consecutive ranked rows; inside a
 * bucket start from its first row and repeatedly append the remaining row
 * of highest Jaccard similarity to the last appended row (ties: lower row
 * id). */
void oracle_order_jaccard(int m, int k, const int *rowptr, const int *colind, int *order) {
  rank_t *rk = (rank_t *)malloc(sizeof(rank_t) * (size_t)(m > 0 ? m : 1));
  for (int r = 0; r < m; ++r) {
    uint64_t s = UINT64_MAX;
    for (int p = rowptr[r]; p < rowptr[r + 1]; ++p) {
      uint64_t h = splitmix64((uint64_t)(uint32_t)colind[p]);
      if (h < s) s = h;
    }
    rk[r].sig = s; rk[r].first = first_col(r, k, rowptr, colind); rk[r].row = r;
  }
  qsort(rk, (size_t)m, sizeof(rank_t), cmp_rank);
  int out = 0;
  int rem[64];
  for (int base = 0; base < m; base += 64) {
    int end = base + 64 < m ? base + 64 : m;
    int n = 0;
    for (int i = base + 1; i < end; ++i) rem[n++] = rk[i].row;
    int cur = rk[base].row;
    order[out++] = cur;
    while (n > 0) {
      int best = 0;
      double bs = -1.0;
      for (int c = 0; c < n; ++c) {
        double s = jaccard(cur, rem[c], rowptr, colind);
        if (s > bs || (s == bs && rem[c] < rem[best])) { bs = s; best = c; }
      }
      cur = rem[best];
      order[out++] = cur;
      for (int c = best; c + 1 < n; ++c) rem[c] = rem[c + 1];
      --n;
    }
  }
  free(rk);
}

/* Non-empty rows in order (the sparse-row physicalisation, CFE:483-488).
 * Returns the count. */
int oracle_order_sparse_rows(int m, const int *rowptr, int *order) {
  int n = 0;
  for (int r = 0; r < m; ++r)
    if (rowptr[r] != rowptr[r + 1]) order[n++] = r;
  return n;
}

/* Generated-operator packing (CFE:496-640) for BH x BW tiles:
 *   packing 0 = column-condensed dense (modes 2 and 4), 1 = active fixed
 *   blocks dense (mode 3, tile columns 8j..8j+7 clamped to k-1);
 *   duplicates are summed; rows follow order[0..P) (new -> original).
 * count pass: fills soff[ceil(P/BH)+1], returns the tile count (or -1 on an
 * out-of-range column). fill pass writes sidx[BW*tiles], val[BH*BW*tiles]. */
static int64_t pack_window(const int *rowptr, const int *colind, const float *values,
                           int k, int bh, int bw, int packing, const int *order, int P, int w,
                           int64_t **buf, int64_t *cap, int *sidx, float *val) {
  int64_t n = 0;
  for (int nr = w * bh; nr < (w + 1) * bh && nr < P; ++nr) {
    int orow = order[nr];
    for (int p = rowptr[orow]; p < rowptr[orow + 1]; ++p) {
      if (colind[p] < 0 || colind[p] >= k) return -1;
      if (n >= *cap) { *cap = *cap < 256 ? 256 : *cap * 2; *buf = (int64_t *)realloc(*buf, sizeof(int64_t) * 2 * (size_t)*cap); }
      (*buf)[2 * n] = packing == 0 ? colind[p] : colind[p] / bw;
      (*buf)[2 * n + 1] = ((int64_t)(nr - w * bh) << 32) | (uint32_t)p;
      ++n;
    }
  }
  qsort(*buf, (size_t)n, 2 * sizeof(int64_t), cmp_key2);
  /* distinct keys in order */
  int64_t nk = 0;
  for (int64_t i = 0; i < n; ++i)
    if (i == 0 || (*buf)[2 * i] != (*buf)[2 * i - 2]) ++nk;
  int64_t tiles = packing == 0 ? (nk + bw - 1) / bw : nk;
  if (!sidx) return tiles;
  int64_t key_idx = -1;
  for (int64_t i = 0; i < n; ++i) {
    if (i == 0 || (*buf)[2 * i] != (*buf)[2 * i - 2]) ++key_idx;
    int64_t key = (*buf)[2 * i];
    int lrow = (int)((*buf)[2 * i + 1] >> 32);
    int p = (int)((*buf)[2 * i + 1] & 0xffffffff);
    int64_t tile, lcol;
    if (packing == 0) { tile = key_idx / bw; lcol = key_idx % bw; }
    else { tile = key_idx; lcol = colind[p] % bw; }
    (void)key;
    val[tile * bh * bw + oracle_swizzle(lrow * bw + (int)lcol)] += values[p];
  }
  /* tile columns */
  key_idx = -1;
  for (int64_t i = 0; i < n; ++i) {
    if (!(i == 0 || (*buf)[2 * i] != (*buf)[2 * i - 2])) continue;
    ++key_idx;
    int64_t key = (*buf)[2 * i];
    if (packing == 0) sidx[key_idx] = (int)key;
    else for (int c = 0; c < bw; ++c) { int64_t col = key * bw + c; sidx[key_idx * bw + c] = (int)(col < k - 1 ? col : k - 1); }
  }
  if (packing == 0 && nk % bw) {
    int last = sidx[nk - 1];
    for (int64_t i = nk; i < tiles * bw; ++i) sidx[i] = last;
  }
  return tiles;
}

int64_t oracle_pack_count(const int *rowptr, const int *colind, int k, int bh, int bw, int packing,
                          const int *order, int P, int *soff) {
  int W = (P + bh - 1) / bh;
  int64_t *buf = NULL, cap = 0, total = 0;
  for (int w = 0; w < W; ++w) {
    soff[w] = (int)total;
    int64_t t = pack_window(rowptr, colind, NULL, k, bh, bw, packing, order, P, w, &buf, &cap, NULL, NULL);
    if (t < 0) { free(buf); return -1; }
    total += t;
  }
  soff[W] = (int)total;
  free(buf);
  return total;
}

void oracle_pack_fill(const int *rowptr, const int *colind, const float *values, int k, int bh, int bw,
                      int packing, const int *order, int P, const int *soff, int *sidx, float *val) {
  int W = (P + bh - 1) / bh;
  int64_t *buf = NULL, cap = 0;
  memset(val, 0, sizeof(float) * (size_t)((int64_t)soff[W] * bh * bw));
  for (int w = 0; w < W; ++w)
    pack_window(rowptr, colind, values, k, bh, bw, packing, order, P, w, &buf, &cap,
                sidx + (int64_t)soff[w] * bw, val + (int64_t)soff[w] * bh * bw);
  free(buf);
}
