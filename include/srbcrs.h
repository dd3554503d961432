/*
 * srbcrs.h -- C ABI of the MI355X (gfx950) SR-BCRS SpMM backend.
 *
 * Plain pointers and sizes only.  Every function returns SRBCRS_OK (0) or a
 * negative status; srbcrs_last_error() then holds a message for the calling
 * thread.  "d_" pointers are device (HBM) pointers, others host pointers.
 * `stream` is a hipStream_t (NULL = the null stream).
 *
 * Reference interfaces replaced (paths relative to the reference root):
 *   SRK = examples/src_fp32/sr_bcrs/testbed/SRBCRSSpMM_kernel.cu
 *   SRC = examples/src_fp32/sr_bcrs/testbed/SRBCRSSpMM.cpp
 *   CFE = examples/src_fp32/acc/testbed/custom_format_e2e.cu
 */
#ifndef MASK_AMD_SRBCRS_H
#define MASK_AMD_SRBCRS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SRBCRS_OK 0
#define SRBCRS_EINVAL (-1)   /* bad argument (the reference's TORCH_CHECK failures) */
#define SRBCRS_EHIP (-2)     /* HIP runtime error */
#define SRBCRS_ENOMEM (-3)   /* allocation failed */
#define SRBCRS_ESTATE (-4)   /* wrong object state (e.g. run on another device) */

typedef struct srbcrs_plan srbcrs_plan;
typedef struct srbcrs_schedule srbcrs_schedule;

/* Message of the last failing call on this thread ("" if none). */
const char *srbcrs_last_error(void);

/* Library version string. */
const char *srbcrs_version(void);

/* ---- Host conversion CSR -> SR-BCRS (bit-exact with SRK:226-282 for 16x8
 * and SRK:284-340 for 32x32; the per-window block count and the padding /
 * swizzle / last-write-wins rules of preprocess_gpu_srcfp32_srbcrs).
 * Two calls: count fills soff[Mo+1] (Mo = ceil(num_nodes/blk_h)) and the
 * total block count; fill writes sidx[blk_w*total], val[blk_h*blk_w*total]
 * and, when non-NULL, block_partition[Mo], edge_to_row[nnz],
 * edge_to_col[nnz] (entries of edges outside rows [0, num_nodes) untouched).
 * (blk_h, blk_w) must be (16, 8) or (32, 32). */
int srbcrs_convert_count(const int32_t *rowptr, const int32_t *colind, int32_t num_nodes,
                         int64_t nnz, int32_t blk_h, int32_t blk_w, int32_t *soff,
                         int64_t *total_blocks);
int srbcrs_convert_fill(const int32_t *rowptr, const int32_t *colind, const float *values,
                        int32_t num_nodes, int64_t nnz, int32_t blk_h, int32_t blk_w,
                        const int32_t *soff, int32_t *sidx, float *val, int32_t *block_partition,
                        int32_t *edge_to_row, int32_t *edge_to_col);

/* ---- Plans: the device-resident SR-BCRS matrix.  Replaces the reference's
 * preprocess_gpu_srcfp32_srbcrs + its process-global CacheEntry
 * (SRK:27-45, SRK:172-393; pybind preprocess_gpu_16x8 / preprocess_gpu at
 * SRC:77-118).  is_device: 0 = the CSR arrays are on the host; 1 = on the
 * device, converted on the device (radix sort of (window, column) keys, no
 * host round trip); 2 = on the device, copied to the host and converted
 * there as the reference does (SRK:203-205).  All three give the same
 * arrays bit for bit.  On success *out owns device copies of soff / sidx /
 * val on the current device. */
int srbcrs_plan_create(const int32_t *rowptr, const int32_t *colind, const float *values,
                       int32_t num_nodes, int64_t nnz, int32_t blk_h, int32_t blk_w,
                       int32_t is_device, void *stream, srbcrs_plan **out);
void srbcrs_plan_destroy(srbcrs_plan *plan);

/* Plan metadata.  d_soff / d_sidx / d_val are owned by the plan. */
typedef struct srbcrs_plan_desc {
  int32_t num_nodes;
  int32_t blk_h, blk_w;
  int32_t row_windows;    /* Mo */
  int32_t max_col;        /* largest column index in the CSR, -1 if nnz == 0 */
  int32_t device;
  int64_t nnz;
  int64_t total_blocks;
  const int32_t *d_soff;  /* row_window_offset, Mo + 1 */
  const int32_t *d_sidx;  /* tcblocktile_id, blk_w * total_blocks */
  const float *d_val;     /* swizzled block values, blk_h * blk_w * total_blocks */
  int64_t packed_rows;    /* rows in the packed order (num_nodes unless sparse rows) */
  const int32_t *d_row_map; /* packed row -> output row, NULL for the identity order */
  int32_t packing;        /* SRBCRS_PACK_* */
  int32_t dup_policy;     /* SRBCRS_DUP_* */
  int64_t stored_values;  /* values in the compact copy of val (-1: no copy) */
  const void *d_a_words;  /* compact copy: one {mask, base} uint32 pair per 32 block positions (NULL: none) */
  const float *d_a_packed; /* compact copy: the stored values in logical order, then 16 zero floats */
} srbcrs_plan_desc;
int srbcrs_plan_get(const srbcrs_plan *plan, srbcrs_plan_desc *out);

/* Write block_partition[Mo], edge_to_col[nnz] and edge_to_row[nnz] (device
 * buffers) as preprocess does, each only when its buffer length is at least
 * the needed size (SRK:355-366).  NULL / short buffers are skipped. */
int srbcrs_plan_write_edges(const srbcrs_plan *plan, int32_t *d_block_partition,
                            int64_t block_partition_len, int32_t *d_edge_to_col,
                            int64_t edge_to_col_len, int32_t *d_edge_to_row,
                            int64_t edge_to_row_len, void *stream);

/* Copy the plan's row_window_offset (Mo + 1) and tcblocktile_id
 * (blk_w * total_blocks) into caller-owned device buffers: the first and
 * third members of preprocess's result tuple (SRK:343-392).  A NULL buffer
 * is skipped; a short one is an error. */
int srbcrs_plan_export_index(const srbcrs_plan *plan, int32_t *d_row_window_offset,
                             int64_t row_window_offset_len, int32_t *d_tcblocktile_id,
                             int64_t tcblocktile_id_len, void *stream);

/* Copy the plan's swizzled block values (blk_h * blk_w * total_blocks
 * floats, the reference's tcblock_val, SRK:329-330) into a caller-owned
 * device buffer.  A short buffer is an error. */
int srbcrs_plan_export_values(const srbcrs_plan *plan, float *d_val, int64_t val_len,
                              void *stream);

/* ---- Generated-operator packings (the reference's custom-format bridge,
 * CFE:157-349 row reorders, CFE:483-488 sparse rows, CFE:496-640 packing,
 * CFE:1083-1100 inverse output map).  A packed plan stores its rows in a
 * new order (new row p <- original row order[p]); runs write each packed
 * row straight to its original output row (the inverse map is fused into
 * the kernel's store) and zero the rows the order leaves out. */
#define SRBCRS_ORDER_IDENTITY 0
#define SRBCRS_ORDER_RCM 1          /* reverse Cuthill-McKee (square matrices) */
#define SRBCRS_ORDER_FIRST_COL 2    /* by first structural column */
#define SRBCRS_ORDER_JACCARD 3      /* minhash buckets of 64, greedy Jaccard */
#define SRBCRS_ORDER_SPARSE_ROWS 4  /* non-empty rows only */
#define SRBCRS_ORDER_EXPLICIT 5     /* caller's order (distinct rows) */
#define SRBCRS_PACK_CONDENSED 0     /* column-condensed dense tiles (SR-BCRS) */
#define SRBCRS_PACK_FIXED_BLOCKS 1  /* active BW-aligned column blocks, dense */
#define SRBCRS_DUP_LAST 0           /* duplicate (row, col): last value wins (preprocess_gpu) */
#define SRBCRS_DUP_SUM 1            /* duplicates summed in edge order (CFE packing) */

typedef struct srbcrs_pack_opts {
  int32_t blk_h, blk_w;     /* (16, 8) or (32, 32) */
  int32_t packing;          /* SRBCRS_PACK_* */
  int32_t dup_policy;       /* SRBCRS_DUP_* */
  int32_t row_order;        /* SRBCRS_ORDER_* */
  const int32_t *order;     /* host, SRBCRS_ORDER_EXPLICIT only */
  int32_t order_len;
  int32_t K;                /* column count; required (> 0) for fixed blocks, -1 = unchecked */
} srbcrs_pack_opts;

/* Row order of a CSR matrix by `method` (SRBCRS_ORDER_RCM .. SPARSE_ROWS,
 * or IDENTITY).  order has num_nodes entries; *order_len receives the
 * number used (fewer than num_nodes only for SPARSE_ROWS). */
int srbcrs_row_order(const int32_t *rowptr, const int32_t *colind, int32_t num_nodes, int64_t nnz,
                     int32_t K, int32_t method, int32_t *order, int32_t *order_len);

/* Host packing with explicit options (opts->row_order IDENTITY or
 * EXPLICIT; resolve the other orders with srbcrs_row_order first).  soff
 * has ceil(rows / blk_h) + 1 entries, rows = order_len or num_nodes. */
int srbcrs_pack_count(const int32_t *rowptr, const int32_t *colind, int32_t num_nodes, int64_t nnz,
                      const srbcrs_pack_opts *opts, int32_t *soff, int64_t *total_tiles);
int srbcrs_pack_fill(const int32_t *rowptr, const int32_t *colind, const float *values,
                     int32_t num_nodes, int64_t nnz, const srbcrs_pack_opts *opts,
                     const int32_t *soff, int32_t *sidx, float *val);

/* srbcrs_plan_create with packing options (NULL = the canonical 16x8
 * preprocess_gpu conversion).  Edge maps (srbcrs_plan_write_edges) exist
 * only for canonical plans. */
int srbcrs_plan_create_ex(const int32_t *rowptr, const int32_t *colind, const float *values,
                          int32_t num_nodes, int64_t nnz, const srbcrs_pack_opts *opts,
                          int32_t is_device, void *stream, srbcrs_plan **out);

/* The plan's row order (new -> original).  order needs room for
 * num_nodes entries; *len receives the packed row count. */
int srbcrs_plan_row_order(const srbcrs_plan *plan, int32_t *order, int32_t capacity, int32_t *len);

/* ---- Execution schedules (host logic).  policy:
 *   "row"        one task per row window, written straight into C
 *                (the plain kernel's mapping, kernel.inc:1590-1700);
 *   "split"      row windows cut into segments of at most `param` blocks
 *                (0 = automatic p95 / heavy-tail rule of CFE:640-699);
 *   "strict_lb"  fixed-work groups of `param` blocks (0 = 64), the
 *                fragmenting of strict_load_balance
 *                (main_strict_lb_16x8.cu:208-256, CFE:719-749);
 *   "multi_bind" windows above 2x the mean split into ceil(x/mean) parts
 *                (main_multi_bind_16x8.cu:211-270, CFE:750-780);
 *   "auto"       "split" (param 0) when the longest window exceeds
 *                max(64, 4 x the 95th-percentile window), else "row" (the
 *                split rule's own heavy-tail test; param ignored).
 * Partial windows go to private partial tiles that a deterministic segment
 * reduction (fixed slot order) sums into C: no atomics anywhere, unlike
 * the reference's atomicAdd edges (kernel_lb.inc:9-58).
 * Export arrays (host) sized from srbcrs_schedule_info:
 *   group_off[n_groups+1], task_begin/end/window/slot[n_tasks]
 *   (slot -1 = direct store), red_window[n_red], red_slot_off[n_red+1]. */
int srbcrs_schedule_build(const int32_t *soff, int32_t row_windows, const char *policy,
                          int32_t param, srbcrs_schedule **out);
int srbcrs_schedule_info(const srbcrs_schedule *s, int32_t *n_groups, int32_t *n_tasks,
                         int32_t *n_slots, int32_t *n_red);
int srbcrs_schedule_export(const srbcrs_schedule *s, int32_t *group_off, int32_t *task_begin,
                           int32_t *task_end, int32_t *task_window, int32_t *task_slot,
                           int32_t *red_window, int32_t *red_slot_off);
void srbcrs_schedule_destroy(srbcrs_schedule *s);

/* Select the schedule a plan runs with (default "row").  Uploads the task
 * tables to the plan's device. */
int srbcrs_plan_set_schedule(srbcrs_plan *plan, const char *policy, int32_t param);

/* ---- SpMM.  C[0:c_rows, 0:N] = A * B with A the plan's matrix (16x8 or
 * 32x32 blocks)
 * (replaces run_spmm_srcfp32_srbcrs, SRK:395-557, pybind run_SRBCRS_16x8 /
 * run_SRBCRS and the *_balance aliases, SRC:120-192).  B is K x N
 * row-major with leading dimension ldb, C is c_rows x N with ldc.
 * Requirements: N % 16 == 0, K > max column, c_rows >=
 * num_nodes (rows beyond num_nodes are not written).  Every row
 * < num_nodes of C is overwritten (zeros for empty windows).  Schedules
 * other than "row" use a plan-owned partial buffer, grown (hipMalloc, to at
 * least twice its size) when a run needs more slots x ldc than it holds.
 * Growth never frees: replaced buffers and replaced task tables are retired
 * and stay allocated until srbcrs_plan_trim or srbcrs_plan_destroy, so a HIP
 * graph captured on an earlier run keeps valid addresses.  Capture after one
 * eager run with the same N, ldc and schedule (a growing run allocates,
 * which graph capture forbids).  A call that is refused (a negative status)
 * has launched nothing and left C untouched. */
int srbcrs_run(srbcrs_plan *plan, const float *d_B, int64_t K, int64_t N, int64_t ldb,
               float *d_C, int64_t ldc, int64_t c_rows, void *stream);

/* Free the device buffers the plan has retired (partial buffers it grew
 * out of, task tables of earlier schedules) after synchronizing `stream`.
 * Retired buffers are what graphs captured on earlier runs may still
 * address: call this only when no such graph will be replayed again and no
 * launch that used them is in flight on another stream.  Without it they
 * are freed with the plan.  No reference counterpart (the reference keeps
 * one global cache entry). */
int srbcrs_plan_trim(srbcrs_plan *plan, void *stream);

/* Launch knobs of the SR-BCRS kernels (template parameters; each maps a
 * knob of the reference's strategy schema, strategy_agent.py:81-130):
 *   depth        blocks in flight per wave: 2, 4 or 8 (0 = 2); the
 *                software-pipeline depth (the reference's 2-buffer,
 *                3-stage pipeline, sr_bcrs_ops.py:684-708); indices are
 *                fetched one further ring ahead (its stage shift);
 *   tile_b       16, 32 or 64: caps the columns one lane group covers per
 *                MFMA sweep (16 * vector width) (0 = widest legal); the
 *                reference's N tile (SRBCRSSpMM_kernel.cu:435-475);
 *   wg_cols      columns per workgroup, a power of two in 64..512
 *                (0 = 128); 32x32 blocks run 128-column waves (two
 *                64-column groups per lane) in workgroups of 256 columns
 *                or more, 64-column waves below; 16x8 blocks run
 *                256-column waves (four groups per lane, N % 256 == 0) in
 *                workgroups of 256 columns or more, 128-column waves at 128,
 *                64-column waves at 64;
 *   grid_order   0 = default (chunk-major), 1 = chunk-major: one column
 *                chunk of every window before the next chunk (narrower B
 *                working set per XCD), 2 = window-major, 3 = chunk sweep:
 *                chunk-major in dispatch order, all XCDs on one chunk at a
 *                time (its B rows shared through the memory-side cache),
 *                4 = merged windows ("row" schedule, 16x8 blocks with the
 *                compact A copy, vector width 4): one wave per
 *                windows_per_wave windows (4 or 8; 0 = 8 at 64 columns,
 *                4 at 128) and wg_cols columns (64 or 128; 0 = 64), walking the
 *                windows' blocks interleaved (block r of each window in
 *                turn) so that it sweeps its B rows once in ascending order,
 *                the column chunk pinned to one XCD (N / wg_cols must divide
 *                8 or be a multiple of 8); depth 2 or 4 (8 windows: only
 *                at 64 columns and depth 2).  The first run per
 *                windows_per_wave builds the interleaved copy of the block
 *                indices and A words on the host (it allocates),
 *                5 = nonzero sweep: the vector kernel for low block density
 *                ("row" schedule, 16x8 blocks with the compact A copy).
 *                One wave per windows_per_wave windows (4 or 8; 0 = 8)
 *                and 64 columns walks the windows' stored values in the
 *                merged order (one 256-byte B-row gather and one LDS
 *                read-add-write per value, no padded block arithmetic);
 *                tile_b = values per sub-batch (16, 32 or 64; 0 = 32),
 *                depth = sub-batches of gathers in flight (2 or 4; 0 = 2;
 *                4 only with tile_b 16 or 32); wg_cols 0 or 64.  Needs N a
 *                multiple of 64 (each 64-column chunk pinned to one XCD
 *                when N / 64 divides 8 or is a multiple of 8, unpinned
 *                otherwise), ldb and ldc multiples of 4, 16-byte aligned
 *                B and C, K * ldb * 4 < 2^32, ldb * 4 < 2^24 and column indices
 *                below 2^24; a matrix whose stream would be mostly
 *                padding (a row with far more values than its group's
 *                others: over 8 entries per value and 2^22 entries) is
 *                refused, before the stream is built when the groups'
 *                lower bounds already pass that size.  C[r, :] is the sum of fl(v * B[c, :]) over
 *                the row's stored values in ascending column order, each
 *                product rounded before it is added (the fp32 CSR product,
 *                not the MFMA kernels' bits).  The first run per setting
 *                builds its value stream on the host (it allocates; kept
 *                until the plan is destroyed);
 *   windows_per_wave  "row" schedule: consecutive row windows one wave
 *                streams through its register ring (0 = 1), in [0, 4096];
 *   a_operand    see SRBCRS_A_* below;
 *   b_stage      where the ring holds the gathered B rows: SRBCRS_B_DEFAULT
 *                (= registers), SRBCRS_B_REGISTERS, or SRBCRS_B_LDS: LDS
 *                slots filled by direct-to-LDS loads (global_load_lds) and
 *                read back in the MFMA layout; the reference's cp.async
 *                double buffer (kernel.inc:584-642) in gfx950 form.  LDS
 *                staging applies at vector width 4 (tile_b 64 and 16-byte
 *                aligned B, ldb % 4 == 0); other launches use registers;
 *   epilogue     SRBCRS_EPILOGUE_NONE (0) or SRBCRS_EPILOGUE_RELU (1): the
 *                kernel that writes an output value applies relu to it
 *                (x < 0 -> +0; NaN and zeros unchanged), on every grid
 *                order and schedule (on split schedules in the segment
 *                reduction, not on the partial tiles); rows a packing
 *                leaves out stay 0.  No counterpart in the reference's
 *                SpMM: it fuses the GCN's relu(A (X W1)) into the SpMM's
 *                store.  Not a launch knob: a tuned setting (all other
 *                fields 0) runs with it.
 * Values outside these sets are rejected.  Every MFMA setting (grid orders
 * 0-4) yields the same bits: the per-element accumulation order does not
 * depend on them; the nonzero sweep (grid order 5) yields the fp32 CSR
 * product's bits, equal to the others within fp32 rounding. */
typedef struct srbcrs_run_opts {
  int32_t depth;
  int32_t tile_b;
  int32_t wg_cols;
  int32_t grid_order;
  int32_t windows_per_wave;
  int32_t a_operand;
  int32_t b_stage;
  int32_t epilogue;
} srbcrs_run_opts;

/* a_operand: where the kernel reads the block values from.  Both give the
 * same bits.  COMPACT reads the plan's compact copy (per 32 block positions
 * a {mask, base} word plus the stored values; built at plan creation); DENSE
 * reads the reference-layout value array.  DEFAULT = COMPACT for 16x8
 * blocks when the plan has the copy (it is skipped when it would not fit)
 * and at most half of the block positions hold values, else DENSE (always
 * DENSE for 32x32 blocks). */
#define SRBCRS_A_DEFAULT 0
#define SRBCRS_A_COMPACT 1
#define SRBCRS_A_DENSE 2

#define SRBCRS_B_DEFAULT 0
#define SRBCRS_B_REGISTERS 1
#define SRBCRS_B_LDS 2

#define SRBCRS_GRID_DEFAULT 0
#define SRBCRS_GRID_CHUNK_MAJOR 1
#define SRBCRS_GRID_WINDOW_MAJOR 2
#define SRBCRS_GRID_CHUNK_SWEEP 3
#define SRBCRS_GRID_MERGED 4
#define SRBCRS_GRID_NZSWEEP 5

#define SRBCRS_EPILOGUE_NONE 0
#define SRBCRS_EPILOGUE_RELU 1

/* srbcrs_run with explicit knobs (opts NULL = defaults). */
int srbcrs_run_ex(srbcrs_plan *plan, const float *d_B, int64_t K, int64_t N, int64_t ldb,
                  float *d_C, int64_t ldc, int64_t c_rows, const srbcrs_run_opts *opts,
                  void *stream);

/* srbcrs_run_ex that allocates nothing (no hipMalloc / hipFree, no
 * allocating library call).  No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid it).  The split / strict_lb / multi_bind
 * schedules keep their partial tiles in a fixed device array of
 * srbcrs_noalloc_scratch_floats() floats (64 MiB) that each GPU the library
 * runs on holds until the process ends; a run whose partial tiles need more
 * (slots x blk_h x ldc floats) is rejected with SRBCRS_EINVAL.  The "row"
 * schedule needs no scratch.  All calls on one GPU share that array, so calls
 * that overlap on one GPU (other streams, other threads) race; calls in
 * stream order do not.  Results are bit-identical to srbcrs_run_ex with the
 * same arguments.  The plan's schedule tables must exist already
 * (srbcrs_plan_set_schedule allocates them), and so must the host-built
 * stream of a merged-window or nonzero-sweep setting (the first
 * srbcrs_run_ex with those knobs builds it); otherwise SRBCRS_EINVAL. */
int srbcrs_run_noalloc(srbcrs_plan *plan, const float *d_B, int64_t K, int64_t N, int64_t ldb,
                       float *d_C, int64_t ldc, int64_t c_rows, const srbcrs_run_opts *opts,
                       void *stream);
size_t srbcrs_noalloc_scratch_floats(void);

/* Time candidate launch settings on this plan for a dense width N and keep
 * one.  Candidates, in preference order: for the compact A operand (16x8
 * blocks, when the plan has the copy and at most 3/4 of the block positions
 * hold values), then for the dense one (unless, for 16x8, under 1/4 hold
 * values and the compact copy exists): grid order chunk-major /
 * chunk sweep x wg_cols 128 / 64 / 256 x depth 2 / 4, then (16x8) the
 * LDS-staged B ring at wg_cols 64, chunk sweep, depth 2 / 4, then, on the
 * "row" schedule, wg_cols 128 / 256 x 4 / 8 windows per wave x depth
 * 2 / 4 / 8 (chunk-major), and last, for the compact A source on the "row"
 * schedule, the merged-window grid at (wg_cols, windows, depth) = (128, 4,
 * 4), (128, 4, 2), (64, 8, 2), (64, 4, 4) where N allows it (a setting the
 * operands' alignment refuses is skipped).  Each gets one warm-up
 * and `reps` timed launches on `stream`; the first candidate within 3 % of
 * the fastest wins, so near-ties resolve the same way on every run.  Later
 * srbcrs_run calls, and srbcrs_run_ex calls whose knobs are all 0, use it
 * at that N until the schedule changes.  C is overwritten (with the
 * product).  Every candidate gives the same bits: tuning changes only the
 * time (srbcrs_plan_tune_ex can add candidates that do not).  best (may be NULL) receives the choice.  Not thread-safe against a
 * concurrent srbcrs_run* on the same plan.  No reference counterpart: the
 * reference fixes its launch shape offline (strategy_agent.py:81-130). */
int srbcrs_plan_tune(srbcrs_plan *plan, const float *d_B, int64_t K, int64_t N, int64_t ldb,
                     float *d_C, int64_t ldc, int64_t c_rows, int32_t reps, srbcrs_run_opts *best,
                     void *stream);

/* srbcrs_plan_tune with flags (srbcrs_plan_tune = flags 0).
 * SRBCRS_TUNE_NONZERO_SWEEP adds, last, the nonzero sweep (grid order 5;
 * "row" schedule, 16x8 blocks with the compact copy) at (windows_per_wave,
 * tile_b, depth) = (8, 32, 2), (4, 16, 2), (4, 16, 4), (8, 32, 4): a choice
 * among them gives the fp32 CSR product's bits instead of the MFMA
 * kernels' (equal within fp32 rounding), the caller's opt-in, as the
 * reference's SPARSENE_ALLOW_CSR_FALLBACK is (external_backend_spmm.py:40-95).
 * Each stream a candidate needs is built on the host at its first run.
 * Other flag bits are rejected.  No reference counterpart. */
#define SRBCRS_TUNE_NONZERO_SWEEP 1
int srbcrs_plan_tune_ex(srbcrs_plan *plan, const float *d_B, int64_t K, int64_t N, int64_t ldb,
                        float *d_C, int64_t ldc, int64_t c_rows, int32_t reps, int32_t flags,
                        srbcrs_run_opts *best, void *stream);

/* ---- Sharding over GPUs (design support; this build runs on one GPU).
 * Cut the row windows into n_shards contiguous ranges of near-equal cost
 * (blocks + one output tile per window): shard s owns windows
 * [bounds[s], bounds[s+1]), i.e. rows [16 * bounds[s], 16 * bounds[s+1])
 * for 16-row windows, and writes its C rows with no reduction.  bounds has
 * n_shards + 1 entries.  No reference counterpart (the reference is
 * single-GPU). */
int srbcrs_shard_windows(const int32_t *soff, int32_t row_windows, int32_t n_shards, int32_t *bounds);

/* ---- CSR fallback for low block density: C[r, :] = sum_e val[e] *
 * B[col[e], :], fp32, edge order.  The arithmetic of csr_spmm_value_kernel
 * (SRK:66-105), one wave64 per row.  max_col (host-known bound on colind,
 * -1 if unknown) is checked against K. */
int srbcrs_csr_spmm(const int32_t *d_rowptr, const int32_t *d_colind, const float *d_values,
                    int32_t M, int64_t nnz, int32_t max_col, const float *d_B, int64_t K,
                    int64_t N, int64_t ldb, float *d_C, int64_t ldc, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MASK_AMD_SRBCRS_H */
