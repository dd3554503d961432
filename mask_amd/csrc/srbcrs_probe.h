/*
 * srbcrs_probe.h -- measurement probes of libmask_srbcrs.so.  Internal: not
 * part of the public C ABI (include/srbcrs.h) and bound only by bench.py.
 * They move memory the way a roofline needs to be calibrated on the same
 * GPU in the same run; they compute nothing a caller uses.  No reference
 * counterparts.
 */
#ifndef MASK_AMD_SRBCRS_PROBE_H
#define MASK_AMD_SRBCRS_PROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Streaming-rate probe: one launch of a plain float4 grid-stride kernel
 * over n_floats floats (a multiple of 4, 16-byte aligned buffers) with
 * `blocks` workgroups of 256 threads: kind 0 copies d_a to d_b, 1 reads d_a
 * (d_b receives at most one float), 2 writes d_b. */
int srbcrs_stream_probe(int32_t kind, const float *d_a, float *d_b, int64_t n_floats, int32_t blocks,
                        void *stream);

/* Gather probe: one launch in which wave w of column chunk c reads the row
 * segments B[rows[i]][c*seg .. (c+1)*seg) for i in [row_off[g], row_off[g+1])
 * of its group g, seg = 256 / rows_per_instr floats (rows_per_instr 1, 2, 4
 * or 8: 1 KB, 512 B, 256 B or 128 B per row segment; every load instruction
 * of the wave moves 1 KB), and sums them.  Nothing but the loads and a
 * 256-byte store per wave (d_out, 64 floats per workgroup of the grid) is
 * done, so the launch time is the gather time of that index stream.  Group
 * row counts must be multiples of 8.  mapping: 0 chunk-major in dispatch
 * order, 1 chunk-major with each XCD given a contiguous range of workgroups
 * (the SpMM kernel's default grid), 2 XCD-affine chunks (workgroup id % 8 is
 * its XCD; XCD x takes chunk x % n_chunks, n_chunks must divide 8).  The
 * grid has n_groups * n_chunks workgroups of one wave, rounded up to a
 * multiple of 8 (d_out needs 64 floats for each). */
int srbcrs_gather_probe(const int32_t *d_rows, const int64_t *d_row_off, int32_t n_groups,
                        int32_t rows_per_instr, const float *d_B, int64_t ldb, int32_t n_chunks,
                        int32_t mapping, float *d_out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MASK_AMD_SRBCRS_PROBE_H */
