"""Write the hand-derived known-answer fixtures of this directory.

Nothing here runs a converter or the oracle: every expected array is
written out by hand from the conversion rules of the reference's
preprocess_gpu_srcfp32_srbcrs (examples/src_fp32/sr_bcrs/testbed/
SRBCRSSpMM_kernel.cu:226-282 for 16x8, :284-340 for 32x32) and from the
CuTe Swizzle<2,2,3> offset map o ^ ((o & 0x60) >> 3), o = BW*r + c:
per BH-row window, the sorted distinct columns cut into BW-column blocks
padded with the window's last column; each value at its swizzled offset,
the last write winning for a duplicate (row, column).  The reference ships
no golden vectors for this path, so these are the fixed answers the CPU and
GPU tests share.  Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
from pathlib import Path

HERE = Path(__file__).resolve().parent


def csr(rows, n_rows):
    rowptr, colind, values = [0], [], []
    for r in range(n_rows):
        for c, v in rows.get(r, []):
            colind.append(c)
            values.append(v)
        rowptr.append(len(colind))
    return rowptr, colind, values


def case_16x8():
    # 18 rows -> two 16-row windows (the second holds rows 16, 17 only)
    rows = {0: [(3, 1.0), (10, 2.0)],
            1: [(10, 3.0), (1, 4.0)],                 # unsorted columns
            3: [(30 + i, 10.0 + i) for i in range(8)],
            5: [(20, 5.0), (3, 6.0)],
            12: [(1, 7.0)],
            16: [(7, 8.0)],
            17: [(7, 9.0), (7, 11.0)]}               # duplicate: the last write wins
    rowptr, colind, values = csr(rows, 18)
    # window 0 columns 1 3 10 20 30..37 (12) -> 2 blocks, the second padded with 37
    val = [0.0] * (3 * 128)
    val[1] = 1.0                  # r0 col 3  -> c1, o 1
    val[2] = 2.0                  # r0 col 10 -> c2, o 2
    val[10] = 3.0                 # r1 col 10 -> o 10
    val[8] = 4.0                  # r1 col 1  -> o 8
    for i in range(4):            # r3 cols 30..33 -> c4..7, o 28..31
        val[28 + i] = 10.0 + i
    val[47] = 5.0                 # r5 col 20 -> o 43 -> swizzled 47
    val[45] = 6.0                 # r5 col 3  -> o 41 -> 45
    val[108] = 7.0                # r12 col 1 -> o 96 -> 108
    for i in range(4):            # block 1: r3 cols 34..37 -> c0..3, o 24..27
        val[128 + 24 + i] = 14.0 + i
    val[256 + 0] = 8.0            # window 1 block: r0 (row 16) col 7
    val[256 + 8] = 11.0           # r1 (row 17) col 7, the last of its two writes
    return {"blk": [16, 8], "num_nodes": 18, "rowptr": rowptr, "colind": colind, "values": values,
            "total": 3, "soff": [0, 2, 3], "block_partition": [2, 1],
            "sidx": [1, 3, 10, 20, 30, 31, 32, 33, 34, 35, 36, 37, 37, 37, 37, 37] + [7] * 8,
            "val": val,
            "edge_to_row": [0, 0, 1, 1] + [3] * 8 + [5, 5, 12, 16, 17, 17],
            "edge_to_col": [1, 2, 2, 0] + list(range(4, 12)) + [3, 1, 0, 0, 0, 0]}


def case_32x32():
    # one 32-row window, 33 distinct columns -> 2 blocks of 32
    rows = {0: [(100 + i, 1.0 + i) for i in range(33)], 31: [(5, 34.0)]}
    rowptr, colind, values = csr(rows, 32)
    val = [0.0] * 2048
    for i in range(31):           # row 0 cols 100..130 -> c1..31 of block 0
        val[1 + i] = 1.0 + i
    val[1024 + 0] = 32.0          # col 131 -> block 1 c0
    val[1024 + 1] = 33.0          # col 132 -> block 1 c1
    val[1004] = 34.0              # row 31 col 5 -> c0, o 992 -> swizzled 1004
    return {"blk": [32, 32], "num_nodes": 32, "rowptr": rowptr, "colind": colind, "values": values,
            "total": 2, "soff": [0, 2], "block_partition": [2],
            "sidx": [5] + list(range(100, 131)) + [131, 132] + [132] * 30, "val": val,
            # edge_to_col is the position in the window's sorted distinct columns
            # (SRBCRSSpMM_kernel.cu:326-328), not the column inside the block
            "edge_to_row": [0] * 33 + [31], "edge_to_col": list(range(1, 32)) + [32, 33] + [0]}


def spmm_exact():
    # A 5x6 with power-of-two values, B 6x16 small integers: every product
    # and partial sum is exact in fp32, so C is known exactly.
    rows = {0: [(0, 1.0), (5, 2.0)], 1: [(2, -0.5)], 3: [(1, 4.0), (3, 0.25), (4, -1.0)], 4: [(5, 8.0)]}
    rowptr, colind, values = csr(rows, 5)
    B = [[(r * 16 + j) % 7 - 3 for j in range(16)] for r in range(6)]
    C = [[0.0] * 16 for _ in range(5)]
    for r, ents in rows.items():
        for c, v in ents:
            for j in range(16):
                C[r][j] += v * B[c][j]
    return {"num_nodes": 5, "K": 6, "N": 16, "rowptr": rowptr, "colind": colind, "values": values,
            "B": B, "C": C}


if __name__ == "__main__":
    for name, obj in (("convert_16x8_hand.json", case_16x8()), ("convert_32x32_hand.json", case_32x32()),
                      ("spmm_exact.json", spmm_exact())):
        (HERE / name).write_text(json.dumps(obj, indent=None, separators=(",", ":")) + "\n")
        print("wrote", name)
