"""Write tests/golden/sym_unsorted_dup.mtx: a small MatrixMarket input for the
reference's real-matrix path (examples/src/mmio_highlevel.cu:255-402) with
the features that path must handle: a symmetric header (mirrored entries),
entries in no particular order, a diagonal, a duplicate (row, col) entry and
an empty row.  Seeded; rerun to regenerate the identical file."""
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "sym_unsorted_dup.mtx"


def main():
    rng = np.random.default_rng(20260)
    n = 90
    lower = [(i, j) for i in range(n) for j in range(i + 1) if rng.random() < 0.06 and i != 41 and j != 41]
    entries = [(i, j, float(np.float32(rng.uniform(-2, 2)))) for i, j in lower]
    rng.shuffle(entries)
    i, j, _ = entries[7]
    entries.insert(30, (i, j, 0.75))        # duplicate of an earlier entry (last write wins in preprocess)
    with open(OUT, "w") as f:
        f.write("%%MatrixMarket matrix coordinate real symmetric\n")
        f.write("% symmetric, unsorted, one duplicate, row/column 41 empty (tests/golden/make_mtx_fixture.py)\n")
        f.write(f"{n} {n} {len(entries)}\n")
        for a, b, v in entries:
            f.write(f"{a + 1} {b + 1} {v!r}\n")


if __name__ == "__main__":
    main()
