"""Format-spec -> executable backend selection for the gfx950 target.

Mirrors the reference's ``select_backend`` / ``BackendPlan``
(python/sparsene/op_gen/backend_registry.py:16-36, :77-303, :482-520) for
the formats this backend executes: the two-level column-condensed dense
hierarchy (SR-BCRS, backend_registry.py:128-142).  The spec is the same
plain mapping the reference consumes (``levels`` / ``atomic`` / ``params``,
e.g. python/test/run_builtin_backend_e2e.py:27-57).  Matching is on
hierarchy and atomic semantics, never on a format name.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Any, Mapping

GFX950_TARGETS = {"gfx950", "mi355x"}
SUPPORTED_REORDERS = {"row_rcm", "first_col_sort", "jaccard_greedy"}
# block shapes the converter and the kernel templates implement
SUPPORTED_BLOCKS = {(16, 8), (32, 32)}


@dataclass(frozen=True)
class BackendPlan:
    backend: str
    codegen_format_name: str
    target: str
    compute_capability: int
    logical_blk_m: int
    logical_blk_k: int
    physical_blk_m: int
    physical_blk_k: int
    tile_n: int
    mma_m: int
    mma_n: int
    mma_k: int
    max_tiles_per_execution_segment: int
    packing_mode: str
    row_reorder: str | None
    notes: tuple[str, ...]
    logical_inner_blk_k: int | None = None

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)


def _axis_map(level: Mapping[str, Any]) -> dict[str, Mapping[str, Any]]:
    return {str(a.get("name")): a for a in level.get("axes", [])}


def _expect(axes, name: str, types: set[str], direction: str):
    a = axes.get(name)
    if a is None:
        raise ValueError(f"column-condensed backend requires axis {name}")
    if a.get("type") not in types or a.get("direction") != direction:
        raise ValueError(f"axis {name} must be {'/'.join(sorted(types))}/{direction}, "
                         f"got {a.get('type')}/{a.get('direction')}")
    return a


def select_backend(spec: Mapping[str, Any], *, target: str = "gfx950", tile_n: int = 64,
                   max_tiles_per_execution_segment: int = 32,
                   allow_physicalization: bool = True) -> BackendPlan:
    """Select the gfx950 backend for a Format-DSL spec, or raise ValueError.

    Accepted: two levels [X_o df ROW, Y_s sv COL, X_i df ROW] /
    [Y_so df|dv COL, Y_si df COL, X_i df ROW] with a dense row-major atomic
    leaf on (X_i, Y_si), i.e. SR-BCRS, with (BLK_M, BLK_K) in
    {(16, 8), (32, 32)}.  ``allow_physicalization`` is accepted for
    signature parity; no canonical fallback format exists here, so a
    rejected spec always raises.
    """
    del allow_physicalization
    if str(target).lower() not in GFX950_TARGETS:
        raise ValueError(f"Unknown target {target!r}; available target: gfx950 (MI355X)")
    levels = spec.get("levels", [])
    atomic = spec.get("atomic", {})
    params = spec.get("params", {})
    if atomic.get("type") != "dense":
        raise ValueError("gfx950 backend requires a dense atomic leaf (SR-BCRS)")
    if len(levels) == 2:
        # backend_registry.py:128-142: column-condensed dense (SR-BCRS)
        outer, inner = _axis_map(levels[0]), _axis_map(levels[1])
        x_outer = _expect(outer, "X_o", {"df"}, "ROW")
        _expect(outer, "Y_s", {"sv"}, "COL")
        _expect(outer, "X_i", {"df"}, "ROW")
        _expect(inner, "Y_so", {"df", "dv"}, "COL")
        _expect(inner, "Y_si", {"df"}, "COL")
        _expect(inner, "X_i", {"df"}, "ROW")
        leaf = ("X_i", "Y_si")
        packing, backend = "column_condensed_dense", "sr_bcrs_dense_mfma_gfx950_v1"
    elif len(levels) == 1:
        # backend_registry.py:143-164: active fixed blocks with a dense leaf
        block = _axis_map(levels[0])
        x_outer = _expect(block, "X_o", {"df"}, "ROW")
        _expect(block, "Y_o_s", {"sv"}, "COL")
        _expect(block, "X_i", {"df"}, "ROW")
        _expect(block, "Y_i", {"df"}, "COL")
        leaf = ("X_i", "Y_i")
        packing, backend = "active_fixed_blocks_dense", "bit_bsr_dense_mfma_gfx950_v1"
    elif len(levels) == 3:
        # backend_registry.py:165-192: sparse-row column-condensed dense
        rows, outer, inner = (_axis_map(lv) for lv in levels)
        x_outer = _expect(rows, "X_s", {"sv"}, "ROW")
        _expect(rows, "Y", {"df"}, "COL")
        _expect(outer, "X_so", {"df"}, "ROW")
        _expect(outer, "Y_s", {"sv"}, "COL")
        _expect(outer, "X_si", {"df"}, "ROW")
        _expect(inner, "Y_so", {"df", "dv"}, "COL")
        _expect(inner, "Y_si", {"df"}, "COL")
        _expect(inner, "X_si", {"df"}, "ROW")
        leaf = ("X_si", "Y_si")
        packing, backend = "sparse_row_column_condensed_dense", "sparse_row_sr_bcrs_dense_mfma_gfx950_v1"
    else:
        raise ValueError("No executable gfx950 backend for this hierarchy: expected two-level column "
                         "condensation, one-level active fixed blocks, or sparse-row SR-BCRS")
    if atomic.get("x_axis") != leaf[0] or atomic.get("y_axis") != leaf[1]:
        raise ValueError(f"dense leaf must map x_axis={leaf[0]} and y_axis={leaf[1]}")
    if atomic.get("layout", "row_major") != "row_major":
        raise ValueError("gfx950 backend requires a row-major atomic leaf")
    reorders = {a.get("reorder") for lv in levels for a in lv.get("axes", []) if a.get("reorder") is not None}
    if len(reorders) > 1 or not reorders.issubset(SUPPORTED_REORDERS):
        raise ValueError(f"Unsupported reorder contract: {sorted(reorders)}")
    row_reorder = next(iter(reorders), None)
    if row_reorder and x_outer.get("reorder") != row_reorder:
        raise ValueError("row reorder must be attached to the outer sparse/dense row axis")
    if packing == "sparse_row_column_condensed_dense" and row_reorder:
        raise ValueError("sparse-row physicalization does not yet compose with an additional row reorder")
    try:
        bm, bk = int(params["BLK_M"]), int(params["BLK_K"])
    except (KeyError, TypeError, ValueError) as exc:
        raise ValueError("backend requires concrete integer BLK_M and BLK_K") from exc
    if (bm, bk) not in SUPPORTED_BLOCKS:
        raise ValueError(f"gfx950 SR-BCRS supports BLK_M x BLK_K in {sorted(SUPPORTED_BLOCKS)}, got {bm}x{bk}")
    if tile_n < 16 or tile_n % 16:
        raise ValueError(f"tile_n must be a positive multiple of 16, got {tile_n}")
    if max_tiles_per_execution_segment < 1:
        raise ValueError("max_tiles_per_execution_segment must be positive")
    notes = [
        "Format conversion is outside timing; every launch (including split reductions) is inside.",
        "fp32 MFMA v_mfma_f32_16x16x4_f32, wave64; each 16-row half of a block and each 8-column unit "
        "is two k-steps.",
        "Partial row windows of split schedules are summed by a deterministic reduction (no atomics).",
    ]
    if packing == "active_fixed_blocks_dense":
        notes.append("Each active fixed block column id expands to BLK_K consecutive scalar columns "
                     "(clamped to K-1) for the dense SR-BCRS kernel.")
    if packing == "sparse_row_column_condensed_dense":
        notes.append("Only structurally non-empty rows are packed; the kernel writes them to their "
                     "original rows and the omitted rows are zeroed.")
    if row_reorder:
        notes.append(f"Rows are packed in {row_reorder} order; the inverse map is applied in the "
                     "kernel's store (no separate unpack pass).")
    return BackendPlan(backend=backend, codegen_format_name="SR_BCRS", target="gfx950",
                       compute_capability=950, logical_blk_m=bm, logical_blk_k=bk, physical_blk_m=bm,
                       physical_blk_k=bk, tile_n=tile_n, mma_m=16, mma_n=16, mma_k=4,
                       max_tiles_per_execution_segment=max_tiles_per_execution_segment,
                       packing_mode=packing, row_reorder=row_reorder, notes=tuple(notes))


def plan_options(plan: BackendPlan) -> dict:
    """Keyword arguments for ``mask_amd.SRBCRSSpMM.Plan`` that realise a
    BackendPlan's physical packing (the generated-operator bridge sums
    duplicates, custom_format_e2e.cu:554-595)."""
    packing = {"column_condensed_dense": "column_condensed_dense",
               "sparse_row_column_condensed_dense": "column_condensed_dense",
               "active_fixed_blocks_dense": "active_fixed_blocks_dense"}[plan.packing_mode]
    order = plan.row_reorder or ("sparse_rows" if plan.packing_mode.startswith("sparse_row") else "identity")
    return dict(blk_h=plan.physical_blk_m, blk_w=plan.physical_blk_k, packing=packing, dup="sum", row_order=order)


def fixed_block_spec(blk_m: int = 16, blk_k: int = 8) -> dict:
    """One-level active fixed blocks with a dense leaf (BIT-BSR dense)."""
    return {
        "format_name": f"FIXED_BLOCK_{blk_m}x{blk_k}",
        "levels": [{"level": 1, "name": "active_block", "axes": [
            {"name": "X_o", "type": "df", "direction": "ROW", "length": "M/BLK_M"},
            {"name": "Y_o_s", "type": "sv", "direction": "COL", "length": "K/BLK_K"},
            {"name": "X_i", "type": "df", "direction": "ROW", "length": "BLK_M"},
            {"name": "Y_i", "type": "df", "direction": "COL", "length": "BLK_K"}]}],
        "atomic": {"type": "dense", "x_axis": "X_i", "y_axis": "Y_i", "layout": "row_major"},
        "params": {"BLK_M": blk_m, "BLK_K": blk_k},
    }


def sparse_row_spec(blk_m: int = 16, blk_k: int = 8) -> dict:
    """Sparse-row domain over a column-condensed dense SR-BCRS hierarchy."""
    return {
        "format_name": f"SPARSE_ROW_SR_BCRS_{blk_m}x{blk_k}",
        "levels": [
            {"level": 1, "name": "sparse_rows", "axes": [
                {"name": "X_s", "type": "sv", "direction": "ROW", "length": "M"},
                {"name": "Y", "type": "df", "direction": "COL", "length": "K"}]},
            {"level": 2, "name": "row_window", "axes": [
                {"name": "X_so", "type": "df", "direction": "ROW", "length": "M/BLK_M"},
                {"name": "Y_s", "type": "sv", "direction": "COL", "length": "K"},
                {"name": "X_si", "type": "df", "direction": "ROW", "length": "BLK_M"}]},
            {"level": 3, "name": "condensed_block", "axes": [
                {"name": "Y_so", "type": "dv", "direction": "COL", "length": "K/BLK_K"},
                {"name": "Y_si", "type": "df", "direction": "COL", "length": "BLK_K"},
                {"name": "X_si", "type": "df", "direction": "ROW", "length": "BLK_M"}]},
        ],
        "atomic": {"type": "dense", "x_axis": "X_si", "y_axis": "Y_si", "layout": "row_major"},
        "params": {"BLK_M": blk_m, "BLK_K": blk_k},
    }


def sr_bcrs_spec(blk_m: int = 16, blk_k: int = 8) -> dict:
    """The SR-BCRS format spec (python/sparsene/formats/SR_BCRS.py:5-20 as a
    mapping, as python/test/run_builtin_backend_e2e.py:27-57 writes it)."""
    return {
        "format_name": f"SR_BCRS_{blk_m}x{blk_k}",
        "levels": [
            {"level": 1, "name": "row_window", "axes": [
                {"name": "X_o", "type": "df", "direction": "ROW", "length": "M"},
                {"name": "Y_s", "type": "sv", "direction": "COL", "length": "K"},
                {"name": "X_i", "type": "df", "direction": "ROW", "length": "BLK_M"}]},
            {"level": 2, "name": "condensed_block", "axes": [
                {"name": "Y_so", "type": "df", "direction": "COL", "length": "K/BLK_K"},
                {"name": "Y_si", "type": "df", "direction": "COL", "length": "BLK_K"},
                {"name": "X_i", "type": "df", "direction": "ROW", "length": "BLK_M"}]},
        ],
        "atomic": {"type": "dense", "x_axis": "X_i", "y_axis": "Y_si", "layout": "row_major"},
        "params": {"BLK_M": blk_m, "BLK_K": blk_k},
    }
