"""SR-BCRS part of the GCN script's external SpMM bridge, on the gfx950 module.

Interface kept from the reference bridge (end2end/gcn/external_backend_spmm.py):
the entry ``srbcrs_spmm(rowptr, colind, values, dense, num_rows, feat_dim,
num_nodes_ori)`` (:1471-1485), the generic ``spmm_external`` dispatcher, the
SPARSENE_* environment variables, the variant spellings and the error text of
the disabled CSR fallback (:40-59).  The code below is this package's own: a
plan cache keyed by the caller's CSR storage, feature widths rounded up to a
tile the kernel accepts, and the SR-BCRS module of ``mask_amd.SRBCRSSpMM``
doing the work.  There is no non-HIP path: the fallback, when enabled, is the
native CSR kernel.

Variants (SPARSENE_SRBCRS_VARIANT):
  base / strict_lb / multi_binding            32x32 blocks
  16x8 / 16x8_strict_lb / 16x8_multi_binding  16x8 blocks
The *_strict_lb / *_multi_binding variants run the matching atomic-free
schedule.
"""
from __future__ import annotations

import functools
import os
from contextlib import nullcontext
from typing import Dict, NamedTuple, Optional, Tuple

import torch

from . import SRBCRSSpMM

Tensor = torch.Tensor


# ---- variants -------------------------------------------------------------------------

class Variant(NamedTuple):
    """What a variant name means for the gfx950 module."""
    block: Tuple[int, int]          # SR-BCRS block (rows, columns)
    schedule: Tuple[str, int]       # srbcrs_plan_set_schedule policy and parameter


VARIANTS: Dict[str, Variant] = {
    "base": Variant((32, 32), ("row", 0)),
    "strict_lb": Variant((32, 32), ("strict_lb", 0)),
    "multi_binding": Variant((32, 32), ("multi_bind", 0)),
    "16x8": Variant((16, 8), ("row", 0)),
    "16x8_strict_lb": Variant((16, 8), ("strict_lb", 0)),
    "16x8_multi_binding": Variant((16, 8), ("multi_bind", 0)),
}


_SCHEDULE_WORDS = {"": "", "base": "", "default": "", "strict_lb": "strict_lb", "strictlb": "strict_lb",
                   "multi_bind": "multi_binding", "multi_binding": "multi_binding", "multibind": "multi_binding"}


def canonical_variant(name: Optional[str]) -> str:
    """The canonical variant for a user spelling.  Case, blanks, '-' vs '_',
    an srbcrs / sr_bcrs prefix and the position of the 16x8 (or 16_8) token
    do not matter; unknown names come back normalised and run as ``base``."""
    key = (name or "").strip().lower().replace("-", "_")
    for prefix in ("srbcrs", "sr_bcrs"):
        if key == prefix or key.startswith(prefix + "_"):
            key = key[len(prefix):].lstrip("_")
    small = False
    for tok in ("16x8", "16_8"):
        if key == tok or key.startswith(tok + "_") or key.endswith("_" + tok):
            key = key.replace(tok, "", 1).strip("_")
            small = True
            break
    word = _SCHEDULE_WORDS.get(key)
    if word is None:
        return (name or "").strip().lower()
    if small:
        return f"16x8_{word}" if word else "16x8"
    return word or "base"


# ---- feature-width tiles ------------------------------------------------------------

_TILES = (64, 32, 16)


def _round_up(x: int, t: int) -> int:
    return -(-x // t) * t


@functools.lru_cache(maxsize=None)
def _notice(msg: str) -> None:
    """Print a warning once per distinct message."""
    print(f"[WARN] {msg}")


def _forced_tile(env_name: str) -> Optional[int]:
    raw = os.getenv(env_name, "auto").strip().lower()
    if raw in ("", "auto"):
        return None
    if raw.isdigit() and int(raw) in _TILES:
        return int(raw)
    _notice(f"Invalid {env_name}={raw}, expected auto/16/32/64; using auto")
    return None


def _select_tile_b(feat_dim: int, env_name: str) -> int:
    """Tile of the dense width: the forced one, else the tile whose padded
    width is smallest, the wider tile on equal widths."""
    forced = _forced_tile(env_name)
    if forced is not None:
        return forced
    return min(_TILES, key=lambda t: (_round_up(feat_dim, t), -t))


def _pad_dense_to_tile(dense: Tensor, tile_b: int) -> Tuple[Tensor, int]:
    """(dense widened with zero columns to a multiple of tile_b, its original width)."""
    rows, cols = int(dense.shape[0]), int(dense.shape[1])
    width = _round_up(cols, tile_b)
    if width == cols:
        return dense.contiguous(), cols
    wide = dense.new_zeros((rows, width))
    wide[:, :cols].copy_(dense)
    return wide, cols


# ---- roctx ranges -------------------------------------------------------------------

@functools.lru_cache(maxsize=1)
def _markers_work() -> bool:
    """Whether roctx ranges can be pushed here (torch.cuda.nvtx maps to roctx on ROCm)."""
    if not torch.cuda.is_available():
        return False
    try:
        torch.cuda.nvtx.range_push("sparsene.probe")
        torch.cuda.nvtx.range_pop()
        return True
    except Exception:
        return False


def _range(name: str):
    """A roctx range around a region, on unless SPARSENE_ENABLE_NVTX=0."""
    if os.getenv("SPARSENE_ENABLE_NVTX", "1") == "1" and _markers_work():
        return torch.cuda.nvtx.range(name)
    return nullcontext()


# ---- CSR fallback -------------------------------------------------------------------

def _fallback_allowed() -> bool:
    return os.getenv("SPARSENE_ALLOW_CSR_FALLBACK", "0") == "1"


def _csr_or_raise(reason: str, rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor,
                  num_rows: int) -> Tensor:
    """The native CSR kernel when SPARSENE_ALLOW_CSR_FALLBACK=1, else the
    reference's error."""
    if not _fallback_allowed():
        raise RuntimeError(f"{reason}. CSR fallback is disabled. "
                           "Set SPARSENE_ALLOW_CSR_FALLBACK=1 to re-enable fallback.")
    _notice(f"{reason}; fallback to the CSR kernel")
    with _range("spmm.fallback.csr_kernel"):
        return SRBCRSSpMM.csr_spmm(rowptr.to(torch.int32).contiguous(), colind.to(torch.int32).contiguous(),
                                   values.to(torch.float32).contiguous(), dense.contiguous(), num_rows)


# ---- the backend ----------------------------------------------------------------------

class _Prepared(NamedTuple):
    arrays: tuple                   # the preprocess 6-tuple
    block: Tuple[int, int]
    keep: tuple                     # caller tensors and converted copies kept alive with the entry


class SRBCRSBackend:
    """One SR-BCRS variant: converts each distinct CSR once and runs the
    module's ``run_SRBCRS*`` on it."""

    def __init__(self, variant: str) -> None:
        self.variant = canonical_variant(variant)
        self._prepared: Dict[tuple, _Prepared] = {}

    @property
    def spec(self) -> Variant:
        return VARIANTS.get(self.variant, VARIANTS["base"])

    def _block(self) -> Tuple[int, int]:
        bh, bw = self.spec.block
        return (int(os.getenv("SPARSENE_SRBCRS_BLK_H", str(bh))), int(os.getenv("SPARSENE_SRBCRS_BLK_W", str(bw))))

    def _prepare(self, rowptr: Tensor, colind: Tensor, values: Tensor, num_rows: int) -> Optional[_Prepared]:
        if not (rowptr.is_cuda and colind.is_cuda and values.is_cuda):
            return None
        block = self._block()
        key = (rowptr.data_ptr(), colind.data_ptr(), values.data_ptr(), int(num_rows), colind.numel(), block)
        hit = self._prepared.get(key)
        if hit is not None:
            return hit
        rp = rowptr if rowptr.dtype == torch.int32 else rowptr.to(torch.int32)
        ci = colind if colind.dtype == torch.int32 else colind.to(torch.int32)
        vv = values if values.dtype == torch.float32 else values.to(torch.float32)
        rp, ci, vv = rp.contiguous(), ci.contiguous(), vv.contiguous()
        bh, bw = block
        windows = _round_up(int(num_rows), bh) // bh
        i32 = dict(dtype=torch.int32, device=rowptr.device)
        edge_maps = (torch.zeros(windows, **i32), torch.zeros(ci.numel(), **i32), torch.zeros(ci.numel(), **i32))
        prep = SRBCRSSpMM.preprocess_gpu_16x8 if block == (16, 8) else SRBCRSSpMM.preprocess_gpu
        with _range("srbcrs.preprocess.extension"):
            arrays = prep(ci, rp, vv, int(num_rows), bh, bw, *edge_maps)
        entry = _Prepared(arrays, block, (rowptr, colind, values, rp, ci, vv))
        self._prepared[key] = entry
        return entry

    def _exeplan(self) -> str:
        plan = os.getenv("SPARSENE_SRBCRS_EXEPLAN", "")
        if plan:
            return plan
        policy, param = self.spec.schedule
        return "" if policy == "row" else f"{policy}:{param}"

    def run(self, rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int, feat_dim: int,
            num_nodes_ori: int) -> Tensor:
        if self.variant not in VARIANTS:
            _notice(f"Unknown SR-BCRS variant={self.variant}, fallback to base dispatch")
        with _range(f"srbcrs.run.entry.{self.variant}"):
            prepared = self._prepare(rowptr, colind, values, num_rows)
            if prepared is None:
                return _csr_or_raise(f"SR-BCRS preprocess unavailable for variant={self.variant}",
                                     rowptr, colind, values, dense, num_rows)
            if os.getenv("SPARSENE_SRBCRS_FORCE_N64_ALIGN", "0") == "1" and "SPARSENE_SRBCRS_TILE_B" not in os.environ:
                os.environ["SPARSENE_SRBCRS_TILE_B"] = "64"
            tile = _select_tile_b(int(dense.shape[1]), "SPARSENE_SRBCRS_TILE_B")
            os.environ["SRBCRS_TILE_B"] = str(tile)   # the module validates the width against it
            with _range(f"srbcrs.run.pad_tile{tile}"):
                wide, width = _pad_dense_to_tile(dense, tile)
            rwo, _rowid, tile_id, toff, a2x, _total = prepared.arrays
            balance = os.getenv("SPARSENE_SRBCRS_BALANCE", "0") == "1"
            small = prepared.block == (16, 8)
            try:
                with _range("srbcrs.run.balance" if balance else "srbcrs.run.default"):
                    if balance:
                        f = SRBCRSSpMM.run_SRBCRS_16x8_balance if small else SRBCRSSpMM.run_SRBCRS_balance
                        res = f(wide, rwo, tile_id, toff, a2x, int(num_rows), self._exeplan())
                    else:
                        f = SRBCRSSpMM.run_SRBCRS_16x8 if small else SRBCRSSpMM.run_SRBCRS
                        res = f(wide, rwo, tile_id, toff, a2x, int(num_rows), colind.numel(), self._exeplan())
            except RuntimeError as exc:
                return _csr_or_raise(f"SR-BCRS run failed for variant={self.variant}: {exc}",
                                     rowptr, colind, values, dense, num_rows)
            out = res[0] if isinstance(res, (list, tuple)) else res
            return out if out.shape[1] == width else out[:, :width].contiguous()


_backends: Dict[str, SRBCRSBackend] = {}


def reset_backend_state() -> None:
    """Forget every backend instance and the CSR conversions they hold."""
    _backends.clear()


def _backend(variant: str) -> SRBCRSBackend:
    v = canonical_variant(variant)
    if v not in _backends:
        _backends[v] = SRBCRSBackend(v)
    return _backends[v]


def _env_variant() -> str:
    return os.getenv("SPARSENE_SRBCRS_VARIANT", os.getenv("SPARSENE_SPMM_VARIANT", "") or "base")


def spmm_external(rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int, feat_dim: int,
                  num_nodes_ori: int) -> Tensor:
    """The generic dispatcher: SPARSENE_SPMM_BACKEND must name sr_bcrs (the
    only backend of this package)."""
    name = os.getenv("SPARSENE_SPMM_BACKEND", "sr_bcrs").strip().lower() or "sr_bcrs"
    if name != "sr_bcrs":
        raise RuntimeError(f"backend '{name}' is not part of the gfx950 SR-BCRS backend; "
                           "use SPARSENE_SPMM_BACKEND=sr_bcrs")
    b = _backend(_env_variant())
    with _range(f"spmm.dispatch.sr_bcrs.{b.variant}"):
        return b.run(rowptr, colind, values, dense, num_rows, feat_dim, num_nodes_ori)


def srbcrs_spmm(rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int, feat_dim: int,
                num_nodes_ori: int) -> Tensor:
    """C = A @ dense for the CSR A (external_backend_spmm.py:1471-1485)."""
    return _backend(_env_variant()).run(rowptr, colind, values, dense, num_rows, feat_dim, num_nodes_ori)
