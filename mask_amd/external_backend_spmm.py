"""Drop-in for the reference's GCN SpMM backend bridge, SR-BCRS part.

Mirrors end2end/gcn/external_backend_spmm.py: the module-level entry
``srbcrs_spmm(rowptr, colind, values, dense, num_rows, feat_dim,
num_nodes_ori)`` (:1471-1485), the ``SRBCRSBackend`` variant router
(:494-942), tile selection / padding (:62-94), the preprocess cache keyed by
the CSR tensors (:789-841) and the SPARSENE_* environment knobs.  The work
is done by ``mask_amd.SRBCRSSpMM`` (the gfx950 C ABI); there is no
non-HIP path.

Variants (SPARSENE_SRBCRS_VARIANT, same spellings as the reference):
  base / strict_lb / multi_binding            32x32 blocks
  16x8 / 16x8_strict_lb / 16x8_multi_binding  16x8 blocks
The *_strict_lb / *_multi_binding variants run the matching atomic-free
schedule (the reference's SRBCRSSpMM module has no such entry points and
falls through to the plain kernel, external_backend_spmm.py:632-763).
"""
from __future__ import annotations

import os
from contextlib import contextmanager
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from . import SRBCRSSpMM

Tensor = torch.Tensor

_WARNED = set()


def _warn_once(msg: str) -> None:
    if msg not in _WARNED:
        print(f"[WARN] {msg}")
        _WARNED.add(msg)


def _csr_fallback_enabled() -> bool:
    # external_backend_spmm.py:40-42: disabled unless SPARSENE_ALLOW_CSR_FALLBACK=1
    return os.getenv("SPARSENE_ALLOW_CSR_FALLBACK", "0") == "1"


def _csr_kernel_spmm(rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int) -> Tensor:
    """The fallback: the native CSR HIP kernel (the reference falls back to
    torch.sparse.mm, external_backend_spmm.py:115-124)."""
    with _range("spmm.fallback.csr_kernel"):
        return SRBCRSSpMM.csr_spmm(rowptr.to(torch.int32).contiguous(), colind.to(torch.int32).contiguous(),
                                   values.to(torch.float32).contiguous(), dense.contiguous(), num_rows)


def _fallback_or_raise(msg: str, rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor,
                       num_rows: int) -> Tensor:
    if _csr_fallback_enabled():
        _warn_once(f"{msg}; fallback to the CSR kernel")
        return _csr_kernel_spmm(rowptr, colind, values, dense, num_rows)
    raise RuntimeError(f"{msg}. CSR fallback is disabled. "
                       "Set SPARSENE_ALLOW_CSR_FALLBACK=1 to re-enable fallback.")


def _parse_tile_env(tile_env: str) -> Optional[int]:
    raw = os.getenv(tile_env, "auto").strip().lower()
    if raw in {"", "auto"}:
        return None
    if raw in {"16", "32", "64"}:
        return int(raw)
    _warn_once(f"Invalid {tile_env}={raw}, expected auto/16/32/64; using auto")
    return None


def _select_tile_b(feat_dim: int, tile_env: str) -> int:
    """Least padding wins, ties go to the larger tile (external_backend_spmm.py:72-84)."""
    forced = _parse_tile_env(tile_env)
    candidates = [64, 32, 16] if forced is None else [forced]
    best, best_pad = candidates[0], -(-feat_dim // candidates[0]) * candidates[0] - feat_dim
    for t in candidates[1:]:
        pad = -(-feat_dim // t) * t - feat_dim
        if pad < best_pad or (pad == best_pad and t > best):
            best, best_pad = t, pad
    return best


def _pad_dense_to_tile(dense: Tensor, tile_b: int) -> Tuple[Tensor, int]:
    cols = int(dense.shape[1])
    padded = -(-cols // tile_b) * tile_b
    if padded == cols:
        return dense.contiguous(), cols
    return torch.nn.functional.pad(dense, (0, padded - cols)).contiguous(), cols


@contextmanager
def _range(name: str):
    """roctx range (torch.cuda.nvtx maps to roctx on ROCm), like the
    reference's NVTX ranges (external_backend_spmm.py:97-112)."""
    pushed = False
    if os.getenv("SPARSENE_ENABLE_NVTX", "1") == "1" and torch.cuda.is_available():
        try:
            torch.cuda.nvtx.range_push(name)
            pushed = True
        except Exception:
            pushed = False
    try:
        yield
    finally:
        if pushed:
            try:
                torch.cuda.nvtx.range_pop()
            except Exception:
                pass


@dataclass(frozen=True)
class BackendConfig:
    name: str
    variant: str


_VARIANT_ALIASES = {
    "base": {"", "base", "default", "srbcrs", "sr_bcrs"},
    "16x8": {"16x8", "16_8", "srbcrs_16x8", "sr_bcrs_16x8"},
    "multi_binding": {"multi_bind", "multi-binding", "multi_binding", "multibind"},
    "strict_lb": {"strict_lb", "strict-lb", "strictlb"},
    "16x8_multi_binding": {"16x8_multi_bind", "16x8_multibind", "16x8_multi_binding", "multi_bind_16x8",
                           "multi_binding_16x8", "multibind_16x8", "srbcrs_16x8_multi_bind",
                           "sr_bcrs_16x8_multi_bind"},
    "16x8_strict_lb": {"16x8_strict_lb", "16x8_strictlb", "strict_lb_16x8", "strictlb_16x8",
                       "srbcrs_16x8_strict_lb", "sr_bcrs_16x8_strict_lb"},
}

# variant -> (block shape, schedule)
_VARIANT_PLAN = {
    "base": ((32, 32), ("row", 0)),
    "strict_lb": ((32, 32), ("strict_lb", 0)),
    "multi_binding": ((32, 32), ("multi_bind", 0)),
    "16x8": ((16, 8), ("row", 0)),
    "16x8_strict_lb": ((16, 8), ("strict_lb", 0)),
    "16x8_multi_binding": ((16, 8), ("multi_bind", 0)),
}


class SRBCRSBackend:
    """SR-BCRS backend (external_backend_spmm.py:494-942) on the gfx950 module."""

    def __init__(self, variant: str) -> None:
        self.variant = self._normalize_variant(variant)
        self._cache: Dict[Tuple, Tuple] = {}
        self._i32_cache: Dict[Tuple, Tensor] = {}
        self._f32_cache: Dict[Tuple, Tensor] = {}

    @staticmethod
    def _normalize_variant(variant: str) -> str:
        v = (variant or "base").strip().lower()
        for name, spellings in _VARIANT_ALIASES.items():
            if v in spellings:
                return name
        return v

    @staticmethod
    def _variant_tile_shape(variant: str) -> Tuple[int, int]:
        return _VARIANT_PLAN.get(variant, _VARIANT_PLAN["base"])[0]

    def _to_i32_cached(self, t: Tensor) -> Tensor:
        if t.dtype == torch.int32 and t.is_contiguous():
            return t
        key = (int(t.data_ptr()), tuple(t.shape), str(t.device), t.dtype)
        c = self._i32_cache.get(key)
        if c is None:
            c = self._i32_cache[key] = t.to(torch.int32).contiguous()
        return c

    def _to_f32_cached(self, t: Tensor) -> Tensor:
        if t.dtype == torch.float32 and t.is_contiguous():
            return t
        key = (int(t.data_ptr()), tuple(t.shape), str(t.device), t.dtype)
        c = self._f32_cache.get(key)
        if c is None:
            c = self._f32_cache[key] = t.to(torch.float32).contiguous()
        return c

    def _get_preprocessed(self, rowptr: Tensor, colind: Tensor, values: Tensor, num_rows: int):
        if not (rowptr.is_cuda and colind.is_cuda and values.is_cuda):
            return None
        dh, dw = self._variant_tile_shape(self.variant)
        bh = int(os.getenv("SPARSENE_SRBCRS_BLK_H", str(dh)))
        bw = int(os.getenv("SPARSENE_SRBCRS_BLK_W", str(dw)))
        key = (int(rowptr.data_ptr()), int(colind.data_ptr()), int(values.data_ptr()), int(num_rows),
               int(colind.numel()), f"{self.variant}:{bh}x{bw}")
        hit = self._cache.get(key)
        if hit is not None:
            return hit
        mo = -(-num_rows // bh)
        nnz = int(colind.numel())
        dev = rowptr.device
        bp = torch.zeros(mo, dtype=torch.int32, device=dev)
        e2c = torch.zeros(nnz, dtype=torch.int32, device=dev)
        e2r = torch.zeros(nnz, dtype=torch.int32, device=dev)
        fn = SRBCRSSpMM.preprocess_gpu_16x8 if (bh, bw) == (16, 8) else SRBCRSSpMM.preprocess_gpu
        with _range("srbcrs.preprocess.extension"):
            prep = fn(self._to_i32_cached(colind), self._to_i32_cached(rowptr), self._to_f32_cached(values),
                      int(num_rows), bh, bw, bp, e2c, e2r)
        # keep the caller's tensors alive with the entry so the pointer key stays valid
        self._cache[key] = (prep, (rowptr, colind, values), (bh, bw))
        return self._cache[key]

    def _run_variant(self, rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int) -> Tensor:
        with _range(f"srbcrs.run.entry.{self.variant}"):
            got = self._get_preprocessed(rowptr, colind, values, num_rows)
            if got is None:
                return _fallback_or_raise(f"SR-BCRS preprocess unavailable for variant={self.variant}",
                                          rowptr, colind, values, dense, num_rows)
            (rwo, _rowid, tile_id, toff, a2x, _count), _, (bh, bw) = got
            if os.getenv("SPARSENE_SRBCRS_FORCE_N64_ALIGN", "0") == "1" and "SPARSENE_SRBCRS_TILE_B" not in os.environ:
                os.environ["SPARSENE_SRBCRS_TILE_B"] = "64"
            tile_b = _select_tile_b(int(dense.shape[1]), "SPARSENE_SRBCRS_TILE_B")
            os.environ["SRBCRS_TILE_B"] = str(tile_b)
            with _range(f"srbcrs.run.pad_tile{tile_b}"):
                dense_in, out_cols = _pad_dense_to_tile(dense, tile_b)
            exeplan = os.getenv("SPARSENE_SRBCRS_EXEPLAN", "")
            if not exeplan:
                pol, param = _VARIANT_PLAN.get(self.variant, _VARIANT_PLAN["base"])[1]
                exeplan = f"{pol}:{param}" if pol != "row" else ""
            use_balance = os.getenv("SPARSENE_SRBCRS_BALANCE", "0") == "1"
            is16 = (bh, bw) == (16, 8)
            try:
                with _range("srbcrs.run.balance" if use_balance else "srbcrs.run.default"):
                    if use_balance:
                        fn = SRBCRSSpMM.run_SRBCRS_16x8_balance if is16 else SRBCRSSpMM.run_SRBCRS_balance
                        out = fn(dense_in, rwo, tile_id, toff, a2x, int(num_rows), exeplan)
                    else:
                        fn = SRBCRSSpMM.run_SRBCRS_16x8 if is16 else SRBCRSSpMM.run_SRBCRS
                        out = fn(dense_in, rwo, tile_id, toff, a2x, int(num_rows), int(colind.numel()), exeplan)
            except RuntimeError as exc:
                return _fallback_or_raise(f"SR-BCRS run failed for variant={self.variant}: {exc}",
                                          rowptr, colind, values, dense, num_rows)
            out = out[0] if isinstance(out, (tuple, list)) else out
            if out.dim() == 2 and int(out.shape[1]) != out_cols:
                out = out[:, :out_cols].contiguous()
            return out

    def run(self, rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int, feat_dim: int,
            num_nodes_ori: int) -> Tensor:
        if self.variant not in _VARIANT_PLAN:
            _warn_once(f"Unknown SR-BCRS variant={self.variant}, fallback to base dispatch")
        return self._run_variant(rowptr, colind, values, dense, num_rows)


class BackendRouter:
    """Backend instances per config (external_backend_spmm.py:1377-1401);
    only the SR-BCRS backend exists here."""

    def __init__(self) -> None:
        self._instances: Dict[BackendConfig, SRBCRSBackend] = {}

    def get(self, cfg: BackendConfig) -> SRBCRSBackend:
        if cfg.name != "sr_bcrs":
            raise RuntimeError(f"backend '{cfg.name}' is not part of the gfx950 SR-BCRS backend; "
                               "use SPARSENE_SPMM_BACKEND=sr_bcrs")
        inst = self._instances.get(cfg)
        if inst is None:
            inst = self._instances[cfg] = SRBCRSBackend(cfg.variant)
        return inst


_ROUTER = BackendRouter()


def reset_backend_state() -> None:
    global _ROUTER
    _ROUTER = BackendRouter()


def _resolve_config() -> BackendConfig:
    name = os.getenv("SPARSENE_SPMM_BACKEND", "sr_bcrs").strip().lower()
    variant = os.getenv("SPARSENE_SPMM_VARIANT", "").strip().lower()
    if name == "sr_bcrs":
        v = os.getenv("SPARSENE_SRBCRS_VARIANT", variant or "base").strip().lower()
        return BackendConfig("sr_bcrs", v or "base")
    return BackendConfig(name or "sr_bcrs", variant or "base")


def spmm_external(rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int, feat_dim: int,
                  num_nodes_ori: int) -> Tensor:
    cfg = _resolve_config()
    with _range(f"spmm.dispatch.{cfg.name}.{cfg.variant}"):
        return _ROUTER.get(cfg).run(rowptr, colind, values, dense, num_rows, feat_dim, num_nodes_ori)


def srbcrs_spmm(rowptr: Tensor, colind: Tensor, values: Tensor, dense: Tensor, num_rows: int, feat_dim: int,
                num_nodes_ori: int) -> Tensor:
    """external_backend_spmm.py:1471-1485."""
    cfg = BackendConfig("sr_bcrs", os.getenv("SPARSENE_SRBCRS_VARIANT",
                                             os.getenv("SPARSENE_SPMM_VARIANT", "base")).strip().lower())
    return _ROUTER.get(cfg).run(rowptr, colind, values, dense, num_rows, feat_dim, num_nodes_ori)
