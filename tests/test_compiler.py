"""Compiler-side boundary (no GPU): select_backend for gfx950 and the HIP
emitter's structure, knob mapping and determinism."""
from __future__ import annotations

import copy
import json
from types import SimpleNamespace

import pytest

from mask_amd.backend_registry import BackendPlan, select_backend, sr_bcrs_spec
from mask_amd.emitter import HipCodeGenerator, KernelParams, emit_source, operator_sha256, params_from_strategy


def test_select_backend_sr_bcrs():
    p = select_backend(sr_bcrs_spec(), target="gfx950")
    assert isinstance(p, BackendPlan)
    assert (p.codegen_format_name, p.packing_mode, p.target) == ("SR_BCRS", "column_condensed_dense", "gfx950")
    assert (p.physical_blk_m, p.physical_blk_k) == (16, 8)
    assert (p.mma_m, p.mma_n, p.mma_k) == (16, 16, 4)
    assert select_backend(sr_bcrs_spec(32, 32), target="MI355X").physical_blk_m == 32
    # the inner condensed-block axis may be a variable-length sequence (dv)
    spec = sr_bcrs_spec()
    spec["levels"][1]["axes"][0]["type"] = "dv"
    assert select_backend(spec).codegen_format_name == "SR_BCRS"


@pytest.mark.parametrize("mutate,msg", [
    (lambda s: s.update(atomic={"type": "mco", "x_axis": "X_i", "y_axis": "Y_si"}), "dense atomic"),
    (lambda s: s["levels"].pop(), "requires axis Y_o_s"),
    (lambda s: s["levels"][0]["axes"][1].update(type="df"), "axis Y_s"),
    (lambda s: s["atomic"].update(y_axis="Y_so"), "x_axis=X_i and y_axis=Y_si"),
    (lambda s: s["atomic"].update(layout="col_major"), "row-major"),
    (lambda s: s["params"].update(BLK_M=8), "BLK_M x BLK_K"),
    (lambda s: s["params"].pop("BLK_K"), "concrete integer"),
    (lambda s: s["levels"][0]["axes"][0].update(reorder="random"), "reorder contract"),
    (lambda s: s["levels"][0]["axes"][1].update(reorder="row_rcm"), "outer sparse/dense row axis"),
    (lambda s: s["levels"].extend([s["levels"][0], s["levels"][1]]), "hierarchy"),
    (lambda s: s["levels"].append(s["levels"][0]), "requires axis X_s"),
])
def test_select_backend_rejects(mutate, msg):
    spec = copy.deepcopy(sr_bcrs_spec())
    mutate(spec)
    with pytest.raises(ValueError, match=msg):
        select_backend(spec)


def test_select_backend_other_sr_bcrs_hierarchies():
    from mask_amd.backend_registry import fixed_block_spec, plan_options, sparse_row_spec
    fb = select_backend(fixed_block_spec())
    assert (fb.packing_mode, fb.codegen_format_name) == ("active_fixed_blocks_dense", "SR_BCRS")
    assert plan_options(fb)["packing"] == "active_fixed_blocks_dense"
    sr = select_backend(sparse_row_spec(32, 32))
    assert sr.packing_mode == "sparse_row_column_condensed_dense" and sr.physical_blk_m == 32
    assert plan_options(sr)["row_order"] == "sparse_rows" and plan_options(sr)["dup"] == "sum"
    spec = sr_bcrs_spec()
    spec["levels"][0]["axes"][0]["reorder"] = "jaccard_greedy"
    p = select_backend(spec)
    assert p.row_reorder == "jaccard_greedy" and plan_options(p)["row_order"] == "jaccard_greedy"
    bad = sparse_row_spec()
    bad["levels"][0]["axes"][0]["reorder"] = "row_rcm"
    with pytest.raises(ValueError, match="does not yet compose"):
        select_backend(bad)
    bad = fixed_block_spec()
    bad["atomic"]["y_axis"] = "Y_o_s"
    with pytest.raises(ValueError, match="y_axis=Y_i"):
        select_backend(bad)


def test_select_backend_targets_and_tiles():
    with pytest.raises(ValueError, match="Unknown target"):
        select_backend(sr_bcrs_spec(), target="sm80")
    with pytest.raises(ValueError, match="tile_n"):
        select_backend(sr_bcrs_spec(), tile_n=24)


def _strategy(**kw):
    tp = SimpleNamespace(tile_b=kw.get("tile_b", 64), b_smem_swizzle="swizzle_323",
                         materialize_b_array_ref_to_smem=kw.get("b_smem", False),
                         b_array_ref_mode=kw.get("b_mode", "cp_async_1x4"))
    pl = SimpleNamespace(enable_async_pipeline=kw.get("pipe", True), max_wait_prior=kw.get("mwp"),
                         stage_shifts=kw.get("shifts", []))
    rs = SimpleNamespace(execution_policy=kw.get("policy", "auto"), task_group_tiles=kw.get("tgt", 64),
                         runtime_max_tiles_per_segment=kw.get("cap", 0))
    return SimpleNamespace(tensor_placement=tp, pipeline=pl, runtime_schedule=rs)


def test_strategy_knob_mapping():
    plan = select_backend(sr_bcrs_spec())
    p = params_from_strategy(None, plan)
    assert p == KernelParams()
    assert params_from_strategy(_strategy(tile_b=32), plan).vec == 2
    assert params_from_strategy(_strategy(tile_b=32), plan).col_groups == 1
    assert params_from_strategy(_strategy(mwp=3), plan).depth == 8
    assert params_from_strategy(_strategy(shifts=[2, 1]), plan).depth == 4
    assert params_from_strategy(_strategy(mwp=3, pipe=False), plan).depth == 2
    sl = params_from_strategy(_strategy(policy="strict_lb", tgt=32), plan)
    assert (sl.schedule, sl.schedule_param) == ("strict_lb", 32)
    sp = params_from_strategy(_strategy(cap=48), plan)
    assert (sp.schedule, sp.schedule_param) == ("split", 48)
    # dict form of the strategy works too
    assert params_from_strategy({"tensor_placement": {"tile_b": 16}}, plan).vec == 1
    p32 = params_from_strategy(None, select_backend(sr_bcrs_spec(32, 32)))
    assert (p32.blk_m, p32.blk_k, p32.col_groups) == (32, 32, 1)
    # B placement: LDS staging only for the gfx950 mode global_load_lds, at vec 4; the
    # reference's default shared-memory staging maps to the (faster) register ring
    assert params_from_strategy(_strategy(b_smem=True, b_mode="global_load_lds"), plan).b_lds
    assert not params_from_strategy(_strategy(b_smem=True), plan).b_lds
    assert not params_from_strategy(_strategy(b_smem=True, b_mode="global_load_lds", tile_b=32), plan).b_lds
    assert not params_from_strategy(_strategy(b_mode="global_load_lds"), plan).b_lds
    assert params_from_strategy({"tensor_placement": {"materialize_b_array_ref_to_smem": True,
                                                      "b_array_ref_mode": "global_load_lds"}}, plan).b_lds


def test_emitted_source_structure_and_determinism():
    plan = select_backend(sr_bcrs_spec())
    prog = SimpleNamespace(name="SR_BCRS_16x8", attrs={
        "format_name": "SR_BCRS", "strategy_decision": _strategy(tile_b=64, mwp=2),
        "specialized_parameters": {"NNZ_HINT": 7}, "launch_contract": {"synchronization": "warp"}})
    gen = HipCodeGenerator(plan)
    src = gen.dump_nvop_program(prog)
    assert src == gen.dump_nvop_program(prog)
    for needle in ("#define SPARSENE_GENERATED_TILE_B 64", "#define SPARSENE_GENERATED_SUPPORTS_TASK_MAPPING 1",
                   "#define SPARSENE_GENERATED_WAVE_SIZE 64", "#define SPARSENE_GENERATED_PIPELINE_DEPTH 4",
                   "constexpr int NNZ_HINT = 7;", '#include "srbcrs_stream.hpp"',
                   "srbcrs::spmm_stream<Src, kBH, kBW, kVEC, kG, kWAVES, kDEPTH, AF, kBSTAGE>",
                   "srbcrs::CompactA{", "srbcrs::DenseA{",
                   "constexpr int kBSTAGE = 0;",
                   'extern "C" int sparsene_generated_run(', 'extern "C" int sparsene_generated_run_tasks(',
                   'extern "C" int sparsene_generated_reduce('):
        assert needle in src, needle
    meta = json.loads(src.split('R"JSON(')[1].split(')JSON"')[0])
    assert meta["kernel_params"]["depth"] == 4 and meta["format_name"] == "SR_BCRS"
    assert meta["kernel_parameter_order"][:5] == ["dB_val", "dC_val", "dval_len_offset", "dval_new",
                                                  "dval_sidx_new"]
    assert meta["notes"]["ignored_knobs"]["b_smem_swizzle"] == "swizzle_323"
    assert "cp.async" not in src and "__syncwarp" not in src and "mma.sync" not in src
    assert operator_sha256(src) != operator_sha256(emit_source(KernelParams()))


def test_emitter_rejects_other_formats_and_bad_params():
    gen = HipCodeGenerator()
    with pytest.raises(NotImplementedError):
        gen.dump_nvop_program(SimpleNamespace(name="x", attrs={"format_name": "ME_TCF"}))
    with pytest.raises(ValueError, match="specialized"):
        gen.dump_nvop_program(SimpleNamespace(name="x", attrs={"format_name": "SR_BCRS",
                                                               "specialized_parameters": {"BLK_M": 4}}))
    with pytest.raises(ValueError):
        emit_source(KernelParams(depth=3))
    with pytest.raises(ValueError):
        emit_source(KernelParams(vec=2, col_groups=1, b_lds=True))
    emit_source(KernelParams(blk_m=32, blk_k=32, col_groups=2))   # 128-column 32x32 waves, as in the library


def test_generated_operators_are_built():
    """build() emitted and compiled the generated operators (travel with the tree)."""
    from mask_amd.build import GENERATED, GENERATED_SHAPES
    for bm, bk, lds in GENERATED_SHAPES:
        so = GENERATED / f"sr_bcrs_{bm}x{bk}{'_lds' if lds else ''}.so"
        assert so.exists(), so
        import ctypes
        L = ctypes.CDLL(str(so))
        L.sparsene_generated_metadata.restype = ctypes.c_char_p
        meta = json.loads(L.sparsene_generated_metadata().decode())
        assert meta["kernel_params"]["blk_m"] == bm and meta["target"] == "gfx950"
        assert meta["kernel_params"]["b_lds"] == lds


# ---- the reference compiler's SR_BCRS program (tests/golden/sr_bcrs_nvir_abi.json) ----

def _fixture():
    from pathlib import Path
    return json.loads((Path(__file__).resolve().parent / "golden" / "sr_bcrs_nvir_abi.json").read_text())


def _program_from_fixture(entry):
    gmem = {n: SimpleNamespace(dtype=v["dtype"], shape=v["shape"]) for n, v in entry["gmem_inouts"].items()}
    return SimpleNamespace(name=entry["program_name"], attrs=copy.deepcopy(entry["attrs"]), gmem_inouts=gmem)


def test_emitter_accepts_the_reference_sr_bcrs_program():
    """The gmem interface the reference's middle end produces for SR_BCRS is
    exactly the operand set the emitted operator's run entry takes, in the
    reference kernel's parameter order; its strategy attributes map onto the
    template parameters."""
    from mask_amd.emitter import SR_BCRS_GMEM_ABI, SR_BCRS_VARLENS, check_gmem_abi
    fx = _fixture()["programs"]
    for key, entry in fx.items():
        assert set(entry["gmem_inouts"]) == set(SR_BCRS_GMEM_ABI), key
        assert tuple(entry["varlens"]) == SR_BCRS_VARLENS
        prog = _program_from_fixture(entry)
        check_gmem_abi(prog)
        src = HipCodeGenerator(select_backend(sr_bcrs_spec())).dump_nvop_program(prog)
        meta = json.loads(src.split('R"JSON(')[1].split(')JSON"')[0])
        assert meta["kernel_parameter_order"] == entry["kernel_parameter_order"], key
        # the run entry's first ten parameters, as declared in the source
        decl = src.split('extern "C" int sparsene_generated_run(')[1].split(")")[0]
        names = [a.strip().split()[-1].lstrip("*") for a in decl.split(",")][:10]
        assert names == entry["kernel_parameter_order"], names
    p_default = params_from_strategy(fx["default"]["attrs"]["strategy_decision"], select_backend(sr_bcrs_spec()))
    assert (p_default.vec, p_default.depth, p_default.b_lds, p_default.schedule) == (4, 2, False, "auto")
    p32 = params_from_strategy(fx["tile32_wait2"]["attrs"]["strategy_decision"], select_backend(sr_bcrs_spec()))
    assert (p32.vec, p32.col_groups, p32.depth) == (2, 1, 4)


@pytest.mark.parametrize("mutate,msg", [
    (lambda g: g.pop("val_sidx_new"), "missing"),
    (lambda g: g.update(extra_ptr=SimpleNamespace(dtype="int", shape="(Varlen(M))")), "unexpected"),
    (lambda g: g.update(val_new=SimpleNamespace(dtype="half", shape=g["val_new"].shape)), "dtype"),
    (lambda g: g.update(val_len_offset=SimpleNamespace(dtype="int", shape="(Varlen(Mo), Param(X))")), "rank"),
])
def test_emitter_rejects_a_mismatched_gmem_interface(mutate, msg):
    prog = _program_from_fixture(_fixture()["programs"]["default"])
    mutate(prog.gmem_inouts)
    with pytest.raises(ValueError, match=msg):
        HipCodeGenerator().dump_nvop_program(prog)


def test_lower_format_operator_signature_and_result(tmp_path, monkeypatch):
    """lower_format_operator takes the reference's keyword-only arguments
    and returns its keys (generate_custom_format_operators.py:88-157)."""
    import inspect
    from mask_amd import emitter
    sig = inspect.signature(emitter.lower_format_operator)
    for name in ("format_obj", "codegen_format_name", "operator_path", "ir_dir", "strategy_dir",
                 "strategy_decision", "specialized_parameters", "preserve_scalar_offset_divisors",
                 "explicit_sequential_iteration", "diagnostic_program_transform"):
        assert sig.parameters[name].kind is inspect.Parameter.KEYWORD_ONLY, name
    compiled = []

    def fake_compile(source, out_path):
        compiled.append(out_path)
        out_path.with_suffix(".hip").write_text(source)
        return out_path
    monkeypatch.setattr(emitter, "compile_operator", fake_compile)
    seen = []
    res = emitter.lower_format_operator(format_obj=sr_bcrs_spec(), codegen_format_name="SR_BCRS",
                                        operator_path=tmp_path / "op.so", ir_dir=tmp_path / "ir",
                                        strategy_dir=tmp_path / "st", strategy_decision={"pipeline": {"max_wait_prior": 3}},
                                        specialized_parameters={"NNZ_HINT": 3},
                                        diagnostic_program_transform=seen.append)
    assert {"operator_sha256", "lowered_block_barriers", "strategy_decision", "gmem_inouts"} <= set(res)
    assert res["lowered_block_barriers"] == 0 and len(seen) == 1
    assert set(res["gmem_inouts"]) == set(_fixture()["programs"]["default"]["gmem_inouts"])
    assert res["kernel_params"]["depth"] == 8
    src = (tmp_path / "op.hip").read_text()
    import hashlib
    assert res["operator_sha256"] == hashlib.sha256(src.encode()).hexdigest()
    assert "constexpr int NNZ_HINT = 3;" in src and (tmp_path / "ir" / "06_nvir_before_pipeline.txt").exists()
    with pytest.raises(NotImplementedError):
        emitter.lower_format_operator(format_obj=sr_bcrs_spec(), codegen_format_name="ME_TCF",
                                      operator_path=tmp_path / "x.so", ir_dir=tmp_path, strategy_dir=tmp_path)


def test_generated_operator_passes_gmem_pointers_in_declared_order():
    """GeneratedOperator hands the five gmem pointers to the generated entry
    in the order the operator declares (dB_val, dC_val, dval_len_offset,
    dval_new, dval_sidx_new): values before column indices.  A transposed
    pair makes the kernel read block values as B-row indices."""
    from mask_amd.build import GENERATED
    from mask_amd.emitter import GeneratedOperator
    so = GENERATED / "sr_bcrs_16x8.so"
    if not so.exists():
        pytest.skip("generated operators not built")
    op = GeneratedOperator(so)
    t = lambda p: SimpleNamespace(data_ptr=lambda: p)
    desc = SimpleNamespace(d_soff=3, d_val=4, d_sidx=5)
    assert op._gmem(t(1), t(2), desc) == (1, 2, 3, 4, 5)
    assert op.metadata["kernel_parameter_order"][:5] == ["dB_val", "dC_val", "dval_len_offset", "dval_new",
                                                         "dval_sidx_new"]
