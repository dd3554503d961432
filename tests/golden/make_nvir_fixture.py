"""Write tests/golden/sr_bcrs_nvir_abi.json: the gmem interface and the
attributes of the reference compiler's SR_BCRS NVIR program (the operands a
generated operator receives, in the order its kernel takes them, and the
strategy / launch attributes an emitter reads), for two strategies.

Runs only in the build container, where the reference tree is mounted
(REFERENCE_ROOT, default /root/reference); the GPU box never runs it.  It
drives the reference's own middle end the way its test
python/test/test_nvir_semantic_fusion.py:48-62 does (Format -> RTS ->
Computent -> OPIR -> varlen lowering -> cval flattening -> generate_nvir with
a fixed StrategyDecision) and records, as data only: the program name, each
gmem in/out's name, dtype and shape, the varlen parameters, and the kernel
parameter order of codegen.py:2092-2140 (gmem pointers sorted by name, then
varlens sorted).  No reference source text is copied into the fixture.
"""
from __future__ import annotations

import contextlib
import copy
import io
import json
import os
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "sr_bcrs_nvir_abi.json"


def main() -> None:
    ref = Path(os.environ.get("REFERENCE_ROOT", "/root/reference"))
    sys.path.insert(0, str(ref / "python"))
    from sparsene.formats.SR_BCRS import SR_BCRS_FORMAT
    from sparsene.op_gen.computent.computent import computent_from_rts
    from sparsene.op_gen.nvir.generate import generate_nvir
    from sparsene.op_gen.opir.cValFlattenPass import CValFlattenPass
    from sparsene.op_gen.opir.generate import generate_from_computent
    from sparsene.op_gen.opir.varlenLoweringPass import VarlenLoweringPass
    from sparsene.op_gen.strategy_agent import PipelineStrategy, StrategyDecision, TensorPlacementStrategy
    from sparsene.transform.rts import derive_rts

    import dataclasses

    strategies = {
        "default": StrategyDecision(provider="fixture", rationale="gmem ABI fixture",
                                    tensor_placement=TensorPlacementStrategy(), pipeline=PipelineStrategy()),
        "tile32_wait2": StrategyDecision(provider="fixture", rationale="gmem ABI fixture",
                                         tensor_placement=TensorPlacementStrategy(
                                             tile_b=32, materialize_b_array_ref_to_smem=False),
                                         pipeline=PipelineStrategy(max_wait_prior=2)),
    }
    programs = {}
    for key, strategy in strategies.items():
        with contextlib.redirect_stdout(io.StringIO()):
            computent = computent_from_rts("SR_BCRS", derive_rts(copy.deepcopy(SR_BCRS_FORMAT)))
            ops = generate_from_computent(computent)
            lowered = VarlenLoweringPass(op_builder=None,
                                         varlen2LenArrayTable=computent.varlen2LenArrayTable).run(ops)
            flat = CValFlattenPass(op_builder=None).run(lowered)
            program = generate_nvir(opir=flat, format_name="SR_BCRS", strategy_decision_override=strategy,
                                    strategy_log_dir_override="")
        gmem = {name: {"dtype": str(io_.dtype), "shape": str(io_.shape)}
                for name, io_ in program.gmem_inouts.items()}
        varlens = sorted(str(v) for v in program.all_varlens())
        attrs = {}
        for k, v in program.attrs.items():
            if dataclasses.is_dataclass(v):
                v = dataclasses.asdict(v)
            try:
                json.dumps(v)
            except TypeError:
                v = str(v)
            attrs[k] = v
        programs[key] = {
            "program_name": str(program.name),
            "gmem_inouts": gmem,
            "varlens": varlens,
            "kernel_parameter_order": [f"d{n}" for n in sorted(gmem)] + varlens,
            "attrs": attrs,
        }
    fixture = {
        "source": "reference compiler, SR_BCRS format (python/sparsene/formats/SR_BCRS.py), generate_nvir",
        "programs": programs,
    }
    OUT.write_text(json.dumps(fixture, indent=1, sort_keys=True) + "\n")
    print(json.dumps(fixture, indent=1, sort_keys=True))


if __name__ == "__main__":
    main()
