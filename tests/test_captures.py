"""The capture-format report for the reference's ``fastkernels bench`` harness
(fastkernels_amd/captures/decode_step_configs.json): it is what the generator
writes, and every entry binds to the candidate classes the way the harness binds
it (bench.py:274-300 discovery, :962-987 forward-argument binding, capture.py:464-494
constructor recipes)."""
from __future__ import annotations

import importlib.util
import inspect
import json
from pathlib import Path

import pytest

from fastkernels_amd.captures import make_reports

ROOT = Path(__file__).resolve().parents[1]
REPORT = ROOT / "fastkernels_amd" / "captures" / "decode_step_configs.json"
CAND = ROOT / "fastkernels_amd" / "candidate" / "L1"


def _cls(qualname):
    mod, cls = qualname.split(":")
    stem = mod.rsplit(".", 1)[-1]
    spec = importlib.util.spec_from_file_location(f"_cap_{stem}", CAND / f"{stem}.py")
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return getattr(m, cls)


def test_report_is_generated_file():
    assert json.loads(REPORT.read_text()) == json.loads(json.dumps(make_reports.build()))


def _is_tensor(v):
    return isinstance(v, dict) and isinstance(v.get("shape"), list) and isinstance(v.get("dtype"), str)


@pytest.mark.parametrize("qualname", sorted(make_reports.build()["operators"]))
def test_entries_bind_to_candidates(qualname):
    assert ".tasks.baseline." in qualname
    entry = make_reports.build()["operators"][qualname]
    cls = _cls(qualname)
    init_params = inspect.signature(cls.__init__).parameters
    for v in entry["init"]["variants"]:
        for name in v["args"]:
            assert name in init_params, f"{qualname}: unknown constructor arg {name}"
        cls(**v["args"])  # constructible from the recipe (scalars only)
    fwd = list(inspect.signature(cls.forward).parameters.values())[1:]
    n_init = len(entry["init"]["variants"])
    for v in entry["forward"]["variants"]:
        assert all(0 <= i < n_init for i in v["init_variant_ids"])
        args = v["args"]
        for p in fwd:
            if p.kind is p.VAR_KEYWORD:
                assert isinstance(args.get(p.name, {}), dict)
            elif p.default is inspect.Parameter.empty:
                assert p.name in args, f"{qualname}: missing required forward arg {p.name}"
        names = {p.name for p in fwd}
        assert set(args) <= names, f"{qualname}: unknown forward args {set(args) - names}"
        for name, val in args.items():
            if isinstance(val, dict) and "shape" in val:
                assert _is_tensor(val)
                if "stride" in val:
                    assert len(val["stride"]) == len(val["shape"])
