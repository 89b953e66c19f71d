"""Bitwise regression of the HIP path against committed output digests.

Old-against-new bit equality, the reference's own check for kernel changes
(npu_ops/python/test_pad_regress.py:1-18): every case of
tests/golden/make_regress.py is recomputed and its SHA-256 compared with
tests/golden/output_digests.json.  A mismatch means a kernel or a plan now
produces different output bits: run the parity suite, and if the change is
intended, regenerate the digests with that script.
"""
from __future__ import annotations

import importlib.util
import json
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _module():
    spec = importlib.util.spec_from_file_location("make_regress", GOLDEN / "make_regress.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


MR = _module()
DOC = json.loads((GOLDEN / "output_digests.json").read_text())


@pytest.mark.parametrize("name", sorted(MR.CASES))
def test_output_bits_unchanged(pkg, dev, name):
    if MR.cu_count() != DOC["cu_count"]:
        pytest.skip(f"digests recorded on {DOC['cu_count']} CUs (the plans follow the CU count)")
    print(f"regress case {name}", flush=True)
    got = MR.CASES[name][1](pkg, dev)
    assert got == DOC["digests"][name], f"{name} ({MR.CASES[name][0]}): output bits changed"


def test_every_case_has_a_digest():
    assert set(DOC["digests"]) == set(MR.CASES)
