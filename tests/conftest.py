"""Shared test setup.

Markers: ``gpu`` -- needs an MI355X (run with ``-m gpu``); everything else runs
on the CPU.  The package directory is not a Python identifier, so it is
imported through ``__graft_entry__.package()``.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X GPU (gfx950)")


# (tag, outputs checked, outputs that needed the float64 value) per output check
# of the parity tests, reported at the end of the session
OUTPUT_CHECKS: list = []


def pytest_terminal_summary(terminalreporter):
    if not OUTPUT_CHECKS:
        return
    n = sum(c[1] for c in OUTPUT_CHECKS)
    fb = [c for c in OUTPUT_CHECKS if c[2]]
    terminalreporter.write_line(
        f"bf16 output bar: {len(OUTPUT_CHECKS)} checks, {n} outputs; {sum(c[2] for c in fb)} outside 1 ulp of "
        f"the fp32 oracle, all within 1 ulp of the float64 value, in {len(fb)} checks")
    for tag, size, k in fb[:40]:
        terminalreporter.write_line(f"  {tag}: {k} of {size}")


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.package()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def bf16_bits_tensor(bits: np.ndarray):
    """uint16 numpy bf16 bits -> torch.bfloat16 tensor (CPU)."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def tensor_bf16_bits(t) -> np.ndarray:
    """torch.bfloat16 tensor -> uint16 numpy bits."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def tie_rows(n_rows: int = 64, K: int = 256, seed: int = 0) -> np.ndarray:
    """bf16 rows (uint16 bits [n_rows, K]) full of exact half-way quotients x/s = k + 0.5.

    Each row's absmax fixes a bf16 scale s = bf16(amax/127) whose fp32 reciprocal
    is inexact, and the rest of the row are bf16 values x with x/s an exact
    half-integer, so round-half-to-even is exercised where a reciprocal multiply
    would round the other way.
    """
    from oracle import w4a8 as ow
    rng = np.random.default_rng(seed)
    rows = []
    e_choices = list(range(-20, 4))
    while len(rows) < n_rows:
        e = int(rng.choice(e_choices))
        m = int(rng.integers(128, 256))
        amax = np.float32(m * 2.0 ** (e - 7)) * np.float32(127.0)
        ab = ow.f32_to_bf16_bits(np.array([amax], np.float32))
        s_b = ow.group_params_sym(ow.bf16_bits_to_f32(ab)[None, :], 8)[0]
        s = float(ow.bf16_bits_to_f32(np.array([s_b]))[0])
        ties = []
        for k in range(-127, 127):
            x = np.float32((k + 0.5) * s)
            xb = ow.f32_to_bf16_bits(np.array([x], np.float32))
            if float(ow.bf16_bits_to_f32(xb)[0]) == float(x) and abs(float(x)) <= float(ow.bf16_bits_to_f32(ab)[0]):
                ties.append(int(xb[0]))
        if not ties:
            continue
        row = np.array([ties[i % len(ties)] for i in range(K)], np.uint16)
        row[int(rng.integers(0, K))] = ab[0]
        rows.append(row)
    return np.stack(rows)
