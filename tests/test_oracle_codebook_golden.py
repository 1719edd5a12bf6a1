"""The oracle's W4A8 codebook choice against the reference's own.

tests/golden/codebook_golden.json holds the tables that the reference's `_codebook_for` (and
through it `_fit_codebook`, CK/backends/eager/w4a8_int8.py:23-97) returned on the CPU for seeded
group-normalised inputs: heavy-tailed rows (fitted tables) with and without the sampling of the
kurtosis gate and of the fit, and Gaussian rows (the fixed table). Bar: bit-exact. Planted
mistakes in a copy of the oracle's fit (one Lloyd update fewer; the median instead of the mean
of a cell; the quantile start shifted by half a step) must each miss the golden tables.
"""

import importlib.util
import json
import pathlib

import numpy as np
import pytest

from oracle import w4a8_quant as wq

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _maker():
    spec = importlib.util.spec_from_file_location("make_codebook_golden", GOLDEN / "make_codebook_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)  # defines the input generator only; the reference is imported by main()
    return mod


CASES = json.loads((GOLDEN / "codebook_golden.json").read_text())["cases"]


def _case_input(case):
    mk = _maker()
    x = mk.normalized_case(case["seed"], *case["shape"], case["kind"])
    assert mk.digest(x) == case["sha256"], "input generator drifted from the fixture's inputs"
    return x


def _table(case):
    return np.array(case["table_f32_bits"], dtype=np.uint32).view(np.float32)


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_codebook_equals_reference(case):
    x = _case_input(case)
    got = wq.codebook_for(x)
    assert np.array_equal(got.astype(np.float32).view(np.uint32), _table(case).view(np.uint32)), (got, _table(case))
    assert case["fitted"] == (not np.array_equal(got, wq.FIXED_LUT))


def _planted_fit(normalized, variant, levels=16, iterations=25, sample_size=300000):
    """The oracle's fit with one planted mistake (`variant`)."""
    import torch

    samples = torch.from_numpy(np.ascontiguousarray(normalized, dtype=np.float32)).flatten()
    if samples.numel() > sample_size:
        gen = torch.Generator().manual_seed(0)
        samples = samples[torch.randint(0, samples.numel(), (sample_size,), generator=gen)]
    q = torch.linspace(0, 1, levels)
    if variant == "shifted_start":
        q = (torch.arange(levels, dtype=torch.float32) + 0.5) / levels
    cb = torch.quantile(samples, q)
    for _ in range(iterations - (1 if variant == "one_fewer" else 0)):
        assign = (samples.unsqueeze(-1) - cb).abs().argmin(-1)
        upd = cb.clone()
        for i in range(levels):
            sel = assign == i
            if sel.any():
                upd[i] = samples[sel].median() if variant == "median" else samples[sel].mean()
        cb = upd
    return cb.numpy().astype(np.float32)


@pytest.mark.parametrize("variant", ["one_fewer", "median", "shifted_start"])
def test_planted_fit_mistakes_miss_the_reference(variant):
    fitted = [c for c in CASES if c["fitted"]]
    assert fitted
    misses = 0
    for case in fitted[:2]:
        got = _planted_fit(_case_input(case), variant)
        misses += not np.array_equal(got.view(np.uint32), _table(case).view(np.uint32))
    assert misses > 0
