"""GPU: the lane pairings of the DPP / permlane wave reductions (mxq_common.h) that the
quantizers' row statistics use. lane_xor4 must hand lane i the value of lane i ^ 4, and the
16-lane float64 sum and the float32 wave sum must pair lanes in their documented order, which
the oracles restate. The inputs make the pairing visible: in each 16-lane row the quads hold
1, 2^60, -2^60, 1, so pairing quad 0 with quad 1 (i ^ 4) gives (1 + 2^60) + (-2^60 + 1) = 0
in float64, while pairing it with quad 3 (i ^ 12) would give 2."""

import numpy as np
import pytest
import torch

def _pair_sum(v, masks):
    v = v.copy()
    for m in masks:
        v = v + v[np.arange(v.size) ^ m]
    return v


def _inputs():
    quad = np.array([0.25, 2.0 ** 58, -(2.0 ** 58), 0.25])
    row = np.repeat(quad, 4)
    # rows 1-3 vary the pattern (quads rotated, scaled) so each row's result is its own
    rows = [row, np.roll(row, 4) * 2.0, np.roll(row, 8) * 0.5, np.repeat(np.array([3.0, -1.5, 0.125, 7.0]), 4)]
    return np.concatenate(rows).astype(np.float64)


def test_pairing_emulation_tells_i4_from_i12():
    v = _inputs()
    good = np.concatenate([_pair_sum(v[r * 16:(r + 1) * 16], [1, 2, 4, 8]) for r in range(4)])
    bad = np.concatenate([_pair_sum(v[r * 16:(r + 1) * 16], [1, 2, 12, 8]) for r in range(4)])
    assert not np.array_equal(good, bad)


@pytest.mark.gpu
def test_lane_exchange_pairings(dev):
    from mx_qlinear import _lib as L
    from mx_qlinear.ops import _p, _stream

    v = _inputs()
    vin = torch.from_numpy(v).to(dev)
    xor4 = torch.zeros(64, dtype=torch.int32, device=dev)
    row16 = torch.zeros(64, dtype=torch.float64, device=dev)
    wsum = torch.zeros(64, dtype=torch.float32, device=dev)
    L.call("mxq_probe_lane_exchange", _p(vin), _p(xor4), _p(row16), _p(wsum), _stream(dev))
    assert np.array_equal(xor4.cpu().numpy(), np.arange(64) ^ 4)
    want16 = np.concatenate([_pair_sum(v[r * 16:(r + 1) * 16], [1, 2, 4, 8]) for r in range(4)])
    assert np.array_equal(row16.cpu().numpy().view(np.uint64), want16.view(np.uint64))
    want32 = _pair_sum(v.astype(np.float32), [32, 16, 8, 4, 2, 1])
    assert np.array_equal(wsum.cpu().numpy().view(np.uint32), want32.view(np.uint32))
