"""CPU tests that pin the gated residual update of the oracle, and the host-side segment map
(no GPU). The update is pinned against the routine the reference calls: torch's bfloat16
``addcmul_`` per modulation segment."""

import numpy as np
import pytest
import torch

from _util import activations, bits, gen
from oracle import eager_np
from oracle.bf16 import bf16_bits, bf16_to_f32

SEGMENTS = ((0, 7, 2), (7, 40, 0), (40, 64, 1))


def _torch_gated(residual, update, gate, segments):
    """h3serve/native_engine/model/layers.py:944-960 as the reference runs it (CPU)."""
    out = residual.clone()
    for start, stop, row in segments:
        out[start:stop].addcmul_(update[start:stop], gate[row].to(update.dtype))
    return out


@pytest.mark.parametrize("gate_dtype", [torch.bfloat16, torch.float32])
def test_gated_residual_matches_torch_addcmul(gate_dtype):
    res = activations(64, 768, 1) * 4
    upd = activations(64, 768, 2)
    gate = torch.randn(3, 768, generator=gen(3)).to(gate_dtype)
    ref = _torch_gated(res, upd, gate, SEGMENTS)
    rows = eager_np.segment_row_map(64, SEGMENTS)
    got = eager_np.gated_residual_bf16(bits(res), bits(upd), bits(gate.to(torch.bfloat16)), rows)
    assert np.array_equal(got, bits(ref))


def test_gated_residual_planted_double_rounding_is_caught():
    """Rounding the product to bfloat16 before the add (a plausible mistake) differs from
    torch on these inputs, so the test above would catch it."""
    res = activations(64, 768, 4) * 4
    upd = activations(64, 768, 5)
    gate = torch.randn(3, 768, generator=gen(6)).to(torch.bfloat16)
    ref = bits(_torch_gated(res, upd, gate, SEGMENTS))
    rows = eager_np.segment_row_map(64, SEGMENTS)
    prod = bf16_bits(bf16_to_f32(bits(upd)) * bf16_to_f32(bits(gate))[rows])
    wrong = bf16_bits(bf16_to_f32(bits(res)) + bf16_to_f32(prod))
    assert not np.array_equal(wrong, ref)
    shifted = eager_np.gated_residual_bf16(bits(res), bits(upd), bits(gate), np.roll(rows, 1))
    assert not np.array_equal(shifted, ref)


def test_segment_row_map_and_its_errors():
    rows = eager_np.segment_row_map(64, SEGMENTS)
    assert rows.dtype == np.int32 and rows[0] == 2 and rows[7] == 0 and rows[63] == 1
    with pytest.raises(ValueError):
        eager_np.segment_row_map(64, ((0, 7, 0), (8, 64, 1)))
    with pytest.raises(ValueError):
        eager_np.segment_row_map(64, ((0, 7, 0), (7, 60, 1)))
    with pytest.raises(ValueError):
        eager_np.segment_row_map(64, ((0, 0, 0), (0, 64, 1)))


def test_host_segment_row_map_matches_oracle():
    import mx_qlinear

    got = mx_qlinear.segment_row_map(64, SEGMENTS, "cpu")
    assert np.array_equal(got.numpy(), eager_np.segment_row_map(64, SEGMENTS))
    assert mx_qlinear.segment_row_map(64, SEGMENTS, "cpu") is got  # cached
    with pytest.raises(ValueError):
        mx_qlinear.segment_row_map(64, ((0, 7, 0), (8, 64, 1)), "cpu")
