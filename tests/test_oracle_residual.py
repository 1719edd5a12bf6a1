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


# ---- RMS adaLN -------------------------------------------------------------------------------

def _rms_inputs(m=48, d=1024, seed=30):
    x = activations(m, d, seed) * 2
    w = (1 + 0.2 * torch.randn(d, generator=gen(seed + 1))).to(torch.bfloat16)
    scale = (0.1 * torch.randn(3, d, generator=gen(seed + 2))).to(torch.bfloat16)
    shift = (0.1 * torch.randn(3, d, generator=gen(seed + 3))).to(torch.bfloat16)
    return x, w, scale, shift


def test_rms_adaln_matches_the_reference_eager_composition():
    """kernels.py:7629-7639 run with torch on the CPU: norm(x), then in-place mul_/add_ per
    segment, against the oracle."""
    x, w, scale, shift = _rms_inputs()
    segs = ((0, 5, 2), (5, 30, 0), (30, 48, 1))
    h = torch.nn.functional.rms_norm(x, (x.shape[-1],), weight=w, eps=1e-6)
    for a, b, row in segs:
        h[a:b].mul_(1.0 + scale[row].to(h.dtype)).add_(shift[row].to(h.dtype))
    got = eager_np.rms_adaln(bits(x), bits(w), 1e-6, bits(scale), bits(shift), eager_np.segment_row_map(48, segs))
    assert np.array_equal(got, bits(h))


def test_rms_norm_routine_is_one_rounding_of_the_float64_value():
    """torch's bfloat16 rms_norm is within one bfloat16 ulp of the float64 value (its float32
    statistics and single final rounding), which bounds the device kernel's freedom."""
    from oracle.bf16 import bf16_ulp

    x, w, _, _ = _rms_inputs(64, 5120, 40)
    n = bf16_to_f32(eager_np.rms_norm_bf16(bits(x), bits(w), 1e-6)).astype(np.float64)
    e = eager_np.rms_norm_f64(bits(x), bits(w), 1e-6)
    assert np.all(np.abs(n - e) <= bf16_ulp(np.abs(e).astype(np.float32)))
    # a planted mistake (weight applied after an intermediate bfloat16 rounding) breaks equality
    r = 1.0 / np.sqrt((bf16_to_f32(bits(x)).astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
    two = bf16_bits(bf16_to_f32(bf16_bits((bf16_to_f32(bits(x)) * r.astype(np.float32)))) * bf16_to_f32(bits(w)))
    assert not np.array_equal(two, eager_np.rms_norm_bf16(bits(x), bits(w), 1e-6))
