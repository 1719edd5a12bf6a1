"""The oracle's stochastic-rounding quantizer (oracle/eager_np.py:quantize_int8_rowwise_stochastic)
pinned on the CPU against the reference's torch op sequence with given uniform draws
(quantization.py:803-826, 857-875), a closed form, and planted mistakes."""

import numpy as np
import pytest
import torch

from _util import activations, bits, gen
from oracle import eager_np
from oracle.bf16 import bf16_to_f32


def _torch_sequence(x: torch.Tensor, noise: torch.Tensor):
    """quantize_int8_rowwise with the rng replaced by `noise` (the reference's op sequence)."""
    abs_max = x.abs().amax(dim=-1, keepdim=True)
    scale = (abs_max.float() / 127.0).clamp(min=1e-30)
    s = scale.to(dtype=x.dtype)
    s = torch.where(s == 0, torch.full_like(s, torch.finfo(x.dtype).tiny), s)
    scaled = x / s
    return scaled.add_(noise).floor_().clamp_(-128.0, 127.0).to(torch.int8), scale


@pytest.mark.parametrize("seed", [1, 7, 12345])
def test_stochastic_oracle_equals_the_torch_sequence(seed):
    x = activations(64, 1024, seed)
    noise = torch.rand(x.shape, dtype=torch.bfloat16, generator=gen(seed + 1))
    q, s = eager_np.quantize_int8_rowwise_stochastic(bits(x), bits(noise))
    qt, st = _torch_sequence(x.clone(), noise)
    assert np.array_equal(q, qt.numpy()) and np.array_equal(s, st.numpy())


def test_zero_noise_is_floor_of_the_scaled_value():
    x = activations(8, 256, 3)
    q, _ = eager_np.quantize_int8_rowwise_stochastic(bits(x), np.zeros(x.shape, np.uint16))
    xf = bf16_to_f32(bits(x))
    s = np.maximum(np.abs(xf).max(-1, keepdims=True) / np.float32(127), np.float32(1e-30)).astype(np.float32)
    sb = bf16_to_f32(bits(torch.from_numpy(s).to(torch.bfloat16)))
    scaled = bf16_to_f32(bits(torch.from_numpy((xf / sb).astype(np.float32)).to(torch.bfloat16)))
    assert np.array_equal(q, np.clip(np.floor(scaled), -128, 127).astype(np.int8))


def test_planted_mistakes_are_caught(monkeypatch):
    x = activations(32, 512, 5)
    noise = torch.rand(x.shape, dtype=torch.bfloat16, generator=gen(6))
    qt, _ = _torch_sequence(x.clone(), noise)
    # round-to-nearest instead of the stochastic floor
    q0, _ = eager_np.quantize_int8_rowwise(bits(x))
    assert not np.array_equal(q0, qt.numpy())

    # the bf16 roundings left out (the quotient and the noisy sum kept in fp32)
    def no_round(a):
        return np.asarray(a, np.float32)

    with monkeypatch.context() as m:
        m.setattr(eager_np, "round_bf16", no_round)
        q1, _ = eager_np.quantize_int8_rowwise_stochastic(bits(x), bits(noise))
    assert not np.array_equal(q1, qt.numpy())
