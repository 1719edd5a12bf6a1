"""GPU parity of the SwiGLU fc1 epilogue and the H3 MLP chain built on it (bit-exact bf16):
fc1 with SwiGLU in the epilogue equals fc1 followed by the SwiGLU input activation, and the
chain equals the reference's default route (int8_linear fc1 -> int8_linear fc2 with
input_act="swiglu", convrot=True -> addcmul_ per segment)."""

import numpy as np
import pytest
import torch

from _util import activations, bf16_vec, bits, gen, int8_weight
from oracle import convrot as cr
from oracle import eager_np
from oracle.bf16 import bf16_bits

pytestmark = pytest.mark.gpu


def _mx():
    import mx_qlinear

    return mx_qlinear


@pytest.mark.parametrize("m,f,k,bias,per_channel", [(300, 512, 1024, True, True), (257, 48, 256, False, True),
                                                    (64, 1024, 512, True, False), (1, 80, 128, True, True)])
def test_swiglu_fc1_matches_oracle(dev, m, f, k, bias, per_channel):
    print(f"swiglu fc1 m={m} f={f} k={k}", flush=True)
    x = activations(m, k, m + f)
    w, ws = int8_weight(2 * f, k, k + f)
    if not per_channel:
        ws = ws[:1].clone()
    b = bf16_vec(2 * f, 3, 0.05) if bias else None
    q, s = eager_np.quantize_int8_rowwise(bits(x))
    fc1 = _mx().prepare_swiglu_fc1(w.to(dev), ws.to(dev), None if b is None else b.to(dev))
    h = _mx().int8_swiglu_fc1(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), fc1)
    y = eager_np.dequant_epilogue(eager_np.int8_matmul(q, w.numpy()), s, ws.numpy(), None if b is None else bits(b), "bf16")
    assert h.shape == (m, f)
    assert np.array_equal(bits(h), cr.swiglu_bf16(bf16_bits(y)))


def test_swiglu_fc1_every_gate_pattern(dev):
    """All 65,536 bf16 gate patterns (NaN, infinities, zeros, subnormals, both signs) through the
    GEMM epilogue's SiLU: zero activations make every fc1 output its bias, so the gate half of the
    bias runs over every pattern and the up half over random values. 512 tiles of 256 on two
    rounds: the looping workgroups' epilogues run beside the next tile's first loads."""
    m, f, k = 40, 65536, 16
    print(f"swiglu fc1 every gate pattern m={m} f={f}", flush=True)
    gate_bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    up = torch.randn(f, generator=gen(31)).to(torch.bfloat16)
    b = torch.cat([gate_bits.view(torch.bfloat16), up])
    w, ws = int8_weight(2 * f, k, 32)
    q = np.zeros((m, k), dtype=np.int8)
    s = np.full((m, 1), 0.5, dtype=np.float32)
    fc1 = _mx().prepare_swiglu_fc1(w.to(dev), ws.to(dev), b.to(dev))
    from mx_qlinear import _lib

    plan = _lib.gemm_plan(m, 2 * f, k, 2)
    assert plan["persistent"] and plan["tiles"] == 512, plan
    h = _mx().int8_swiglu_fc1(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), fc1)
    y = eager_np.dequant_epilogue(np.zeros((m, 2 * f), dtype=np.int32), s, ws.numpy(), bits(b), "bf16")
    assert np.array_equal(bits(h), cr.swiglu_bf16(bf16_bits(y)))


@pytest.mark.parametrize("m,f,k", [(4096, 4096, 512), (4100, 4112, 400)])
def test_swiglu_fc1_multi_round_matches_oracle(dev, m, f, k):
    """Looping ping-pong workgroups over 512+ tiles (ragged edges in the second case): sampled
    rows against the oracle, bit for bit."""
    print(f"swiglu fc1 multi-round m={m} f={f} k={k}", flush=True)
    from mx_qlinear import _lib

    assert _lib.gemm_plan(m, 2 * f, k, 2)["persistent"]
    x = activations(m, k, m + 3)
    w, ws = int8_weight(2 * f, k, f + 4)
    b = bf16_vec(2 * f, 5, 0.05)
    q, s = eager_np.quantize_int8_rowwise(bits(x))
    fc1 = _mx().prepare_swiglu_fc1(w.to(dev), ws.to(dev), b.to(dev))
    h = _mx().int8_swiglu_fc1(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), fc1).cpu()
    rows = np.unique(np.concatenate([[0, m - 1], np.random.default_rng(m).choice(m, 30, replace=False)]))
    acc = (q[rows].astype(np.float64) @ w.numpy().astype(np.float64).T).astype(np.int64).astype(np.int32)
    y = eager_np.dequant_epilogue(acc, s[rows], ws.numpy(), bits(b), "bf16")
    assert np.array_equal(bits(h[rows]), cr.swiglu_bf16(bf16_bits(y)))


def test_swiglu_fc1_equals_linear_then_swiglu_on_device(dev):
    m, f, k = 200, 768, 512
    x = activations(m, k, 5).to(dev)
    w, ws = int8_weight(2 * f, k, 6)
    b = bf16_vec(2 * f, 7, 0.02)
    w, ws, b = w.to(dev), ws.to(dev), b.to(dev)
    raw = _mx().int8_linear(x, w, ws, b)
    q, s = _mx().quantize_int8_rowwise(x)
    h = _mx().int8_swiglu_fc1(q, s, _mx().prepare_swiglu_fc1(w, ws, b))
    assert torch.equal(h, _mx().apply_input_act(raw, "swiglu"))


def _mlp_layer(dev, d, f, seed):
    w1, s1 = int8_weight(2 * f, d, seed)
    w2, s2 = int8_weight(d, f, seed + 1)
    b1, b2 = bf16_vec(2 * f, seed + 2, 0.02), bf16_vec(d, seed + 3, 0.02)
    return [t.to(dev) for t in (w1, s1, b1, w2, s2, b2)]


def test_swiglu_mlp_chain_equals_the_reference_route(dev):
    m, d, f = 150, 512, 1024
    w1, s1, b1, w2, s2, b2 = _mlp_layer(dev, d, f, 11)
    hidden = activations(m, d, 12).to(dev)
    gate = torch.randn(3, d, generator=gen(13)).to(torch.bfloat16).to(dev)
    segs = ((0, 20, 2), (20, 64, 1), (64, 150, 0))
    res0 = (activations(m, d, 14) * 2).to(dev)
    # reference route: raw = fc1(hidden); fused_down_gated_residual(raw, ...)
    ref = res0.clone()
    raw = _mx().int8_linear(hidden, w1, s1, b1, convrot=True)
    _mx().fused_down_gated_residual(raw, ref, gate, _mx().segment_row_map(m, segs, dev), w2, s2, b2)
    got = res0.clone()
    q, s = _mx().quantize_int8_rowwise_convrot(hidden, 256)
    _mx().swiglu_mlp_gated_residual_(got, q, s, _mx().prepare_swiglu_fc1(w1, s1, b1), w2, s2, b2, gate, segs)
    assert torch.equal(got, ref)


def test_h3_mlp_chain_equals_its_parts(dev):
    m, d, f = 96, 1024, 512
    w1, s1, b1, w2, s2, b2 = _mlp_layer(dev, d, f, 21)
    norm_w = (1 + 0.1 * torch.randn(d, generator=gen(22))).to(torch.bfloat16).to(dev)
    scale = (0.1 * torch.randn(3, d, generator=gen(23))).to(torch.bfloat16).to(dev)
    shift = (0.1 * torch.randn(3, d, generator=gen(24))).to(torch.bfloat16).to(dev)
    gate = (0.1 * torch.randn(3, d, generator=gen(25))).to(torch.bfloat16).to(dev)
    segs = ((0, 10, 0), (10, 40, 1), (40, 96, 2))
    res0 = (activations(m, d, 26) * 2).to(dev)
    ref = res0.clone()
    hidden = _mx().rms_adaln(ref, (norm_w, 1e-6), shift, scale, segs)
    raw = _mx().int8_linear(hidden, w1, s1, b1, convrot=True)
    _mx().fused_down_gated_residual(raw, ref, gate, _mx().segment_row_map(m, segs, dev), w2, s2, b2)
    got = res0.clone()
    _mx().h3_mlp_(got, (norm_w, 1e-6), shift, scale, gate, segs, _mx().prepare_swiglu_fc1(w1, s1, b1), w2, s2, b2)
    assert torch.equal(got, ref)


def test_prepare_swiglu_fc1_rejects_bad_widths(dev):
    w, ws = int8_weight(40, 64, 1)
    with pytest.raises(NotImplementedError):
        _mx().prepare_swiglu_fc1(w.to(dev), ws.to(dev))
