"""GPU parity of fc2 with the gated residual epilogue against the oracle (bit-exact bf16):
int8_linear followed by the per-segment addcmul_ of the reference."""

import numpy as np
import pytest
import torch

from _util import activations, bf16_vec, bits, gen, int8_weight
from oracle import convrot as cr
from oracle import eager_np

pytestmark = pytest.mark.gpu


def _mx():
    import mx_qlinear

    return mx_qlinear


def _segments(m, parts):
    cuts = sorted({0, m, *[(m * i) // parts for i in range(1, parts)]})
    return tuple((a, b, i % 3) for i, (a, b) in enumerate(zip(cuts[:-1], cuts[1:])))


def _expected(res, x, w, ws, b, gate, rows, g=0, act=None):
    if g or act:
        q, s, _ = cr.convrot_quantize_bf16(bits(x), g, act)
    else:
        q, s = eager_np.quantize_int8_rowwise(bits(x))
    y = eager_np.dequant_epilogue(eager_np.int8_matmul(q, w.numpy()), s, ws.numpy(),
                                  None if b is None else bits(b), "bf16")
    from oracle.bf16 import bf16_bits

    return eager_np.gated_residual_bf16(bits(res), bf16_bits(y), bits(gate), rows)


@pytest.mark.parametrize("m,n,k,bias", [(300, 512, 1024, True), (257, 200, 640, False), (1, 256, 256, True),
                                        (64, 3072, 3072, True), (515, 776, 208, True)])
def test_gated_residual_matches_oracle(dev, m, n, k, bias):
    print(f"gated residual m={m} n={n} k={k} bias={bias}", flush=True)
    x = activations(m, k, m + n)
    w, ws = int8_weight(n, k, k)
    b = bf16_vec(n, 5, 0.02) if bias else None
    gate = torch.randn(3, n, generator=gen(7)).to(torch.bfloat16)
    res = activations(m, n, 8) * 3
    segs = _segments(m, 4)
    rows = eager_np.segment_row_map(m, segs)
    out = res.to(dev)
    r = _mx().int8_linear_gated_residual_(out, x.to(dev), w.to(dev), ws.to(dev), None if b is None else b.to(dev),
                                          gate.to(dev), segs)
    assert r is out
    assert np.array_equal(bits(out), _expected(res, x, w, ws, b, gate, rows))


def test_gated_residual_equals_linear_then_addcmul_on_device(dev):
    """The fused update equals the reference's two-step composition run with torch on the GPU."""
    m, n, k = 200, 384, 512
    x = activations(m, k, 1).to(dev)
    w, ws = int8_weight(n, k, 2)
    w, ws = w.to(dev), ws.to(dev)
    b = bf16_vec(n, 3, 0.02).to(dev)
    gate = torch.randn(2, n, generator=gen(4)).to(dev)          # float32 gate, rounded per use
    res = (activations(m, n, 5) * 2).to(dev)
    segs = ((0, 50, 1), (50, 200, 0))
    ref = res.clone()
    y = _mx().int8_linear(x, w, ws, b)
    for a, c, row in segs:
        ref[a:c].addcmul_(y[a:c], gate[row].to(y.dtype))
    _mx().int8_linear_gated_residual_(res, x, w, ws, b, gate, segs)
    assert torch.equal(res, ref)


def test_gated_residual_strided_residual_and_row_tensor(dev):
    """A residual that is a column slice of a wider buffer (row stride > N, unaligned start,
    so the element-wise store path runs) and gate rows passed as a tensor."""
    m, n, k = 130, 200, 256
    x = activations(m, k, 11)
    w, ws = int8_weight(n, k, 12)
    gate = torch.randn(4, n, generator=gen(13)).to(torch.bfloat16)
    rows = torch.randint(0, 4, (m,), generator=gen(14), dtype=torch.int32)
    base = (activations(m, n + 9, 15) * 2)
    res = base[:, 3:3 + n]
    want = _expected(res, x, w, ws, None, gate, rows.numpy())
    dbase = base.to(dev)
    dres = dbase[:, 3:3 + n]
    _mx().int8_linear_gated_residual_(dres, x.to(dev), w.to(dev), ws.to(dev), None, gate.to(dev), rows.to(dev))
    assert np.array_equal(bits(dres), want)
    # the columns outside the slice are untouched
    assert torch.equal(dbase[:, :3].cpu(), base[:, :3]) and torch.equal(dbase[:, 3 + n:].cpu(), base[:, 3 + n:])


def test_fused_down_gated_residual_swiglu_convrot(dev):
    m, inner, n = 96, 1024, 512
    hidden = activations(m, 2 * inner, 21, outlier_frac=0.0)
    w, ws = int8_weight(n, inner, 22)
    b = bf16_vec(n, 23, 0.01)
    gate = torch.randn(2, n, generator=gen(24)).to(torch.bfloat16)
    res = activations(m, n, 25)
    segs = ((0, 32, 1), (32, 96, 0))
    rows = _mx().segment_row_map(m, segs, dev)
    out = res.to(dev)
    _mx().fused_down_gated_residual(hidden.to(dev), out, gate.to(dev), rows, w.to(dev), ws.to(dev), b.to(dev))
    want = _expected(res, hidden, w, ws, b, gate, rows.cpu().numpy(), g=256, act="swiglu")
    assert np.array_equal(bits(out), want)


def test_gated_residual_rejects_bad_maps(dev):
    m, n, k = 16, 64, 64
    x = activations(m, k, 1).to(dev)
    w, ws = int8_weight(n, k, 2)
    gate = torch.zeros(2, n, dtype=torch.bfloat16, device=dev)
    res = torch.zeros(m, n, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        _mx().int8_linear_gated_residual_(res, x, w.to(dev), ws.to(dev), None, gate,
                                          torch.full((m,), 2, dtype=torch.int32))
    with pytest.raises(ValueError):
        _mx().int8_linear_gated_residual_(res, x, w.to(dev), ws.to(dev), None, gate, ((0, 8, 0), (9, 16, 1)))
    with pytest.raises(ValueError):
        _mx().int8_linear_gated_residual_(res[:8], x, w.to(dev), ws.to(dev), None, gate, ((0, 16, 0),))
