"""GPU parity of the float16 input paths: the input activations (tanh-GELU, SwiGLU) and the
ConvRot rotation quantizer on float16 activations, and int8_linear on them.

Oracle: the reference's own torch CPU ops in float16 for the activations and the row quantizer
(oracle/eager_torch.py: CK/backends/_activations.py:40-53, CK/backends/eager/quantization.py:
857-875), the exact rotation rounded once to float16 (oracle/convrot.py convrot_quantize_f16,
its rounding pinned in test_oracle_f16_rounding.py). Bar: bit-exact, NaN patterns included.
"""

import numpy as np
import pytest
import torch

from _util import gen
from oracle import convrot as cr
from oracle import eager_np, eager_torch
from oracle.bf16 import bf16_bits

pytestmark = pytest.mark.gpu


def _mx():
    import mx_qlinear

    return mx_qlinear


def _all_f16() -> torch.Tensor:
    return torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(torch.float16)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_gelu_f16_every_input(dev):
    x = _all_f16().reshape(256, 256)
    got = _mx().ops.apply_input_act(x.to(dev), "gelu_tanh").cpu()
    ref = eager_torch.apply_input_act(x, "gelu_tanh")
    assert np.array_equal(_bits(got), _bits(ref))


def test_swiglu_f16_every_gate(dev):
    """Every float16 gate against ups drawn from all float16 patterns (NaN payloads, infinities,
    zeros, subnormals among them), so NaN passing and 0 * inf are exercised too."""
    gate = _all_f16()
    up = torch.from_numpy(np.random.default_rng(3).integers(0, 65536, 65536).astype(np.uint16).view(np.int16)).view(torch.float16)
    up[:8] = torch.tensor([0x7C00, 0xFC00, 0x0000, 0x8000, 0x7D23, 0xFE01, 0x0001, 0x3C00], dtype=torch.int32).to(torch.int16).view(torch.float16)
    x = torch.cat([gate.reshape(256, 256), up.reshape(256, 256)], dim=1)
    got = _mx().ops.apply_input_act(x.to(dev), "swiglu").cpu()
    ref = eager_torch.apply_input_act(x, "swiglu")
    assert np.array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("m,k", [(33, 1000), (8, 16384)])
def test_quantize_gelu_f16(dev, m, k):
    x = (torch.randn(m, k, generator=gen(m + k)) * 3).to(torch.float16)
    x[1] = 0
    x[2, 5] = float("inf")
    q, s = _mx().quantize_int8_rowwise(x.to(dev), input_act="gelu_tanh")
    q_ref, s_ref = eager_torch.quantize_int8_rowwise(eager_torch.apply_input_act(x, "gelu_tanh"))
    assert torch.equal(q.cpu(), q_ref) and torch.equal(s.cpu(), s_ref)


def _f16_rows(m, k, seed):
    x = (torch.randn(m, k, generator=gen(seed)) * 2).to(torch.float16)
    x[0] = 0                                   # zero row: scale 1e-30 -> float16 tiny
    x[1, :7] = torch.tensor([60000.0, -60000.0, 1e-7, -1e-7, 6e-5, 65504.0, -3.0])
    if m > 3:
        x[3] = torch.randn(k, generator=gen(seed + 1)).to(torch.float16) * 1e-4  # subnormal results
    return x


@pytest.mark.parametrize("act", [None, "gelu_tanh", "swiglu"])
@pytest.mark.parametrize("g", [0, 16, 64, 256, 1024])
@pytest.mark.parametrize("m,k", [(5, 1024), (17, 3072), (4, 5376)])
def test_convrot_quantize_f16(dev, act, g, m, k):
    if g and k % g:
        pytest.skip("group does not divide K")
    width = 2 * k if act == "swiglu" else k
    print(f"convrot f16 m={m} k={k} g={g} act={act}", flush=True)
    x = _f16_rows(m, width, m * 7 + k + g)
    q, s = _mx().quantize_int8_rowwise_convrot(x.to(dev), g, act)
    q_ref, s_ref, _ = cr.convrot_quantize_f16(x.numpy(), g, act)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    _same_scales(s.cpu().numpy(), s_ref)


def _same_scales(got, ref):
    """Bit-equal scales; a row whose rotation meets inf - inf has a NaN scale on both sides, whose
    payload follows the order the rotation meets it in (not part of the contract)."""
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_convrot_f16_non_finite_rows(dev):
    x = _f16_rows(4, 2048, 9)
    x[1, 100] = float("nan")
    x[2, 7] = float("inf")
    for g in (0, 256):
        q, s = _mx().quantize_int8_rowwise_convrot(x.to(dev), g, None)
        q_ref, s_ref, _ = cr.convrot_quantize_f16(x.numpy(), g, None)
        assert np.array_equal(q.cpu().numpy(), q_ref)
        _same_scales(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("convrot,act", [(True, None), (True, "gelu_tanh"), (False, "swiglu"), (False, "gelu_tanh")])
def test_int8_linear_f16_inputs(dev, convrot, act):
    """int8_linear on float16 activations: the quantizer's output (checked above) through the
    INT8 GEMM and the dequant epilogue, against the oracle's composition (bf16 output)."""
    m, k, n = 70, 1024, 384
    width = 2 * k if act == "swiglu" else k
    x = (torch.randn(m, width, generator=gen(41)) * 2).to(torch.float16)
    w = torch.randint(-127, 128, (n, k), generator=gen(42), dtype=torch.int8)
    ws = torch.rand(n, generator=gen(43)) * 0.01 + 1e-3
    b = (torch.randn(n, generator=gen(44)) * 0.1).to(torch.bfloat16)
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), b.to(dev), convrot=convrot, input_act=act).cpu()
    q_ref, s_ref, _ = cr.convrot_quantize_f16(x.numpy(), 256 if convrot else 0, act)
    acc = eager_np.int8_matmul(q_ref, w.numpy())
    ref = eager_np.dequant_epilogue(acc, s_ref.reshape(-1), ws.numpy(), bf16_bits(b.float().numpy()), "bf16")
    assert np.array_equal(y.view(torch.int16).numpy().view(np.uint16), bf16_bits(ref))


def _f16_ulp(v: np.ndarray) -> np.ndarray:
    return np.spacing(np.abs(np.asarray(v, dtype=np.float32)).astype(np.float16)).astype(np.float64)


# Fraction of float16 adaLN / RMS adaLN outputs that may differ from torch's CPU result by the
# bounded amount: the statistics are reductions in another order than torch's, and float16 (eleven
# significant bits) meets a rounding boundary more often than bfloat16. Measured on one MI355X:
# adaLN 3.3e-5 to 1.2e-4, RMS adaLN 3.3e-5 to 4.3e-5 on the shapes below.
F16_NORM_MISMATCH_BOUND = 5e-4


@pytest.mark.parametrize("m,d,groups", [(64, 5120, 1), (33, 1000, 1), (40, 768, 4)])
def test_adaln_f16(dev, m, d, groups):
    """Modulated float16 within 2 ulp(n.t) + ulp(y) of torch's CPU adaln in float16; the int8
    quantization of the kernel's own modulated rows bit-exact (torch's quantizer sequence)."""
    x = (torch.randn(m, d, generator=gen(m + d)) * 2 + 0.3).to(torch.float16)
    sc = (torch.randn(groups, d, generator=gen(5)) * 0.1).to(torch.float16)
    sh = (torch.randn(groups, d, generator=gen(6)) * 0.1).to(torch.float16)
    q, s, y = _mx().adaln_quantize_int8(x.to(dev), sc.to(dev), sh.to(dev), 1e-6, return_modulated=True)
    rep = m // groups
    scr, shr = sc.repeat_interleave(rep, 0), sh.repeat_interleave(rep, 0)
    y_ref = eager_torch.adaln(x, scr, shr, 1e-6)
    yv, rv = y.cpu().float().numpy(), y_ref.float().numpy()
    x64 = x.double().numpy()
    mu = x64.mean(-1, keepdims=True)
    n64 = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(-1, keepdims=True) + 1e-6)
    t = (1 + scr.float()).half().float().numpy()
    tol = 2 * _f16_ulp(n64 * t) + _f16_ulp(np.maximum(np.abs(rv), np.abs(yv)))
    assert np.all(np.abs(yv.astype(np.float64) - rv) <= tol)
    rate = float(np.mean(_bits(y.cpu()) != _bits(y_ref)))
    print(f"adaLN float16 mismatch rate vs torch CPU ({m}x{d}): {rate:.2e}", flush=True)
    assert rate <= F16_NORM_MISMATCH_BOUND
    q_ref, s_ref = eager_torch.quantize_int8_rowwise(y.cpu())
    assert torch.equal(q.cpu(), q_ref) and torch.equal(s.cpu(), s_ref)
    assert torch.equal(_mx().adaln(x.to(dev), sc.to(dev), sh.to(dev), 1e-6), y)


@pytest.mark.parametrize("g", [0, 256])
@pytest.mark.parametrize("m,d", [(48, 5376), (20, 3072)])
def test_rms_adaln_f16(dev, m, d, g):
    """RMS adaLN on float16 within 2 ulp(n.t) + ulp(y) of torch's CPU sequence in float16 (three
    segments); q / scales bit-exact against the oracle's rotation and quantizer on the kernel's
    own modulated rows."""
    from mx_qlinear import ops

    x = (torch.randn(m, d, generator=gen(m * 3 + d)) * 1.5).to(torch.float16)
    w = (1 + 0.1 * torch.randn(d, generator=gen(7))).to(torch.float16)
    sc = (torch.randn(3, d, generator=gen(8)) * 0.1).to(torch.float16)
    sh = (torch.randn(3, d, generator=gen(9)) * 0.1).to(torch.float16)
    segs = [(0, m // 3, 0), (m // 3, 2 * m // 3, 2), (2 * m // 3, m, 1)]
    q, s, y = ops.rms_adaln_quantize_int8(x.to(dev), (w.to(dev), 1e-6), sh.to(dev), sc.to(dev), segs, g,
                                          return_modulated=True)
    y_ref = eager_torch.rms_adaln(x.clone(), w, 1e-6, sh, sc, segs)
    yv, rv = y.cpu().float().numpy(), y_ref.float().numpy()
    x64 = x.double().numpy()
    n64 = x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + 1e-6) * w.double().numpy()
    rows = np.concatenate([np.full(b - a, r) for a, b, r in segs])
    t = (1 + sc.float()).half().float().numpy()[rows]
    tol = 2 * _f16_ulp(n64 * t) + _f16_ulp(np.maximum(np.abs(rv), np.abs(yv)))
    assert np.all(np.abs(yv.astype(np.float64) - rv) <= tol)
    rate = float(np.mean(_bits(y.cpu()) != _bits(y_ref)))
    print(f"RMS adaLN float16 mismatch rate vs torch CPU ({m}x{d}, G={g}): {rate:.2e}", flush=True)
    assert rate <= F16_NORM_MISMATCH_BOUND
    q_ref, s_ref, _ = cr.convrot_quantize_f16(y.cpu().numpy(), g, None)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    _same_scales(s.cpu().numpy(), s_ref)


def test_int8_ffn_gelu_f16_input(dev):
    """The fused FFN chain on a float16 input equals the two-call composition (int8_linear with
    bf16 output, then int8_linear with input_act='gelu_tanh'), bit for bit."""
    m, k, h, n = 96, 512, 1024, 384
    x = (torch.randn(m, k, generator=gen(61)) * 2).to(torch.float16).to(dev)
    w1 = torch.randint(-127, 128, (h, k), generator=gen(62), dtype=torch.int8).to(dev)
    w2 = torch.randint(-127, 128, (n, h), generator=gen(63), dtype=torch.int8).to(dev)
    s1 = (torch.rand(h, generator=gen(64)) * 0.01 + 1e-3).to(dev)
    s2 = (torch.rand(n, generator=gen(65)) * 0.01 + 1e-3).to(dev)
    b1 = (torch.randn(h, generator=gen(66)) * 0.1).to(torch.bfloat16).to(dev)
    b2 = (torch.randn(n, generator=gen(67)) * 0.1).to(torch.bfloat16).to(dev)
    mx = _mx()
    y = mx.int8_ffn_gelu(x, w1, s1, b1, w2, s2, b2)
    ref = mx.int8_linear(mx.int8_linear(x, w1, s1, b1), w2, s2, b2, input_act="gelu_tanh")
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
