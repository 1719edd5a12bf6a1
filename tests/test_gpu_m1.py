"""GPU parity of the single-token (M = 1) INT8 linear: the fused quantizer + GEMV launch and the
prequantized GEMV, against the oracle and against the batched path's rows (bit-exact)."""

import numpy as np
import pytest
import torch

from _util import activations, bf16_vec, bits, int8_weight
from oracle import convrot as cr
from oracle import eager_np
from oracle.bf16 import bf16_bits

pytestmark = pytest.mark.gpu

_NAMES = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def _mx():
    import mx_qlinear

    return mx_qlinear


def _as_u32(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("with_bias,per_channel", [(True, True), (False, False)])
@pytest.mark.parametrize("n,k", [(3072, 3072), (7, 16), (1, 16384), (3073, 5120)])
def test_m1_linear_matches_oracle(dev, out_dtype, with_bias, per_channel, n, k):
    print(f"m1 linear n={n} k={k} {out_dtype} bias={with_bias} per_channel={per_channel}", flush=True)
    x = activations(1, k, n + k)
    w, ws = int8_weight(n, k, k)
    if not per_channel:
        ws = ws[:1].clone()
    bias = bf16_vec(n, 3, 0.02) if with_bias else None
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), None if bias is None else bias.to(dev),
                          out_dtype=out_dtype)
    ref = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), None if bias is None else bits(bias),
                               _NAMES[out_dtype])
    assert y.shape == (1, n) and y.dtype == out_dtype
    assert np.array_equal(_as_u32(y), ref.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("g,act", [(256, None), (64, None), (1024, None), (256, "swiglu"), (0, "gelu_tanh"),
                                   (256, "gelu_tanh"), (0, "swiglu"), (16, None)])
def test_m1_linear_convrot_and_acts(dev, g, act):
    n, k = 640, 5120 if g != 1024 else 4096
    width = 2 * k if act == "swiglu" else k
    x = activations(1, width, g + 5, outlier_frac=0.0 if act else 0.005)
    w, ws = int8_weight(n, k, 9)
    b = bf16_vec(n, 10, 0.01)
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), b.to(dev), convrot=bool(g), convrot_groupsize=g or 256,
                          input_act=act)
    q, s, _ = cr.convrot_quantize_bf16(bits(x), g, act)
    ref = eager_np.dequant_epilogue(eager_np.int8_matmul(q, w.numpy()), s, ws.numpy(), bits(b), "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))


def test_m1_rows_equal_the_batched_rows(dev):
    """A token alone (one launch, GEMV) gives the same bits as inside a batch (GEMM)."""
    m, n, k = 5, 1536, 3072
    x = activations(m, k, 77).to(dev)
    w, ws = int8_weight(n, k, 78)
    w, ws = w.to(dev), ws.to(dev)
    b = bf16_vec(n, 79, 0.02).to(dev)
    for convrot in (False, True):
        full = _mx().int8_linear(x, w, ws, b, convrot=convrot)
        for i in range(m):
            one = _mx().int8_linear(x[i:i + 1], w, ws, b, convrot=convrot)
            assert torch.equal(one[0], full[i])
    x3 = x[:1].reshape(1, 1, k)
    assert torch.equal(_mx().int8_linear(x3, w, ws, b)[0, 0], _mx().int8_linear(x, w, ws, b)[0])


def test_gemv_dequant_matches_prequantized_gemm(dev):
    n, k = 2000, 2048
    x = activations(2, k, 90)
    q, s = eager_np.quantize_int8_rowwise(bits(x))
    w, ws = int8_weight(n, k, 91)
    b = bf16_vec(n, 92, 0.02)
    args = (w.to(dev), torch.from_numpy(s[:1]).to(dev), ws.to(dev), b.to(dev), torch.bfloat16)
    y = _mx().int8_gemv_dequant(torch.from_numpy(q[:1]).to(dev), *args)
    ref = eager_np.dequant_epilogue(eager_np.int8_matmul(q[:1], w.numpy()), s[:1], ws.numpy(), bits(b), "bf16")
    assert y.shape == (1, n)
    assert np.array_equal(bits(y), bf16_bits(ref))
    both = _mx().int8_linear_prequantized(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), w.to(dev),
                                          ws.to(dev), b.to(dev))
    assert torch.equal(both[:1], y)


def test_m1_k_outside_the_gemv_range_uses_the_gemm(dev):
    """K not a multiple of 16 (and K above 16384) take the padded GEMM; values are unchanged."""
    for n, k in ((96, 72), (64, 16400)):
        x = activations(1, k, k)
        w, ws = int8_weight(n, k, k + 1)
        y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev))
        ref = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), None, "bf16")
        assert np.array_equal(bits(y), bf16_bits(ref))
