"""GPU parity: INT8 GEMM (int32), fused dequant epilogues, int8_linear and the FFN chain.

Bar: int32 accumulators bit-exact; bf16/fp16/fp32 outputs bit-exact against the oracle's
restatement of the eager recipe (which is within 1 bf16 ulp of any other rounding order).
"""

import numpy as np
import pytest
import torch

import mx_qlinear._lib as L
from _util import activations, bf16_vec, bits, gen, int8_weight
from oracle import eager_np
from oracle.bf16 import bf16_bits

pytestmark = pytest.mark.gpu


def _mx():
    import mx_qlinear

    return mx_qlinear


def _i8(shape, seed, lo=-128, hi=128):
    return torch.randint(lo, hi, shape, generator=gen(seed), dtype=torch.int8)


@pytest.mark.parametrize(
    "m,n,k",
    [(1, 1, 16), (256, 256, 128), (257, 384, 3072), (300, 200, 144), (64, 1000, 4096), (513, 257, 1040)],
)
def test_gemm_i32_exact(dev, m, n, k):
    print(f"gemm i32 m={m} n={n} k={k}", flush=True)
    a, w = _i8((m, k), m + k), _i8((n, k), n * 3 + k)
    c = _mx().mm_int8(a.to(dev), w.to(dev).t())
    assert np.array_equal(c.cpu().numpy(), eager_np.int8_matmul(a.numpy(), w.numpy()))


def test_gemm_i32_bruteforce_small(dev):
    a, w = _i8((19, 48), 1), _i8((23, 48), 2)
    c = _mx().mm_int8(a.to(dev), w.to(dev).t())
    assert np.array_equal(c.cpu().numpy(), eager_np.int8_matmul_bruteforce(a.numpy(), w.numpy()))


def test_gemm_extremes_and_structure(dev):
    """Saturation-free extremes, identity and permutation weights."""
    k = 20480
    a = torch.full((3, k), -128, dtype=torch.int8)
    a[1] = 127
    w = torch.full((2, k), -128, dtype=torch.int8)
    c = _mx().mm_int8(a.to(dev), w.to(dev).t()).cpu()
    assert c[0, 0] == k * 128 * 128 and c[1, 0] == -k * 127 * 128
    k = 512
    a = _i8((300, k), 5)
    eye = torch.eye(k, dtype=torch.int8)
    assert torch.equal(_mx().mm_int8(a.to(dev), eye.to(dev)).cpu(), a.to(torch.int32))
    perm = torch.randperm(k, generator=gen(6))
    c = _mx().mm_int8(a.to(dev), eye[:, perm].contiguous().to(dev)).cpu()
    assert torch.equal(c, a[:, perm].to(torch.int32))


def test_gemm_largest_k(dev):
    """K = 131056, the largest K whose int32 sums cannot overflow (131056 * 128 * 128 < 2^31):
    extreme operands sum exactly; one 16 beyond is rejected."""
    k = 131056
    a = torch.full((3, k), -128, dtype=torch.int8)
    a[1] = 127
    a[2, ::2] = 5
    w = torch.full((2, k), -128, dtype=torch.int8)
    w[1, 1::2] = 3
    c = _mx().mm_int8(a.to(dev), w.to(dev).t()).cpu()
    assert np.array_equal(c.numpy(), eager_np.int8_matmul(a.numpy(), w.numpy()))
    assert c[0, 0] == k * 128 * 128 == 2147221504
    with pytest.raises(RuntimeError, match="exceeds the int32 accumulator bound"):
        _mx().mm_int8(torch.zeros(2, k + 16, dtype=torch.int8, device=dev),
                      torch.zeros(k + 16, 2, dtype=torch.int8, device=dev))


def test_gemm_i32_strided_output(dev):
    m, n, k, ldc = 100, 300, 256, 512
    a, w = _i8((m, k), 8), _i8((n, k), 9)
    c = torch.full((m, ldc), 7, dtype=torch.int32, device=dev)
    from mx_qlinear.ops import _p, _stream

    ad, wd = a.to(dev), w.to(dev)
    L.call("mxq_int8_gemm_i32", _p(ad), _p(wd), _p(c), m, n, k, ldc, None, 0, _stream(dev))
    c = c.cpu().numpy()
    assert np.array_equal(c[:, :n], eager_np.int8_matmul(a.numpy(), w.numpy()))
    assert np.all(c[:, n:] == 7)


@pytest.mark.parametrize("m,n,tile_n", [(260, 520, 96), (1000, 192, 128)])  # both deep-ring tile forms
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("per_channel", [False, True])
def test_dequant_epilogue_matches_oracle(dev, out_dtype, with_bias, per_channel, m, n, tile_n):
    from mx_qlinear import _lib

    k = 1024
    assert _lib.gemm_plan(m, n, k)["tile_n"] == tile_n
    print(f"dequant epilogue m={m} n={n} out={out_dtype} bias={with_bias} per_channel={per_channel}", flush=True)
    x = activations(m, k, 41)
    w, ws = int8_weight(n, k, 42)
    if not per_channel:
        ws = ws[:1].clone()
    bias = bf16_vec(n, 43, 0.01) if with_bias else None
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), None if bias is None else bias.to(dev),
                          out_dtype=out_dtype)
    name = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[out_dtype]
    # a bf16 bias is cast to the output dtype before the add (bias.to(result.dtype))
    ref = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), None if bias is None else bits(bias), name)
    got = y.float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def test_int8_linear_config1(dev):
    """W8A8 single linear, X [1024, 3072] with 0.5% outlier channels, W [3072, 3072]."""
    m, k, n = 1024, 3072, 3072
    x = activations(m, k, 20261201)
    w, ws = int8_weight(n, k, 20261202)
    bias = bf16_vec(n, 20261203, 0.01)
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.reshape(n, 1).to(dev), bias.to(dev))
    ref = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), bits(bias), "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))


def test_int8_linear_leading_dims_and_empty(dev):
    x = activations(2 * 3 * 5, 256, 3).reshape(2, 3, 5, 256)
    w, ws = int8_weight(64, 256, 4)
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev))
    assert y.shape == (2, 3, 5, 64)
    ref = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), None, "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))
    e = _mx().int8_linear(x[:0].to(dev), w.to(dev), ws.to(dev))
    assert e.shape == (0, 3, 5, 64)


def test_int8_linear_k_not_multiple_of_16(dev):
    x = activations(40, 100, 12)
    w, ws = int8_weight(48, 100, 13)
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev))
    ref = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), None, "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))


def test_padded_weight_form_follows_updates(dev):
    """A weight whose K needs padding has its GEMM form cached on the tensor: an in-place update
    through the tensor, a prepare_int8_weight call after a write through .data, and a
    load_state_dict into a module all make later calls use the new contents; mm_int8's generic
    right operand is never cached."""
    from mx_qlinear.modules import ComfyQuantSpec, ConvRotInt8Linear

    x = activations(40, 100, 14)
    w0, ws = int8_weight(48, 100, 15)
    w1, _ = int8_weight(48, 100, 16)
    wd = w0.to(dev)
    xd, wsd = x.to(dev), ws.to(dev)

    def want(w):
        return bf16_bits(eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), None, "bf16"))

    assert np.array_equal(bits(_mx().int8_linear(xd, wd, wsd)), want(w0))
    wd.copy_(w1.to(dev))  # through the tensor: its version moves
    assert np.array_equal(bits(_mx().int8_linear(xd, wd, wsd)), want(w1))
    wd.data.copy_(w0.to(dev))  # through .data: the caller re-prepares
    _mx().prepare_int8_weight(wd)
    assert np.array_equal(bits(_mx().int8_linear(xd, wd, wsd)), want(w0))
    spec = ComfyQuantSpec(format="int8_tensorwise", convrot=False)
    layer = ConvRotInt8Linear(w1.to(dev), ws.reshape(-1, 1).to(dev), spec=spec)
    assert np.array_equal(bits(layer(xd)), want(w1))
    layer.load_state_dict({"qweight": w0.to(dev), "scale": ws.reshape(-1, 1).to(dev)})
    assert np.array_equal(bits(layer(xd)), want(w0))
    a = _i8((33, 100), 17)
    b = _i8((100, 24), 18)
    bd = b.to(dev)
    assert np.array_equal(_mx().mm_int8(a.to(dev), bd).cpu().numpy(), eager_np.int8_matmul(a.numpy(), b.numpy().T))
    assert not hasattr(bd, "_mxq_gemm_weight")
    bd.copy_(_i8((100, 24), 19).to(dev))
    assert np.array_equal(_mx().mm_int8(a.to(dev), bd).cpu().numpy(),
                          eager_np.int8_matmul(a.numpy(), bd.cpu().numpy().T))


def test_int8_linear_gelu_input_act(dev):
    x = (torch.randn(96, 512, generator=gen(21)) * 2).to(torch.bfloat16)
    w, ws = int8_weight(256, 512, 22)
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), input_act="gelu_tanh")
    ref = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), None, "bf16", input_act="gelu_tanh")
    assert np.array_equal(bits(y), bf16_bits(ref))


def test_int8_linear_rejects_bad_arguments(dev):
    x = activations(4, 64, 1).to(dev)
    w, ws = int8_weight(8, 64, 2)
    with pytest.raises(ValueError):
        _mx().int8_linear(x, w[:, :32].contiguous().to(dev), ws.to(dev))
    with pytest.raises(ValueError):
        _mx().int8_linear(x, w.to(dev), ws[:3].to(dev))
    with pytest.raises(ValueError):
        _mx().int8_linear(x, w.to(dev), ws.to(dev), input_act="relu")


def test_prequantized_accepts_unaligned_views(dev):
    """Operands that start off a 16-byte boundary (views into a flat buffer) give the same int32
    products and outputs as aligned copies."""
    m, n, k = 48, 40, 64
    a, w = torch.randint(-128, 128, (m, k), generator=gen(7), dtype=torch.int8), torch.randint(
        -128, 128, (n, k), generator=gen(8), dtype=torch.int8)
    buf = torch.zeros(m * k + 3, dtype=torch.int8, device=dev)
    av = buf[3:].view(m, k)
    av.copy_(a.to(dev))
    assert av.data_ptr() % 16 and av.is_contiguous()
    c = _mx().mm_int8(av, w.to(dev).t())
    assert np.array_equal(c.cpu().numpy(), eager_np.int8_matmul(a.numpy(), w.numpy()))
    xs = torch.rand(m, 1, generator=gen(9)) * 1e-2
    ws = torch.rand(n, generator=gen(10)) * 1e-2
    y = _mx().int8_linear_prequantized(av, xs.to(dev), w.to(dev), ws.to(dev))
    ref = eager_np.dequant_epilogue(eager_np.int8_matmul(a.numpy(), w.numpy()), xs.numpy(), ws.numpy(), None, "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))


def test_output_and_scale_arguments_are_checked(dev):
    """Buffers a kernel would write or read past are rejected before any launch."""
    m, f, k = 32, 64, 128
    q = torch.zeros(m, k, dtype=torch.int8, device=dev)
    s = torch.ones(m, 1, device=dev)
    w, ws = int8_weight(2 * f, k, 11)
    fc1 = _mx().prepare_swiglu_fc1(w.to(dev), ws.to(dev))
    for bad in (torch.empty(m, f - 8, dtype=torch.bfloat16, device=dev),
                torch.empty(m, f, dtype=torch.float16, device=dev),
                torch.empty(m, 2 * f, dtype=torch.bfloat16, device=dev)[:, ::2]):
        with pytest.raises(ValueError):
            _mx().int8_swiglu_fc1(q, s, fc1, out=bad)
    qd = torch.zeros(f, k // 2, dtype=torch.int8, device=dev)
    gs = torch.ones(k // 128, f, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="x_scale"):
        _mx().w4a8_grouped_linear(q, qd, gs, 128, x_scale=s[: m // 2])
    with pytest.raises(ValueError, match="codebook"):
        _mx().dequantize_int4_grouped_to_int8(qd, torch.ones(f, k // 16, device=dev), torch.zeros(8, device=dev), 16)


# the last case is wider than the GELU quantizer's 32768 columns: fc1 applies GELU in its epilogue
@pytest.mark.parametrize("m,k,hidden,n", [(300, 256, 1024, 256), (64, 512, 2048, 384), (40, 128, 32784, 256)])
def test_ffn_chain_matches_oracle(dev, m, k, hidden, n):
    print(f"ffn m={m} k={k} hidden={hidden} n={n}", flush=True)
    x = activations(m, k, 500 + m)
    w1, s1 = int8_weight(hidden, k, 501)
    w2, s2 = int8_weight(n, hidden, 502)
    b1, b2 = bf16_vec(hidden, 503, 0.01), bf16_vec(n, 504, 0.01)
    out, h = _mx().int8_ffn_gelu(x.to(dev), w1.to(dev), s1.to(dev), b1.to(dev), w2.to(dev), s2.to(dev),
                                 b2.to(dev), return_hidden=True)
    ref_out, ref_h = eager_np.ffn_gelu_int8(bits(x), w1.numpy(), s1.numpy(), bits(b1), w2.numpy(),
                                            s2.numpy(), bits(b2))
    assert np.array_equal(bits(h), bf16_bits(ref_h))
    assert np.array_equal(bits(out), bf16_bits(ref_out))
    # same result as the unfused two-call composition of the public API
    y1 = _mx().int8_linear(x.to(dev), w1.to(dev), s1.to(dev), b1.to(dev))
    y2 = _mx().int8_linear(y1, w2.to(dev), s2.to(dev), b2.to(dev), input_act="gelu_tanh")
    assert torch.equal(y2, out)
