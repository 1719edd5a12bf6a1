"""GPU parity: int4 grouped decode, reference-format W4A8 linear and group-scaled W4A8 GEMM.

Bar: decoded int8 weights bit-exact; outputs bit-exact against the oracle's restatement of the
same summation order; the group-scaled GEMM additionally within its float32 error bound of the
float64 value and exact where the arithmetic is exact (unit / power-of-two scales).
"""

import numpy as np
import pytest
import torch

from _util import activations, bf16_vec, bits, gen, group_scales, packed_int4
from oracle import eager_np
from oracle.bf16 import bf16_bits, bf16_ulp

pytestmark = pytest.mark.gpu


def _mx():
    import mx_qlinear

    return mx_qlinear


@pytest.mark.parametrize("g", [4, 8, 16, 32, 48, 128])
@pytest.mark.parametrize("e4m3", [False, True])
@pytest.mark.parametrize("codebook", [False, True])
def test_decode_matches_oracle(dev, g, e4m3, codebook):
    """Every group size form of the decode: 4 and 8 (four and two scales per 16 weights), 16 and
    its multiples, a power of two or not (one scale per 16 weights)."""
    n, k = 96, 480 if g == 48 else 512
    qd = packed_int4(n, k, 7 + g)
    s = torch.rand(n, k // g, generator=gen(g)) * 30
    if e4m3:
        s = s.to(torch.float8_e4m3fn)
    cb = torch.linspace(-7.5, 7.5, 16) if codebook else None
    w8 = _mx().dequantize_int4_grouped_to_int8(qd.to(dev), s.to(dev), None if cb is None else cb.to(dev), g)
    s_np = s.view(torch.uint8).numpy() if e4m3 else s.numpy()
    ref = eager_np.dequant_int4_grouped_to_int8(qd.numpy(), s_np, None if cb is None else cb.numpy(), g,
                                                s_rel_is_e4m3=e4m3)
    assert np.array_equal(w8.cpu().numpy(), ref)


def test_decode_unit_scale_is_code_minus_8(dev):
    n, k = 16, 64
    codes = np.arange(n * k).reshape(n, k) % 16
    qd = torch.from_numpy(eager_np.pack_int4(codes))
    w8 = _mx().dequantize_int4_grouped_to_int8(qd.to(dev), torch.ones(n, k // 16, device=dev), None, 16)
    assert np.array_equal(w8.cpu().numpy(), codes - 8)


def _format_r_storage(n, k, g, use_codebook, source):
    """Random codes and scales, or storage made by quantize_w4a8_int8_weight from an N(0, 0.02)
    bf16 weight (the reference's codebook or uniform symmetric mode, e4m3 s_rel)."""
    if source == "prepared":
        w = (torch.randn(n, k, generator=gen(36)) * 0.02).to(torch.bfloat16)
        qd, s_rel, s_ch, _, cb = _mx().quantize_w4a8_int8_weight(w.cuda(), g, 256, codebook=use_codebook)
        return qd.cpu(), s_rel.cpu(), s_ch.cpu(), None if cb is None else cb.cpu()
    qd = packed_int4(n, k, 32)
    s_rel = (torch.rand(n, k // g, generator=gen(33)) * 15 + 1).to(torch.float8_e4m3fn)
    s_ch = torch.rand(n, generator=gen(34)) * 1e-3
    return qd, s_rel, s_ch, torch.linspace(-7.5, 7.5, 16) if use_codebook else None


@pytest.mark.parametrize("source", ["random", "prepared"])
@pytest.mark.parametrize("m,n,k,use_codebook", [(200, 300, 1024, True), (64, 4232, 256, False)])
def test_w4a8_reference_format_linear(dev, m, n, k, use_codebook, source):
    g = 16
    x = activations(m, k, 31)
    qd, s_rel, s_ch, cb = _format_r_storage(n, k, g, use_codebook, source)
    bias = bf16_vec(n, 35, 0.01)
    y = _mx().w4a8_int8_linear(x.to(dev), qd.to(dev), s_rel.to(dev), s_ch.to(dev),
                               codebook=None if cb is None else cb.to(dev),
                               bias=bias.to(dev), group_size=g, convrot_groupsize=0)
    ref = eager_np.w4a8_reference_linear(bits(x), qd.numpy(), s_rel.view(torch.uint8).numpy(), s_ch.numpy(),
                                         None if cb is None else cb.numpy(), g, bits(bias), "bf16", s_rel_is_e4m3=True)
    assert np.array_equal(bits(y), bf16_bits(ref))


def test_w4a8_reference_format_chunking_changes_nothing(dev):
    """Through the C-ABI: the decode-then-GEMM over column chunks of 4232 (one chunk, as
    w4a8_decode_chunk picks here), 4096 + 136, 1000 and 136 columns gives the same output bit for
    bit, each chunk's GEMM writing its output column slice."""
    from mx_qlinear import _lib
    from mx_qlinear.ops import _gemm_ws, _p, _stream

    m, n, k, g = 64, 4232, 256, 16
    assert _mx().ops.w4a8_decode_chunk(n, k) == n
    qd, s_rel, s_ch, cb = (t.to(dev) for t in _format_r_storage(n, k, g, True, "random"))
    xq = torch.randint(-127, 128, (m, k), generator=gen(36), dtype=torch.int8).to(dev)
    xs = (torch.rand(m, generator=gen(37)) * 1e-2).to(dev)
    bias = bf16_vec(n, 38, 0.01).to(dev)
    outs = []
    for chunk in (n, 4096, 1000, 136):
        work = torch.empty((chunk, k), dtype=torch.int8, device=dev)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        _lib.call("mxq_w4a8_codebook_gemm", _p(xq), _p(qd), _p(s_rel), _lib.DTYPE_E4M3, _p(cb), _p(s_ch), _p(xs),
                  _p(bias), _p(work), _p(out), m, n, k, g, chunk, _lib.DTYPE_BF16, *_gemm_ws(dev), _stream(dev))
        outs.append(out)
    for out in outs[1:]:
        assert torch.equal(out, outs[0])


def _int_input(m, k, seed):
    return torch.randint(-128, 128, (m, k), generator=gen(seed), dtype=torch.int8)


@pytest.mark.parametrize("m", [64, 2048])
def test_grouped_unit_scales_are_exact(dev, m):
    """scale = 1, xs = 1, fp32 out: the output is the exact integer sum of A * (c - 8)."""
    n, k, g = 384, 1024, 128
    a = _int_input(m, k, m)
    qd = packed_int4(n, k, m + 1)
    gs = torch.ones(k // g, n, dtype=torch.float16)
    y = _mx().w4a8_grouped_linear(a.to(dev), qd.to(dev), gs.to(dev), g, out_dtype=torch.float32,
                                  x_scale=torch.ones(m, device=dev))
    w = eager_np.unpack_int4(qd.numpy()) - 8
    exact = a.numpy().astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(y.cpu().numpy(), exact.astype(np.float32))


def test_grouped_power_of_two_scales_are_exact(dev):
    """Per-group scales 2^-(g % 5): every fp32 step is exact, so the group indexing is pinned."""
    m, n, k, g = 96, 256, 2048, 128
    a = _int_input(m, k, 3)
    qd = packed_int4(n, k, 4)
    gs = torch.tensor([2.0 ** -(i % 5) for i in range(k // g)], dtype=torch.float16)[:, None].repeat(1, n)
    gs[:, 7] = 4.0
    y = _mx().w4a8_grouped_linear(a.to(dev), qd.to(dev), gs.to(dev), g, out_dtype=torch.float32,
                                  x_scale=torch.ones(m, device=dev))
    p = eager_np.w4a8_group_partials(a.numpy(), qd.numpy(), g).astype(np.float64)
    exact = (p * gs.double().numpy()[:, None, :]).sum(axis=0)
    assert np.array_equal(y.cpu().numpy().astype(np.float64), exact)


# group 128 with N % 8 == 0 runs the pipelined kernel (edge tiles in M and N included; K of one
# and two groups, shorter than its 3-stage ring): with 64-row tiles below 512 tiles of 128 rows,
# with 128-row tiles from there (2056 x 4104: 17 x 33 tiles, both edges partial); group 256 and
# N = 70 run the general kernel.
@pytest.mark.parametrize("m,n,k,g", [(512, 1024, 5120, 128), (2048, 640, 1024, 128), (100, 200, 1024, 128),
                                     (257, 136, 640, 128), (64, 256, 128, 128), (130, 264, 256, 128),
                                     (2056, 4104, 384, 128), (100, 200, 1024, 256), (33, 70, 512, 128)])
def test_grouped_matches_oracle(dev, m, n, k, g):
    print(f"w4a8 grouped m={m} n={n} k={k} g={g}", flush=True)
    x = activations(m, k, 1000 + m, outlier_frac=0.0)
    qd = packed_int4(n, k, 1001 + n)
    gs = group_scales(k, n, g, 1002)
    y = _mx().w4a8_grouped_linear(x.to(dev), qd.to(dev), gs.to(dev), g)
    a, xs = eager_np.quantize_int8_rowwise(bits(x))
    ref = eager_np.w4a8_grouped_linear(a, xs, qd.numpy(), gs.numpy(), g)
    assert np.array_equal(bits(y), bf16_bits(ref))
    # independent float64 pin: |y - exact| <= 1 ulp(y) + fp32 accumulation bound
    exact, mag = eager_np.w4a8_grouped_linear_f64(a, xs, qd.numpy(), gs.numpy(), g)
    yv = y.float().cpu().numpy().astype(np.float64)
    bound = bf16_ulp(np.abs(exact).astype(np.float32)).astype(np.float64) + (k // g + 2) * 2.0 ** -24 * mag
    assert np.all(np.abs(yv - exact) <= bound)


# The 128-row tile form over K loops that wrap its 3-stage ring several times, with a group count
# that is not a multiple of 3 (10 and 40 groups: the unrolled-by-three stage loop plus one leftover
# stage), on both edges partial (2056 x 4104: 17 x 33 = 561 tiles, above the 512 that select the
# form), on the checkpoint and the prepared layout. Sampled rows (first, last, random) against the
# oracle, which computes per-group partials of every sampled row.
@pytest.mark.parametrize("k", [1280, 5120])
@pytest.mark.parametrize("prepared", [False, True])
def test_grouped_128_row_tiles_deep_k(dev, k, prepared):
    m, n, g = 2056, 4104, 128
    assert ((m + 127) // 128) * ((n + 127) // 128) >= 512 and (k // g) % 3 != 0
    print(f"w4a8 grouped 128-row tiles m={m} n={n} k={k} prepared={prepared}", flush=True)
    x = activations(m, k, 1100 + k, outlier_frac=0.0)
    qd = packed_int4(n, k, 1101 + k)
    gs = group_scales(k, n, g, 1102 + k)
    bias = bf16_vec(n, 1103, 0.01)
    qdd = qd.to(dev)
    y = _mx().w4a8_grouped_linear(x.to(dev), _mx().prepare_w4a8_grouped(qdd) if prepared else qdd, gs.to(dev), g,
                                  bias=bias.to(dev))
    rnd = np.random.default_rng(k).choice(np.arange(8, m - 8), size=48, replace=False)
    rows = np.unique(np.concatenate([np.arange(8), np.arange(m - 8, m), rnd]))
    a, xs = eager_np.quantize_int8_rowwise(bits(x[torch.from_numpy(rows)]))
    ref = eager_np.w4a8_grouped_linear(a, xs, qd.numpy(), gs.numpy(), g, bits(bias))
    got = y[torch.from_numpy(rows).to(dev)]
    assert np.array_equal(bits(got), bf16_bits(ref))


# The 128-row tile form on a larger problem (4100 x 4360: 33 x 35 tiles, both edges partial) over
# K of 1, 3, 5 and 10 groups (its ring holds three), on both weight layouts, with a bias, and
# fp16 / fp32 outputs. Sampled rows against the oracle.
@pytest.mark.parametrize("k,prepared,out_dtype", [(128, True, torch.bfloat16), (384, False, torch.bfloat16),
                                                  (640, True, torch.float16), (1280, False, torch.float32),
                                                  (1280, True, torch.bfloat16)])
def test_grouped_128_row_tiles_outputs(dev, k, prepared, out_dtype):
    m, n, g = 4100, 4360, 128
    assert -(-m // 128) * -(-n // 128) >= 512
    print(f"w4a8 grouped 128-row tiles m={m} n={n} k={k} prepared={prepared} out={out_dtype}", flush=True)
    x = activations(m, k, 1200 + k, outlier_frac=0.0)
    qd = packed_int4(n, k, 1201 + k)
    gs = group_scales(k, n, g, 1202 + k)
    bias = bf16_vec(n, 1203, 0.01)
    qdd = qd.to(dev)
    y = _mx().w4a8_grouped_linear(x.to(dev), _mx().prepare_w4a8_grouped(qdd) if prepared else qdd, gs.to(dev), g,
                                  bias=bias.to(dev), out_dtype=out_dtype)
    rnd = np.random.default_rng(k).choice(np.arange(8, m - 8), size=40, replace=False)
    rows = np.unique(np.concatenate([np.arange(8), np.arange(m - 8, m), rnd]))
    a, xs = eager_np.quantize_int8_rowwise(bits(x[torch.from_numpy(rows)]))
    code = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[out_dtype]
    ref = eager_np.w4a8_grouped_linear(a, xs, qd.numpy(), gs.numpy(), g, bits(bias), code)
    got = y[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("m,n", [(64, 256), (130, 200)])
def test_grouped_with_bias(dev, m, n):
    k, g = 512, 128
    x = activations(m, k, 70)
    qd = packed_int4(n, k, 71 + m)
    gs = group_scales(k, n, g, 72)
    bias = bf16_vec(n, 73, 0.01)
    y = _mx().w4a8_grouped_linear(x.to(dev), qd.to(dev), gs.to(dev), g, bias=bias.to(dev))
    a, xs = eager_np.quantize_int8_rowwise(bits(x))
    ref = eager_np.w4a8_grouped_linear(a, xs, qd.numpy(), gs.numpy(), g, bits(bias))
    assert np.array_equal(bits(y), bf16_bits(ref))


# ---- the prepared (load) layout of the group-128 kernel ------------------------------------

@pytest.mark.parametrize("n,k", [(136, 640), (3, 8), (1024, 5120)])
def test_prepare_matches_oracle(dev, n, k):
    qd = packed_int4(n, k, 900 + n)
    got = _mx().prepare_w4a8_grouped(qd.to(dev)).qdata.cpu().numpy()
    assert np.array_equal(got, eager_np.prepare_w4a8_grouped(qd.numpy()))


@pytest.mark.parametrize("m,n,k,bias,out_dtype", [(512, 1024, 5120, False, torch.bfloat16),
                                                  (257, 136, 640, True, torch.bfloat16),
                                                  (2056, 4104, 256, False, torch.bfloat16),
                                                  (2056, 4104, 128, True, torch.float16),
                                                  (64, 256, 128, False, torch.float16),
                                                  (130, 264, 256, True, torch.float32)])
def test_prepared_equals_checkpoint_layout(dev, m, n, k, bias, out_dtype):
    print(f"w4a8 prepared m={m} n={n} k={k} bias={bias} out={out_dtype}", flush=True)
    x = activations(m, k, 910 + m).to(dev)
    qd = packed_int4(n, k, 911 + n).to(dev)
    gs = group_scales(k, n, 128, 912).to(dev)
    b = bf16_vec(n, 913, 0.01).to(out_dtype).to(dev) if bias else None
    ref = _mx().w4a8_grouped_linear(x, qd, gs, 128, bias=b, out_dtype=out_dtype)
    got = _mx().w4a8_grouped_linear(x, _mx().prepare_w4a8_grouped(qd), gs, 128, bias=b, out_dtype=out_dtype)
    assert torch.equal(got.view(torch.int16 if out_dtype != torch.float32 else torch.int32),
                       ref.view(torch.int16 if out_dtype != torch.float32 else torch.int32))
    if not bias and out_dtype == torch.bfloat16:
        a, xs = eager_np.quantize_int8_rowwise(bits(x.cpu()))
        want = eager_np.w4a8_grouped_linear(a, xs, qd.cpu().numpy(), gs.cpu().numpy(), 128)
        assert np.array_equal(bits(got), bf16_bits(want))


def test_prepared_needs_group_128(dev):
    qd = packed_int4(64, 512, 920).to(dev)
    x = activations(16, 512, 921).to(dev)
    with pytest.raises(RuntimeError, match="group 128"):
        _mx().w4a8_grouped_linear(x, _mx().prepare_w4a8_grouped(qd), group_scales(512, 64, 256, 922).to(dev), 256)


# ---- the correction term of asymmetric int4 weights (reference CUDA backend) ---------------

@pytest.mark.parametrize("g,out_dtype,code", [(16, torch.bfloat16, "bf16"), (4, torch.float16, "fp16"),
                                              (32, torch.float32, "fp32")])
def test_group_sums_match_oracle(dev, g, out_dtype, code):
    from mx_qlinear import _lib as L
    from mx_qlinear.ops import _p, _stream

    m, k = 37, 640
    xq = torch.randint(-128, 128, (m, k), generator=gen(950), dtype=torch.int8)
    xs = torch.rand(m, generator=gen(951)) * 0.01
    out = torch.empty(m, k // g, dtype=out_dtype, device=dev)
    xqd, xsd = xq.to(dev), xs.to(dev)
    L.call("mxq_int8_group_sums", _p(xqd), _p(xsd), _p(out), m, k, g,
           {torch.bfloat16: L.DTYPE_BF16, torch.float16: L.DTYPE_F16, torch.float32: L.DTYPE_F32}[out_dtype], _stream(dev))
    want = eager_np.w4a8_correction_lhs(xq.numpy(), xs.numpy(), g, code)
    assert np.array_equal(out.float().cpu().numpy(), want)


def _corr_case(dev, m, n, k, g):
    x = activations(m, k, 960).to(dev)
    qd = packed_int4(n, k, 961).to(dev)
    s_rel = (torch.rand(n, k // g, generator=gen(962)) * 0.75 + 0.25).to(torch.float8_e4m3fn).to(dev)
    s_ch = (torch.rand(n, generator=gen(963)) * 1e-3).to(dev)
    corr = (torch.randn(k // g, n, generator=gen(964)) * 0.01).to(torch.bfloat16).to(dev)
    bias = bf16_vec(n, 965, 0.01).to(dev)
    return x, qd, s_rel, s_ch, corr, bias


def test_correction_equals_the_reference_composition(dev):
    """With a correction the output is the reference CUDA backend's composition run with torch on
    the same device: the W8A8 result, then out.addmm_(bf16(group sums) * bf16(xs), correction)."""
    m, n, k, g = 150, 264, 512, 16
    x, qd, s_rel, s_ch, corr, bias = _corr_case(dev, m, n, k, g)
    got = _mx().w4a8_int8_linear(x, qd, s_rel, s_ch, correction=corr, bias=bias, group_size=g, convrot_groupsize=256)
    base = _mx().w4a8_int8_linear(x, qd, s_rel, s_ch, bias=bias, group_size=g, convrot_groupsize=256)
    xq, xs = _mx().quantize_int8_rowwise_convrot(x, 256)
    sx = xq.view(m, k // g, g).sum(-1, dtype=torch.int32).to(torch.bfloat16) * xs.reshape(-1, 1).to(torch.bfloat16)
    ref = base.clone().addmm_(sx, corr)
    assert torch.equal(got, ref)
    # and within 1 ulp + the float32 accumulation bound of the exact value of that expression
    lhs = eager_np.w4a8_correction_lhs(xq.cpu().numpy(), xs.cpu().numpy(), g, "bf16").astype(np.float64)
    terms = lhs[:, :, None] * corr.float().cpu().numpy().astype(np.float64)[None, :, :]
    exact = base.float().cpu().numpy().astype(np.float64) + terms.sum(1)
    mag = np.abs(base.float().cpu().numpy()).astype(np.float64) + np.abs(terms).sum(1)
    bound = bf16_ulp(np.abs(exact).astype(np.float32)).astype(np.float64) + (k // g + 2) * 2.0 ** -24 * mag
    assert np.all(np.abs(got.float().cpu().numpy().astype(np.float64) - exact) <= bound)


def test_correction_through_the_module(dev):
    m, n, k, g = 64, 136, 256, 16
    x, qd, s_rel, s_ch, corr, bias = _corr_case(dev, m, n, k, g)
    from mx_qlinear.modules import ConvRotW4A8Linear, W4A8QuantSpec, w4a8_kernel

    layer = ConvRotW4A8Linear(qd, s_rel, s_ch, correction=corr, bias=bias,
                              spec=W4A8QuantSpec(group_size=g, convrot_groupsize=256), kernel=w4a8_kernel)
    want = _mx().w4a8_int8_linear(x, qd, s_rel, s_ch, correction=corr, bias=bias, group_size=g, convrot_groupsize=256)
    assert torch.equal(layer(x), want)
