"""GPU parity of the 256 x 256-tile INT8 GEMM (the configuration every model-sized shape runs),
of the 128 x 128 one at a mid-sized shape with partial edge tiles, and of the 128 x 128 one with
the deep operand ring (one workgroup per CU, four stages in flight) that problems of at most 256
such tiles run.

The library runs a GEMM with 256 x 256 tiles once it has at least 256 of them, unless its rounds of
128 x 128 tiles (512 per round, ~0.55 of a 256-tile round) would finish first; the small-shape tests
cover 128 x 128 tiles. These shapes (4100 x 7432: 17 x 30 = 510 tiles of 256, two full rounds,
both edges partial) keep the 256 x 256 kernel for every epilogue. K is chosen
at the boundaries of the K loop: a single stage (128), stages that are all full with and without
steady-state iterations (256, 384, 1024) and a partial last stage after zero, one or two steady
iterations (144, 400, 528). Every epilogue is covered: int32, dequant (+ bias) to bf16 (alone
and as the FFN chain's fc1 and fc2), GELU + row absmax (the FFN chain's path for hidden widths
beyond 32768), SwiGLU and the gated residual.

Bar: int32 and every bf16 output bit-exact against the oracle.
"""

import numpy as np
import pytest
import torch

from _util import activations, bf16_vec, bits, gen, int8_weight
from oracle import convrot as cr
from oracle import eager_np
from oracle.bf16 import bf16_bits

pytestmark = pytest.mark.gpu

M, N = 4100, 7432  # 17 x 30 tiles of 256, both edges partial


def _mx():
    import mx_qlinear

    return mx_qlinear


def _i8(shape, seed):
    return torch.randint(-128, 128, shape, generator=gen(seed), dtype=torch.int8)


@pytest.mark.parametrize("k", [128, 144, 256, 384, 400, 528, 1024])
def test_gemm_i32_256_tiles(dev, k):
    print(f"gemm i32 256-tile m={M} n={N} k={k}", flush=True)
    a, w = _i8((M, k), 40 + k), _i8((N, k), 41 + k)
    c = _mx().mm_int8(a.to(dev), w.to(dev).t())
    assert np.array_equal(c.cpu().numpy(), eager_np.int8_matmul(a.numpy(), w.numpy()))


@pytest.mark.parametrize("k,bias", [(400, True), (1024, False)])
def test_int8_linear_256_tiles(dev, k, bias):
    print(f"int8_linear 256-tile m={M} n={N} k={k} bias={bias}", flush=True)
    x = activations(M, k, 50 + k)
    w, ws = int8_weight(N, k, 51 + k)
    b = bf16_vec(N, 52, 0.01) if bias else None
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), None if b is None else b.to(dev))
    ref = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), None if b is None else bits(b), "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))


def test_ffn_chain_256_tiles(dev):
    """fc1 (the bf16 dequant GEMM, then the one-pass GELU quantizer) runs 256 x 256 tiles; fc2
    (17 x 16 tiles of 256, just over one round) runs 128 x 128 tiles."""
    m, k, hidden, n = M, 400, 4112, 4096  # hidden: a multiple of 16 with a partial edge tile
    print(f"ffn 256-tile m={m} k={k} hidden={hidden} n={n}", flush=True)
    x = activations(m, k, 60)
    w1, s1 = int8_weight(hidden, k, 61)
    w2, s2 = int8_weight(n, hidden, 62)
    b1, b2 = bf16_vec(hidden, 63, 0.01), bf16_vec(n, 64, 0.01)
    out = _mx().int8_ffn_gelu(x.to(dev), w1.to(dev), s1.to(dev), b1.to(dev), w2.to(dev), s2.to(dev), b2.to(dev))
    ref, _ = eager_np.ffn_gelu_int8(bits(x), w1.numpy(), s1.numpy(), bits(b1), w2.numpy(), s2.numpy(), bits(b2))
    assert np.array_equal(bits(out), bf16_bits(ref))


@pytest.mark.parametrize("k", [144, 400])
def test_gelu_absmax_epilogue_256_tiles(dev, k):
    import mx_qlinear._lib as L
    from mx_qlinear import ops

    assert L.gemm_plan(M, N, k, True)["tile"] == 256
    print(f"gelu+absmax 256-tile m={M} n={N} k={k}", flush=True)
    a, w = _i8((M, k), 90 + k), _i8((N, k), 91 + k)
    xs = torch.rand(M, generator=gen(92)) * 1e-3
    ws = torch.rand(N, generator=gen(93)) * 1e-2
    b = bf16_vec(N, 94, 0.5)
    dv = [t.to(dev) for t in (a, w, xs, ws, b)]
    h = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    amax = torch.zeros(M, dtype=torch.float32, device=dev)
    L.call("mxq_int8_gemm_dequant_gelu_absmax", *map(ops._p, dv[:4]), N, ops._p(dv[4]), ops._p(h),
           ops._p(amax), M, N, k, N, *ops._gemm_ws(dev), ops._stream(dev))
    y = eager_np.dequant_epilogue(eager_np.int8_matmul(a.numpy(), w.numpy()), xs.numpy(), ws.numpy(), bits(b), "bf16")
    hb = eager_np.gelu_tanh_bf16(bf16_bits(y))
    assert np.array_equal(bits(h), hb)
    amax_bits = (hb & np.uint16(0x7FFF)).max(axis=1).astype(np.uint32) << np.uint32(16)
    assert np.array_equal(amax.cpu().numpy().view(np.uint32), amax_bits)


def test_swiglu_fc1_256_tiles(dev):
    m, f, k = M, 4096, 528
    print(f"swiglu fc1 256-tile m={m} f={f} k={k}", flush=True)
    x = activations(m, k, 70)
    w, ws = int8_weight(2 * f, k, 71)
    b = bf16_vec(2 * f, 72, 0.05)
    q, s = eager_np.quantize_int8_rowwise(bits(x))
    fc1 = _mx().prepare_swiglu_fc1(w.to(dev), ws.to(dev), b.to(dev))
    h = _mx().int8_swiglu_fc1(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), fc1)
    y = eager_np.dequant_epilogue(eager_np.int8_matmul(q, w.numpy()), s, ws.numpy(), bits(b), "bf16")
    assert np.array_equal(bits(h), cr.swiglu_bf16(bf16_bits(y)))


def test_gated_residual_256_tiles(dev):
    k = 384
    print(f"gated residual 256-tile m={M} n={N} k={k}", flush=True)
    x = activations(M, k, 80)
    w, ws = int8_weight(N, k, 81)
    b = bf16_vec(N, 82, 0.02)
    gate = torch.randn(3, N, generator=gen(83)).to(torch.bfloat16)
    res = activations(M, N, 84) * 3
    segs = ((0, 1000, 2), (1000, 2500, 0), (2500, M, 1))
    out = res.to(dev)
    _mx().int8_linear_gated_residual_(out, x.to(dev), w.to(dev), ws.to(dev), b.to(dev), gate.to(dev), segs)
    q, s = eager_np.quantize_int8_rowwise(bits(x))
    y = eager_np.dequant_epilogue(eager_np.int8_matmul(q, w.numpy()), s, ws.numpy(), bits(b), "bf16")
    want = eager_np.gated_residual_bf16(bits(res), bf16_bits(y), bits(gate), eager_np.segment_row_map(M, segs))
    assert np.array_equal(bits(out), want)


# ---- the deep-ring configurations: at most 256 tiles, one workgroup per CU with four stages in
# flight, as 128 x 128 tiles or, where more of them then fit on the CUs at once, 128 x 96 tiles
# (four 32-row strips of three blocks per wave; 12 KB B chunks). K covers one partial stage (16),
# one full (128), the loop's tail with three, two and one stages left after a partial last stage
# (144 .. 656), steady iterations (1024) and a long loop ending in a partial stage (3088).

DEEP = {
    "square": (1900, 2000, 128),  # 15 x 16 = 240 tiles of 128 (315 of 128 x 96 would not fit)
    "128x96": (1100, 1800, 96),   # 9 x 19 = 171 tiles of 128 x 96 (135 of 128), both edges partial
}


def _assert_deep(m, n, k, tile_n):
    import mx_qlinear._lib as L

    plan = L.gemm_plan(m, n, k)
    assert (plan["tile"], plan["tile_n"], plan["ahead"]) == (128, tile_n, 4), plan


@pytest.mark.parametrize("form", list(DEEP))
@pytest.mark.parametrize("k", [16, 128, 144, 400, 528, 656, 1024, 3088])
def test_gemm_i32_deep_ring(dev, k, form):
    md, nd, tile_n = DEEP[form]
    _assert_deep(md, nd, k, tile_n)
    print(f"gemm i32 deep-ring {form} m={md} n={nd} k={k}", flush=True)
    a, w = _i8((md, k), 240 + k), _i8((nd, k), 241 + k)
    c = _mx().mm_int8(a.to(dev), w.to(dev).t())
    assert np.array_equal(c.cpu().numpy(), eager_np.int8_matmul(a.numpy(), w.numpy()))


@pytest.mark.parametrize("m,n,tile_n,k,bias", [(1024, 3072, 96, 400, True), (1024, 3072, 96, 3072, False),
                                               (1900, 2000, 128, 400, True)])
def test_int8_linear_deep_ring(dev, m, n, tile_n, k, bias):
    _assert_deep(m, n, k, tile_n)
    print(f"int8_linear deep-ring m={m} n={n} k={k} bias={bias}", flush=True)
    x = activations(m, k, 250 + k)
    w, ws = int8_weight(n, k, 251 + k)
    b = bf16_vec(n, 252, 0.01) if bias else None
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), None if b is None else b.to(dev))
    ref = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), None if b is None else bits(b), "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))


@pytest.mark.parametrize("out", ["fp32", "fp16"])
def test_dequant_deep_ring_128x96_wide_outputs(dev, out):
    """fp32 outputs leave the odd third block through the staged 128-byte lines, fp16 ones by runs."""
    md, nd, tile_n = DEEP["128x96"]
    k = 528
    _assert_deep(md, nd, k, tile_n)
    print(f"dequant deep-ring 128x96 m={md} n={nd} k={k} out={out}", flush=True)
    dt = torch.float32 if out == "fp32" else torch.float16
    a, w = _i8((md, k), 255), _i8((nd, k), 256)
    xs = torch.rand(md, generator=gen(257)) * 1e-3
    ws = torch.rand(nd, generator=gen(258)) * 1e-2
    b = (torch.randn(nd, generator=gen(259)) * 0.5).to(dt)
    y = _mx().int8_linear_prequantized(a.to(dev), xs.to(dev), w.to(dev), ws.to(dev), b.to(dev), out_dtype=dt)
    ref = eager_np.dequant_epilogue(eager_np.int8_matmul(a.numpy(), w.numpy()), xs.numpy(), ws.numpy(),
                                    b.float().numpy(), out, bias_dtype="f32")
    want = ref.astype(np.float32 if out == "fp32" else np.float16)
    assert np.array_equal(y.cpu().numpy().view(want.dtype.str.replace("f", "u")), want.view(want.dtype.str.replace("f", "u")))


@pytest.mark.parametrize("form", list(DEEP))
def test_gated_residual_deep_ring(dev, form):
    md, nd, tile_n = DEEP[form]
    k = 528
    _assert_deep(md, nd, k, tile_n)
    print(f"gated residual deep-ring {form} m={md} n={nd} k={k}", flush=True)
    x = activations(md, k, 260)
    w, ws = int8_weight(nd, k, 261)
    b = bf16_vec(nd, 262, 0.02)
    gate = torch.randn(2, nd, generator=gen(263)).to(torch.bfloat16)
    res = activations(md, nd, 264) * 3
    segs = ((0, 600, 1), (600, md, 0))
    out = res.to(dev)
    _mx().int8_linear_gated_residual_(out, x.to(dev), w.to(dev), ws.to(dev), b.to(dev), gate.to(dev), segs)
    q, s = eager_np.quantize_int8_rowwise(bits(x))
    y = eager_np.dequant_epilogue(eager_np.int8_matmul(q, w.numpy()), s, ws.numpy(), bits(b), "bf16")
    want = eager_np.gated_residual_bf16(bits(res), bf16_bits(y), bits(gate), eager_np.segment_row_map(md, segs))
    assert np.array_equal(bits(out), want)


# ---- the 128 x 128-tile configuration: at least 256 tiles of 128, fewer than 256 of 256 ------

M128, N128 = 2050, 2056  # 17 x 17 tiles of 128 (9 x 9 of 256), both edges partial


@pytest.mark.parametrize("k", [128, 400, 1024])
def test_gemm_i32_128_tiles(dev, k):
    print(f"gemm i32 128-tile m={M128} n={N128} k={k}", flush=True)
    a, w = _i8((M128, k), 140 + k), _i8((N128, k), 141 + k)
    c = _mx().mm_int8(a.to(dev), w.to(dev).t())
    assert np.array_equal(c.cpu().numpy(), eager_np.int8_matmul(a.numpy(), w.numpy()))


def test_int8_linear_and_gated_residual_128_tiles(dev):
    k = 528
    x = activations(M128, k, 150)
    w, ws = int8_weight(N128, k, 151)
    b = bf16_vec(N128, 152, 0.01)
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), b.to(dev))
    assert np.array_equal(bits(y), bf16_bits(eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), bits(b), "bf16")))
    gate = torch.randn(2, N128, generator=gen(153)).to(torch.bfloat16)
    res = activations(M128, N128, 154) * 3
    segs = ((0, 700, 1), (700, M128, 0))
    out = res.to(dev)
    _mx().int8_linear_gated_residual_(out, x.to(dev), w.to(dev), ws.to(dev), b.to(dev), gate.to(dev), segs)
    q, s = eager_np.quantize_int8_rowwise(bits(x))
    yy = eager_np.dequant_epilogue(eager_np.int8_matmul(q, w.numpy()), s, ws.numpy(), bits(b), "bf16")
    want = eager_np.gated_residual_bf16(bits(res), bf16_bits(yy), bits(gate), eager_np.segment_row_map(M128, segs))
    assert np.array_equal(bits(out), want)
