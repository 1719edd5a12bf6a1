"""CPU tests that pin the oracle itself (no GPU).

Each oracle function is checked against something other than its own formula: hand-derived
known answers, brute force, a second independent restatement (torch-CPU eager op sequence),
float64 bounds, the golden fixtures, and planted mistakes that the known answers must catch.
"""

import pathlib

import numpy as np
import pytest
import torch

from _util import activations, bf16_vec, bits, from_bits, gen, int8_weight, packed_int4
from oracle import eager_np, eager_torch
from oracle.bf16 import bf16_bits, bf16_to_f32, bf16_ulp, e4m3fn_to_f32, round_bf16

GOLDEN = pathlib.Path(__file__).parent / "golden"


# ---- quantizer ---------------------------------------------------------------------------

def _kat_rows():
    k = 16
    rows, expect = [], []
    # constant 1.0: s = 1/127, bf16(s) = 0.00787353515625 (rounded down), 1/bf16(s) = 127.008
    # -> bf16 127 -> 127.
    rows.append(np.full(k, 1.0, np.float32)); expect.append({i: 127 for i in range(k)})
    # constant 3.0: bf16(3/127) = 0.023681640625 (rounded up), 3/bf16(s) = 126.68 -> bf16 126.5
    # -> half-to-even 126: a constant row does not always reach 127.
    rows.append(np.full(k, 3.0, np.float32)); expect.append({i: 126 for i in range(k)})
    rows.append(np.zeros(k, np.float32)); expect.append({i: 0 for i in range(k)})
    r = np.zeros(k, np.float32); r[5] = -2.5; rows.append(r); expect.append({5: -127, 4: 0})
    r = np.zeros(k, np.float32); r[:6] = [127, 0.5, 1.5, 2.5, -3.5, 126.5]; rows.append(r)
    expect.append({0: 127, 1: 0, 2: 2, 3: 2, 4: -4, 5: 126})
    r = np.zeros(k, np.float32); r[:3] = [-42.5, 1.0, 42.5]; rows.append(r)
    expect.append({0: -128, 1: 3, 2: 127})
    return np.stack([bf16_bits(r) for r in rows]), expect


def _check_kats(quant):
    xb, expect = _kat_rows()
    q, s = quant(xb)
    ok = s[2, 0] == np.float32(1e-30)
    for row, exp in enumerate(expect):
        for col, val in exp.items():
            ok &= int(q[row, col]) == val
    return bool(ok)


def test_quantizer_known_answers():
    assert _check_kats(eager_np.quantize_int8_rowwise)


def _variant(mistake):
    def quant(xb):
        xf = bf16_to_f32(xb)
        amax = np.max(np.abs(xf), axis=-1, keepdims=True)
        s = np.maximum(amax / np.float32(127), np.float32(1e-30)).astype(np.float32)
        sm = s if mistake == "no_scale_rounding" else round_bf16(s)
        qf = xf / sm if mistake == "no_quotient_rounding" else round_bf16(xf / sm)
        if mistake == "half_away":
            r = np.sign(qf) * np.floor(np.abs(qf) + 0.5)
        else:
            r = np.rint(qf)
        lo = -127 if mistake == "symmetric_clamp" else -128
        return np.clip(r, lo, 127).astype(np.int8), s
    return quant


@pytest.mark.parametrize("mistake", ["no_scale_rounding", "no_quotient_rounding", "half_away",
                                     "symmetric_clamp"])
def test_quantizer_kats_catch_planted_mistakes(mistake):
    assert not _check_kats(_variant(mistake))


@pytest.mark.parametrize("m,k", [(33, 3072), (5, 100), (64, 5120)])
def test_quantizer_numpy_matches_torch_eager(m, k):
    x = activations(m, k, 7 + k)
    q1, s1 = eager_np.quantize_int8_rowwise(bits(x))
    q2, s2 = eager_torch.quantize_int8_rowwise(x)
    assert np.array_equal(q1, q2.numpy()) and np.array_equal(s1, s2.numpy())


def test_quantizer_row_slice_invariance():
    xb = bits(activations(50, 256, 1))
    q, s = eager_np.quantize_int8_rowwise(xb)
    q2, s2 = eager_np.quantize_int8_rowwise(xb[10:20])
    assert np.array_equal(q[10:20], q2) and np.array_equal(s[10:20], s2)


def test_reciprocal_multiply_equals_division_for_all_bf16_pairs():
    """bf16(x * rn(1/s)) == bf16(x / s) for every positive finite bf16 x and every bf16 s
    significand, at exponent offsets covering the quantizer's range (the device kernels rely
    on it). Signs are symmetric under IEEE rounding."""
    x = bf16_to_f32(np.arange(0x0000, 0x7F80, dtype=np.uint16))
    sig = bf16_to_f32(np.arange(0x3F80, 0x4000, dtype=np.uint16))
    with np.errstate(over="ignore"):
        for e in (-126, -100, -20, 0, 20, 60, 100):
            s = (sig * np.float32(2.0 ** e)).astype(np.float32)
            r = (np.float32(1.0) / s).astype(np.float32)
            a = bf16_bits(x[None, :] / s[:, None])
            b = bf16_bits(x[None, :] * r[:, None])
            assert np.array_equal(a, b), e


# ---- int32 GEMM ---------------------------------------------------------------------------

def test_int8_matmul_matches_bruteforce():
    a = torch.randint(-128, 128, (37, 200), generator=gen(1), dtype=torch.int8).numpy()
    w = torch.randint(-128, 128, (29, 200), generator=gen(2), dtype=torch.int8).numpy()
    assert np.array_equal(eager_np.int8_matmul(a, w), eager_np.int8_matmul_bruteforce(a, w))
    a[0] = -128
    w[0] = -128
    assert eager_np.int8_matmul(a, w)[0, 0] == 200 * 16384


def test_int8_matmul_matches_torch_int_mm():
    a = torch.randint(-128, 128, (64, 136), generator=gen(3), dtype=torch.int8)
    w = torch.randint(-128, 128, (40, 136), generator=gen(4), dtype=torch.int8)
    assert np.array_equal(eager_np.int8_matmul(a.numpy(), w.numpy()), eager_torch.int8_matmul(a, w).numpy())


# ---- epilogue / int8_linear ------------------------------------------------------------------

def test_dequant_epilogue_closed_form():
    """Power-of-two scales make every product exact: y = acc * 2^-(a+b) (+ bias)."""
    acc = np.array([[3, -5, 100], [255, 1, -256]], np.int32)
    xs = np.array([2.0 ** -3, 2.0 ** 2], np.float32)
    ws = np.array([2.0 ** -1, 1.0, 2.0 ** -4], np.float32)
    y = eager_np.dequant_epilogue(acc, xs, ws, None, "bf16")
    exp = acc * xs[:, None] * ws[None, :]
    assert np.array_equal(y, exp.astype(np.float32))
    bias = bf16_bits(np.array([0.5, 0.25, -1.0], np.float32))
    y = eager_np.dequant_epilogue(acc, xs, ws, bias, "fp32")
    assert np.array_equal(y, (exp + np.array([0.5, 0.25, -1.0])).astype(np.float32))


def test_dequant_rounds_twice_like_eager():
    """bias is added to the already-rounded bf16 product: a case where one rounding differs."""
    acc = np.array([[257]], np.int32)  # 257 needs 9 bits: bf16(257) = 256
    y = eager_np.dequant_epilogue(acc, np.array([1.0], np.float32), np.array([1.0], np.float32),
                                  bf16_bits(np.array([0.75], np.float32)), "bf16")
    # two roundings: bf16(257) = 256, bf16(256 + 0.75) = 256; one rounding would give 258
    assert y[0, 0] == 256.0


@pytest.mark.parametrize("out", ["bf16", "fp16", "fp32"])
def test_int8_linear_numpy_matches_torch_eager(out):
    x = activations(70, 512, 5)
    w, ws = int8_weight(96, 512, 6)
    b = bf16_vec(96, 7, 0.01)
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[out]
    y1 = eager_np.int8_linear(bits(x), w.numpy(), ws.numpy(), bits(b), out)
    y2 = eager_torch.int8_linear(x, w, ws, b, out_dtype=dt)
    assert np.array_equal(y1, y2.float().numpy())


def test_ffn_chain_numpy_matches_torch_eager():
    x = activations(40, 128, 9)
    w1, s1 = int8_weight(256, 128, 10)
    w2, s2 = int8_weight(64, 256, 11)
    b1, b2 = bf16_vec(256, 12, 0.01), bf16_vec(64, 13, 0.01)
    out, _ = eager_np.ffn_gelu_int8(bits(x), w1.numpy(), s1.numpy(), bits(b1), w2.numpy(), s2.numpy(), bits(b2))
    ref = eager_torch.ffn_gelu_int8(x, w1, s1, b1, w2, s2, b2)
    assert np.array_equal(out, ref.float().numpy())


# ---- GELU ----------------------------------------------------------------------------------

def test_gelu_oracle_matches_golden_table():
    golden = np.load(GOLDEN / "gelu_tanh_bf16.npy")
    assert golden.shape == (65536,) and golden.dtype == np.uint16
    assert np.array_equal(eager_np.gelu_tanh_table(), golden)


def test_gelu_golden_is_close_to_the_mathematical_function():
    """torch's values are within 1 bf16 ulp of the float64 tanh-GELU plus the fp32 error of
    ``1 + tanh(u)``: torch evaluates 0.5 x (1 + tanh(u)) in fp32, whose cancellation for
    x < -3 costs up to ~0.5|x| 2^-22 absolute (several bf16 ulps of the tiny result)."""
    golden = np.load(GOLDEN / "gelu_tanh_bf16.npy")
    with np.errstate(invalid="ignore"):
        x = bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16)).astype(np.float64)
    fin = np.isfinite(x)
    with np.errstate(all="ignore"):
        g = 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))
    y = bf16_to_f32(golden).astype(np.float64)
    ulp = bf16_ulp(np.abs(g).astype(np.float32)).astype(np.float64)
    bound = ulp + 0.5 * np.abs(x) * 2.0 ** -22
    assert np.all(np.abs(y[fin] - g[fin]) <= bound[fin])
    # and exact to 1 ulp away from the cancelling tail
    calm = fin & (x > -3.0)
    assert np.all(np.abs(y[calm] - g[calm]) <= ulp[calm] + 1e-38)


def test_device_gelu_table_matches_golden():
    """The table compiled into the kernels, plus its closed-form rules, reproduce the fixture."""
    inc = (pathlib.Path(__file__).parents[1] / "x-minimaxh3_amd" / "csrc" / "gelu_tanh_bf16_table.inc").read_text()
    defs = dict(line.split()[1:3] for line in inc.splitlines() if line.startswith("#define"))
    e_lo, e_hi = int(defs["MXQ_GELU_E_LO"]), int(defs["MXQ_GELU_E_HI"])
    nan = int(defs["MXQ_GELU_NAN"].rstrip("u"), 16)
    body = inc[inc.index("{") + 1:inc.rindex("}")]
    table = np.array([int(v, 16) for v in body.replace("\n", "").split(",") if v.strip()], np.uint32)
    golden = np.load(GOLDEN / "gelu_tanh_bf16.npy").astype(np.uint32)
    b = np.arange(65536, dtype=np.uint32)
    e = (b >> 7) & 0xFF
    sign, mag = b & 0x8000, b & 0x7FFF
    v = mag & 0xFF
    half = sign | np.where(e >= 2, mag - 0x80, (v >> 1) + ((v & 1) & ((v >> 1) & 1)))
    ei = np.clip(e.astype(np.int64) - e_lo, 0, e_hi - e_lo - 1)
    looked = table[((b >> 15) * (e_hi - e_lo) + ei) * 128 + (b & 0x7F)]
    big = np.where(sign != 0, 0x8000, b)
    special = np.where(b == 0x7F80, 0x7F80, nan)
    dev = np.where(e < e_lo, half, np.where(e < e_hi, looked, np.where(e < 255, big, special)))
    assert np.array_equal(dev, golden)


# ---- adaLN -----------------------------------------------------------------------------------

def test_adaln_numpy_matches_torch_eager():
    x = activations(20, 1024, 3)
    sc, sh = bf16_vec(1024, 4, 0.1), bf16_vec(1024, 5, 0.1)
    y1 = eager_np.adaln(bits(x), bits(sc), bits(sh))
    y2 = eager_torch.adaln(x, sc, sh)
    assert np.array_equal(y1, bits(y2))


def test_adaln_layernorm_within_float64_bound():
    """torch's normalised bf16 values are within 1 bf16 ulp of the float64 LayerNorm."""
    x = activations(16, 2048, 8)
    n = torch.nn.functional.layer_norm(x, (2048,), eps=1e-6)
    ref = eager_np.layer_norm_f64(bits(x))
    nv = bf16_to_f32(bits(n)).astype(np.float64)
    assert np.all(np.abs(nv - ref) <= bf16_ulp(np.abs(ref).astype(np.float32)))


# ---- W4 formats -------------------------------------------------------------------------------

def test_e4m3_decode_matches_torch():
    golden = np.load(GOLDEN / "e4m3fn_to_f32.npy")
    mine = e4m3fn_to_f32(np.arange(256, dtype=np.uint8))
    assert np.array_equal(np.isnan(mine), np.isnan(golden))
    fin = ~np.isnan(golden)
    assert np.array_equal(mine[fin], golden[fin])


def test_pack_unpack_roundtrip_and_nibble_order():
    codes = torch.randint(0, 16, (8, 64), generator=gen(1)).numpy()
    p = eager_np.pack_int4(codes)
    assert np.array_equal(eager_np.unpack_int4(p), codes)
    # even k in the low nibble
    p1 = eager_np.pack_int4(np.array([[3, 12]]))
    assert p1.view(np.uint8)[0, 0] == 0xC3


def test_prepared_w4a8_layout():
    """The load layout of the group-128 GEMM: a known word, the round trip, and the device's
    unpack rule ((w << 4) & 0xF0F0F0F0, w & 0xF0F0F0F0 -> 16 (c - 8) in natural k order)."""
    p = eager_np.pack_int4(np.arange(8).reshape(1, 8))
    assert p.view(np.uint8).tolist() == [[0x10, 0x32, 0x54, 0x76]]
    q = eager_np.prepare_w4a8_grouped(p)
    assert q.view(np.uint8).tolist() == [[0xC8, 0xD9, 0xEA, 0xFB]]
    codes = np.random.default_rng(5).integers(0, 16, size=(7, 64))
    q = eager_np.prepare_w4a8_grouped(eager_np.pack_int4(codes))
    assert np.array_equal(eager_np.unprepare_w4a8_grouped(q), codes)

    def device_unpack(prepared):
        w = np.ascontiguousarray(prepared).view(np.uint32)  # little-endian words
        lo = ((w << 4) & 0xF0F0F0F0).astype(np.uint32)
        hi = (w & 0xF0F0F0F0).astype(np.uint32)
        b = np.stack([lo, hi], axis=-1).view(np.int8)      # per word: 4 bytes of lo, then 4 of hi
        return b.reshape(prepared.shape[0], -1).astype(np.int32)

    assert np.array_equal(device_unpack(q), 16 * (codes - 8))
    # a planted mistake (nibble halves swapped) fails the unpack rule
    bad = q.view(np.uint8)
    bad = (((bad & 0xF) << 4) | (bad >> 4)).astype(np.uint8).view(np.int8)
    assert not np.array_equal(device_unpack(bad), 16 * (codes - 8))


def test_w4a8_correction_lhs_matches_torch_composition():
    """The correction operand equals the reference's torch expression on the CPU
    (CK/backends/cuda/__init__.py:2295-2296), and a known row."""
    import torch

    rng = np.random.default_rng(9)
    xq = rng.integers(-128, 128, size=(5, 64)).astype(np.int8)
    xs = (rng.random(5) * 0.01).astype(np.float32)
    for g, dt, tdt in [(16, "bf16", torch.bfloat16), (4, "fp16", torch.float16), (32, "fp32", torch.float32)]:
        t = torch.from_numpy(xq).view(5, 64 // g, g).sum(-1, dtype=torch.int32).to(tdt)
        t = (t * torch.from_numpy(xs).reshape(-1, 1).to(tdt)).float().numpy()
        assert np.array_equal(eager_np.w4a8_correction_lhs(xq, xs, g, dt), t)
    row = np.array([[127] * 16 + [-128] * 16], dtype=np.int8)
    got = eager_np.w4a8_correction_lhs(row, np.array([0.5], dtype=np.float32), 16, "bf16")
    assert got.tolist() == [[1016.0, -1024.0]]  # 2032 -> bf16 2032 (exact), times 0.5


def test_decode_closed_forms():
    n, k = 4, 64
    codes = (np.arange(n * k) % 16).reshape(n, k)
    p = eager_np.pack_int4(codes)
    w = eager_np.dequant_int4_grouped_to_int8(p, np.ones((n, k // 16), np.float32), None, 16)
    assert np.array_equal(w, codes - 8)
    w = eager_np.dequant_int4_grouped_to_int8(p, np.full((n, k // 16), 8.0, np.float32), None, 16)
    assert np.array_equal(w, np.clip((codes - 8) * 8, -127, 127))
    cb = np.linspace(-7.5, 7.5, 16).astype(np.float32)
    w = eager_np.dequant_int4_grouped_to_int8(p, np.full((n, k // 4), 2.0, np.float32), cb, 4)
    assert np.array_equal(w, np.rint(cb[codes] * 2.0).astype(np.int8))  # half-integers * 2: exact


def test_decode_numpy_matches_torch_eager():
    qd = packed_int4(32, 256, 5)
    s = torch.rand(32, 256 // 16, generator=gen(6)) * 20
    cb = torch.linspace(-7.5, 7.5, 16)
    for c in (None, cb):
        a = eager_np.dequant_int4_grouped_to_int8(qd.numpy(), s.numpy(), None if c is None else c.numpy(), 16)
        b = eager_torch.dequant_int4_grouped_to_int8(qd, s, c, 16)
        assert np.array_equal(a, b.numpy())


def test_group_partials_bruteforce():
    a = torch.randint(-128, 128, (5, 256), generator=gen(1), dtype=torch.int8).numpy()
    qd = packed_int4(7, 256, 2).numpy()
    p = eager_np.w4a8_group_partials(a, qd, 128)
    w = eager_np.unpack_int4(qd) - 8
    for g in range(2):
        sl = slice(128 * g, 128 * (g + 1))
        assert np.array_equal(p[g], a[:, sl].astype(np.int64) @ w[:, sl].astype(np.int64).T)


def test_grouped_linear_within_float64_bound():
    a = torch.randint(-128, 128, (20, 1024), generator=gen(3), dtype=torch.int8).numpy()
    xs = (np.random.default_rng(0).random(20) * 0.05).astype(np.float32)
    qd = packed_int4(30, 1024, 4).numpy()
    gs = (torch.randn(8, 30, generator=gen(5)).abs() * 0.01).to(torch.float16).numpy()
    y = eager_np.w4a8_grouped_linear(a, xs, qd, gs, 128, out_dtype="fp32").astype(np.float64)
    exact, mag = eager_np.w4a8_grouped_linear_f64(a, xs, qd, gs, 128)
    assert np.all(np.abs(y - exact) <= 10 * 2.0 ** -24 * mag + 2.0 ** -24 * np.abs(exact))
    yt = eager_torch.w4a8_grouped_linear(torch.from_numpy(a), torch.from_numpy(xs), torch.from_numpy(qd),
                                         torch.from_numpy(gs), 128, torch.float32).double().numpy()
    assert np.all(np.abs(yt - exact) <= 10 * 2.0 ** -24 * mag + 2.0 ** -24 * np.abs(exact))


def test_bits_helpers_roundtrip():
    x = torch.randn(100).to(torch.bfloat16)
    assert torch.equal(from_bits(bits(x)), x)
    assert np.array_equal(bf16_bits(bf16_to_f32(bits(x))), bits(x))
