"""The oracle's offline W4A8 weight preparation (oracle/w4a8_quant.py) pinned on the CPU:

* the reduction order it uses for group sums and its float8_e4m3fn rounding against torch's own
  CPU routines (what the reference's torch code calls);
* bit-exact agreement with a second restatement written as the reference's torch op sequence
  (oracle/eager_torch.py:quantize_rotated_w4a8) over all modes, scale dtypes and group sizes;
* closed forms: constant groups give known codes and scales in every mode, a group of known
  values gives known codes, s_rel * s_channel equals the group scale (absmax / 7 in the uniform
  mode), decoding stays within the quantization bound of the grid, and a planted mistake in the
  refinement order or the tie rule is caught.
"""

import numpy as np
import pytest
import torch

from _util import gen
from oracle import eager_np, eager_torch
from oracle import w4a8_quant as wq
from oracle.bf16 import bf16_bits, bf16_to_f32, e4m3fn_to_f32

F32 = np.float32


@pytest.mark.parametrize("n", [4, 8, 16, 24, 32])
def test_group_sum_order_is_torchs(n):
    x = torch.randn(3000, 50, n, generator=gen(n)) * torch.rand(3000, 50, 1, generator=gen(n + 1)) * 10
    assert np.array_equal(wq.sum_last_f32(x.numpy()), x.sum(-1).numpy())


def test_group_sum_order_catches_a_sequential_sum():
    x = torch.randn(3000, 50, 16, generator=gen(3)) * 7
    seq = x.numpy()[..., 0].copy()
    for i in range(1, 16):
        seq = seq + x.numpy()[..., i]
    assert not np.array_equal(seq, x.sum(-1).numpy())


def test_e4m3_rounding_is_torchs():
    vals = [0.0, -0.0, 448.0, 456.0, 464.0, 464.5, 470.0, 480.0, 1e9, 2.0 ** -6, 2.0 ** -9, 2.0 ** -10,
            1.5 * 2.0 ** -10, 3 * 2.0 ** -10, 0.0019, 0.001, 1.0625, 1.0626, 1.1875, 129.5, 127.9]
    bf = bf16_to_f32(np.arange(0, 0x7F80, dtype=np.uint16))  # every finite positive bf16
    rnd = (torch.rand(200000, generator=gen(9)).numpy() * 500.0).astype(F32)
    x = np.concatenate([np.array(vals, F32), bf, -bf, rnd, -rnd]).astype(F32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = wq.f32_to_e4m3fn_bits(x)
    nan_w = (want & 0x7F) == 0x7F
    assert np.array_equal(nan_w, (got & 0x7F) == 0x7F)
    assert np.array_equal(got[~nan_w], want[~nan_w])


def _rotated(n, k, seed, scale=0.02):
    w = (torch.randn(n, k, generator=gen(seed)) * scale).to(torch.bfloat16)
    return wq.rotate_weight(w.float().numpy(), "bf16", 256)


@pytest.mark.parametrize("mode", ["codebook", "symmetric", "asymmetric"])
@pytest.mark.parametrize("sdt", [torch.float8_e4m3fn, torch.float32])
@pytest.mark.parametrize("g", [4, 8, 16, 32])
def test_oracle_equals_the_torch_op_sequence(mode, sdt, g):
    rot = _rotated(64, 512, 100 + g)
    cb = wq.FIXED_LUT if mode == "codebook" else None
    sym = mode != "asymmetric"
    p, s, c, corr, _ = wq.quantize_rotated(rot, g, sym, "e4m3" if sdt != torch.float32 else "f32", cb, "bf16")
    rt = torch.from_numpy(rot).to(torch.bfloat16)
    pt, st, ct, corrt = eager_torch.quantize_rotated_w4a8(rt, g, sym, sdt, None if cb is None else torch.from_numpy(cb))
    assert np.array_equal(p, pt.numpy())
    assert np.array_equal(s, st.view(torch.uint8).numpy() if sdt != torch.float32 else st.numpy())
    assert np.array_equal(c, ct.numpy())
    if mode == "asymmetric":
        assert np.array_equal(bf16_bits(corr), corrt.view(torch.int16).numpy().view(np.uint16))


def test_oracle_equals_torch_with_a_fitted_codebook():
    rot = _rotated(64, 512, 7)
    g = rot.reshape(64, 512 // 16, 16)
    normalized = g / np.maximum(np.abs(g).max(axis=-1, keepdims=True), F32(1e-8))
    cb = wq.fit_codebook(normalized.astype(F32))
    assert cb.shape == (16,) and np.all(np.diff(cb) > 0)
    p, s, c, _, _ = wq.quantize_rotated(rot, 16, True, "e4m3", cb)
    pt, st, ct, _ = eager_torch.quantize_rotated_w4a8(torch.from_numpy(rot).to(torch.bfloat16), 16, True,
                                                      torch.float8_e4m3fn, torch.from_numpy(cb))
    assert np.array_equal(p, pt.numpy()) and np.array_equal(s, st.view(torch.uint8).numpy())
    assert np.array_equal(c, ct.numpy())


def test_constant_groups_known_answers():
    """Row 0: one group of 2.0 (the row's largest) and one of 0.5; known codes and scales."""
    w = np.zeros((1, 32), F32)
    w[0, :16], w[0, 16:] = 2.0, 0.5
    # uniform symmetric: s = amax / 7, every code 7 + 8 = 15, s_channel = 7 s / 127
    p, s, c, _, _ = wq.quantize_rotated(w, 16, True, "f32", None)
    assert np.all(eager_np.unpack_int4(p) == 15)
    assert c[0] == F32(F32(F32(2.0) / F32(7.0)) * F32(7.0)) / F32(127.0)
    assert s[0, 0] == F32(F32(2.0) / F32(7.0)) / c[0] and s[0, 1] == F32(F32(0.5) / F32(7.0)) / c[0]
    # codebook: every code the top level 0.980671, the refined scale w / 0.980671, decoded levels
    # rne(0.980671 * e4m3(127 / 0.980671)) = rne(0.980671 * 128) = 126 -> code 15 again
    p, s, c, _, _ = wq.quantize_rotated(w, 16, True, "e4m3", wq.FIXED_LUT)
    assert np.all(eager_np.unpack_int4(p)[0, :16] == 15)
    assert e4m3fn_to_f32(s[0, 0]) == 128.0
    assert abs(float(c[0]) - 2.0 / 127) < 1e-8
    # asymmetric: max == min gives s = 1e-8, codes 0, correction 8e-8 + w
    p, s, c, corr, _ = wq.quantize_rotated(w, 16, False, "f32", None, "fp32")
    assert np.all(eager_np.unpack_int4(p) == 0)
    assert corr[0, 0] == F32(F32(8.0) * F32(1e-8)) + F32(2.0) and corr[1, 0] == F32(F32(8.0) * F32(1e-8)) + F32(0.5)


def test_known_group_codes():
    """Uniform mode on k / 8, k = -8 .. 7: s = fp32(1 / 7) = 0.14285715 (rounded up), so the
    quotients 7 k / 8 come out just below their exact values in magnitude and the would-be ties
    +-3.5 round to +-3: codes 1 2 3 4 5 5 6 7 8 9 10 11 11 12 13 14."""
    w = (np.arange(-8, 8, dtype=F32) / F32(8.0)).reshape(1, 16)
    p, s, c, _, _ = wq.quantize_rotated(w, 16, True, "f32", None)
    assert list(eager_np.unpack_int4(p)[0]) == [1, 2, 3, 4, 5, 5, 6, 7, 8, 9, 10, 11, 11, 12, 13, 14]
    assert c[0] == F32(F32(F32(1.0) / F32(7.0)) * F32(7.0)) / F32(127.0)


@pytest.mark.parametrize("sdt", ["f32", "e4m3"])
def test_relative_times_channel_scale_is_the_group_scale(sdt):
    rot = _rotated(32, 256, 11)
    p, s, c, _, _ = wq.quantize_rotated(rot, 16, True, sdt, None)
    gs = np.maximum(np.abs(rot.reshape(32, 16, 16)).max(-1) / F32(7.0), F32(1e-8)).astype(F32)
    sv = e4m3fn_to_f32(s) if sdt == "e4m3" else s
    rel = np.abs(sv * c[:, None] - gs) / gs
    assert rel.max() <= (2.0 ** -4 if sdt == "e4m3" else 2.0 ** -22)


def test_decode_stays_within_the_grid_bound():
    """Uniform mode, fp32 s_rel: |w / s_channel - w8| <= s_rel / 2 + 1/2 (the code's rounding in
    units of the group scale, then the int8 grid's)."""
    rot = _rotated(32, 256, 12)
    p, s, c, _, _ = wq.quantize_rotated(rot, 16, True, "f32", None)
    w8 = eager_np.dequant_int4_grouped_to_int8(p, s, None, 16).astype(np.float64)
    err = np.abs(rot.astype(np.float64) / c[:, None] - w8).reshape(32, 16, 16)
    assert np.all(err <= s[:, :, None] / 2 + 0.5 + 1e-6)


def test_dequantize_recovers_the_weight():
    w = (torch.randn(64, 512, generator=gen(13)) * 0.02).to(torch.bfloat16).float().numpy()
    for sym, cb in ((True, True), (True, False), (False, False)):
        p, s, c, corr, table = wq.quantize_w4a8_int8_weight(w, "bf16", 16, 256, sym, "e4m3", cb)
        back = wq.dequantize_w4a8_int8_weight(p, s, c, table, corr, 16, 256, True, "bf16")
        rel = np.linalg.norm(back - w) / np.linalg.norm(w)
        assert rel < 0.2, (sym, cb, rel)


def test_gaussian_weights_take_the_fixed_table():
    w = (torch.randn(128, 1024, generator=gen(14)) * 0.02).to(torch.bfloat16).float().numpy()
    assert np.array_equal(wq.decide_codebook(w, "bf16", 16, 256), wq.FIXED_LUT)


def test_planted_mistakes_are_caught(monkeypatch):
    # every second group a thousand times smaller: its decoded levels rne(cb * s_rel) collide,
    # so the nearest-level search meets exact ties there
    rot = _rotated(64, 512, 15).reshape(64, 32, 16)
    rot[:, 1::2] *= F32(0.001)
    rot = rot.reshape(64, 512).astype(F32)
    p, _, _, _, _ = wq.quantize_rotated(rot, 16, True, "e4m3", wq.FIXED_LUT)
    _, s, c, _, _ = wq.quantize_rotated(rot, 16, True, "f32", wq.FIXED_LUT)

    def last_on_ties(values, levels):  # the last nearest level instead of the first
        lv = np.broadcast_to(np.asarray(levels, F32), np.asarray(values).shape + (16,))
        d = np.abs(np.asarray(values, F32)[..., None] - lv)
        return (15 - np.argmin(d[..., ::-1], axis=-1)).astype(np.int32)

    def sequential_sum(a):  # the group sums in plain index order
        a = np.asarray(a, F32)
        acc = a[..., 0].copy()
        for i in range(1, a.shape[-1]):
            acc = (acc + a[..., i]).astype(F32)
        return acc

    with monkeypatch.context() as m:
        m.setattr(wq, "assign_nearest", last_on_ties)
        p2, _, _, _, _ = wq.quantize_rotated(rot, 16, True, "e4m3", wq.FIXED_LUT)
    assert not np.array_equal(p2, p)
    with monkeypatch.context() as m:
        m.setattr(wq, "sum_last_f32", sequential_sum)
        _, s3, c3, _, _ = wq.quantize_rotated(rot, 16, True, "f32", wq.FIXED_LUT)
    assert not (np.array_equal(s3, s) and np.array_equal(c3, c))
