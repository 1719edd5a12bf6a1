"""Offline W4A8 weight preparation (the reference's ``quantize_w4a8_int8_weight``) and its inverse,
restated in numpy. Test infrastructure only (see the package docstring).

Reference (CK = backends/turbo/vendor/comfy_kitchen, eager backend w4a8_int8.py):
  * validate_w4a8_weight_shape (99-119), quantize_w4a8_int8_weight (315-341) and its chunked
    driver _quantize_w4a8_chunked (243-312), _decide_codebook (221-240);
  * _quantize_rotated_w4a8_int8_weight (122-209): the three storage modes
      - symmetric + codebook (the default): a 16-level Lloyd-Max codebook, group scale from the
        group absmax, codes by nearest level, three least-squares refinements of the group scale,
        then s_channel = max |codebook[code] * s_group| / 127, s_rel = s_group / s_channel
        (float8_e4m3fn or fp32), and the final codes by the nearest decoded int8 level
        round(codebook * s_rel) to w / s_channel;
      - symmetric uniform: s_group = absmax / 7, code = clamp(round(w / s_group), -8, 7) + 8;
      - asymmetric: s_group = (max - min) / 15, code = clamp(round((w - min) / s_group), 0, 15),
        correction = 8 s_group + min in the weight's dtype ([K/G, N]);
    packed two codes per byte, even k in the low nibble (200-202);
  * _codebook_for / _assign_codes / _assign_grid / _fit_codebook (24-97) and the fixed table
    _FIXED_LUT (13-16);
  * dequantize_w4a8_int8_weight (404-437): decode to the int8 grid, * s_channel (+ correction),
    rotate back.

Arithmetic: every float32 operation is one IEEE operation with round-to-nearest-even, as torch
performs it on the CPU. The 16-term group sums of the refinement follow torch's CPU reduction
order for a last dimension of at most 32 float32 values (eight interleaved partial sums, then
added in order; fewer than eight terms: in order), which tests/test_oracle_w4a8_quant.py checks
against torch. The ConvRot rotation is the exact product rounded once to the weight's dtype (as
for activations, oracle.convrot). The codebook choice (kurtosis of a sampled set, k-means fit)
runs torch's own CPU routines, the functions the reference calls.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits, bf16_to_f32, e4m3fn_to_f32
from .convrot import fht_f64, log4, round_f64_to_bf16
from .eager_np import dequant_int4_grouped_to_int8, pack_int4

F32 = np.float32

# Lloyd-Max levels for a group-normalised Gaussian (CK/backends/eager/w4a8_int8.py:13-16): the
# table is part of the storage format (codes index it), so its values are the reference's.
FIXED_LUT = np.array([
    -0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
    0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671,
], dtype=F32)
GATE_KURTOSIS = -0.1          # w4a8_int8.py:19
KURTOSIS_SAMPLE = 1 << 19     # w4a8_int8.py:20
QUANT_ROW_ELEM_BUDGET = 1 << 22   # w4a8_int8.py:215
CODEBOOK_SAMPLE_ELEMS = 1 << 22   # w4a8_int8.py:218
_FLOOR = F32(1e-8)


def validate_shape(n_k: tuple[int, int], group_size: int, convrot_groupsize: int) -> None:
    """CK/backends/eager/w4a8_int8.py:99-119 (same condition and message)."""
    k = n_k[1]
    if (k % 16 != 0 or k % group_size != 0 or k % convrot_groupsize != 0 or group_size < 4
            or (16 % group_size != 0 and group_size % 16 != 0)):
        raise ValueError(
            f"K={k} must be divisible by 16, group_size={group_size}, and "
            f"convrot_groupsize={convrot_groupsize}; group_size must be >=4 "
            f"and divide 16 or be a multiple of 16"
        )


def sum_last_f32(a: np.ndarray) -> np.ndarray:
    """float32 sum over the last axis in torch's CPU order for up to 32 terms: eight partial
    sums s_j = a_j + a_{j+8} + ... (each in order), then s_0 + s_1 + ... + s_7 in order; fewer
    than eight terms are added in order."""
    a = np.asarray(a, dtype=F32)
    n = a.shape[-1]
    if n < 8:
        acc = a[..., 0].copy()
        for i in range(1, n):
            acc = (acc + a[..., i]).astype(F32)
        return acc
    parts = [a[..., j].copy() for j in range(8)]
    for i in range(8, n):
        parts[i % 8] = (parts[i % 8] + a[..., i]).astype(F32)
    acc = parts[0]
    for j in range(1, 8):
        acc = (acc + parts[j]).astype(F32)
    return acc


_E4M3_POS = None


def f32_to_e4m3fn_bits(x) -> np.ndarray:
    """float32 -> float8_e4m3fn bits as torch converts (round to nearest, ties to the even code;
    the format has no infinity, and magnitudes that round beyond 448 become NaN 0x7F | sign)."""
    global _E4M3_POS
    if _E4M3_POS is None:
        codes = np.arange(0x7F, dtype=np.uint8)               # 0 .. 0x7E: +0 .. 448
        _E4M3_POS = np.append(e4m3fn_to_f32(codes).astype(np.float64), 480.0)  # 0x7F: next step, NaN
    x = np.asarray(x, dtype=F32)
    ax = np.abs(x.astype(np.float64))
    hi = np.clip(np.searchsorted(_E4M3_POS, ax, side="left"), 1, 0x7F)
    lo = hi - 1
    dlo, dhi = ax - _E4M3_POS[lo], _E4M3_POS[hi] - ax
    pick = np.where(dhi < dlo, hi, np.where(dlo < dhi, lo, np.where(hi % 2 == 0, hi, lo)))
    pick = np.where(ax >= _E4M3_POS[-1], 0x7F, pick)
    out = pick.astype(np.uint8) | np.where(np.signbit(x), np.uint8(0x80), np.uint8(0))
    return np.where(np.isnan(x), np.uint8(0x7F), out).astype(np.uint8)


def rotate_weight(w: np.ndarray, dtype: str, convrot_groupsize: int) -> np.ndarray:
    """ConvRot rotation of the weight rows (W_grouped @ H^T; H is symmetric), the exact product
    rounded once to ``dtype`` ('bf16' or 'fp32'); float32 values."""
    log4(convrot_groupsize)
    y = fht_f64(np.asarray(w, dtype=np.float64), convrot_groupsize)
    if dtype == "bf16":
        return bf16_to_f32(round_f64_to_bf16(y))
    return y.astype(F32)


def assign_nearest(values: np.ndarray, levels: np.ndarray) -> np.ndarray:
    """Index of the nearest level, the first one on ties (|v - level| in float32, strict <;
    CK/backends/eager/w4a8_int8.py:35-45, 48-63). ``levels`` broadcasts against
    ``values[..., None]``."""
    values = np.asarray(values, dtype=F32)
    lv = np.broadcast_to(np.asarray(levels, dtype=F32), values.shape + (16,))
    best = np.abs(values - lv[..., 0]).astype(F32)
    idx = np.zeros(values.shape, dtype=np.int32)
    for i in range(1, 16):
        d = np.abs(values - lv[..., i]).astype(F32)
        closer = d < best
        best = np.where(closer, d, best)
        idx = np.where(closer, i, idx)
    return idx


def codebook_for(normalized: np.ndarray) -> np.ndarray:
    """The fixed table unless the group-normalised weights are heavy-tailed, then a fit
    (CK/backends/eager/w4a8_int8.py:24-32): torch's CPU sampling, moments and fit."""
    import torch

    x = torch.from_numpy(np.ascontiguousarray(normalized, dtype=F32)).flatten()
    if x.numel() > KURTOSIS_SAMPLE:
        gen = torch.Generator().manual_seed(0)
        x = x[torch.randint(0, x.numel(), (KURTOSIS_SAMPLE,), generator=gen)]
    excess = ((x - x.mean()) / (x.std() + 1e-9)).pow(4).mean() - 3.0
    if excess.item() <= GATE_KURTOSIS:
        return FIXED_LUT.copy()
    return fit_codebook(normalized)


def fit_codebook(normalized: np.ndarray, levels: int = 16, iterations: int = 25,
                 sample_size: int = 300000) -> np.ndarray:
    """Lloyd-Max fit on a sample (CK/backends/eager/w4a8_int8.py:66-97), torch CPU routines."""
    import torch

    samples = torch.from_numpy(np.ascontiguousarray(normalized, dtype=F32)).flatten()
    if samples.numel() > sample_size:
        gen = torch.Generator().manual_seed(0)
        samples = samples[torch.randint(0, samples.numel(), (sample_size,), generator=gen)]
    cb = torch.quantile(samples, torch.linspace(0, 1, levels))
    for _ in range(iterations):
        assign = (samples.unsqueeze(-1) - cb).abs().argmin(-1)
        upd = cb.clone()
        for i in range(levels):
            sel = assign == i
            if sel.any():
                upd[i] = samples[sel].mean()
        cb = upd
    return cb.numpy().astype(F32)


def decide_codebook(w: np.ndarray, dtype: str, group_size: int, convrot_groupsize: int) -> np.ndarray:
    """One table for the whole tensor from evenly strided rows (w4a8_int8.py:221-240)."""
    import torch

    n, k = w.shape
    max_rows = max(1, CODEBOOK_SAMPLE_ELEMS // max(k, 1))
    if n > max_rows:
        idx = torch.linspace(0, n - 1, max_rows).long().numpy()
        sample = w[idx]
    else:
        sample = w
    rot = rotate_weight(sample, dtype, convrot_groupsize)
    g = rot.reshape(sample.shape[0], k // group_size, group_size)
    amax = np.maximum(np.abs(g).max(axis=-1, keepdims=True), _FLOOR)
    return codebook_for((g / amax).astype(F32))


def quantize_rotated(w_rot: np.ndarray, group_size: int = 16, symmetric: bool = True,
                     scale_dtype: str = "e4m3", codebook: np.ndarray | None = None,
                     orig_dtype: str = "bf16"):
    """Storage of an already rotated float32 weight [N, K] (w4a8_int8.py:122-209).

    ``codebook``: the 16-level table for the symmetric codebook mode (None: uniform symmetric
    codes, or the asymmetric mode when ``symmetric`` is False). Returns ``(packed int8 [N, K/2],
    s_rel [N, K/G] (e4m3 bits uint8 or float32), s_channel float32 [N], correction [K/G, N] as
    float32 values of ``orig_dtype`` or None, codebook or None)``."""
    w = np.asarray(w_rot, dtype=F32)
    n, k = w.shape
    groups = k // group_size
    gw = w.reshape(n, groups, group_size)
    correction = None
    if symmetric and codebook is not None:
        cb = np.asarray(codebook, dtype=F32)
        gs = np.maximum(np.abs(gw).max(axis=-1, keepdims=True), _FLOOR)
        codes = assign_nearest((gw / gs).astype(F32), cb)
        for _ in range(3):
            qc = cb[codes]
            num = sum_last_f32((gw * qc).astype(F32))[..., None]
            den = np.maximum(sum_last_f32((qc * qc).astype(F32)), _FLOOR)[..., None]
            gs = np.maximum((num / den).astype(F32), _FLOOR)
            codes = assign_nearest((gw / gs).astype(F32), cb)
        shifted = (cb[codes] * gs).astype(F32)
    elif symmetric:
        gs = np.maximum((np.abs(gw).max(axis=-1, keepdims=True) / F32(7.0)).astype(F32), _FLOOR)
        signed = np.clip(np.rint((gw / gs).astype(F32)), -8, 7).astype(np.int32)
        codes = signed + 8
        shifted = (signed.astype(F32) * gs).astype(F32)
    else:
        mn = gw.min(axis=-1, keepdims=True)
        gs = np.maximum(((gw.max(axis=-1, keepdims=True) - mn) / F32(15.0)).astype(F32), _FLOOR)
        codes = np.clip(np.rint(((gw - mn) / gs).astype(F32)), 0, 15).astype(np.int32)
        shifted = ((codes - 8).astype(F32) * gs).astype(F32)
        corr = (F32(8.0) * gs + mn).astype(F32)[..., 0].T
        correction = bf16_to_f32(bf16_bits(corr)) if orig_dtype == "bf16" else corr
    s_channel = np.maximum((np.abs(shifted).max(axis=(1, 2)) / F32(127.0)).astype(F32), _FLOOR)
    s_rel = (gs[..., 0] / s_channel[:, None]).astype(F32)
    s_rel_val = s_rel
    if scale_dtype == "e4m3":
        s_rel = f32_to_e4m3fn_bits(s_rel)
        s_rel_val = e4m3fn_to_f32(s_rel)
    if symmetric and codebook is not None:
        levels = np.clip(np.rint((cb[None, None, :] * s_rel_val[..., None]).astype(F32)), -127, 127).astype(F32)
        target = (gw / s_channel[:, None, None]).astype(F32)
        codes = assign_nearest(target, levels[:, :, None, :])
    packed = pack_int4(codes.reshape(n, k))
    return packed, s_rel, s_channel, correction, (None if codebook is None or not symmetric else np.asarray(codebook, F32))


def quantize_w4a8_int8_weight(w: np.ndarray, dtype: str = "bf16", group_size: int = 16,
                              convrot_groupsize: int = 256, symmetric: bool = True,
                              scale_dtype: str = "e4m3", codebook: bool = True,
                              codebook_tensor: np.ndarray | None = None):
    """Rotate and store a floating weight [N, K] (values exactly representable in ``dtype``),
    w4a8_int8.py:315-341 with the chunked driver 243-312 (rows are independent once the table
    is chosen, so the chunking does not change the result)."""
    w = np.asarray(w, dtype=F32)
    if w.ndim != 2:
        raise ValueError(f"W4A8 weight must be 2D, got shape {tuple(w.shape)}")
    validate_shape(w.shape, group_size, convrot_groupsize)
    table = None
    if symmetric and codebook:
        table = (np.asarray(codebook_tensor, dtype=F32) if codebook_tensor is not None
                 else decide_codebook(w, dtype, group_size, convrot_groupsize))
    rot = rotate_weight(w, dtype, convrot_groupsize)
    return quantize_rotated(rot, group_size, symmetric, scale_dtype, table, dtype)


def dequantize_w4a8_int8_weight(packed, s_rel, s_channel, codebook=None, correction=None,
                                group_size: int = 16, convrot_groupsize: int = 256,
                                s_rel_is_e4m3: bool = True, out_dtype: str = "bf16") -> np.ndarray:
    """w4a8_int8.py:404-437: the int8 grid (344-363), * s_channel (+ correction^T) in float32,
    rounded to ``out_dtype``, then rotated back (the rotation is its own inverse) and rounded."""
    w8 = dequant_int4_grouped_to_int8(packed, s_rel, codebook, group_size, s_rel_is_e4m3)
    n, k = w8.shape
    v = w8.astype(F32).reshape(n, k // group_size, group_size) * np.asarray(s_channel, F32).reshape(n, 1, 1)
    if correction is not None:
        v = (v + np.asarray(correction, F32).T[:, :, None]).astype(F32)
    v = v.reshape(n, k).astype(F32)
    if out_dtype == "bf16":
        v = bf16_to_f32(bf16_bits(v))
    return rotate_weight(v, out_dtype, convrot_groupsize)
