"""numpy restatement of the reference's eager W8A8 / W4A8 linear path.

Test infrastructure only (see the package docstring). Paths are relative to the
reference tree; ``CK`` stands for ``backends/turbo/vendor/comfy_kitchen``.

Conventions: bfloat16 tensors are ``uint16`` bit arrays, int8 tensors are
``int8`` arrays, scales are ``float32``. Every float32 operation below is one
IEEE-754 operation with round-to-nearest-even, exactly as torch performs it on
the CPU for the same dtypes.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits, bf16_to_f32, e4m3fn_to_f32, round_bf16, round_to

F32 = np.float32
_SCALE_FLOOR = F32(1e-30)          # CK/backends/eager/quantization.py:873 (clamp(min=1e-30))
_BF16_TINY = F32(2.0 ** -126)      # torch.finfo(torch.bfloat16).tiny, quantization.py:815-818


# ---------------------------------------------------------------------------
# a1: per-token symmetric absmax quantizer
# ---------------------------------------------------------------------------

def quantize_int8_rowwise(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row INT8 quantization of a bfloat16 tensor ``[..., K]``.

    Follows CK/backends/eager/quantization.py:857-875 with the helpers at
    815-818 (``_int8_scale_for_math``) and 821-826 (``_round_int8``):
      amax = max |x| over the row (exact in bfloat16),
      s    = max(fp32(amax) / 127, 1e-30)              (fp32 division),
      q    = clamp(rne(bf16(x / bf16(s))), -128, 127)   (bf16 division = fp32
             division rounded to bf16; ``round`` is half-to-even).
    Returns ``(q int8 [..., K], s float32 [..., 1])``.
    """
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    if x_bits.shape[-1] == 0:
        raise ValueError("quantize_int8_rowwise needs a non-empty last dimension")
    xf = bf16_to_f32(x_bits)
    amax = np.max(np.abs(xf), axis=-1, keepdims=True)
    scale = np.maximum(amax / F32(127.0), _SCALE_FLOOR).astype(F32)
    s_math = round_bf16(scale)
    s_math = np.where(s_math == 0, _BF16_TINY, s_math)
    qf = round_bf16(xf / s_math)
    with np.errstate(invalid="ignore"):
        q = np.clip(np.rint(qf), -128.0, 127.0)
    q = np.nan_to_num(q, nan=0.0).astype(np.int8)
    return q, scale


def quantize_int8_rowwise_stochastic(x_bits: np.ndarray, noise_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The same quantizer with stochastic rounding on bfloat16 (quantization.py:803-826): the
    scaled value ``bf16(x / bf16(s))`` gets the uniform draw ``noise`` (bf16, the reference's
    ``torch.rand`` in the input dtype) added in bfloat16 (``scaled.add_(rng)``: an fp32 sum rounded
    once), then ``floor``, clamp to [-128, 127]; NaN -> 0 as in the rounding path."""
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    xf = bf16_to_f32(x_bits)
    amax = np.max(np.abs(xf), axis=-1, keepdims=True)
    scale = np.maximum(amax / F32(127.0), _SCALE_FLOOR).astype(F32)
    s_math = round_bf16(scale)
    s_math = np.where(s_math == 0, _BF16_TINY, s_math)
    qf = round_bf16(xf / s_math)
    t = round_bf16((qf + bf16_to_f32(np.asarray(noise_bits, dtype=np.uint16))).astype(F32))
    with np.errstate(invalid="ignore"):
        q = np.clip(np.floor(t), -128.0, 127.0)
    q = np.nan_to_num(q, nan=0.0).astype(np.int8)
    return q, scale


def quantize_int8_rowwise_with_absmax(x_bits: np.ndarray, amax: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Same quantizer with the row absmax supplied (it must equal max |x|)."""
    xf = bf16_to_f32(np.asarray(x_bits, dtype=np.uint16))
    amax = np.asarray(amax, dtype=F32).reshape(xf.shape[:-1] + (1,))
    scale = np.maximum(amax / F32(127.0), _SCALE_FLOOR).astype(F32)
    s_math = round_bf16(scale)
    qf = round_bf16(xf / s_math)
    q = np.clip(np.rint(qf), -128.0, 127.0).astype(np.int8)
    return q, scale


# ---------------------------------------------------------------------------
# a2: exact int8 x int8 -> int32 GEMM
# ---------------------------------------------------------------------------

def int8_matmul(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """``C[m, n] = sum_k A[m, k] * W[n, k]`` in int32.

    The reference computes ``torch._int_mm(x_8, weight.T)`` after zero padding
    (CK/backends/eager/quantization.py:749-782, 1028); padding adds zero terms.
    Here the products are summed in float64: every product is an integer of
    magnitude <= 2**14 and every partial sum stays below 2**53 for K < 2**39,
    so each step is exact whatever order BLAS uses.
    """
    a = np.asarray(a, dtype=np.int8)
    w = np.asarray(w, dtype=np.int8)
    if a.shape[-1] != w.shape[-1]:
        raise ValueError(f"K mismatch: {a.shape[-1]} vs {w.shape[-1]}")
    k = a.shape[-1]
    if k * 128 * 128 >= 2 ** 31:
        raise ValueError("K too large for an int32 accumulator")
    return (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int32)


def int8_matmul_bruteforce(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """int64 brute force of :func:`int8_matmul` for small shapes."""
    a64 = np.asarray(a, dtype=np.int64)
    w64 = np.asarray(w, dtype=np.int64)
    return np.einsum("mk,nk->mn", a64, w64).astype(np.int32)


# ---------------------------------------------------------------------------
# a3: dequant epilogue and the whole int8_linear
# ---------------------------------------------------------------------------

def dequant_epilogue(acc: np.ndarray, x_scale: np.ndarray, w_scale: np.ndarray,
                     bias_bits: np.ndarray | None = None, out_dtype: str = "bf16",
                     bias_dtype: str = "bf16") -> np.ndarray:
    """``y = out(fp32(acc) * (xs[m] * ws[n]))`` then ``y = out(y + out(bias))``.

    CK/backends/eager/quantization.py:1034-1054: the chunk loop computes
    ``chunk.float() * (x_scale * weight_scale)`` (two fp32 products, the scale
    product first), converts to ``out_dtype``, and the bias is added afterwards
    in ``out_dtype`` (``bias.to(result.dtype)``). Returns float32 values that are
    exactly representable in ``out_dtype``.
    """
    acc = np.asarray(acc, dtype=np.int32)
    xs = np.asarray(x_scale, dtype=F32).reshape(-1, 1)
    ws = np.asarray(w_scale, dtype=F32).reshape(1, -1)
    scales = (xs * ws).astype(F32)
    y = round_to(acc.astype(F32) * scales, out_dtype)
    if bias_bits is not None:
        b = _as_float(bias_bits, bias_dtype)
        y = round_to(y + round_to(b.reshape(1, -1), out_dtype), out_dtype)
    return y


def _as_float(t, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_to_f32(t)
    return np.asarray(t, dtype=F32)


def int8_linear(x_bits: np.ndarray, weight: np.ndarray, weight_scale: np.ndarray,
                bias_bits: np.ndarray | None = None, out_dtype: str = "bf16",
                input_act: str | None = None) -> np.ndarray:
    """Eager ``int8_linear`` (CK/backends/eager/quantization.py:971-1056), convrot=False.

    ``input_act`` ('gelu_tanh' or None) is applied to the bfloat16 input first
    (CK/backends/_activations.py:40-53). Returns float32 values representable in
    ``out_dtype`` with shape ``[..., N]``.
    """
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    if input_act == "gelu_tanh":
        x_bits = gelu_tanh_bf16(x_bits)
    elif input_act not in (None, "none"):
        raise ValueError(f"unsupported input_act: {input_act!r}")
    if x_bits.shape[-1] != weight.shape[-1]:
        raise ValueError("Input and weight inner dimensions must match")
    ws = np.asarray(weight_scale, dtype=F32).reshape(-1)
    if ws.size not in (1, weight.shape[0]):
        raise ValueError("INT8 weight scale must be scalar or per-output-channel")
    lead = x_bits.shape[:-1]
    x2 = x_bits.reshape(-1, x_bits.shape[-1])
    q, s = quantize_int8_rowwise(x2)
    acc = int8_matmul(q, weight)
    y = dequant_epilogue(acc, s, ws, bias_bits, out_dtype)
    return y.reshape(lead + (weight.shape[0],))


# ---------------------------------------------------------------------------
# a4: tanh-GELU on bfloat16
# ---------------------------------------------------------------------------

_GELU_TABLE: np.ndarray | None = None


def gelu_tanh_table() -> np.ndarray:
    """All 65,536 bfloat16 inputs through ``torch.nn.functional.gelu(approximate='tanh')``.

    The reference applies torch's CPU GELU to the bfloat16 tensor
    (CK/backends/_activations.py:47-48); torch is the routine, so the oracle
    evaluates it once over every bfloat16 bit pattern in one vectorised call
    and looks results up. The golden fixture tests/golden/gelu_tanh_bf16.npy
    pins this table.
    """
    global _GELU_TABLE
    if _GELU_TABLE is None:
        import torch

        bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16)
        y = torch.nn.functional.gelu(bits.view(torch.bfloat16), approximate="tanh")
        _GELU_TABLE = y.view(torch.int16).numpy().view(np.uint16).copy()
    return _GELU_TABLE


def gelu_tanh_bf16(x_bits: np.ndarray) -> np.ndarray:
    return gelu_tanh_table()[np.asarray(x_bits, dtype=np.uint16)]


# ---------------------------------------------------------------------------
# gated residual after fc2
# ---------------------------------------------------------------------------

def segment_row_map(length: int, segments) -> np.ndarray:
    """Modulation row of every token from ordered (start, stop, row) segments
    (h3serve/native_engine/model/fused_mlp.py:34-55; same partition checks)."""
    out = np.empty(length, dtype=np.int32)
    previous = 0
    for start, stop, row in segments:
        if start != previous or stop <= start:
            raise ValueError("modulation segments must be an ordered partition")
        out[start:stop] = row
        previous = stop
    if previous != length:
        raise ValueError("modulation segments do not cover the packed sequence")
    return out


def gated_residual_bf16(residual_bits: np.ndarray, update_bits: np.ndarray, gate_bits: np.ndarray,
                        gate_rows: np.ndarray) -> np.ndarray:
    """``residual[m] = bf16(residual[m] + update[m] * gate[gate_rows[m]])`` on bfloat16 bits.

    h3serve/native_engine/model/layers.py:944-960: ``residual[a:b].addcmul_(update[a:b],
    gate[row].to(update.dtype))`` per segment. addcmul_ evaluates in float32; the product of
    two bfloat16 values is exact in float32, so the value is one float32 addition rounded to
    bfloat16 (the gate is already bfloat16 bits here)."""
    r = bf16_to_f32(residual_bits)
    u = bf16_to_f32(update_bits)
    g = bf16_to_f32(np.asarray(gate_bits, dtype=np.uint16)[np.asarray(gate_rows)])
    return bf16_bits((r + u * g).astype(F32))


# ---------------------------------------------------------------------------
# a6: adaLN (LayerNorm without affine, then modulation)
# ---------------------------------------------------------------------------

def adaln(x_bits: np.ndarray, scale_bits: np.ndarray, shift_bits: np.ndarray,
          eps: float = 1e-6) -> np.ndarray:
    """``bf16(bf16(bf16(LN(x)) * bf16(1 + scale)) + shift)``.

    CK/backends/eager/adaln.py:11-14 evaluates ``layer_norm(x) * (1 + scale) +
    shift`` on bfloat16 tensors: four bfloat16 roundings. The LayerNorm itself
    is torch's CPU ``layer_norm`` (the routine the reference calls). Returns
    bfloat16 bits.
    """
    import torch

    xt = torch.from_numpy(np.asarray(x_bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
    n = torch.nn.functional.layer_norm(xt, xt.shape[-1:], eps=eps)
    n32 = bf16_to_f32(n.view(torch.int16).numpy().view(np.uint16))
    t = round_bf16(F32(1.0) + bf16_to_f32(scale_bits))
    y = round_bf16(n32 * t)
    y = round_bf16(y + bf16_to_f32(shift_bits))
    return bf16_bits(y)


def layer_norm_f64(x_bits: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """float64 LayerNorm (biased variance), used to bound torch's result."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps)


# ---------------------------------------------------------------------------
# RMS adaLN (the H3 block's norm + segmented modulation)
# ---------------------------------------------------------------------------

def rms_norm_bf16(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """``F.rms_norm(x, (D,), weight=w, eps)`` on bfloat16 with torch's CPU routine, the
    function the reference's RMSNorm calls (h3serve/native_engine/model/layers.py:39-48)."""
    import torch

    xt = torch.from_numpy(np.asarray(x_bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
    wt = torch.from_numpy(np.asarray(w_bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
    n = torch.nn.functional.rms_norm(xt, xt.shape[-1:], weight=wt, eps=eps)
    return n.view(torch.int16).numpy().view(np.uint16).copy()


def rms_norm_f64(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """float64 x / sqrt(mean(x^2) + eps) * w, used to bound torch's result."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    r = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return x * r * bf16_to_f32(w_bits).astype(np.float64)


def modulate_bf16(n_bits: np.ndarray, scale_bits: np.ndarray, shift_bits: np.ndarray,
                  rows: np.ndarray) -> np.ndarray:
    """``h[a:b].mul_(1.0 + scale[row].to(bf16)).add_(shift[row].to(bf16))`` per segment
    (h3serve/native_engine/model/kernels.py:7629-7639): three bfloat16 roundings."""
    rows = np.asarray(rows)
    t = round_bf16(F32(1.0) + bf16_to_f32(np.asarray(scale_bits, dtype=np.uint16)[rows]))
    y = round_bf16(bf16_to_f32(n_bits) * t)
    return bf16_bits(round_bf16(y + bf16_to_f32(np.asarray(shift_bits, dtype=np.uint16)[rows])))


def rms_adaln(x_bits: np.ndarray, w_bits: np.ndarray, eps: float, scale_bits: np.ndarray,
              shift_bits: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """rms_adaln (kernels.py:7594-7640, eager branch): RMSNorm then the segmented modulation."""
    return modulate_bf16(rms_norm_bf16(x_bits, w_bits, eps), scale_bits, shift_bits, rows)


# ---------------------------------------------------------------------------
# a7 / a9: int4 packing and grouped decode to the int8 grid
# ---------------------------------------------------------------------------

def pack_int4(codes: np.ndarray) -> np.ndarray:
    """Pack unsigned 4-bit codes ``[N, K]`` two per byte, even k in the low nibble.

    CK/backends/eager/w4a8_int8.py:200-202.
    """
    u = np.asarray(codes).astype(np.int32)
    if u.shape[-1] % 2:
        raise ValueError("K must be even to pack int4")
    packed = (u[:, 0::2] & 0xF) | ((u[:, 1::2] & 0xF) << 4)
    return packed.astype(np.uint8).view(np.int8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """Inverse of :func:`pack_int4`: codes 0..15 as int32 ``[N, K]``.

    CK/backends/eager/w4a8_int8.py:351-355.
    """
    p = np.asarray(packed).view(np.uint8).astype(np.int32)
    n, kh = p.shape
    codes = np.empty((n, kh * 2), dtype=np.int32)
    codes[:, 0::2] = p & 0xF
    codes[:, 1::2] = (p >> 4) & 0xF
    return codes


def prepare_w4a8_grouped(packed: np.ndarray) -> np.ndarray:
    """The GEMM's load layout of packed offset-8 codes ``[N, K/2]`` (this build's own layout; the
    reference has none): per 8 consecutive k (one 32-bit word), byte j holds ``c[j] ^ 8`` in its
    low nibble and ``c[4 + j] ^ 8`` in its high nibble (``c ^ 8`` is ``c - 8`` as a 4-bit two's
    complement value)."""
    codes = unpack_int4(packed)
    n, k = codes.shape
    if k % 8:
        raise ValueError("K must be a multiple of 8")
    v = (codes ^ 8).reshape(n, k // 8, 8)
    out = v[:, :, 0:4] | (v[:, :, 4:8] << 4)
    return out.reshape(n, k // 2).astype(np.uint8).view(np.int8)


def unprepare_w4a8_grouped(prepared: np.ndarray) -> np.ndarray:
    """Offset-8 codes ``[N, K]`` (int32) of a :func:`prepare_w4a8_grouped` layout."""
    p = np.asarray(prepared).view(np.uint8).astype(np.int32)
    n, kh = p.shape
    q = p.reshape(n, kh // 4, 4)
    codes = np.concatenate([q & 0xF, (q >> 4) & 0xF], axis=2) ^ 8
    return codes.reshape(n, kh * 2)


def w4a8_correction_lhs(xq: np.ndarray, x_scale: np.ndarray, group_size: int, out_dtype: str = "bf16") -> np.ndarray:
    """Left operand of the W4A8 correction term, as float32 values of ``out_dtype``:
    ``o(o(sum of xq over each group) * o(xs))`` (CK/backends/cuda/__init__.py:2294-2296:
    ``xq.view(m, groups, G).sum(-1, dtype=int32).to(out_dtype) * xs.to(out_dtype)``)."""
    q = np.asarray(xq, dtype=np.int64)
    m, k = q.shape
    sums = q.reshape(m, k // group_size, group_size).sum(-1).astype(F32)  # |sum| < 2^24: exact
    xs = np.asarray(x_scale, dtype=F32).reshape(-1, 1)
    return round_to(round_to(sums, out_dtype) * round_to(xs, out_dtype), out_dtype)


def quantize_int4_symmetric(w: np.ndarray) -> np.ndarray:
    """Signed int4 values in [-8, 7] -> offset-8 codes (``u = v + 8``, w4a8_int8.py:171-173)."""
    v = np.asarray(w, dtype=np.int32)
    if v.min(initial=0) < -8 or v.max(initial=0) > 7:
        raise ValueError("int4 values must lie in [-8, 7]")
    return v + 8


def dequant_int4_grouped_to_int8(qdata: np.ndarray, s_rel: np.ndarray,
                                 codebook: np.ndarray | None, group_size: int,
                                 s_rel_is_e4m3: bool = False) -> np.ndarray:
    """Decode packed int4 to the int8 grid the GEMM consumes.

    CK/backends/eager/w4a8_int8.py:344-363:
      v  = codebook[c] (fp32) if a codebook is given, else c - 8,
      w8 = clamp(rne(v * fp32(s_rel[n, k // G])), -127, 127).
    ``s_rel`` is float32, or float8_e4m3fn bits when ``s_rel_is_e4m3``.
    """
    codes = unpack_int4(qdata)
    n, k = codes.shape
    if k % group_size:
        raise ValueError("K must be a multiple of group_size")
    if codebook is not None:
        values = np.asarray(codebook, dtype=F32)[codes]
    else:
        values = (codes - 8).astype(F32)
    sr = e4m3fn_to_f32(s_rel) if s_rel_is_e4m3 else np.asarray(s_rel, dtype=F32)
    sr = sr.reshape(n, k // group_size)
    prod = values.reshape(n, k // group_size, group_size) * sr[:, :, None]
    return np.clip(np.rint(prod), -127, 127).astype(np.int8).reshape(n, k)


def w4a8_reference_linear(x_bits, qdata, s_rel, s_channel, codebook, group_size,
                          bias_bits=None, out_dtype="bf16", s_rel_is_e4m3=False):
    """Reference-format W4A8 linear without ConvRot: decode, then int8_linear.

    CK/backends/eager/w4a8_int8.py:494-508 (the reference always rotates with
    ConvRot first; this restatement covers the rotation-free composition).
    """
    w8 = dequant_int4_grouped_to_int8(qdata, s_rel, codebook, group_size, s_rel_is_e4m3)
    return int8_linear(x_bits, w8, s_channel, bias_bits, out_dtype)


# ---------------------------------------------------------------------------
# a8 (grouped-scale form): int32 partials per K group, fp32 group scales
# ---------------------------------------------------------------------------

def w4a8_group_partials(a: np.ndarray, qdata: np.ndarray, group_size: int) -> np.ndarray:
    """Exact per-group int32 partials ``P[g, m, n] = sum_{k in g} A[m,k] * (c[n,k] - 8)``."""
    codes = unpack_int4(qdata)
    w = (codes - 8).astype(np.float64)
    a = np.asarray(a, dtype=np.int8).astype(np.float64)
    m, k = a.shape
    n = w.shape[0]
    g = k // group_size
    out = np.empty((g, m, n), dtype=np.int32)
    for i in range(g):
        sl = slice(i * group_size, (i + 1) * group_size)
        out[i] = (a[:, sl] @ w[:, sl].T).astype(np.int32)
    return out


def w4a8_grouped_linear_f64(a: np.ndarray, x_scale: np.ndarray, qdata: np.ndarray,
                            group_scale: np.ndarray, group_size: int):
    """float64 value of ``xs[m] * sum_g fp32(scale[g, n]) * P_g[m, n]`` and its error budget.

    Returns ``(value, magnitude)`` where ``magnitude = xs * sum_g |scale * P_g|``
    bounds the float32 accumulation error of any summation order.
    """
    p = w4a8_group_partials(a, qdata, group_size).astype(np.float64)
    gs = np.asarray(group_scale, dtype=np.float16).astype(np.float64)  # [G, N]
    xs = np.asarray(x_scale, dtype=F32).astype(np.float64).reshape(-1, 1)
    terms = p * gs[:, None, :]
    return xs * terms.sum(axis=0), xs * np.abs(terms).sum(axis=0)


def w4a8_grouped_linear(a: np.ndarray, x_scale: np.ndarray, qdata: np.ndarray,
                        group_scale: np.ndarray, group_size: int,
                        bias_bits: np.ndarray | None = None, out_dtype: str = "bf16") -> np.ndarray:
    """The grouped-scale W4A8 output in the kernel's own summation order.

    acc = sum over g = 0, 1, ... of fp32(P_g) * fp32(scale[g, n]) accumulated
    with fused multiply-adds in float32 (emulated exactly in float64 per step),
    then y = out(acc * xs[m]), then y = out(y + out(bias)).
    """
    p = w4a8_group_partials(a, qdata, group_size)
    gs = np.asarray(group_scale, dtype=np.float16).astype(F32)
    acc = np.zeros(p.shape[1:], dtype=F32)
    for g in range(p.shape[0]):
        # fma(float(P), s, acc): the product (<= 29 significant bits) is exact in the x87
        # 64-bit significand, and so is its sum with acc unless the two differ by more than
        # 2**35, where the lost bits cannot move the single rounding to fp32.
        prod = p[g].astype(F32).astype(np.longdouble) * gs[g][None, :].astype(np.longdouble)
        acc = (prod + acc.astype(np.longdouble)).astype(F32)
    xs = np.asarray(x_scale, dtype=F32).reshape(-1, 1)
    y = round_to(acc * xs, out_dtype)
    if bias_bits is not None:
        y = round_to(y + round_to(bf16_to_f32(bias_bits).reshape(1, -1), out_dtype), out_dtype)
    return y


# ---------------------------------------------------------------------------
# The INT8 FFN chain (fc1 -> tanh-GELU -> per-token re-quant -> fc2)
# ---------------------------------------------------------------------------

def ffn_gelu_int8(x_bits, w1, s1, b1_bits, w2, s2, b2_bits):
    """``int8_linear(gelu_tanh(int8_linear(x, fc1)), fc2)``; returns (out, h) as float32.

    The reference chains two ``int8_linear`` calls with ``input_act`` on the
    second (CK/backends/eager/quantization.py:971-1056, _activations.py:40-53).
    ``h`` is the bfloat16 GELU output fed to the second quantizer.
    """
    y1 = int8_linear(x_bits, w1, s1, b1_bits, "bf16")
    h = gelu_tanh_bf16(bf16_bits(y1))
    out = int8_linear(h, w2, s2, b2_bits, "bf16")
    return out, bf16_to_f32(h)
