"""ConvRot (regular Hadamard) rotation before the per-token quantizer, and the SwiGLU input
activation. Test infrastructure only (see the package docstring).

Reference semantics (CK = backends/turbo/vendor/comfy_kitchen):
  * H_G = kron(h4, ..., h4) / sqrt(G), h4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]], G a
    power of 4 (CK/tensor/int8_utils.py:11-38);
  * activations: x_rot = x_grouped @ H_G per group of G columns (int8_utils.py:58-74), then
    the row quantizer (CK/backends/eager/quantization.py:1012-1025, 857-875);
  * weights (offline): W_rot = W_grouped @ H_G^T, then the row quantizer (quantization.py:898-906).
The reference multiplies in the tensor's dtype with torch's CPU matmul, whose accumulation order
is internal to the library. This restatement fixes the value instead: the rotated activation is
the exact product rounded once to the tensor's dtype. It is computed as a radix-4 transform in
float64 (every float64 operation below is exact while a group's exponent spread is at most 37
bits, so the result is then the correctly rounded product) in one fixed operation order, which
the device kernel repeats. The tests pin it against x @ H in exact arithmetic and against
torch's CPU matmul.

SwiGLU (CK/backends/_activations.py:50-52): gate, up = x.chunk(2, -1); y = silu(gate) * up in
bfloat16: bf16(bf16(silu(gate)) * up), silu from torch's CPU routine (golden table).
"""

from __future__ import annotations

import pathlib

import numpy as np

from .bf16 import bf16_bits, bf16_to_f32

F32 = np.float32
_H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
_GOLDEN = pathlib.Path(__file__).resolve().parents[1] / "tests" / "golden"


def log4(g: int) -> int:
    if g < 4 or g & (g - 1) or (g.bit_length() - 1) % 2:
        raise ValueError(f"Regular Hadamard size must be a power of 4, got {g}")
    return (g.bit_length() - 1) // 2


def hadamard(g: int) -> np.ndarray:
    """H_G as float64 (int8_utils.py:11-38: repeated kron of h4, divided by sqrt(G))."""
    d = log4(g)
    h = _H4
    for _ in range(d - 1):
        h = np.kron(h, _H4)
    return h / float(2 ** d)


def fht_f64(x: np.ndarray, g: int) -> np.ndarray:
    """x @ H_G per group of g columns, float64 in, float64 out, in the kernel's operation order.

    For digit t = 0 .. log4(g) - 1 of the in-group index (stride 4**t), each quad
    (x0, x1, x2, x3) becomes y_k = S - 2 x_{3-k} (column k of h4 is all ones except -1 in row
    3-k), evaluated as the kernel does: for t <= 3 (digits it applies inside a lane) as
    S - (x_{3-k} + x_{3-k}) with S = (x0 + x1) + (x2 + x3); for t >= 4 (digits exchanged across
    lanes) as (x_k + x_{k^1}) + (x_{k^2} - x_{k^3}). The product with the 1/sqrt(g) factor (a power
    of two) comes last.
    """
    d = log4(g)
    x = np.asarray(x, dtype=np.float64)
    lead, k = x.shape[:-1], x.shape[-1]
    if k % g:
        raise ValueError(f"features {k} not divisible by group_size {g}")
    y = x.reshape(-1, k // g, g)
    for t in range(d):
        v = y.reshape(y.shape[0], y.shape[1], g // 4 ** (t + 1), 4, 4 ** t)
        out = np.empty_like(v)
        if t < 4:
            s = (v[:, :, :, 0] + v[:, :, :, 1]) + (v[:, :, :, 2] + v[:, :, :, 3])
            for kk in range(4):
                p = v[:, :, :, 3 - kk]
                out[:, :, :, kk] = s - (p + p)
        else:
            for kk in range(4):
                out[:, :, :, kk] = (v[:, :, :, kk] + v[:, :, :, kk ^ 1]) + (v[:, :, :, kk ^ 2] - v[:, :, :, kk ^ 3])
        y = out.reshape(y.shape)
    return (y * (1.0 / 2 ** d)).reshape(*lead, k)


def round_f64_to_bf16(x: np.ndarray) -> np.ndarray:
    """float64 -> bfloat16 bits, one round-to-nearest-even rounding.

    Through float32 (RNE), which is exact except where the float32 value is itself a bfloat16
    midpoint that x is not: then x lies strictly on one side and the midpoint is broken
    toward it (the device kernel does the same)."""
    x = np.asarray(x, dtype=np.float64)
    f = x.astype(F32)
    b = bf16_bits(f).astype(np.uint32)
    u = f.view(np.uint32)
    with np.errstate(invalid="ignore"):
        tie = ((u & 0xFFFF) == 0x8000) & (f.astype(np.float64) != x) & np.isfinite(x)
        up = np.abs(x) > np.abs(f.astype(np.float64))
    fixed = (u >> 16) + up.astype(np.uint32)
    return np.where(tie, fixed, b).astype(np.uint16)


def silu_table() -> np.ndarray:
    return np.load(_GOLDEN / "silu_bf16.npy")


def gelu_table() -> np.ndarray:
    return np.load(_GOLDEN / "gelu_tanh_bf16.npy")


def swiglu_bf16(x_bits: np.ndarray) -> np.ndarray:
    """[..., 2K] bf16 bits -> [..., K] bf16 bits: bf16(bf16(silu(gate)) * up)."""
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    k2 = x_bits.shape[-1]
    if k2 % 2:
        raise ValueError("swiglu needs an even last dimension")
    gate, up = x_bits[..., : k2 // 2], x_bits[..., k2 // 2:]
    a = bf16_to_f32(silu_table()[gate])
    with np.errstate(over="ignore", invalid="ignore"):  # fp32 overflow to inf and inf * 0 = NaN, as in torch
        return bf16_bits(a * bf16_to_f32(up))


def apply_input_act_bf16(x_bits: np.ndarray, input_act: str | None) -> np.ndarray:
    if input_act in (None, "none"):
        return np.asarray(x_bits, dtype=np.uint16)
    if input_act == "gelu_tanh":
        return gelu_table()[np.asarray(x_bits, dtype=np.uint16)]
    if input_act == "swiglu":
        return swiglu_bf16(x_bits)
    raise ValueError(f"unsupported input_act: {input_act!r}")


def quantize_rows_f32(xf: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The row quantizer on float32 values (quantization.py:857-875 with T = float32):
    s = max(amax / 127, 1e-30); q = clamp(rne(x / s), -128, 127)."""
    xf = np.asarray(xf, dtype=F32)
    amax = np.max(np.abs(xf), axis=-1, keepdims=True)
    scale = np.maximum(amax / F32(127.0), F32(1e-30)).astype(F32)
    with np.errstate(invalid="ignore"):
        q = np.clip(np.rint(xf / scale), -128.0, 127.0)
    return np.nan_to_num(q, nan=0.0).astype(np.int8), scale


def convrot_quantize_bf16(x_bits: np.ndarray, group_size: int, input_act: str | None = None):
    """bf16 activations [..., K] (or [..., 2K] for swiglu) -> (q int8, scale fp32 [..., 1],
    rotated bf16 bits). group_size 0 skips the rotation (activation + quantizer only)."""
    from .eager_np import quantize_int8_rowwise

    a = apply_input_act_bf16(x_bits, input_act)
    if group_size:
        rot = round_f64_to_bf16(fht_f64(bf16_to_f32(a).astype(np.float64), group_size))
    else:
        rot = a
    q, s = quantize_int8_rowwise(rot)
    return q, s, rot


def round_f64_to_f16(x: np.ndarray) -> np.ndarray:
    """float64 -> float16, one round-to-nearest-even rounding (numpy converts from the float64
    bits directly; the device goes through a round-to-odd float32, which lands on the same side
    of every float16 rounding boundary)."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float64).astype(np.float16)


def convrot_quantize_f16(x: np.ndarray, group_size: int, input_act: str | None = None):
    """float16 activations [..., K] (or [..., 2K] for swiglu) -> (q int8, scale fp32 [..., 1],
    rotated float16). The activation and the row quantizer are the reference's own torch CPU ops
    in float16 (eager_torch: CK/backends/_activations.py:40-53, CK/backends/eager/
    quantization.py:857-875); the rotation is the exact product rounded once to float16. group_size
    0 skips the rotation."""
    import torch

    from . import eager_torch

    a = eager_torch.apply_input_act(torch.from_numpy(np.asarray(x, dtype=np.float16)), input_act).numpy()
    with np.errstate(invalid="ignore"):  # inf - inf in the rotation: NaN, as in the device's
        rot = round_f64_to_f16(fht_f64(a.astype(np.float64), group_size)) if group_size else a
    q, s = eager_torch.quantize_int8_rowwise(torch.from_numpy(rot))
    return q.numpy(), s.numpy(), rot


def convrot_quantize_f32(x: np.ndarray, group_size: int):
    """float32 activations [..., K] -> (q, scale, rotated float32)."""
    rot = fht_f64(np.asarray(x, dtype=F32).astype(np.float64), group_size).astype(F32)
    q, s = quantize_rows_f32(rot)
    return q, s, rot


def rotate_weight_f64(w: np.ndarray, group_size: int) -> np.ndarray:
    """W_grouped @ H^T in float64 (H is symmetric, so the same transform as activations)."""
    return fht_f64(np.asarray(w, dtype=np.float64), group_size)


def quantize_int8_convrot_weight(w: np.ndarray, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Offline weight preparation for tests: rotate in float64, round to bf16, quantize rows
    (quantization.py:898-906 restated with the exact rotation)."""
    from .eager_np import quantize_int8_rowwise

    rot = round_f64_to_bf16(rotate_weight_f64(w, group_size))
    return quantize_int8_rowwise(rot)
