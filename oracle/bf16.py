"""Bit-exact reduced-precision helpers (numpy). Test infrastructure only.

bfloat16 values are carried as ``uint16`` bit patterns; rounding from float32 is
round-to-nearest-even with NaN mapped to 0x7FC0, the scalar conversion PyTorch's
``c10::BFloat16(float)`` performs.
"""

from __future__ import annotations

import numpy as np

BF16_QNAN = np.uint16(0x7FC0)


def bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bits, round-to-nearest-even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)
    return np.where(np.isnan(x), BF16_QNAN, r)


def bf16_to_f32(bits) -> np.ndarray:
    """bfloat16 bits -> float32 (exact)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 and return them as float32."""
    return bf16_to_f32(bf16_bits(x))


def round_to(x, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` ('bf16', 'fp16' or 'fp32'), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "fp32":
        return x
    raise ValueError(f"unsupported dtype {dtype!r}")


def bf16_ulp(x) -> np.ndarray:
    """Spacing of bfloat16 values at |x| (the ulp of the binade containing x)."""
    x = np.abs(np.asarray(x, dtype=np.float32))
    e = np.floor(np.log2(np.maximum(x, np.float32(2.0 ** -126))))
    return np.float32(2.0) ** (e - 7)


def e4m3fn_to_f32(bits) -> np.ndarray:
    """float8_e4m3fn bits -> float32 (exact; 0x7F / 0xFF are NaN, no infinities)."""
    b = np.asarray(bits, dtype=np.uint8).astype(np.int32)
    sign = np.where(b & 0x80, -1.0, 1.0)
    exp = (b >> 3) & 0xF
    man = b & 0x7
    normal = sign * (1.0 + man / 8.0) * np.exp2(exp - 7.0)
    sub = sign * (man / 8.0) * np.exp2(-6.0)
    out = np.where(exp == 0, sub, normal).astype(np.float32)
    return np.where((b & 0x7F) == 0x7F, np.float32(np.nan), out)
