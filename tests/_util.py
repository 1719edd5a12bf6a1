"""Shared helpers for the test suite: seeded inputs and torch <-> numpy bit views."""

from __future__ import annotations

import numpy as np
import torch


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> numpy uint16 bit array."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def from_bits(b: np.ndarray) -> torch.Tensor:
    """numpy uint16 bits -> CPU bf16 tensor."""
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def activations(m: int, k: int, seed: int, outlier_frac: float = 0.005, outlier_mul: float = 20.0) -> torch.Tensor:
    """bf16 [m, k] ~ N(0, 1) with ceil(outlier_frac * k) channels scaled (CPU)."""
    g = gen(seed)
    x = torch.randn(m, k, generator=g)
    n_out = int(np.ceil(outlier_frac * k))
    if n_out:
        idx = torch.randperm(k, generator=g)[:n_out]
        x[:, idx] *= outlier_mul
    return x.to(torch.bfloat16)


def int8_weight(n: int, k: int, seed: int, std: float = 0.02):
    """int8 [n, k] and fp32 [n] per-channel scales from N(0, std) with the row quantizer."""
    from oracle import eager_np

    g = gen(seed)
    wf = (torch.randn(n, k, generator=g) * std).to(torch.bfloat16)
    q, s = eager_np.quantize_int8_rowwise(bits(wf))
    return torch.from_numpy(q), torch.from_numpy(s.reshape(-1))


def bf16_vec(n: int, seed: int, std: float) -> torch.Tensor:
    return (torch.randn(n, generator=gen(seed)) * std).to(torch.bfloat16)


def packed_int4(n: int, k: int, seed: int) -> torch.Tensor:
    """Random offset-8 int4 codes packed two per byte (low nibble = even k), int8 [n, k/2]."""
    from oracle import eager_np

    codes = torch.randint(0, 16, (n, k), generator=gen(seed)).numpy()
    return torch.from_numpy(eager_np.pack_int4(codes))


def group_scales(k: int, n: int, g: int, seed: int) -> torch.Tensor:
    """fp16 [k/g, n] = |N(0,1)| * 0.01."""
    return (torch.randn(k // g, n, generator=gen(seed)).abs() * 0.01).to(torch.float16)
