"""torch-CPU restatement of the reference's eager op sequence.

Test infrastructure only (see the package docstring). It replays, op for op, the
PyTorch CPU path the reference runs when no GPU backend is present, so that
``bench.py`` can time it as the CPU baseline and the tests can cross-check it
against the numpy restatement in ``eager_np``. Paths are relative to the
reference tree; ``CK`` = ``backends/turbo/vendor/comfy_kitchen``.
"""

from __future__ import annotations

import torch


def quantize_int8_rowwise(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """CK/backends/eager/quantization.py:857-875 (+815-818, 821-826)."""
    abs_max = x.abs().amax(dim=-1, keepdim=True)
    scale = (abs_max.float() / 127.0).clamp(min=1e-30)
    s = scale.to(dtype=x.dtype)
    s = torch.where(s == 0, torch.full_like(s, torch.finfo(x.dtype).tiny), s)
    q = (x / s).round_().clamp_(-128.0, 127.0).to(torch.int8)
    return q, scale


def quantize_int8_rowwise_stochastic(x: torch.Tensor, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference's stochastic path, quantization.py:803-826 + 857-875, on x's device: the
    noise is torch.rand in x's dtype from a generator on x's device seeded with ``seed``. The
    scale is divided on the CPU, as the eager path computes it there (torch on a GPU divides by
    a host scalar through its reciprocal, which can differ in the last bit)."""
    abs_max = x.abs().amax(dim=-1, keepdim=True)
    scale = (abs_max.float().cpu() / 127.0).clamp(min=1e-30).to(x.device)
    s = scale.to(dtype=x.dtype)
    s = torch.where(s == 0, torch.full_like(s, torch.finfo(x.dtype).tiny), s)
    scaled = x / s
    gen = torch.Generator(device=x.device)
    gen.manual_seed(seed)
    rng = torch.rand(scaled.shape, dtype=scaled.dtype, layout=scaled.layout, device=scaled.device, generator=gen)
    q = scaled.add_(rng).floor_().clamp_(-128.0, 127.0).to(torch.int8)
    return q, scale


def int8_matmul(a: torch.Tensor, w_nk: torch.Tensor) -> torch.Tensor:
    """``torch._int_mm`` with the K padding of quantization.py:749-782."""
    b = w_nk.t().contiguous()
    k = a.shape[1]
    pk = (k + 7) // 8 * 8
    if pk != k:
        a = torch.cat((a, a.new_zeros(a.shape[0], pk - k)), dim=1)
        b = torch.cat((b, b.new_zeros(pk - k, b.shape[1])), dim=0)
    n = b.shape[1]
    pn = (n + 7) // 8 * 8
    if pn != n:
        b = torch.cat((b, b.new_zeros(b.shape[0], pn - n)), dim=1)
    out = torch._int_mm(a, b)
    return out[:, :n] if pn != n else out


def dequant(result: torch.Tensor, x_scale: torch.Tensor, weight_scale: torch.Tensor,
            bias: torch.Tensor | None, out_dtype: torch.dtype) -> torch.Tensor:
    """Chunked dequant and bias add of quantization.py:1031-1054."""
    m, n = result.shape
    chunk_size = max(1, min(m, 256 * 1024 * 1024 // (n * 4)))
    ws = weight_scale.to(torch.float32).reshape(1, -1)
    parts = []
    for i in range(0, m, chunk_size):
        e = min(i + chunk_size, m)
        chunk = result[i:e].float()
        parts.append((chunk * (x_scale[i:e].to(torch.float32) * ws)).to(out_dtype))
    out = torch.cat(parts, dim=0)
    if bias is not None:
        out = out + bias.to(dtype=out.dtype).reshape(1, -1)
    return out


def apply_input_act(x: torch.Tensor, input_act: str | None) -> torch.Tensor:
    """CK/backends/_activations.py:40-53."""
    if input_act in (None, "none"):
        return x
    if input_act == "gelu_tanh":
        return torch.nn.functional.gelu(x, approximate="tanh")
    if input_act == "swiglu":
        gate, up = x.chunk(2, dim=-1)
        return torch.nn.functional.silu(gate).mul_(up)
    raise ValueError(f"unsupported input_act: {input_act!r}")


_HADAMARD: dict = {}


def hadamard(g: int, dtype: torch.dtype) -> torch.Tensor:
    """kron(h4, ..., h4) / sqrt(g) (CK/tensor/int8_utils.py:11-38)."""
    key = (g, dtype)
    if key not in _HADAMARD:
        h4 = torch.tensor([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=torch.float64)
        h = h4
        while h.shape[0] < g:
            h = torch.kron(h, h4)
        _HADAMARD[key] = (h / float(g) ** 0.5).to(dtype)
    return _HADAMARD[key]


def rotate(x: torch.Tensor, g: int) -> torch.Tensor:
    """x_grouped @ H_g in x's dtype (CK/tensor/int8_utils.py:58-74)."""
    k = x.shape[-1]
    return torch.matmul(x.reshape(*x.shape[:-1], k // g, g), hadamard(g, x.dtype)).reshape(x.shape)


def int8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                input_act: str | None = None, convrot: bool = False,
                convrot_groupsize: int = 256) -> torch.Tensor:
    """CK/backends/eager/quantization.py:971-1056."""
    x = apply_input_act(x, input_act)
    if convrot:
        x = rotate(x, convrot_groupsize)
    weight_scale = weight_scale.to(torch.float32).reshape(-1)
    x2 = x.reshape(-1, x.shape[-1])
    q, s = quantize_int8_rowwise(x2)
    acc = int8_matmul(q, weight)
    out = dequant(acc, s, weight_scale, bias, out_dtype)
    return out.reshape(*x.shape[:-1], weight.shape[0])


def adaln(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """CK/backends/eager/adaln.py:11-14."""
    normalized = torch.nn.functional.layer_norm(x, x.shape[-1:], eps=eps)
    return normalized * (1 + scale) + shift


def dequant_int4_grouped_to_int8(qdata, s_rel, codebook, group_size):
    """CK/backends/eager/w4a8_int8.py:344-363."""
    n, k_half = qdata.shape
    k = k_half * 2
    packed = qdata.to(torch.int32) & 0xFF
    codes = torch.empty(n, k, dtype=torch.int32)
    codes[:, 0::2] = packed & 0xF
    codes[:, 1::2] = (packed >> 4) & 0xF
    values = codebook.float()[codes] if codebook is not None else codes.float() - 8.0
    values = values.view(n, k // group_size, group_size) * s_rel.float().unsqueeze(-1)
    return values.view(n, k).round().clamp_(-127, 127).to(torch.int8)


def w4a8_grouped_linear(a: torch.Tensor, x_scale: torch.Tensor, qdata: torch.Tensor,
                        group_scale: torch.Tensor, group_size: int,
                        out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Grouped-scale W4A8: per-group ``torch._int_mm`` partials, fp32 group scaling.

    There is no reference implementation of this format; this is the eager
    composition of reference ops (w4a8_int8.py:351-355 unpacking, ``_int_mm``)
    that the CPU baseline times.
    """
    n, k_half = qdata.shape
    k = k_half * 2
    packed = qdata.to(torch.int32) & 0xFF
    codes = torch.empty(n, k, dtype=torch.int8)
    codes[:, 0::2] = ((packed & 0xF) - 8).to(torch.int8)
    codes[:, 1::2] = (((packed >> 4) & 0xF) - 8).to(torch.int8)
    acc = torch.zeros(a.shape[0], n, dtype=torch.float32)
    gs = group_scale.float()
    for g in range(k // group_size):
        sl = slice(g * group_size, (g + 1) * group_size)
        part = int8_matmul(a[:, sl].contiguous(), codes[:, sl].contiguous())
        acc.addcmul_(part.float(), gs[g].reshape(1, -1))
    return (acc * x_scale.reshape(-1, 1).float()).to(out_dtype)


def ffn_gelu_int8(x, w1, s1, b1, w2, s2, b2):
    """fc1 -> tanh-GELU (as fc2's input_act) -> fc2, two eager int8_linear calls."""
    h = int8_linear(x, w1, s1, b1)
    return int8_linear(h, w2, s2, b2, input_act="gelu_tanh")


def rms_adaln(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, shift: torch.Tensor,
              scale: torch.Tensor, segments) -> torch.Tensor:
    """h3serve/native_engine/model/kernels.py:7629-7640 with RMSNorm at layers.py:39-48."""
    hidden = torch.nn.functional.rms_norm(x, (x.shape[-1],), weight=norm_weight.to(x.dtype), eps=eps)
    for start, stop, row in segments:
        hidden[start:stop].mul_(1.0 + scale[row].to(hidden.dtype)).add_(shift[row].to(hidden.dtype))
    return hidden


def gated_residual_(residual: torch.Tensor, update: torch.Tensor, gate: torch.Tensor, segments) -> torch.Tensor:
    """h3serve/native_engine/model/layers.py:944-960."""
    for start, stop, row in segments:
        residual[start:stop].addcmul_(update[start:stop], gate[row].to(update.dtype))
    return residual


def h3_mlp_(residual, norm_weight, eps, shift, scale, gate, segments, w1, s1, b1, w2, s2, b2):
    """The H3 block's MLP half as the reference composes it (layers.py:1138-1150 ->
    fused_mlp.py:386-420): rms_adaln, fc1 (ConvRot 256), SwiGLU folded into fc2's ConvRot
    int8_linear, gated residual update of ``residual`` in place."""
    hidden = rms_adaln(residual, norm_weight, eps, shift, scale, segments)
    raw = int8_linear(hidden, w1, s1, b1, convrot=True)
    projected = int8_linear(raw, w2, s2, b2, input_act="swiglu", convrot=True)
    return gated_residual_(residual, projected, gate, segments)


def quantize_rotated_w4a8(weight: torch.Tensor, group_size: int = 16, symmetric: bool = True,
                          scale_dtype: torch.dtype = torch.float8_e4m3fn,
                          codebook: torch.Tensor | None = None):
    """The reference's storage of an already rotated weight as torch CPU ops
    (CK/backends/eager/w4a8_int8.py:122-209; nearest-level search 35-63): ``codebook`` given
    selects the symmetric codebook mode, None the uniform symmetric mode (or the asymmetric one
    when ``symmetric`` is False). Returns (packed, s_rel, s_channel, correction)."""
    n, k = weight.shape
    groups = k // group_size
    gw = weight.float().view(n, groups, group_size)

    def nearest(values, levels):  # first index of the smallest |values - level|
        best = (values - levels[..., 0]).abs()
        idx = torch.zeros_like(values, dtype=torch.int32)
        for i in range(1, 16):
            d = (values - levels[..., i]).abs()
            closer = d < best
            best = torch.where(closer, d, best)
            idx = torch.where(closer, i, idx)
        return idx

    correction = None
    if symmetric and codebook is not None:
        cb = codebook.float()
        gs = gw.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
        q = nearest(gw / gs, cb)
        for _ in range(3):
            qc = cb[q]
            gs = ((gw * qc).sum(-1, keepdim=True) / (qc * qc).sum(-1, keepdim=True).clamp(min=1e-8)).clamp(min=1e-8)
            q = nearest(gw / gs, cb)
        shifted = cb[q] * gs
    elif symmetric:
        gs = (gw.abs().amax(dim=-1, keepdim=True) / 7.0).clamp(min=1e-8)
        signed = (gw / gs).round().clamp(-8, 7).to(torch.int32)
        q = signed + 8
        shifted = signed * gs
    else:
        mn = gw.amin(dim=-1, keepdim=True)
        gs = ((gw.amax(dim=-1, keepdim=True) - mn) / 15.0).clamp(min=1e-8)
        q = ((gw - mn) / gs).round().clamp(0, 15).to(torch.int32)
        shifted = (q - 8) * gs
        correction = (8.0 * gs + mn).squeeze(-1).t().contiguous().to(weight.dtype)
    s_channel = (shifted.abs().amax(dim=(1, 2)) / 127.0).clamp(min=1e-8)
    s_rel = (gs.squeeze(-1) / s_channel.unsqueeze(1)).float()
    if scale_dtype != torch.float32:
        s_rel = s_rel.to(scale_dtype)
    if symmetric and codebook is not None:
        levels = (cb.view(1, 1, 16) * s_rel.float().unsqueeze(-1)).round_().clamp_(-127, 127)
        target = gw / s_channel.view(-1, 1, 1)
        q = nearest(target, levels.unsqueeze(2))
    u = q.reshape(n, k)
    packed = ((u[:, 0::2] & 0xF) | ((u[:, 1::2] & 0xF) << 4)).to(torch.int8)
    return packed, s_rel, s_channel.float(), correction
