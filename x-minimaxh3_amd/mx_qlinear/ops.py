"""Torch-facing functions of the quantized linear path.

Names, argument order, defaults and error behaviour mirror the reference's Comfy-Kitchen API
(backends/turbo/vendor/comfy_kitchen/__init__.py:110-127, 702-764 and
comfy_kitchen/tensor/w4a8_int8.py:89-115; CK below stands for
backends/turbo/vendor/comfy_kitchen). Every function runs the HIP kernels of libmx_qlinear.so
on the tensors' GPU and current stream; there is no CPU path.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import call

_OUT_CODES = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}
_ACT_CODES = {None: _lib.ACT_NONE, "none": _lib.ACT_NONE, "gelu_tanh": _lib.ACT_GELU_TANH,
              "swiglu": _lib.ACT_SWIGLU}


def _p(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_GEMM_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _gemm_ws(device: torch.device):
    """The INT8 GEMMs' tile-queue workspace for the current stream on ``device``, as the two
    trailing arguments (pointer, bytes) the GEMM entry points take before the stream: the
    counters with which the XCDs share out the last tiles at run time. One zero-filled workspace
    per (device, stream), made on that stream's first GEMM and kept for the process, as the
    reference keeps one per (device, stream) inside its launchers
    (CK/backends/cuda/ops/cutlass_gemm_int8.cu:39-55); the kernels leave it zero after every call.
    Under graph capture no workspace is passed (the static tile order, the same outputs), so a
    captured graph shares no memory with eager calls."""
    with torch.cuda.device(device):
        if torch.cuda.is_current_stream_capturing():
            return None, 0
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream)
    ws = _GEMM_WORKSPACES.get(key)
    if ws is None:
        ws = torch.zeros(_lib.GEMM_WORKSPACE_BYTES, dtype=torch.uint8, device=device)
        _GEMM_WORKSPACES[key] = ws
    return _p(ws), ws.numel()


def _require_gpu(*tensors: torch.Tensor | None) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("mx_qlinear runs on the GPU only; got a tensor on " + str(t.device))
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _act_code(input_act: str | None) -> int:
    try:
        return _ACT_CODES[input_act]
    except KeyError:
        raise ValueError(
            f"unsupported input_act: {input_act!r} (expected one of ['gelu_tanh', 'none', 'swiglu'])"
        ) from None


def _act_width(input_act: str | None) -> int:
    """Raw input columns per activated column (CK/backends/_activations.py:34-36)."""
    return 2 if input_act == "swiglu" else 1


def _check_power_of_four(g: int) -> None:
    if g < 4 or g & (g - 1) or (g.bit_length() - 1) % 2:
        raise ValueError(f"Regular Hadamard size must be a power of 4, got {g}")


def _out_code(dtype: torch.dtype) -> int:
    try:
        return _OUT_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported output dtype {dtype}") from None


# ---------------------------------------------------------------------------------------
# quantizers and adaLN
# ---------------------------------------------------------------------------------------

def quantize_int8_rowwise(x: torch.Tensor, stochastic_rounding: int | None = 0,
                          input_act: str | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row INT8 quantization: ``(q int8 [..., K], scale fp32 [..., 1])``.

    CK/__init__.py:702-709 / CK/backends/eager/quantization.py:857-875. ``stochastic_rounding``
    > 0 is the reference's seed (quantization.py:803-826): the noise is ``torch.rand`` in x's
    dtype from a generator on x's device seeded with it, the same draws the reference makes, and
    the kernel adds it to the scaled value and floors. ``input_act`` ('gelu_tanh' or 'swiglu',
    bf16 or fp16 inputs; CK/backends/_activations.py:40-53) is applied first (not with stochastic
    rounding); with 'swiglu' the input is ``[..., 2K]`` and the result ``[..., K]``.
    """
    act = _act_code(input_act)
    if stochastic_rounding is not None and stochastic_rounding > 0:
        if act:
            raise NotImplementedError("input_act is not provided together with stochastic rounding")
        return _quantize_int8_rowwise_stochastic(x, int(stochastic_rounding))
    if act == _lib.ACT_SWIGLU:
        return quantize_int8_rowwise_convrot(x, 0, input_act)
    dev = _require_gpu(x)
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"unsupported input dtype {x.dtype}")
    if act and x.dtype == torch.float32:
        raise NotImplementedError(f"input_act={input_act!r} is provided for bfloat16 and float16 inputs")
    k = x.shape[-1]
    if k == 0:
        raise ValueError("quantize_int8_rowwise needs a non-empty last dimension")
    x2 = x.reshape(-1, k).contiguous()
    m = x2.shape[0]
    q = torch.empty((m, k), dtype=torch.int8, device=dev)
    s = torch.empty((m, 1), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        call("mxq_quantize_int8_rowwise", _p(x2), _OUT_CODES[x.dtype], _p(q), _p(s), m, k, act, _stream(dev))
    return q.reshape(x.shape), s.reshape(*x.shape[:-1], 1)


def _quantize_int8_rowwise_stochastic(x: torch.Tensor, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    dev = _require_gpu(x)
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"unsupported input dtype {x.dtype}")
    k = x.shape[-1]
    if k == 0:
        raise ValueError("quantize_int8_rowwise needs a non-empty last dimension")
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    noise = torch.rand(x.shape, dtype=x.dtype, layout=x.layout, device=dev, generator=gen)
    x2 = x.reshape(-1, k).contiguous()
    m = x2.shape[0]
    q = torch.empty((m, k), dtype=torch.int8, device=dev)
    s = torch.empty((m, 1), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        call("mxq_quantize_int8_rowwise_stochastic", _p(x2), _OUT_CODES[x.dtype], _p(noise.reshape(m, k)),
             _p(q), _p(s), m, k, _stream(dev))
    return q.reshape(x.shape), s.reshape(*x.shape[:-1], 1)


def quantize_int8_rowwise_convrot(x: torch.Tensor, group_size: int = 256,
                                  input_act: str | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """ConvRot rotation + per-row INT8 quantization in one pass: ``(q, scale [..., 1])``.

    The reference's fused rotate-and-quantize (quantize_int8_rowwise_convrot64 of its CUDA
    backend, CK/backends/cuda/ops/int8_linear.cu:942-1030; eager
    CK/backends/eager/quantization.py:876-895 and 1012-1025): optional activation
    (CK/backends/_activations.py:40-53), then x @ H_G per group of ``group_size`` columns
    (CK/tensor/int8_utils.py:11-74, the exact product rounded once to x's dtype), then the row
    quantizer. ``group_size=0`` skips the rotation. bf16 or fp16 inputs (any activation) or
    fp32 inputs (no activation).
    """
    act = _act_code(input_act)
    dev = _require_gpu(x)
    if group_size:
        _check_power_of_four(group_size)
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32) or (act and x.dtype == torch.float32):
        raise NotImplementedError("the rotation quantizer takes bfloat16 or float16 inputs (or float32 without an "
                                  "activation)")
    width = x.shape[-1]
    if width % _act_width(input_act):
        raise ValueError(f"{input_act} needs an even last dimension, got {width}")
    k = width // _act_width(input_act)
    if k == 0:
        raise ValueError("quantize_int8_rowwise needs a non-empty last dimension")
    if group_size and k % group_size:
        raise ValueError(f"ConvRot group size {group_size} does not divide input features {k}")
    if k % 16:
        raise NotImplementedError(f"the rotation quantizer needs a multiple of 16 columns, got {k}")
    x2 = x.reshape(-1, width).contiguous()
    m = x2.shape[0]
    q = torch.empty((m, k), dtype=torch.int8, device=dev)
    s = torch.empty((m, 1), dtype=torch.float32, device=dev)
    if m:
        with torch.cuda.device(dev):
            call("mxq_quantize_int8_rowwise_convrot", _p(x2), _OUT_CODES[x.dtype], _p(q), _p(s), m, k,
                 group_size, act, _stream(dev))
    return q.reshape(*x.shape[:-1], k), s.reshape(*x.shape[:-1], 1)


def quantize_int8_convrot_weight(weight: torch.Tensor, group_size: int = 256) -> tuple[torch.Tensor, torch.Tensor]:
    """Offline ConvRot weight preparation (CK/backends/eager/quantization.py:898-906): each row's
    groups are rotated (W_grouped @ H_G^T; H_G is symmetric, so the activation transform) and the
    rows quantized: ``(q int8 [N, K], scale fp32 [N, 1])``, the checkpoint's weight and
    weight_scale."""
    if weight.dim() != 2:
        raise ValueError("weight must be 2D [out_features, in_features]")
    return quantize_int8_rowwise_convrot(weight, group_size)


def apply_input_act(x: torch.Tensor, input_act: str | None) -> torch.Tensor:
    """The pre-quantization activation (CK/backends/_activations.py:40-53) for bf16 and fp16 inputs.

    ``gelu_tanh`` is bit-identical to torch's CPU ``gelu(approximate='tanh')`` in the input's dtype;
    ``swiglu`` maps ``[..., 2K]`` to ``[..., K]`` as torch's ``silu(gate).mul_(up)``.
    """
    code = _act_code(input_act)
    if code == _lib.ACT_NONE:
        return x
    dev = _require_gpu(x)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError(f"{input_act} is provided for bfloat16 and float16 tensors")
    xc = x.contiguous()
    if x.dtype == torch.float16:
        width = x.shape[-1]
        if code == _lib.ACT_SWIGLU and width % 2:
            raise ValueError(f"swiglu needs an even last dimension, got {width}")
        k = width // 2 if code == _lib.ACT_SWIGLU else width
        rows = xc.numel() // max(width, 1)
        y = torch.empty((*x.shape[:-1], k), dtype=x.dtype, device=dev)
        if y.numel():
            with torch.cuda.device(dev):
                call("mxq_input_act_f16", _p(xc), _p(y), rows, k, code, _stream(dev))
        return y
    if code == _lib.ACT_SWIGLU:
        if x.shape[-1] % 2:
            raise ValueError(f"swiglu needs an even last dimension, got {x.shape[-1]}")
        k = x.shape[-1] // 2
        rows = xc.numel() // max(x.shape[-1], 1)
        y = torch.empty((*x.shape[:-1], k), dtype=x.dtype, device=dev)
        with torch.cuda.device(dev):
            call("mxq_swiglu_bf16", _p(xc), _p(y), rows, k, _stream(dev))
        return y
    y = torch.empty_like(xc)
    with torch.cuda.device(dev):
        call("mxq_gelu_tanh_bf16", _p(xc), _p(y), xc.numel(), _stream(dev))
    return y


def _modulation(t: torch.Tensor, rows: int, cols: int, dev, name: str, dtype=torch.bfloat16):
    t = t.to(device=dev, dtype=dtype)
    if t.shape[-1] != cols:
        raise ValueError(f"{name} last dimension {t.shape[-1]} != {cols}")
    t2 = t.reshape(-1, cols).contiguous()
    g = t2.shape[0]
    if g == 0 or rows % g != 0:
        raise ValueError(f"{name} with {g} rows does not broadcast over {rows} rows")
    return t2, rows // g


def adaln(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``layer_norm(x) * (1 + scale) + shift`` in x's dtype, bf16 or fp16 (CK/__init__.py:110-127,
    eager adaln.py:11-14).

    ``scale`` / ``shift`` are ``[D]`` or one row per consecutive group of x rows
    (``[G, D]`` with G dividing the number of rows), as the reference's CUDA launcher's
    scale_group / shift_group (CK/backends/cuda/ops/adaln.cu:256-313).
    """
    dev = _require_gpu(x)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError("mx_qlinear.adaln supports bfloat16 and float16 inputs")
    d = x.shape[-1]
    x2 = x.reshape(-1, d).contiguous()
    rows = x2.shape[0]
    out = torch.empty_like(x2)
    if rows == 0:
        return out.reshape(x.shape)
    sc, sg = _modulation(scale, rows, d, dev, "scale", x.dtype)
    sh, hg = _modulation(shift, rows, d, dev, "shift", x.dtype)
    with torch.cuda.device(dev):
        if x.dtype == torch.float16:
            call("mxq_adaln_quantize_int8_f16", _p(x2), _p(sc), _p(sh), sg, hg, float(eps), None, None, _p(out), rows,
                 d, _stream(dev))
        else:
            call("mxq_adaln", _p(x2), _p(sc), _p(sh), _p(out), rows, d, sg, hg, float(eps), _stream(dev))
    return out.reshape(x.shape)


def adaln_quantize_int8(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                        eps: float = 1e-6, return_modulated: bool = False):
    """``quantize_int8_rowwise(adaln(x, scale, shift, eps))`` in one pass over x.

    Returns ``(q, x_scale)`` or ``(q, x_scale, modulated_bf16)`` when ``return_modulated``.
    """
    dev = _require_gpu(x)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError("adaln_quantize_int8 supports bfloat16 and float16 inputs")
    d = x.shape[-1]
    x2 = x.reshape(-1, d).contiguous()
    rows = x2.shape[0]
    q = torch.empty((rows, d), dtype=torch.int8, device=dev)
    s = torch.empty((rows, 1), dtype=torch.float32, device=dev)
    y = torch.empty_like(x2) if return_modulated else None
    if rows:
        sc, sg = _modulation(scale, rows, d, dev, "scale", x.dtype)
        sh, hg = _modulation(shift, rows, d, dev, "shift", x.dtype)
        entry = "mxq_adaln_quantize_int8_f16" if x.dtype == torch.float16 else "mxq_adaln_quantize_int8"
        with torch.cuda.device(dev):
            call(entry, _p(x2), _p(sc), _p(sh), sg, hg, float(eps), _p(q), _p(s), _p(y), rows, d, _stream(dev))
    out = (q.reshape(x.shape), s.reshape(*x.shape[:-1], 1))
    return out + (y.reshape(x.shape),) if return_modulated else out


def _norm_parts(norm, d: int, dev, dtype=torch.bfloat16) -> tuple[torch.Tensor, float]:
    """An RMSNorm module (``.weight`` [d], ``.eps``) or a ``(weight, eps)`` pair ->
    (weight on ``dev`` in x's dtype, eps); the weight is cast like ``weight.to(x.dtype)``."""
    weight, eps = (norm.weight, norm.eps) if hasattr(norm, "weight") else norm
    w = weight.detach().to(device=dev, dtype=dtype).reshape(-1).contiguous()
    if w.numel() != d:
        raise ValueError(f"RMSNorm weight has {w.numel()} entries, expected {d}")
    return w, float(eps)


def _segment_table(t: torch.Tensor, d: int, dev, name: str, dtype=torch.bfloat16) -> torch.Tensor:
    t = t.detach()
    if t.dim() == 1:
        t = t.reshape(1, -1)
    if t.dim() != 2 or t.shape[1] != d:
        raise ValueError(f"{name} must be [rows, {d}], got {tuple(t.shape)}")
    return t.to(device=dev, dtype=dtype).contiguous()


def rms_adaln_quantize_int8(value: torch.Tensor, norm, shift: torch.Tensor, scale: torch.Tensor,
                            segments, convrot_groupsize: int = 256, return_modulated: bool = False):
    """``quantize(rotate(rms_adaln(value, norm, shift, scale, segments)))`` in one launch.

    The H3 block's pre-projection chain (h3serve/native_engine/model/layers.py:1094 ->
    kernels.py:7594 -> the ConvRotInt8Linear quantizer, CK/backends/eager/quantization.py:
    1012-1025). ``segments`` is a sequence of ``(start, stop, row)`` or an int32 row map.
    ``convrot_groupsize`` 0 skips the rotation. Returns ``(q, x_scale)`` or
    ``(q, x_scale, modulated)`` with ``return_modulated``.
    """
    return _rms_adaln_call(value, norm, shift, scale, segments, True, convrot_groupsize, return_modulated)


def rms_adaln(value: torch.Tensor, norm, shift: torch.Tensor, scale: torch.Tensor, segments) -> torch.Tensor:
    """RMSNorm then the segmented modulation ``h[a:b].mul_(1 + scale[row]).add_(shift[row])``
    (h3serve/native_engine/model/kernels.py:7594-7640, same roundings); bfloat16 [rows, D]."""
    return _rms_adaln_call(value, norm, shift, scale, segments, False, 0, True)


def _rms_adaln_call(value, norm, shift, scale, segments, quant: bool, group: int, want_y: bool):
    if value.dim() != 2:
        raise ValueError("rms_adaln expects a 2-D [tokens, hidden] tensor")
    if value.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError("rms_adaln supports bfloat16 and float16 inputs")
    dev = _require_gpu(value)
    rows, d = value.shape
    if quant and group:
        _check_power_of_four(group)
        if d % group:
            raise ValueError(f"ConvRot group size {group} does not divide input features {d}")
    w, eps = _norm_parts(norm, d, dev, value.dtype)
    sc = _segment_table(scale, d, dev, "scale", value.dtype)
    sh = _segment_table(shift, d, dev, "shift", value.dtype)
    if sc.shape[0] != sh.shape[0]:
        raise ValueError("scale and shift must have the same number of rows")
    if isinstance(segments, torch.Tensor):
        mr = _row_map(segments, rows, sc.shape[0], dev, "modulation row map", "modulation row outside the scale/shift tables")
    else:
        mr = segment_row_map(rows, segments, dev)
        if rows and max(int(r) for _, _, r in segments) >= sc.shape[0]:
            raise ValueError("modulation segment row outside the scale/shift tables")
    x = value.contiguous()
    y = torch.empty_like(x) if want_y else None
    q = torch.empty((rows, d), dtype=torch.int8, device=dev) if quant else None
    s = torch.empty((rows, 1), dtype=torch.float32, device=dev) if quant else None
    if rows and d:
        with torch.cuda.device(dev):
            if x.dtype == torch.float16:
                call("mxq_rms_adaln_quantize_int8_f16", _p(x), _p(w), _p(sc), _p(sh), sc.stride(0), sc.shape[0],
                     _p(mr), eps, _p(y), _p(q), _p(s), rows, d, group if quant else 0, _stream(dev))
            else:
                # room for bf16(1 + scale) of each modulation row, formed once per call
                ws = torch.empty(sc.shape[0] * sc.stride(0) * 2 if quant else 0, dtype=torch.uint8, device=dev)
                call("mxq_rms_adaln_quantize_int8", _p(x), _p(w), _p(sc), _p(sh), sc.stride(0), sc.shape[0],
                     _p(mr), eps, _p(y), _p(q), _p(s), rows, d, group if quant else 0, _p(ws), ws.numel(),
                     _stream(dev))
    if not quant:
        return y
    return (q, s, y) if want_y else (q, s)


# ---------------------------------------------------------------------------------------
# INT8 GEMMs
# ---------------------------------------------------------------------------------------

def _gemm_weight(w: torch.Tensor, kp: int, transpose: bool = False) -> torch.Tensor:
    """The int8 weight as the GEMM reads it: ``[N, kp]`` row-major (``w.t()`` with ``transpose``),
    K zero-padded to ``kp`` (zero terms leave the int32 sums unchanged, as the reference's own K
    padding, CK/backends/eager/quantization.py:770-775) and 16-byte aligned. A weight that already
    has that form is used as it is. Otherwise a weight (``transpose`` False: a layer's ``[N, K]``
    parameter or buffer) has the copy made once and kept on the tensor, rebuilt when the tensor's
    version counter moves; an in-place write through ``w.data`` does not move that counter, so a
    weight updated that way must be passed to :func:`prepare_int8_weight` again (or updated through
    the tensor itself). ``transpose`` (mm_int8's generic right operand, which can be any
    activation-like tensor) copies per call and caches nothing."""
    src = w.t() if transpose else w
    if not transpose and src.is_contiguous() and src.shape[1] == kp and src.data_ptr() % 16 == 0:
        return src
    key = (w._version, w.data_ptr(), tuple(w.shape), tuple(w.stride()), kp)
    cached = None if transpose else getattr(w, "_mxq_gemm_weight", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    wp = torch.zeros((src.shape[0], kp), dtype=torch.int8, device=w.device)
    wp[:, : src.shape[1]] = src
    if not transpose:
        try:
            w._mxq_gemm_weight = (key, wp)
        except (AttributeError, RuntimeError):  # tensors that take no attributes: copy per call
            pass
    return wp


def _gemm_activation(q: torch.Tensor, kp: int) -> torch.Tensor:
    """The int8 activation ``[M, kp]``: zero-padded K and 16-byte aligned (copied only when needed)."""
    if q.shape[1] == kp:
        return _aligned16(q)
    qp = torch.zeros((q.shape[0], kp), dtype=torch.int8, device=q.device)
    qp[:, : q.shape[1]] = q
    return qp


def _pad_k(q: torch.Tensor, w: torch.Tensor):
    """Activation and weight for the GEMM with K rounded up to a multiple of 16; the weight's
    padded or realigned form is built once per weight tensor (:func:`_gemm_weight`)."""
    k = q.shape[1]
    kp = (k + 15) // 16 * 16
    return _gemm_activation(q, kp), _gemm_weight(w, kp), kp


def prepare_int8_weight(qweight: torch.Tensor) -> torch.Tensor:
    """Build, once (at load), the GEMM form of an int8 ``[N, K]`` weight when it differs from the
    stored tensor (K not a multiple of 16, or a misaligned start), so later calls do not copy it.
    Calling it again rebuilds that form from the tensor's current contents (after an update
    through ``qweight.data``, which the cache cannot see)."""
    if qweight.dim() == 2 and qweight.dtype == torch.int8 and qweight.is_cuda:
        if hasattr(qweight, "_mxq_gemm_weight"):
            try:
                del qweight._mxq_gemm_weight
            except (AttributeError, RuntimeError):
                pass
        _gemm_weight(qweight, (qweight.shape[1] + 15) // 16 * 16)
    return qweight


def mm_int8(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``C[M, N] = A[M, K] @ B[K, N]`` in int32 (CK/__init__.py:717-719, eager quantization.py:785-800)."""
    if a.dtype != torch.int8 or b.dtype != torch.int8 or a.dim() != 2 or b.dim() != 2:
        raise ValueError("mm_int8 expects two 2-D int8 tensors")
    if a.shape[1] != b.shape[0]:
        raise ValueError(f"K mismatch: {a.shape[1]} vs {b.shape[0]}")
    dev = _require_gpu(a, b)
    m, n = a.shape[0], b.shape[1]
    out = torch.empty((m, n), dtype=torch.int32, device=dev)
    if m == 0 or n == 0:
        return out
    if a.shape[1] == 0:
        return out.zero_()
    k = a.shape[1]
    kp = (k + 15) // 16 * 16
    a2, w2 = _gemm_activation(a.contiguous(), kp), _gemm_weight(b, kp, transpose=True)
    k = kp
    with torch.cuda.device(dev):
        call("mxq_int8_gemm_i32", _p(a2), _p(w2), _p(out), m, n, k, n, *_gemm_ws(dev), _stream(dev))
    return out


def _weight_scale(weight_scale: torch.Tensor, n: int, dev) -> torch.Tensor:
    ws = torch.as_tensor(weight_scale).to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if ws.numel() not in (1, n):
        raise ValueError(
            f"INT8 weight scale must be scalar or per-output-channel, got {tuple(weight_scale.shape)} "
            f"for {n} output channels"
        )
    return ws


def _bias(bias: torch.Tensor | None, n: int, dtype: torch.dtype, dev):
    if bias is None:
        return None
    b = bias.to(device=dev, dtype=dtype).reshape(-1).contiguous()
    if b.numel() != n:
        raise ValueError(f"bias has {b.numel()} entries, expected {n}")
    return b


_M1_MAX_K = 16384


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    """Contiguous, with a 16-byte aligned start (vector loads)."""
    t = t.contiguous()
    return t.clone() if t.data_ptr() % 16 else t


def _m1_ok(k: int) -> bool:
    """Shapes the single-launch M = 1 kernels take (a K tail goes through the padded GEMM)."""
    return 0 < k <= _M1_MAX_K and k % 16 == 0


def int8_gemv_dequant(x_qdata: torch.Tensor, weight: torch.Tensor, x_scale: torch.Tensor,
                      weight_scale: torch.Tensor, bias: torch.Tensor | None,
                      out_dtype: torch.dtype) -> torch.Tensor:
    """Single-row INT8 GEMV with the dequant epilogue, [1, N] (CK/backends/cuda/__init__.py:
    1587-1610); the values of :func:`int8_linear_prequantized` for that row."""
    if x_qdata.numel() != weight.shape[1]:
        raise ValueError("x_qdata must hold one row of K values")
    return int8_linear_prequantized(x_qdata.reshape(1, -1), x_scale, weight, weight_scale, bias, out_dtype)


def int8_linear_prequantized(x_qdata: torch.Tensor, x_scale: torch.Tensor, weight: torch.Tensor,
                             weight_scale: torch.Tensor, bias: torch.Tensor | None = None,
                             out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """INT8 GEMM + dequant epilogue from an already quantized 2-D activation.

    CK/backends/cuda/__init__.py:1934-1957 (``int8_linear_prequantized``).
    """
    if x_qdata.dim() != 2 or x_qdata.dtype != torch.int8:
        raise ValueError("x_qdata must be a 2-D int8 tensor")
    if weight.dim() != 2 or weight.dtype != torch.int8:
        raise ValueError("weight must be a 2-D int8 tensor")
    if x_qdata.shape[1] != weight.shape[1]:
        raise ValueError(
            f"Input and weight inner dimensions must match, got {x_qdata.shape[1]} and {weight.shape[1]}"
        )
    dev = _require_gpu(x_qdata, weight)
    m, n = x_qdata.shape[0], weight.shape[0]
    code = _out_code(out_dtype)
    ws = _weight_scale(weight_scale, n, dev)
    b = _bias(bias, n, out_dtype, dev)
    xs = x_scale.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if xs.numel() != m:
        raise ValueError(f"x_scale has {xs.numel()} entries, expected {m}")
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    if m == 0 or n == 0:
        return out
    k = x_qdata.shape[1]
    if m == 1 and _m1_ok(k):
        with torch.cuda.device(dev):
            call("mxq_int8_gemv_dequant", _p(_aligned16(x_qdata)), _p(xs), _p(_gemm_weight(weight, k)), _p(ws),
                 ws.numel(), _p(b), _p(out), n, k, code, _stream(dev))
        return out
    q2, w2, k = _pad_k(x_qdata.contiguous(), weight)
    with torch.cuda.device(dev):
        call("mxq_int8_gemm_dequant", _p(q2), _p(w2), _p(xs), _p(ws), ws.numel(), _p(b), _p(out),
             m, n, k, n, code, *_gemm_ws(dev), _stream(dev))
    return out


def int8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                bias: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                convrot: bool = False, convrot_groupsize: int = 256,
                input_act: str | None = None) -> torch.Tensor:
    """Dynamically quantized INT8 linear (CK/__init__.py:722-764, eager quantization.py:971-1056).

    x [..., K] (bf16 / fp16 / fp32; [..., 2K] with ``input_act='swiglu'``); weight int8 [N, K];
    weight_scale scalar or [N] (any shape with that many elements); bias [N] or None. Returns
    [..., N] of ``out_dtype`` (default bf16). The activation and the ConvRot rotation are folded
    into the quantizer.
    """
    if out_dtype is None:
        out_dtype = torch.bfloat16
    act = _act_code(input_act)
    width = x.shape[-1] // _act_width(input_act)
    if width != weight.shape[-1] or x.shape[-1] % _act_width(input_act):
        raise ValueError(
            f"Input and weight inner dimensions must match, got {width} and {weight.shape[-1]}"
        )
    if convrot:
        _check_power_of_four(convrot_groupsize)
        if width % convrot_groupsize:
            raise ValueError(f"ConvRot group size {convrot_groupsize} does not divide input features {width}")
    dev = _require_gpu(x, weight)
    n = weight.shape[0]
    _weight_scale(weight_scale, n, dev)  # validate before launching anything
    if act and x.dtype == torch.float32:
        raise NotImplementedError(f"input_act={input_act!r} needs a bfloat16 or float16 input")
    lead = x.shape[:-1]
    if x.numel() == 0:
        return torch.empty((*lead, n), dtype=out_dtype, device=dev)
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[0] == 1 and x.dtype == torch.bfloat16 and _m1_ok(width) and n:
        # one token: the row quantizer, then the weight-streaming GEMV (int8_linear_m1's route)
        ws = _weight_scale(weight_scale, n, dev)
        b = _bias(bias, n, out_dtype, dev)
        out = torch.empty((1, n), dtype=out_dtype, device=dev)
        xq = torch.empty((1, width), dtype=torch.int8, device=dev)
        xs = torch.empty((1, 1), dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            call("mxq_int8_linear_m1", _p(_aligned16(x2)), _p(_gemm_weight(weight, width)), _p(ws), ws.numel(), _p(b),
                 _p(out), n, width, convrot_groupsize if convrot else 0, act, _out_code(out_dtype), _p(xq), _p(xs),
                 _stream(dev))
        return out.reshape(*lead, n)
    if convrot:
        q, s = quantize_int8_rowwise_convrot(x2, convrot_groupsize, input_act)
    else:
        q, s = quantize_int8_rowwise(x2, input_act=input_act)
    out = int8_linear_prequantized(q, s, weight, weight_scale, bias, out_dtype)
    return out.reshape(*lead, n)


# ---------------------------------------------------------------------------------------
# The INT8 FFN chain: fc1 -> tanh-GELU -> per-token re-quant -> fc2
# ---------------------------------------------------------------------------------------

# Widest row the single-pass GELU quantizer (mxq_quantize_int8_rowwise_gelu) holds in registers.
_GELU_QUANT_MAX_COLS = 32768


class FfnWorkspace:
    """Reusable device buffers of :func:`int8_ffn_gelu` for a given (M, K, hidden) shape."""

    def __init__(self, m: int, k: int, hidden: int, device):
        self.shape = (m, k, hidden)
        self.xq = torch.empty((m, k), dtype=torch.int8, device=device)
        self.xs = torch.empty((m, 1), dtype=torch.float32, device=device)
        self.h = torch.empty((m, hidden), dtype=torch.bfloat16, device=device)
        self.hmax = torch.empty((m,), dtype=torch.float32, device=device)
        self.hq = torch.empty((m, hidden), dtype=torch.int8, device=device)
        self.hs = torch.empty((m, 1), dtype=torch.float32, device=device)


def int8_ffn_gelu(x: torch.Tensor, fc1_weight: torch.Tensor, fc1_scale: torch.Tensor,
                  fc1_bias: torch.Tensor | None, fc2_weight: torch.Tensor, fc2_scale: torch.Tensor,
                  fc2_bias: torch.Tensor | None, workspace: FfnWorkspace | None = None,
                  return_hidden: bool = False):
    """``int8_linear(int8_linear(x, fc1), fc2, input_act='gelu_tanh')`` in four launches.

    The reference composes two ``int8_linear`` calls with the activation applied before the
    second quantizer (CK/backends/eager/quantization.py:971-1056,
    CK/backends/_activations.py:40-53). Here fc1 writes its bf16 output and one pass over it
    applies GELU, takes each row's absmax and quantizes (the GELU table in LDS, loaded once per
    CU, its lookups hidden under that pass's HBM traffic); with ``return_hidden`` the same pass
    writes the GELU output over fc1's. Hidden widths beyond that pass's register budget (32768)
    apply GELU and the row absmax in fc1's epilogue instead. Results are identical to the
    two-call composition. x bf16, fp16 or fp32 (the first quantizer reads it in its dtype; fc1's
    output and everything after are bf16, the composition's default out_dtype); bf16 out.
    """
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise NotImplementedError("int8_ffn_gelu takes a bfloat16, float16 or float32 input")
    dev = _require_gpu(x, fc1_weight, fc2_weight)
    k = x.shape[-1]
    hidden, n = fc1_weight.shape[0], fc2_weight.shape[0]
    if fc1_weight.shape[1] != k or fc2_weight.shape[1] != hidden:
        raise ValueError("FFN weight shapes do not chain")
    if k % 16 or hidden % 16:
        raise NotImplementedError("int8_ffn_gelu needs K and the hidden width to be multiples of 16")
    x2 = x.reshape(-1, k).contiguous()
    m = x2.shape[0]
    s1 = _weight_scale(fc1_scale, hidden, dev)
    s2 = _weight_scale(fc2_scale, n, dev)
    b1 = _bias(fc1_bias, hidden, torch.bfloat16, dev)
    b2 = _bias(fc2_bias, n, torch.bfloat16, dev)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    if m == 0:
        return out.reshape(*x.shape[:-1], n)
    reuse = workspace is not None and workspace.shape == (m, k, hidden) and workspace.xq.device == dev
    ws = workspace if reuse else FfnWorkspace(m, k, hidden, dev)
    w1 = _gemm_weight(fc1_weight, k)
    w2 = _gemm_weight(fc2_weight, hidden)
    st = _stream(dev)
    gws = _gemm_ws(dev)
    with torch.cuda.device(dev):
        call("mxq_quantize_int8_rowwise", _p(x2), _OUT_CODES[x.dtype], _p(ws.xq), _p(ws.xs), m, k,
             _lib.ACT_NONE, st)
        if hidden <= _GELU_QUANT_MAX_COLS:
            call("mxq_int8_gemm_dequant", _p(ws.xq), _p(w1), _p(ws.xs), _p(s1), s1.numel(), _p(b1),
                 _p(ws.h), m, hidden, k, hidden, _lib.DTYPE_BF16, *gws, st)
            call("mxq_quantize_int8_rowwise_gelu", _p(ws.h), _p(ws.h) if return_hidden else None,
                 _p(ws.hq), _p(ws.hs), m, hidden, st)
        else:
            call("mxq_fill_f32", _p(ws.hmax), 0.0, m, st)
            call("mxq_int8_gemm_dequant_gelu_absmax", _p(ws.xq), _p(w1), _p(ws.xs), _p(s1), s1.numel(),
                 _p(b1), _p(ws.h), _p(ws.hmax), m, hidden, k, hidden, *gws, st)
            call("mxq_quantize_int8_rowwise_absmax", _p(ws.h), _p(ws.hmax), _p(ws.hq), _p(ws.hs), m,
                 hidden, st)
        call("mxq_int8_gemm_dequant", _p(ws.hq), _p(w2), _p(ws.hs), _p(s2), s2.numel(), _p(b2),
             _p(out), m, n, hidden, n, _lib.DTYPE_BF16, *gws, st)
    out = out.reshape(*x.shape[:-1], n)
    return (out, ws.h.reshape(*x.shape[:-1], hidden)) if return_hidden else out


# ---------------------------------------------------------------------------------------
# fc2 with the gated residual update
# ---------------------------------------------------------------------------------------

_ROW_MAP_CACHE: dict[tuple, torch.Tensor] = {}


def _row_map(t: torch.Tensor, rows: int, count: int, dev, what: str, range_error: str) -> torch.Tensor:
    """An int32 [rows] row map on ``dev`` whose entries index a table of ``count`` rows. The range
    check reads the map back to the host, so it runs once per map tensor (and again only if the
    tensor is modified in place): later calls, including ones under graph capture, do not
    synchronise. The kernels clamp every index into the table, so even an unchecked map cannot
    read out of bounds."""
    m = t.to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
    if m.numel() != rows:
        raise ValueError(f"{what} has {m.numel()} entries, expected {rows}")
    key = (t._version, t.data_ptr(), rows, str(dev))
    checked = getattr(t, "_mxq_row_map_checked", None)
    if rows and not (checked is not None and checked[0] == key and checked[1] <= count):
        lo, hi = torch.aminmax(m)
        lo, hi = int(lo), int(hi)
        if lo < 0 or hi >= count:
            raise ValueError(range_error)
        try:
            t._mxq_row_map_checked = (key, hi + 1)
        except (AttributeError, RuntimeError):
            pass
    return m


def segment_row_map(length: int, segments, device) -> torch.Tensor:
    """int32 [length] modulation row of every token, from ordered ``(start, stop, row)``
    segments that partition ``[0, length)``; cached per device and segmentation
    (h3serve/native_engine/model/fused_mlp.py:34-55, same errors)."""
    normalized = tuple((int(a), int(b), int(r)) for a, b, r in segments)
    device = torch.device(device)
    key = (device.type, device.index, int(length), normalized)
    cached = _ROW_MAP_CACHE.get(key)
    if cached is not None:
        return cached
    host = torch.empty(length, dtype=torch.int32)
    previous = 0
    for start, stop, row in normalized:
        if start != previous or stop <= start:
            raise ValueError("modulation segments must be an ordered partition")
        host[start:stop] = row
        previous = stop
    if previous != length:
        raise ValueError("modulation segments do not cover the packed sequence")
    cached = host.to(device=device)
    if length:
        cached._mxq_row_map_checked = ((cached._version, cached.data_ptr(), int(length), str(device)),
                                       max(r for _, _, r in normalized) + 1)
    _ROW_MAP_CACHE[key] = cached
    return cached


def int8_linear_gated_residual_(residual: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                                weight_scale: torch.Tensor, bias: torch.Tensor | None,
                                gate: torch.Tensor, gate_rows, *, convrot: bool = False,
                                convrot_groupsize: int = 256, input_act: str | None = None) -> torch.Tensor:
    """``residual += int8_linear(x, ...) * gate[gate_rows]`` in place; returns ``residual``.

    The composition the reference runs after fc2 (fused_mlp.py:386-420 and
    layers.py:944-960): ``y = int8_linear(x, weight, weight_scale, bias, convrot=...,
    input_act=...)`` then ``residual[a:b].addcmul_(y[a:b], gate[row].to(bf16))`` per segment.
    Here the quantizer is one launch and the GEMM's epilogue applies the update, so ``y`` is
    never written. ``gate_rows`` is an int32 tensor [rows] or a sequence of segments.
    Bit-identical to the composition; bfloat16 residual.
    """
    if residual.dtype != torch.bfloat16:
        raise NotImplementedError("the gated residual update takes a bfloat16 residual")
    dev = _require_gpu(residual, x, weight)
    n = weight.shape[0]
    rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
    res2 = residual.view(-1, n) if residual.numel() else residual.reshape(0, n)
    if res2.shape[0] != rows or res2.shape[1] != n:
        raise ValueError(f"residual {tuple(residual.shape)} does not match the update [{rows}, {n}]")
    if res2.stride(1) != 1:
        raise ValueError("residual rows must be contiguous")
    if gate.dim() == 1:
        gate = gate.reshape(1, -1)
    if gate.dim() != 2 or gate.shape[1] != n:
        raise ValueError(f"gate must be [rows, {n}], got {tuple(gate.shape)}")
    g = gate.to(device=dev, dtype=torch.bfloat16).contiguous()
    if isinstance(gate_rows, torch.Tensor):
        gr = _row_map(gate_rows, rows, g.shape[0], dev, "gate_rows", "gate_rows index outside the gate")
    else:
        gr = segment_row_map(rows, gate_rows, dev)
        if rows and max(int(r) for _, _, r in gate_rows) >= g.shape[0]:
            raise ValueError("modulation segment row outside the gate")
    if rows == 0 or n == 0:
        return residual
    ws = _weight_scale(weight_scale, n, dev)
    b = _bias(bias, n, torch.bfloat16, dev)
    act = _act_code(input_act)
    width = x.shape[-1] // _act_width(input_act)
    if width != weight.shape[-1] or x.shape[-1] % _act_width(input_act):
        raise ValueError(f"Input and weight inner dimensions must match, got {width} and {weight.shape[-1]}")
    if act and x.dtype == torch.float32:
        raise NotImplementedError(f"input_act={input_act!r} needs a bfloat16 or float16 input")
    x2 = x.reshape(-1, x.shape[-1])
    if convrot:
        _check_power_of_four(convrot_groupsize)
        if width % convrot_groupsize:
            raise ValueError(f"ConvRot group size {convrot_groupsize} does not divide input features {width}")
        q, xs = quantize_int8_rowwise_convrot(x2, convrot_groupsize, input_act)
    else:
        q, xs = quantize_int8_rowwise(x2, input_act=input_act)
    q2, w2, k = _pad_k(q, weight)
    with torch.cuda.device(dev):
        call("mxq_int8_gemm_gated_residual", _p(q2), _p(w2), _p(xs), _p(ws), ws.numel(), _p(b), _p(res2),
             res2.stride(0), _p(g), g.stride(0), g.shape[0], _p(gr), rows, n, k, *_gemm_ws(dev), _stream(dev))
    return residual


def fused_down_gated_residual(hidden: torch.Tensor, residual: torch.Tensor, gate: torch.Tensor,
                              gate_rows: torch.Tensor, qweight: torch.Tensor, weight_scale: torch.Tensor,
                              bias: torch.Tensor | None) -> None:
    """fc2 of the SwiGLU MLP with the gated residual update, in place
    (h3serve/native_engine/model/fused_mlp.py:159-219): ``hidden`` is fc1's raw output
    [rows, 2 * inner] = [gate | up]; SwiGLU, the 256-column ConvRot rotation and the row
    quantizer run in one launch, the GEMM epilogue updates ``residual`` [rows, N]."""
    if weight_scale.numel() not in (1, qweight.shape[0]):
        raise ValueError("fc2 scale must be scalar or per output channel")
    int8_linear_gated_residual_(residual, hidden.reshape(-1, hidden.shape[-1]), qweight, weight_scale, bias,
                                gate, gate_rows, convrot=True, convrot_groupsize=256, input_act="swiglu")


# ---------------------------------------------------------------------------------------
# SwiGLU MLP: fc1 with the SwiGLU epilogue, ConvRot re-quant, fc2 with the gated residual
# ---------------------------------------------------------------------------------------

class PreparedSwiGLUFc1:
    """An INT8 SwiGLU fc1 ([gate | up] rows, [2F, K]) with its rows reordered for the SwiGLU
    epilogue: per block of 32 rows, 16 gate rows then the matching 16 up rows. The weight
    scale and bias follow the same order. Built once per layer (``prepare_swiglu_fc1``)."""

    def __init__(self, qweight: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None, inner: int):
        self.qweight, self.scale, self.bias, self.inner = qweight, scale, bias, inner


def _swiglu_order(n2: int, device) -> torch.Tensor:
    f = n2 // 2
    blk = torch.arange(f // 16, device=device).reshape(-1, 1) * 16
    r = torch.arange(16, device=device).reshape(1, -1)
    return torch.cat([blk + r, f + blk + r], dim=1).reshape(-1)


def prepare_swiglu_fc1(qweight: torch.Tensor, weight_scale: torch.Tensor,
                       bias: torch.Tensor | None = None) -> PreparedSwiGLUFc1:
    """Reorder a SwiGLU fc1 (rows [gate | up], h3serve/native_engine/model/layers.py SwiGLUMLP)
    for ``int8_swiglu_fc1``; the values are unchanged."""
    if qweight.dim() != 2 or qweight.dtype != torch.int8:
        raise ValueError("fc1 weight must be a 2-D int8 tensor")
    n2 = qweight.shape[0]
    if n2 % 32:
        raise NotImplementedError("the SwiGLU epilogue needs 2 x inner to be a multiple of 32")
    dev = qweight.device
    order = _swiglu_order(n2, dev)
    ws = _weight_scale(weight_scale, n2, dev)
    ws = ws if ws.numel() == 1 else ws[order].contiguous()
    b = None if bias is None else bias.to(device=dev, dtype=torch.bfloat16).reshape(-1)[order].contiguous()
    return PreparedSwiGLUFc1(qweight[order].contiguous(), ws, b, n2 // 2)


def int8_swiglu_fc1(x_qdata: torch.Tensor, x_scale: torch.Tensor, fc1: PreparedSwiGLUFc1,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """``swiglu(int8_linear_prequantized(x, fc1))`` as bf16 [M, inner] in one GEMM launch
    (the SwiGLU half of fc2's ``input_act="swiglu"``, CK/backends/_activations.py:50-52)."""
    if x_qdata.dim() != 2 or x_qdata.dtype != torch.int8:
        raise ValueError("x_qdata must be a 2-D int8 tensor")
    if x_qdata.shape[1] != fc1.qweight.shape[1]:
        raise ValueError("Input and weight inner dimensions must match")
    dev = _require_gpu(x_qdata, fc1.qweight)
    m, n2 = x_qdata.shape[0], fc1.qweight.shape[0]
    xs = x_scale.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if xs.numel() != m:
        raise ValueError(f"x_scale has {xs.numel()} entries, expected {m}")
    if out is None:
        h = torch.empty((m, n2 // 2), dtype=torch.bfloat16, device=dev)
    else:
        h = out
        if h.dtype != torch.bfloat16 or h.device != dev or h.dim() != 2 or tuple(h.shape) != (m, n2 // 2):
            raise ValueError(f"out must be a bfloat16 [{m}, {n2 // 2}] tensor on {dev}")
        if h.stride(1) != 1 or h.stride(0) < n2 // 2:
            raise ValueError("out rows must be contiguous and must not overlap")
    if m == 0:
        return h
    q2, w2, k = _pad_k(x_qdata.contiguous(), fc1.qweight)
    with torch.cuda.device(dev):
        call("mxq_int8_gemm_dequant_swiglu", _p(q2), _p(w2), _p(xs), _p(fc1.scale), fc1.scale.numel(),
             _p(fc1.bias), _p(h), m, n2, k, h.stride(0), *_gemm_ws(dev), _stream(dev))
    return h


def swiglu_mlp_gated_residual_(residual: torch.Tensor, x_qdata: torch.Tensor, x_scale: torch.Tensor,
                               fc1: PreparedSwiGLUFc1, fc2_qweight: torch.Tensor, fc2_scale: torch.Tensor,
                               fc2_bias: torch.Tensor | None, gate: torch.Tensor, segments,
                               convrot_groupsize: int = 256) -> torch.Tensor:
    """The H3 MLP after its quantized input, in place on ``residual``: fc1 (+ SwiGLU in the
    epilogue) -> ConvRot re-quant -> fc2 + gated residual. Bit-identical to the reference's
    default route (fused_mlp.py:386-420: ``raw = fc1(hidden)``, ``int8_linear(raw, fc2, convrot=True,
    input_act="swiglu")``, then ``addcmul_`` per segment)."""
    h = int8_swiglu_fc1(x_qdata, x_scale, fc1)
    return int8_linear_gated_residual_(residual, h, fc2_qweight, fc2_scale, fc2_bias, gate, segments,
                                       convrot=True, convrot_groupsize=convrot_groupsize)


def h3_mlp_(residual: torch.Tensor, norm, shift: torch.Tensor, scale: torch.Tensor, gate: torch.Tensor,
            segments, fc1: PreparedSwiGLUFc1, fc2_qweight: torch.Tensor, fc2_scale: torch.Tensor,
            fc2_bias: torch.Tensor | None, convrot_groupsize: int = 256) -> torch.Tensor:
    """The H3 block's MLP half in four launches, in place on ``residual`` (layers.py:1138-1160:
    ``rms_adaln`` -> ``try_fused_gated_mlp``): RMS adaLN + ConvRot quant, fc1 + SwiGLU, ConvRot
    re-quant, fc2 + gated residual."""
    q, s = rms_adaln_quantize_int8(residual, norm, shift, scale, segments, convrot_groupsize=convrot_groupsize)
    return swiglu_mlp_gated_residual_(residual, q, s, fc1, fc2_qweight, fc2_scale, fc2_bias, gate, segments,
                                      convrot_groupsize)


# ---------------------------------------------------------------------------------------
# W4A8
# ---------------------------------------------------------------------------------------

def _srel_code(s_rel: torch.Tensor) -> tuple[torch.Tensor, int]:
    if s_rel.dtype == torch.float8_e4m3fn:
        return s_rel.contiguous().view(torch.uint8), _lib.DTYPE_E4M3
    return s_rel.to(torch.float32).contiguous(), _lib.DTYPE_F32


def dequantize_int4_grouped_to_int8(qdata: torch.Tensor, s_rel: torch.Tensor,
                                    codebook: torch.Tensor | None, group_size: int) -> torch.Tensor:
    """Decode packed int4 to the int8 grid (CK/backends/eager/w4a8_int8.py:344-363)."""
    if qdata.dim() != 2 or qdata.dtype != torch.int8:
        raise ValueError("packed weight must be a 2D int8 tensor")
    dev = _require_gpu(qdata)
    n, kh = qdata.shape
    k = kh * 2
    if group_size <= 0 or k % group_size:
        raise ValueError(f"K={k} must be divisible by group_size={group_size}")
    if tuple(s_rel.shape) != (n, k // group_size):
        raise ValueError(f"s_rel must have shape {(n, k // group_size)}, got {tuple(s_rel.shape)}")
    if codebook is not None and codebook.numel() != 16:
        raise ValueError(f"codebook must have 16 entries, got {codebook.numel()}")
    sr, code = _srel_code(s_rel.to(dev))
    cb = None if codebook is None else codebook.to(device=dev, dtype=torch.float32).contiguous()
    out = torch.empty((n, k), dtype=torch.int8, device=dev)
    with torch.cuda.device(dev):
        call("mxq_dequant_int4_grouped_to_int8", _p(qdata.contiguous()), _p(sr), code, _p(cb), _p(out),
             n, k, group_size, _stream(dev))
    return out


# The decoded weight chunk stays in the 256 MB last-level cache between the decode and the GEMM
# that reads it; the reference bounds its chunk to 4096 columns to save memory on 8 GB boards.
W4A8_DECODE_BYTES = 256 << 20


def w4a8_decode_chunk(n: int, k: int) -> int:
    """Columns per decode chunk of the reference-format W4A8 linear: all ``n`` when the decoded
    ``[n, k]`` int8 weight fits ``W4A8_DECODE_BYTES``, else as many as fit (at least 4096, the
    reference's chunk). Fewer chunks mean fewer partly filled last rounds of GEMM tiles (the H3
    QKV projection at 720p: 7.93 ms per step in six 3584-column chunks, 7.73 ms in one); the
    outputs do not depend on the chunking."""
    return min(n, max(4096, W4A8_DECODE_BYTES // max(k, 1)))


def w4a8_int8_linear(x: torch.Tensor, qdata: torch.Tensor, s_rel: torch.Tensor, s_channel: torch.Tensor,
                     codebook: torch.Tensor | None = None, correction: torch.Tensor | None = None,
                     bias: torch.Tensor | None = None, group_size: int = 16,
                     convrot_groupsize: int = 256, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Reference-format W4A8 linear (CK/tensor/w4a8_int8.py:89-115, eager w4a8_int8.py:457-508):
    the int4 codes are decoded to the int8 grid chunk by chunk and multiplied with the ConvRot-
    rotated, per-token quantized activations (int8_linear with convrot=True).
    ``convrot_groupsize=0`` skips the rotation (for unrotated weights). A ``correction`` [K/G, N]
    (asymmetric int4 weights) is added as the reference's CUDA backend does
    (CK/backends/cuda/__init__.py:2294-2297): ``out += o(o(group sums of xq) * o(xs)) @ correction``
    in the output dtype, the product by a library GEMM (``addmm_``). The reference's eager backend
    instead runs a dense floating-point linear on the dequantized weight.
    """
    if convrot_groupsize:
        _check_power_of_four(convrot_groupsize)
    if qdata.dim() != 2 or qdata.dtype != torch.int8:
        raise ValueError("packed weight must be a 2D int8 tensor")
    n, kh = qdata.shape
    k = kh * 2
    if x.shape[-1] != k:
        raise ValueError(f"Input K={x.shape[-1]} does not match qdata K={k}")
    if (group_size < 4 or k % 16 != 0 or k % group_size != 0
            or (16 % group_size != 0 and group_size % 16 != 0)):
        raise ValueError(
            f"K={k} must be divisible by 16, group_size={group_size}; group_size must be >=4 "
            "and divide 16 or be a multiple of 16"
        )
    if tuple(s_rel.shape) != (n, k // group_size):
        raise ValueError(f"s_rel must have shape {(n, k // group_size)}, got {tuple(s_rel.shape)}")
    if tuple(s_channel.shape) != (n,):
        raise ValueError(f"s_channel must have shape {(n,)}, got {tuple(s_channel.shape)}")
    if codebook is not None and tuple(codebook.shape) != (16,):
        raise ValueError(f"codebook must have shape (16,), got {tuple(codebook.shape)}")
    if correction is not None and tuple(correction.shape) != (k // group_size, n):
        raise ValueError(f"correction must have shape {(k // group_size, n)}, got {tuple(correction.shape)}")
    dev = _require_gpu(x, qdata)
    code = _out_code(out_dtype)
    lead = x.shape[:-1]
    if convrot_groupsize:
        if k % convrot_groupsize:
            raise ValueError(f"ConvRot group size {convrot_groupsize} does not divide input features {k}")
        xq, xs = quantize_int8_rowwise_convrot(x.reshape(-1, k), convrot_groupsize)
    else:
        xq, xs = quantize_int8_rowwise(x.reshape(-1, k))
    m = xq.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    if m == 0:
        return out.reshape(*lead, n)
    sr, scode = _srel_code(s_rel.to(dev))
    cb = None if codebook is None else codebook.to(device=dev, dtype=torch.float32).contiguous()
    sch = s_channel.to(device=dev, dtype=torch.float32).contiguous()
    b = _bias(bias, n, out_dtype, dev)
    chunk = w4a8_decode_chunk(n, k)
    work = torch.empty((chunk, k), dtype=torch.int8, device=dev)
    with torch.cuda.device(dev):
        call("mxq_w4a8_codebook_gemm", _p(xq), _p(qdata.contiguous()), _p(sr), scode, _p(cb), _p(sch),
             _p(xs), _p(b), _p(work), _p(out), m, n, k, group_size, chunk, code, *_gemm_ws(dev), _stream(dev))
        if correction is not None:
            sx = torch.empty((m, k // group_size), dtype=out_dtype, device=dev)
            call("mxq_int8_group_sums", _p(xq), _p(xs), _p(sx), m, k, group_size, code, _stream(dev))
            out.addmm_(sx, correction.to(device=dev, dtype=out_dtype))
    return out.reshape(*lead, n)


class PreparedW4A8Grouped:
    """Group-128 int4 weights in the GEMM's load layout (``prepare_w4a8_grouped``): the same
    ``[N, K/2]`` bytes and codes, each 32-bit word's nibbles reordered so the kernel unpacks them
    with one shift and two masks. Results are identical to the checkpoint layout's."""

    def __init__(self, qdata: torch.Tensor):
        self.qdata = qdata
        self.shape = qdata.shape


def prepare_w4a8_grouped(qdata: torch.Tensor) -> PreparedW4A8Grouped:
    """Re-lay packed offset-8 int4 weights ``[N, K/2]`` (CK/backends/eager/w4a8_int8.py:200-202)
    for ``w4a8_grouped_linear`` at group size 128; done once per layer when weights load."""
    if qdata.dim() != 2 or qdata.dtype != torch.int8:
        raise ValueError("packed weight must be a 2D int8 tensor")
    n, kh = qdata.shape
    if (2 * kh) % 8:
        raise ValueError(f"K={2 * kh} must be a multiple of 8")
    dev = _require_gpu(qdata)
    src = qdata.contiguous()
    out = torch.empty_like(src)
    with torch.cuda.device(dev):
        call("mxq_w4a8_prepare_grouped", _p(src), _p(out), n, 2 * kh, _stream(dev))
    return PreparedW4A8Grouped(out)


def w4a8_grouped_linear(x: torch.Tensor, qdata: torch.Tensor | PreparedW4A8Grouped, group_scale: torch.Tensor,
                        group_size: int = 128, bias: torch.Tensor | None = None,
                        out_dtype: torch.dtype = torch.bfloat16,
                        x_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Group-scaled int4 weights x per-token int8 activations.

    ``x`` is bf16/fp16/fp32 ``[..., K]`` (quantized per token here) or int8 ``[M, K]`` with its
    ``x_scale``; ``qdata`` int8 ``[N, K/2]`` packs offset-8 codes two per byte, even k in the
    low nibble (CK/backends/eager/w4a8_int8.py:200-202), or is that tensor after
    ``prepare_w4a8_grouped`` (group 128 only); ``group_scale`` fp16 ``[K/G, N]``.
    y = out(xs[m] * sum_g fp32(scale[g, n]) * P_g[m, n]), P_g the exact int32 partial of group g.
    """
    prepared = isinstance(qdata, PreparedW4A8Grouped)
    if prepared:
        qdata = qdata.qdata
    if qdata.dim() != 2 or qdata.dtype != torch.int8:
        raise ValueError("packed weight must be a 2D int8 tensor")
    n, kh = qdata.shape
    k = kh * 2
    if x.shape[-1] != k:
        raise ValueError(f"Input K={x.shape[-1]} does not match qdata K={k}")
    if group_size <= 0 or k % group_size:
        raise ValueError(f"K={k} must be divisible by group_size={group_size}")
    if tuple(group_scale.shape) != (k // group_size, n):
        raise ValueError(f"group_scale must have shape {(k // group_size, n)}, got {tuple(group_scale.shape)}")
    dev = _require_gpu(x, qdata, group_scale)
    code = _out_code(out_dtype)
    if x.dtype == torch.int8:
        if x_scale is None:
            raise ValueError("an int8 input needs x_scale")
        xq = x.reshape(-1, k).contiguous()
        xs = x_scale.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        if xs.numel() != xq.shape[0]:
            raise ValueError(f"x_scale has {xs.numel()} entries, expected {xq.shape[0]}")
    else:
        xq, xs = quantize_int8_rowwise(x.reshape(-1, k))
    lead = x.shape[:-1]
    m = xq.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=dev)
    if m == 0:
        return out.reshape(*lead, n)
    gs = group_scale.to(device=dev, dtype=torch.float16).contiguous()
    b = _bias(bias, n, out_dtype, dev)
    entry = "mxq_w4a8_gemm_grouped_prepared" if prepared else "mxq_w4a8_gemm_grouped"
    with torch.cuda.device(dev):
        call(entry, _p(xq), _p(xs), _p(qdata.contiguous()), _p(gs), _p(b), _p(out),
             m, n, k, group_size, n, code, _stream(dev))
    return out.reshape(*lead, n)


# ---------------------------------------------------------------------------------------
# Offline W4A8 weight preparation (the reference's quantize_w4a8_int8_weight)
# ---------------------------------------------------------------------------------------

# Lloyd-Max levels for a group-normalised Gaussian (CK/backends/eager/w4a8_int8.py:13-16): the
# codes of the default storage index this table, so the values are the reference's.
_W4A8_FIXED_LUT = (
    -0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210, -0.050720,
    0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876, 0.980671,
)
_W4A8_GATE_KURTOSIS = -0.1
_W4A8_KURTOSIS_SAMPLE = 1 << 19
_W4A8_CODEBOOK_SAMPLE_ELEMS = 1 << 22
_W4_MODES = {"codebook": 0, "symmetric": 1, "asymmetric": 2, "rotate": 3}


def _validate_w4a8_weight(weight: torch.Tensor, group_size: int, convrot_groupsize: int) -> None:
    """CK/backends/eager/w4a8_int8.py:99-119 (same condition and message)."""
    if weight.dim() != 2:
        raise ValueError(f"W4A8 weight must be 2D, got shape {tuple(weight.shape)}")
    k = weight.shape[1]
    if (k % 16 != 0 or k % group_size != 0 or k % convrot_groupsize != 0 or group_size < 4
            or (16 % group_size != 0 and group_size % 16 != 0)):
        raise ValueError(
            f"K={k} must be divisible by 16, group_size={group_size}, and "
            f"convrot_groupsize={convrot_groupsize}; group_size must be >=4 "
            f"and divide 16 or be a multiple of 16"
        )


def _w4_kernel(weight: torch.Tensor, mode: str, group_size: int, convrot_groupsize: int,
               codebook: torch.Tensor | None = None, e4m3: bool = True, rotated: torch.Tensor | None = None):
    dev = weight.device
    n, k = weight.shape
    code = _OUT_CODES[weight.dtype]
    packed = s_rel = s_ch = corr = None
    if mode != "rotate":
        packed = torch.empty((n, k // 2), dtype=torch.int8, device=dev)
        s_rel = torch.empty((n, k // group_size), dtype=torch.uint8 if e4m3 else torch.float32, device=dev)
        s_ch = torch.empty((n,), dtype=torch.float32, device=dev)
        if mode == "asymmetric":
            corr = torch.empty((k // group_size, n), dtype=weight.dtype, device=dev)
    with torch.cuda.device(dev):
        call("mxq_w4a8_quantize_weight", _p(weight), code, n, k, group_size, convrot_groupsize, _W4_MODES[mode],
             _p(codebook), _lib.DTYPE_E4M3 if e4m3 else _lib.DTYPE_F32, _p(packed), _p(s_rel), _p(s_ch), _p(corr),
             _p(rotated), _stream(dev))
    if s_rel is not None and e4m3:
        s_rel = s_rel.view(torch.float8_e4m3fn)
    return packed, s_rel, s_ch, corr


def rotate_int8_convrot_weight(weight: torch.Tensor, group_size: int) -> torch.Tensor:
    """ConvRot rotation of weight rows, ``W_grouped @ H^T`` per group (CK/backends/eager/
    quantization.py:909-912), as the exact product rounded once to the weight's dtype (bf16 or
    fp32). H is symmetric and orthogonal, so the rotation is its own inverse."""
    _check_power_of_four(group_size)
    if weight.dim() != 2:
        raise ValueError("weight must be 2D [out_features, in_features]")
    if weight.shape[1] % group_size:
        raise ValueError(f"in_features {weight.shape[1]} not divisible by group_size {group_size}")
    _require_gpu(weight)
    if weight.dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError("the weight rotation takes bfloat16 or float32 weights")
    w = weight.contiguous()
    out = torch.empty_like(w)
    if w.numel():
        _w4_kernel(w, "rotate", 16, group_size, rotated=out)
    return out


def _w4a8_codebook_for(normalized: torch.Tensor) -> torch.Tensor:
    """The fixed table unless the group-normalised rotated weights are heavy-tailed
    (CK/backends/eager/w4a8_int8.py:24-32): the excess kurtosis of a seeded sample, drawn with
    torch's generator on the tensor's device as the reference draws it."""
    x = normalized.detach().flatten()
    if x.numel() > _W4A8_KURTOSIS_SAMPLE:
        gen = torch.Generator(device=x.device).manual_seed(0)
        x = x[torch.randint(0, x.numel(), (_W4A8_KURTOSIS_SAMPLE,), device=x.device, generator=gen)]
    x = x.float()
    excess = ((x - x.mean()) / (x.std() + 1e-9)).pow(4).mean() - 3.0
    if excess.item() <= _W4A8_GATE_KURTOSIS:
        return torch.tensor(_W4A8_FIXED_LUT, device=normalized.device, dtype=torch.float32)
    return _w4a8_fit_codebook(normalized)


def _w4a8_fit_codebook(normalized: torch.Tensor, levels: int = 16, iterations: int = 25,
                       sample_size: int = 300000) -> torch.Tensor:
    """Lloyd-Max fit of the 16 levels on a seeded sample (CK/backends/eager/w4a8_int8.py:66-97):
    quantile start, 25 nearest-level / mean updates."""
    samples = normalized.flatten()
    if samples.numel() > sample_size:
        gen = torch.Generator(device=samples.device).manual_seed(0)
        samples = samples[torch.randint(0, samples.numel(), (sample_size,), device=samples.device, generator=gen)]
    samples = samples.float()
    cb = torch.quantile(samples, torch.linspace(0, 1, levels, device=samples.device))
    for _ in range(iterations):
        assign = (samples.unsqueeze(-1) - cb).abs().argmin(-1)
        upd = cb.clone()
        for i in range(levels):
            sel = assign == i
            if sel.any():
                upd[i] = samples[sel].mean()
        cb = upd
    return cb.contiguous()


def _w4a8_decide_codebook(weight: torch.Tensor, group_size: int, convrot_groupsize: int) -> torch.Tensor:
    """One table for the whole tensor from evenly strided rows (CK/backends/eager/w4a8_int8.py:
    221-240), the rows rotated by the HIP kernel."""
    n, k = weight.shape
    max_rows = max(1, _W4A8_CODEBOOK_SAMPLE_ELEMS // max(k, 1))
    if n > max_rows:
        idx = torch.linspace(0, n - 1, max_rows, device=weight.device).long()
        sample = weight.index_select(0, idx).contiguous()
    else:
        sample = weight
    rotated = rotate_int8_convrot_weight(sample, convrot_groupsize)
    grouped = rotated.float().view(sample.shape[0], k // group_size, group_size)
    normalized = grouped / grouped.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
    return _w4a8_codebook_for(normalized)


def quantize_w4a8_int8_weight(weight: torch.Tensor, group_size: int = 16, convrot_groupsize: int = 256,
                              symmetric: bool = True, scale_dtype: torch.dtype = torch.float8_e4m3fn,
                              codebook: bool = True, codebook_tensor: torch.Tensor | None = None):
    """Rotate and store a floating weight ``[N, K]`` in the grouped W4A8 format
    (CK/tensor/w4a8_int8.py:29-63, eager backend CK/backends/eager/w4a8_int8.py:122-209,
    243-341): returns ``(qdata int8 [N, K/2], s_rel [N, K/G] float8_e4m3fn or float32,
    s_channel float32 [N], correction [K/G, N] or None, codebook float32 [16] or None)`` with the
    reference's meaning, ready for ``w4a8_int8_linear`` / ``ConvRotW4A8Linear``.

    The rotation, the group and channel scales, the codes and the packing run in one HIP launch
    (one workgroup per row); the codebook choice (a kurtosis test on a seeded sample and, for
    heavy-tailed weights, a 16-level fit) is made once per tensor as in the reference, or taken
    from ``codebook_tensor``. bf16 or fp32 weights on the GPU, K <= 16384."""
    if scale_dtype not in (torch.float32, torch.float8_e4m3fn):
        raise ValueError(f"scale_dtype must be float32 or float8_e4m3fn, got {scale_dtype}")
    _validate_w4a8_weight(weight, group_size, convrot_groupsize)
    dev = _require_gpu(weight)
    if weight.dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError("W4A8 preparation takes bfloat16 or float32 weights")
    w = weight.contiguous()
    table = None
    if symmetric and codebook:
        table = (codebook_tensor.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
                 if codebook_tensor is not None else _w4a8_decide_codebook(w, group_size, convrot_groupsize))
        if table.numel() != 16:
            raise ValueError(f"codebook must have 16 entries, got {table.numel()}")
        mode = "codebook"
    else:
        mode = "symmetric" if symmetric else "asymmetric"
    packed, s_rel, s_ch, corr = _w4_kernel(w, mode, group_size, convrot_groupsize, table,
                                           e4m3=scale_dtype == torch.float8_e4m3fn)
    return packed, s_rel, s_ch, corr, table


def dequantize_w4a8_int8_weight(qdata: torch.Tensor, s_rel: torch.Tensor, s_channel: torch.Tensor,
                                codebook: torch.Tensor | None = None, correction: torch.Tensor | None = None,
                                group_size: int = 16, convrot_groupsize: int = 256,
                                output_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """The physical ``[N, K]`` weight of W4A8 storage (CK/backends/eager/w4a8_int8.py:404-437):
    the int8 grid (``dequantize_int4_grouped_to_int8``), times ``s_channel`` plus the correction
    in float32, rounded to ``output_dtype``, rotated back to the original basis."""
    _check_power_of_four(convrot_groupsize)
    w8 = dequantize_int4_grouped_to_int8(qdata, s_rel, codebook, group_size)
    n, k = w8.shape
    groups = k // group_size
    if tuple(s_channel.shape) != (n,):
        raise ValueError(f"s_channel must have shape {(n,)}, got {tuple(s_channel.shape)}")
    if correction is not None and tuple(correction.shape) != (groups, n):
        raise ValueError(f"correction must have shape {(groups, n)}, got {tuple(correction.shape)}")
    v = w8.float().view(n, groups, group_size) * s_channel.to(device=w8.device, dtype=torch.float32).view(n, 1, 1)
    if correction is not None:
        v = v + correction.to(w8.device).t().unsqueeze(-1).float()
    return rotate_int8_convrot_weight(v.view(n, k).to(output_dtype), convrot_groupsize)
