"""Quantized-linear modules with the reference's module contract.

Mirrors h3serve/native_engine/model/quantization.py (the drop-in boundary): the kernel
callable types (19-37), the checkpoint spec decoders (98-139, 153-187), ``ConvRotInt8Linear``
(210-413) and ``ConvRotW4A8Linear`` (416-586) keep their constructor arguments, buffer names,
``from_state_dict`` keys, ``forward`` / ``forward_output_slice`` signatures and ValueError /
RuntimeError behaviour. The injected kernels default to this package's HIP path. The
reference's CPU fallback (an fp32 ``F.linear`` on dequantized weights) is not provided:
a CPU input raises RuntimeError.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from typing import Callable, Mapping

import torch
import torch.nn as nn

from . import ops

Int8Kernel = Callable[
    [torch.Tensor, torch.Tensor, torch.Tensor, "torch.Tensor | None", int], torch.Tensor
]
W4A8Kernel = Callable[..., torch.Tensor]


def int8_kernel(value, qweight, scale, bias, convrot_group_size: int) -> torch.Tensor:
    """``Int8Kernel`` bound to :func:`mx_qlinear.int8_linear` (reference binding: quantization.py:40-61)."""
    return ops.int8_linear(value, qweight, scale, bias, value.dtype,
                           convrot=bool(convrot_group_size), convrot_groupsize=convrot_group_size or 256)


def w4a8_kernel(value, qdata, s_rel, s_channel, codebook, correction, bias, group_size: int,
                convrot_group_size: int, output_dtype: torch.dtype) -> torch.Tensor:
    """``W4A8Kernel`` bound to :func:`mx_qlinear.w4a8_int8_linear` (reference: quantization.py:64-95)."""
    return ops.w4a8_int8_linear(value, qdata, s_rel, s_channel, codebook=codebook,
                                correction=correction, bias=bias, group_size=group_size,
                                convrot_groupsize=convrot_group_size, out_dtype=output_dtype)


def _is_power_of_four(size: int) -> bool:
    return size >= 4 and size & (size - 1) == 0 and (size.bit_length() - 1) % 2 == 0


@dataclass(frozen=True)
class ComfyQuantSpec:
    """The ``{prefix}.comfy_quant`` JSON record of an INT8 layer (quantization.py:98-139)."""

    format: str
    convrot: bool = False
    convrot_groupsize: int = 256

    @classmethod
    def decode(cls, raw) -> "ComfyQuantSpec":
        if isinstance(raw, torch.Tensor):
            payload = bytes(raw.detach().cpu().to(torch.uint8).tolist())
        elif isinstance(raw, (bytes, bytearray, memoryview)):
            payload = bytes(raw)
        elif isinstance(raw, str):
            payload = raw.encode("utf-8")
        elif isinstance(raw, Mapping):
            return cls._from_mapping(raw)
        else:
            raise TypeError(f"unsupported comfy_quant payload: {type(raw).__name__}")
        return cls._from_mapping(json.loads(payload.decode("utf-8")))

    @classmethod
    def _from_mapping(cls, data: Mapping) -> "ComfyQuantSpec":
        params = data.get("params", {})
        params = params if isinstance(params, Mapping) else {}
        return cls(
            format=str(data.get("format", "")),
            convrot=bool(data.get("convrot", params.get("convrot", False))),
            convrot_groupsize=int(data.get("convrot_groupsize", params.get("convrot_groupsize", 256))),
        )

    def validate_supported(self) -> None:
        if self.format != "int8_tensorwise":
            raise ValueError(f"native core currently supports int8_tensorwise, got {self.format!r}")
        if self.convrot and not _is_power_of_four(self.convrot_groupsize):
            raise ValueError("ConvRot group size must be a power of four")


@dataclass(frozen=True)
class W4A8QuantSpec:
    """Layout record of a W4A8 layer (quantization.py:153-187)."""

    format: str = "asym_w4a8_int8"
    group_size: int = 16
    convrot: bool = True
    convrot_groupsize: int = 256

    @classmethod
    def from_mapping(cls, data: Mapping) -> "W4A8QuantSpec":
        return cls(
            format=str(data.get("format", "")),
            group_size=int(data.get("group_size", 16)),
            convrot=bool(data.get("convrot", True)),
            convrot_groupsize=int(data.get("convrot_groupsize", 256)),
        )

    def validate_supported(self) -> None:
        if self.format != "asym_w4a8_int8":
            raise ValueError(f"native core currently supports asym_w4a8_int8, got {self.format!r}")
        if self.group_size < 4 or (16 % self.group_size != 0 and self.group_size % 16 != 0):
            raise ValueError("W4A8 group size must be >=4 and divide 16 or be a multiple of 16")
        if not self.convrot:
            raise ValueError("the H3 W4A8 checkpoint requires ConvRot")
        if not _is_power_of_four(self.convrot_groupsize):
            raise ValueError("ConvRot group size must be a power of four")


@dataclass(frozen=True)
class PreparedConvRotInt8Input:
    """One quantized activation shared by later output-slice GEMMs (quantization.py:142-150)."""

    qdata: torch.Tensor
    scale: torch.Tensor
    rows: int
    width: int
    dtype: torch.dtype


def _gpu_only(value: torch.Tensor) -> None:
    if not value.is_cuda:
        raise RuntimeError("mx_qlinear modules run on the GPU only (no CPU fallback)")


class ConvRotInt8Linear(nn.Module):
    """W8A8 linear over a stored int8 ``[out, in]`` weight and fp32 ``[out, 1]`` / scalar scale."""

    def __init__(self, qweight: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None = None, *,
                 spec: ComfyQuantSpec, kernel: Int8Kernel | None = None,
                 output_dtype: torch.dtype | None = None) -> None:
        super().__init__()
        spec.validate_supported()
        if qweight.ndim != 2 or qweight.dtype != torch.int8:
            raise ValueError("qweight must be a rank-two int8 tensor")
        if scale.numel() not in (1, qweight.shape[0]):
            raise ValueError("INT8 scale must be scalar or one value per output row")
        if bias is not None and bias.numel() != qweight.shape[0]:
            raise ValueError("bias does not match qweight output rows")
        if spec.convrot and qweight.shape[1] % spec.convrot_groupsize:
            raise ValueError("qweight input width is not divisible by ConvRot group size")
        self.register_buffer("qweight", ops.prepare_int8_weight(qweight))
        self.register_buffer("scale", scale)
        self.register_buffer("bias", bias)
        self.spec = spec
        self.kernel = kernel if kernel is not None else int8_kernel
        self.output_dtype = output_dtype

    @classmethod
    def from_state_dict(cls, state: Mapping[str, torch.Tensor], prefix: str, *,
                        kernel: Int8Kernel | None = None,
                        output_dtype: torch.dtype | None = None) -> "ConvRotInt8Linear":
        try:
            spec = ComfyQuantSpec.decode(state[f"{prefix}.comfy_quant"])
            qweight = state[f"{prefix}.weight"]
            scale = state[f"{prefix}.weight_scale"]
        except KeyError as error:
            raise KeyError(f"incomplete quantized layer {prefix!r}: missing {error.args[0]!r}") from error
        return cls(qweight, scale, state.get(f"{prefix}.bias"), spec=spec, kernel=kernel,
                   output_dtype=output_dtype)

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)
        # the GEMM form of a weight that needs padding or realignment is rebuilt from the loaded
        # contents (load_state_dict may also have written through .data, which it cannot see)
        ops.prepare_int8_weight(self.qweight)

    @property
    def in_features(self) -> int:
        return int(self.qweight.shape[1])

    @property
    def out_features(self) -> int:
        return int(self.qweight.shape[0])

    def _forward_parameters(self, value, qweight, scale, bias) -> torch.Tensor:
        if value.shape[-1] != self.in_features:
            raise ValueError("input width does not match quantized weight")
        _gpu_only(value)
        out = self.kernel(value, qweight, scale, bias,
                          self.spec.convrot_groupsize if self.spec.convrot else 0)
        want = self.output_dtype or value.dtype
        return out if out.dtype == want else out.to(want)

    def forward(self, value: torch.Tensor) -> torch.Tensor:
        return self._forward_parameters(value, self.qweight, self.scale, self.bias)

    def _slice_params(self, start: int, stop: int):
        scale = self.scale if self.scale.numel() == 1 else self.scale[start:stop]
        bias = None if self.bias is None else self.bias[start:stop]
        return self.qweight[start:stop], scale, bias

    def forward_output_slice(self, value: torch.Tensor, start: int, stop: int) -> torch.Tensor:
        """Project the contiguous output range ``[start, stop)`` (quantization.py:311-337)."""
        start, stop = int(start), int(stop)
        if not 0 <= start < stop <= self.out_features:
            raise ValueError("quantized output slice lies outside the layer")
        return self._forward_parameters(value, *self._slice_params(start, stop))

    def prepare_output_slices(self, value: torch.Tensor) -> PreparedConvRotInt8Input:
        """Quantize a 2-D activation once for later output slices (quantization.py:339-371), with
        the reference's contract: this package's INT8 kernel, a rank-two GPU activation, ConvRot
        group 256 and an input width that is a multiple of 256 in [256, 16384]; RuntimeError
        otherwise (ValueError for a width that does not match the weight), in the same order."""
        if self.kernel is not int8_kernel:
            raise RuntimeError("prepared output slices require the audited HIP INT8 kernel")
        if not value.is_cuda or value.ndim != 2:
            raise RuntimeError("prepared output slices require a rank-two GPU activation")
        if not self.spec.convrot or self.spec.convrot_groupsize != 256:
            raise RuntimeError("prepared output slices require ConvRot group size 256")
        if value.shape[1] != self.in_features:
            raise ValueError("input width does not match quantized weight")
        if not 256 <= self.in_features <= 16_384 or self.in_features % 256:
            raise RuntimeError("prepared output slice width is outside the fused GPU contract")
        contiguous = value if value.is_contiguous() else value.contiguous()
        qdata, scale = ops.quantize_int8_rowwise_convrot(contiguous, 256)
        return PreparedConvRotInt8Input(qdata=qdata, scale=scale, rows=int(value.shape[0]),
                                        width=int(value.shape[1]), dtype=value.dtype)

    def forward_prepared_output_slice(self, value: torch.Tensor, prepared: PreparedConvRotInt8Input,
                                      row_start: int, row_stop: int, output_start: int,
                                      output_stop: int) -> torch.Tensor:
        """Project one row/output rectangle from a shared quantized input (quantization.py:373-413)."""
        row_start, row_stop = int(row_start), int(row_stop)
        output_start, output_stop = int(output_start), int(output_stop)
        if prepared.width != self.in_features:
            raise ValueError("prepared activation width does not match quantized weight")
        if value.ndim != 2 or tuple(value.shape) != (prepared.rows, prepared.width):
            raise ValueError("source activation does not match its prepared INT8 input")
        if not 0 <= row_start < row_stop <= prepared.rows:
            raise ValueError("prepared activation row slice lies outside the input")
        if not 0 <= output_start < output_stop <= self.out_features:
            raise ValueError("quantized output slice lies outside the layer")
        qweight, scale, bias = self._slice_params(output_start, output_stop)
        return ops.int8_linear_prequantized(prepared.qdata[row_start:row_stop],
                                            prepared.scale[row_start:row_stop], qweight, scale, bias,
                                            self.output_dtype or prepared.dtype)


class ConvRotW4A8Linear(nn.Module):
    """Grouped packed-int4 weights with int8 activations (quantization.py:416-586)."""

    def __init__(self, qdata: torch.Tensor, s_rel: torch.Tensor, s_channel: torch.Tensor, *,
                 codebook: torch.Tensor | None = None, correction: torch.Tensor | None = None,
                 bias: torch.Tensor | None = None, spec: W4A8QuantSpec = W4A8QuantSpec(),
                 kernel: W4A8Kernel | None = None, output_dtype: torch.dtype | None = None) -> None:
        super().__init__()
        spec.validate_supported()
        if qdata.ndim != 2 or qdata.dtype != torch.int8:
            raise ValueError("packed W4 weight must be a rank-two int8 tensor")
        out_features, packed_width = qdata.shape
        in_features = packed_width * 2
        if in_features % 16 or in_features % spec.group_size:
            raise ValueError("W4A8 input width is incompatible with its group size")
        if in_features % spec.convrot_groupsize:
            raise ValueError("W4A8 input width is incompatible with ConvRot")
        groups = in_features // spec.group_size
        if tuple(s_rel.shape) != (out_features, groups):
            raise ValueError(f"s_rel must be {(out_features, groups)}, got {tuple(s_rel.shape)}")
        if tuple(s_channel.shape) != (out_features,):
            raise ValueError(f"s_channel must be {(out_features,)}, got {tuple(s_channel.shape)}")
        if codebook is not None and tuple(codebook.shape) != (16,):
            raise ValueError("W4A8 codebook must contain 16 entries")
        if correction is not None and tuple(correction.shape) != (groups, out_features):
            raise ValueError("W4A8 correction must be [groups, out_features]")
        if bias is not None and bias.numel() != out_features:
            raise ValueError("bias does not match W4A8 output rows")
        for name, t in (("qdata", qdata), ("s_rel", s_rel), ("s_channel", s_channel),
                        ("codebook", codebook), ("correction", correction), ("bias", bias)):
            self.register_buffer(name, t)
        self.spec = spec
        self.kernel = kernel if kernel is not None else w4a8_kernel
        self.output_dtype = output_dtype

    @property
    def in_features(self) -> int:
        return int(self.qdata.shape[1]) * 2

    @property
    def out_features(self) -> int:
        return int(self.qdata.shape[0])

    def _forward_parameters(self, value, qdata, s_rel, s_channel, codebook, correction, bias):
        if value.shape[-1] != self.in_features:
            raise ValueError("input width does not match packed W4A8 weight")
        _gpu_only(value)
        return self.kernel(value, qdata, s_rel, s_channel, codebook, correction, bias,
                           self.spec.group_size, self.spec.convrot_groupsize,
                           self.output_dtype or value.dtype)

    def forward(self, value: torch.Tensor) -> torch.Tensor:
        return self._forward_parameters(value, self.qdata, self.s_rel, self.s_channel, self.codebook,
                                        self.correction, self.bias)

    def forward_output_slice(self, value: torch.Tensor, start: int, stop: int) -> torch.Tensor:
        start, stop = int(start), int(stop)
        if not 0 <= start < stop <= self.out_features:
            raise ValueError("W4A8 output slice lies outside the layer")
        return self._forward_parameters(
            value, self.qdata[start:stop], self.s_rel[start:stop], self.s_channel[start:stop],
            self.codebook, None if self.correction is None else self.correction[:, start:stop],
            None if self.bias is None else self.bias[start:stop])


def inspect_quantized_layers(state: Mapping[str, torch.Tensor]) -> dict[str, ComfyQuantSpec]:
    """Map layer prefix -> spec for every ``*.comfy_quant`` entry (quantization.py:589-595)."""
    suffix = ".comfy_quant"
    return {key[: -len(suffix)]: ComfyQuantSpec.decode(v) for key, v in state.items() if key.endswith(suffix)}
