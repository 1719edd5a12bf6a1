"""The quantized-linear checkpoint format: reading, auditing and writing it.

Mirrors the reference's on-disk contract and loaders (paths relative to the reference tree):
  * INT8 ConvRot layers (h3serve/native_engine/model/checkpoint.py:131-157):
      {p}.weight I8 [N, K], {p}.weight_scale F32 [N, 1], {p}.comfy_quant U8 (JSON bytes
      {"format": "int8_tensorwise", "convrot": true, "convrot_groupsize": 256}), optional {p}.bias;
  * W4A8 layers (checkpoint.py:158-190; assembly.py:188-228):
      {p}.weight I8 [N, K/2], {p}.weight_s_rel F8_E4M3 or F32 [N, K/G], {p}.weight_s_channel
      F32 [N], optional {p}.weight_codebook F32 [16], {p}.weight_correction [K/G, N], {p}.bias,
      and the layer's record in the safetensors metadata "_quantization_metadata" -> "layers"
      -> p (assembly.py:106-129);
  * tensor sources (assembly.py:69-153) and the layer factory ``quant_linear``
    (assembly.py:166-228).
Tensors are read lazily from the file and moved to the target device one layer at a time.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from typing import Mapping, Protocol

import torch

from .modules import ComfyQuantSpec, ConvRotInt8Linear, ConvRotW4A8Linear, W4A8QuantSpec

# W4A8 layers of an H3 checkpoint without file-level metadata (assembly.py:199-207).
DEFAULT_W4A8_SPEC = {"format": "asym_w4a8_int8", "group_size": 16, "convrot": True, "convrot_groupsize": 256}

_SAFETENSORS_DTYPES = {
    torch.int8: "I8", torch.uint8: "U8", torch.int16: "I16", torch.int32: "I32", torch.int64: "I64",
    torch.float32: "F32", torch.float16: "F16", torch.bfloat16: "BF16", torch.float64: "F64",
    torch.float8_e4m3fn: "F8_E4M3", torch.float8_e5m2: "F8_E5M2", torch.bool: "BOOL",
}


class TensorSource(Protocol):
    def tensor(self, key: str) -> torch.Tensor: ...

    def has_tensor(self, key: str) -> bool: ...

    def quantization_spec(self, prefix: str) -> Mapping[str, object] | None: ...


class MappingTensorSource:
    """An in-memory state dict with optional per-layer W4A8 records (assembly.py:77-95)."""

    def __init__(self, state: Mapping[str, torch.Tensor],
                 quantization: Mapping[str, Mapping[str, object]] | None = None) -> None:
        self.state = state
        self.quantization = dict(quantization or {})

    def tensor(self, key: str) -> torch.Tensor:
        return self.state[key]

    def has_tensor(self, key: str) -> bool:
        return key in self.state

    def quantization_spec(self, prefix: str) -> Mapping[str, object] | None:
        return self.quantization.get(prefix)


def parse_quantization_metadata(metadata: Mapping[str, str] | None) -> dict[str, dict]:
    """The ``layers`` map of the "_quantization_metadata" JSON record (assembly.py:106-129)."""
    raw = (metadata or {}).get("_quantization_metadata")
    if not raw:
        return {}
    try:
        decoded = json.loads(raw)
        layers = decoded.get("layers", {})
        if not isinstance(layers, Mapping):
            raise TypeError("layers must be a mapping")
        return {str(name): dict(spec) for name, spec in layers.items() if isinstance(spec, Mapping)}
    except (json.JSONDecodeError, TypeError, ValueError, AttributeError) as error:
        raise ValueError("invalid safetensors _quantization_metadata") from error


class SafeTensorSource:
    """Lazy reader of a .safetensors file; use as a context manager (assembly.py:98-153)."""

    def __init__(self, path: str) -> None:
        self.path = str(path)
        self._reader = None
        self._keys: set[str] = set()
        self._quantization: dict[str, dict] = {}

    def __enter__(self) -> "SafeTensorSource":
        try:
            from safetensors import safe_open
        except ImportError as error:
            raise RuntimeError("safetensors is required to load quantized weights") from error
        self._reader = safe_open(self.path, framework="pt", device="cpu")
        self._reader.__enter__()
        self._keys = set(self._reader.keys())
        self._quantization = parse_quantization_metadata(self._reader.metadata())
        return self

    def __exit__(self, *args) -> None:
        if self._reader is not None:
            self._reader.__exit__(*args)
        self._reader = None
        self._keys.clear()
        self._quantization.clear()

    def _open(self):
        if self._reader is None:
            raise RuntimeError("SafeTensorSource must be used as a context manager")
        return self._reader

    def tensor(self, key: str) -> torch.Tensor:
        return self._open().get_tensor(key)

    def has_tensor(self, key: str) -> bool:
        self._open()
        return key in self._keys

    def keys(self) -> set[str]:
        self._open()
        return set(self._keys)

    def quantization_spec(self, prefix: str) -> Mapping[str, object] | None:
        self._open()
        return self._quantization.get(prefix)


def quant_linear(source: TensorSource, prefix: str, *, device: torch.device | str,
                 int8_kernel=None, w4a8_kernel=None, output_dtype: torch.dtype | None = None):
    """Build the quantized module stored under ``prefix`` (assembly.py:166-228): INT8 ConvRot if
    ``{p}.weight_scale`` exists, else W4A8 (KeyError if neither layout is present). As in the
    reference, an INT8 layer is built from its weight, scale and spec only: a stored
    ``{p}.bias`` is not applied to it (W4A8 layers do load theirs)."""
    if source.has_tensor(f"{prefix}.weight_scale"):
        state = {
            f"{prefix}.weight": source.tensor(f"{prefix}.weight").to(device),
            f"{prefix}.weight_scale": source.tensor(f"{prefix}.weight_scale").to(device),
            f"{prefix}.comfy_quant": source.tensor(f"{prefix}.comfy_quant"),
        }
        return ConvRotInt8Linear.from_state_dict(state, prefix, kernel=int8_kernel, output_dtype=output_dtype)
    required = (f"{prefix}.weight_s_rel", f"{prefix}.weight_s_channel")
    if not all(source.has_tensor(key) for key in required):
        raise KeyError(f"quantized layer {prefix!r} is neither ConvRot INT8 nor W4A8")
    raw_spec = source.quantization_spec(prefix)
    spec = W4A8QuantSpec.from_mapping(raw_spec if raw_spec is not None else DEFAULT_W4A8_SPEC)

    def opt(key):
        return source.tensor(key).to(device) if source.has_tensor(key) else None

    return ConvRotW4A8Linear(
        source.tensor(f"{prefix}.weight").to(device),
        source.tensor(f"{prefix}.weight_s_rel").to(device),
        source.tensor(f"{prefix}.weight_s_channel").to(device),
        codebook=opt(f"{prefix}.weight_codebook"),
        correction=opt(f"{prefix}.weight_correction"),
        bias=opt(f"{prefix}.bias"),
        spec=spec,
        kernel=w4a8_kernel,
        output_dtype=output_dtype,
    )


@dataclass
class LayerAudit:
    """Outcome of checking one quantized layer against its expected [out, in] shape."""

    prefix: str
    kind: str = ""          # "int8" | "w4a8" | ""
    issues: list[str] = field(default_factory=list)

    @property
    def ok(self) -> bool:
        return not self.issues


def audit_quantized_layer(source: TensorSource, prefix: str, shape: tuple[int, int],
                          dtype_of=None) -> LayerAudit:
    """The per-layer checks of the reference's checkpoint audit (checkpoint.py:131-190):
    tensor presence, shapes and dtypes, a decodable and supported spec, ConvRot enabled and
    its group dividing the input width. ``dtype_of(key)`` returns a tensor's dtype without
    loading it (defaults to loading)."""
    out_f, in_f = shape
    audit = LayerAudit(prefix)

    def dtype(key):
        return dtype_of(key) if dtype_of is not None else source.tensor(key).dtype

    def expect(key, want_shape, dtypes=None):
        if not source.has_tensor(key):
            audit.issues.append(f"missing {key}")
            return
        t_shape = tuple(source.tensor(key).shape)
        if t_shape != tuple(want_shape):
            audit.issues.append(f"{key}: shape {t_shape}, expected {tuple(want_shape)}")
        if dtypes is not None:
            name = _SAFETENSORS_DTYPES.get(dtype(key), str(dtype(key)))
            if name not in dtypes:
                audit.issues.append(f"{key}: dtype {name}, expected one of {dtypes}")

    if source.has_tensor(f"{prefix}.weight_scale"):
        audit.kind = "int8"
        expect(f"{prefix}.weight", (out_f, in_f), ("I8",))
        expect(f"{prefix}.weight_scale", (out_f, 1), ("F32",))
        quant_key = f"{prefix}.comfy_quant"
        if not source.has_tensor(quant_key):
            audit.issues.append(f"missing {quant_key}")
            return audit
        try:
            spec = ComfyQuantSpec.decode(source.tensor(quant_key))
            spec.validate_supported()
            if not spec.convrot:
                audit.issues.append(f"{prefix}: ConvRot flag is false")
            elif in_f % spec.convrot_groupsize:
                audit.issues.append(f"{prefix}: input width not divisible by ConvRot group")
        except Exception as error:  # the audit reports, it does not raise
            audit.issues.append(f"{quant_key}: {error}")
        return audit

    raw_spec = source.quantization_spec(prefix)
    if not isinstance(raw_spec, Mapping):
        audit.issues.append(f"{prefix}: missing INT8 tensors and W4A8 metadata")
        return audit
    audit.kind = "w4a8"
    try:
        w4 = W4A8QuantSpec.from_mapping(raw_spec)
        w4.validate_supported()
        expect(f"{prefix}.weight", (out_f, in_f // 2), ("I8",))
        expect(f"{prefix}.weight_s_rel", (out_f, in_f // w4.group_size), ("F8_E4M3", "F32"))
        expect(f"{prefix}.weight_s_channel", (out_f,), ("F32",))
        if source.has_tensor(f"{prefix}.weight_codebook"):
            expect(f"{prefix}.weight_codebook", (16,), ("F32",))
        if source.has_tensor(f"{prefix}.weight_correction"):
            expect(f"{prefix}.weight_correction", (in_f // w4.group_size, out_f))
    except Exception as error:
        audit.issues.append(f"{prefix}: {error}")
    return audit


def int8_layer_tensors(prefix: str, weight: torch.Tensor, weight_scale: torch.Tensor,
                       bias: torch.Tensor | None = None, convrot_groupsize: int = 256) -> dict:
    """The tensors of one INT8 ConvRot layer in checkpoint form (checkpoint.py:131-157)."""
    spec = {"format": "int8_tensorwise", "convrot": bool(convrot_groupsize),
            "convrot_groupsize": int(convrot_groupsize or 256)}
    out = {
        f"{prefix}.weight": weight.to(torch.int8).cpu().contiguous(),
        f"{prefix}.weight_scale": weight_scale.to(torch.float32).reshape(-1, 1).cpu().contiguous(),
        f"{prefix}.comfy_quant": torch.tensor(list(json.dumps(spec).encode("utf-8")), dtype=torch.uint8),
    }
    if bias is not None:
        out[f"{prefix}.bias"] = bias.cpu().contiguous()
    return out


def save_checkpoint(path: str, tensors: Mapping[str, torch.Tensor],
                    w4a8_layers: Mapping[str, Mapping[str, object]] | None = None) -> None:
    """Write tensors (and the W4A8 layer records as "_quantization_metadata") to a .safetensors
    file in the reference's layout."""
    from safetensors.torch import save_file

    metadata = {}
    if w4a8_layers:
        metadata["_quantization_metadata"] = json.dumps({"layers": {k: dict(v) for k, v in w4a8_layers.items()}})
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(path), metadata=metadata or None)
