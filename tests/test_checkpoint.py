"""The checkpoint format: writing, reading, auditing and module construction (CPU), and the
loaded layers' forward on the GPU against direct calls. Layout contract:
h3serve/native_engine/model/checkpoint.py:131-190 and assembly.py:69-228 of the reference."""

import json

import numpy as np
import pytest
import torch

from _util import activations, bf16_vec, bits, gen, int8_weight, packed_int4


def _mx():
    import mx_qlinear

    return mx_qlinear


def _layers():
    from mx_qlinear.checkpoint import int8_layer_tensors

    w, ws = int8_weight(192, 512, 1)
    t = int8_layer_tensors("blocks.0.attn.qkv_proj", w, ws, bf16_vec(192, 2, 0.01), 256)
    n, k, g = 128, 512, 16
    t["blocks.0.mlp.fc2.weight"] = packed_int4(n, k, 3)
    t["blocks.0.mlp.fc2.weight_s_rel"] = (torch.rand(n, k // g, generator=gen(4)) + 0.5).to(torch.float8_e4m3fn)
    t["blocks.0.mlp.fc2.weight_s_channel"] = torch.rand(n, generator=gen(5)) * 0.01
    t["blocks.0.mlp.fc2.weight_codebook"] = torch.linspace(-7.5, 7.5, 16)
    meta = {"blocks.0.mlp.fc2": {"format": "asym_w4a8_int8", "group_size": g, "convrot": True,
                                 "convrot_groupsize": 256}}
    return t, meta


def test_roundtrip_read_audit_and_build(tmp_path):
    mx = _mx()
    t, meta = _layers()
    path = tmp_path / "q.safetensors"
    mx.save_checkpoint(path, t, meta)
    with mx.SafeTensorSource(str(path)) as src:
        assert src.quantization_spec("blocks.0.mlp.fc2") == meta["blocks.0.mlp.fc2"]
        assert src.quantization_spec("blocks.0.attn.qkv_proj") is None
        a = mx.audit_quantized_layer(src, "blocks.0.attn.qkv_proj", (192, 512))
        b = mx.audit_quantized_layer(src, "blocks.0.mlp.fc2", (128, 512))
        assert (a.kind, a.ok, b.kind, b.ok) == ("int8", True, "w4a8", True), (a.issues, b.issues)
        l1 = mx.quant_linear(src, "blocks.0.attn.qkv_proj", device="cpu")
        l2 = mx.quant_linear(src, "blocks.0.mlp.fc2", device="cpu")
        with pytest.raises(KeyError):
            mx.quant_linear(src, "blocks.0.attn.out_proj", device="cpu")
    assert isinstance(l1, mx.ConvRotInt8Linear) and l1.spec.convrot and l1.spec.convrot_groupsize == 256
    assert torch.equal(l1.qweight, t["blocks.0.attn.qkv_proj.weight"])
    # the stored INT8 bias is not applied, as in the reference's loader (assembly.py:174-184)
    assert "blocks.0.attn.qkv_proj.bias" in t and l1.bias is None
    assert isinstance(l2, mx.ConvRotW4A8Linear) and l2.spec.group_size == 16
    assert l2.s_rel.dtype == torch.float8_e4m3fn and l2.codebook is not None
    with pytest.raises(RuntimeError):  # the modules run on the GPU only
        l1(torch.zeros(2, 512, dtype=torch.bfloat16))


@pytest.mark.parametrize("corrupt,needle", [
    (lambda t, m: t.__setitem__("blocks.0.attn.qkv_proj.weight_scale", torch.ones(192)), "weight_scale: shape"),
    (lambda t, m: t.__setitem__("blocks.0.attn.qkv_proj.weight", torch.zeros(192, 512, dtype=torch.int16)), "dtype I16"),
    (lambda t, m: t.__setitem__("blocks.0.attn.qkv_proj.comfy_quant",
                                torch.tensor(list(json.dumps({"format": "int8_tensorwise", "convrot": False}).encode()),
                                             dtype=torch.uint8)), "ConvRot flag is false"),
    (lambda t, m: t.__setitem__("blocks.0.attn.qkv_proj.comfy_quant",
                                torch.tensor(list(b"{\"format\": \"fp8\"}"), dtype=torch.uint8)), "int8_tensorwise"),
])
def test_audit_reports_corrupt_int8_layers(tmp_path, corrupt, needle):
    mx = _mx()
    t, meta = _layers()
    corrupt(t, meta)
    path = tmp_path / "bad.safetensors"
    mx.save_checkpoint(path, t, meta)
    with mx.SafeTensorSource(str(path)) as src:
        a = mx.audit_quantized_layer(src, "blocks.0.attn.qkv_proj", (192, 512))
    assert not a.ok and any(needle in i for i in a.issues), a.issues


def test_audit_reports_w4a8_problems(tmp_path):
    mx = _mx()
    t, meta = _layers()
    t["blocks.0.mlp.fc2.weight_s_channel"] = torch.ones(127)
    mx.save_checkpoint(tmp_path / "b.safetensors", t, meta)
    with mx.SafeTensorSource(str(tmp_path / "b.safetensors")) as src:
        a = mx.audit_quantized_layer(src, "blocks.0.mlp.fc2", (128, 512))
        b = mx.audit_quantized_layer(src, "blocks.0.mlp.fc1", (128, 512))
    assert any("weight_s_channel: shape" in i for i in a.issues)
    assert b.issues == ["blocks.0.mlp.fc1: missing INT8 tensors and W4A8 metadata"]


def test_invalid_metadata_is_rejected():
    from mx_qlinear.checkpoint import parse_quantization_metadata

    with pytest.raises(ValueError):
        parse_quantization_metadata({"_quantization_metadata": "{not json"})
    with pytest.raises(ValueError):
        parse_quantization_metadata({"_quantization_metadata": json.dumps({"layers": [1, 2]})})
    assert parse_quantization_metadata({}) == {}


def test_mapping_source_defaults_w4a8_spec():
    mx = _mx()
    t, _ = _layers()
    layer = mx.quant_linear(mx.MappingTensorSource(t), "blocks.0.mlp.fc2", device="cpu")
    assert (layer.spec.group_size, layer.spec.convrot_groupsize) == (16, 256)


@pytest.mark.gpu
def test_loaded_layers_run_on_the_gpu(tmp_path, dev):
    mx = _mx()
    wf = (torch.randn(192, 512, generator=gen(9)) * 0.02).to(torch.bfloat16)
    q, s = mx.quantize_int8_convrot_weight(wf.to(dev), 256)
    from mx_qlinear.checkpoint import int8_layer_tensors

    t = int8_layer_tensors("l", q, s, bf16_vec(192, 10, 0.01), 256)
    mx.save_checkpoint(tmp_path / "g.safetensors", t)
    with mx.SafeTensorSource(str(tmp_path / "g.safetensors")) as src:
        layer = mx.quant_linear(src, "l", device=dev)
    x = activations(24, 512, 11).to(dev)
    y = layer(x)
    assert layer.bias is None  # a stored INT8 bias is not applied (assembly.py:174-184)
    ref = mx.int8_linear(x, q, s, None, convrot=True, convrot_groupsize=256)
    assert torch.equal(y, ref)
    # the stored weights are the rotated, quantized originals: the layer approximates x @ W^T
    dense = x.float() @ wf.float().to(dev).T
    assert ((y.float() - dense).norm() / dense.norm()).item() < 0.05


def test_reads_a_file_written_without_this_package(tmp_path):
    """A checkpoint written directly with safetensors in the layout the reference's loader and
    audit read (h3serve/native_engine/model/assembly.py:105-135, checkpoint.py:130-190,
    quantization.py:105-131): `comfy_quant` as uint8 JSON bytes (here with the nested `params`
    form), INT8 `[N, 1]` fp32 scales, W4A8 layers with fp32 `s_rel`, a codebook, a correction
    term, and the per-layer record in the file's `_quantization_metadata`."""
    from safetensors.torch import save_file

    mx = _mx()
    n, k, g = 64, 512, 16
    w8 = torch.randint(-127, 128, (n, k), generator=gen(31), dtype=torch.int8)
    ws = torch.rand(n, 1, generator=gen(32)) * 1e-3
    cq = json.dumps({"format": "int8_tensorwise", "params": {"convrot": True, "convrot_groupsize": 64}})
    qd = packed_int4(n, k, 33)
    s_rel = torch.rand(n, k // g, generator=gen(34)) * 4 + 0.5
    s_ch = torch.rand(n, generator=gen(35)) * 1e-3
    cb = torch.linspace(-1.0, 1.0, 16)
    corr = (torch.randn(k // g, n, generator=gen(36)) * 1e-3).to(torch.bfloat16)
    tensors = {
        "blocks.3.attn.out_proj.weight": w8,
        "blocks.3.attn.out_proj.weight_scale": ws,
        "blocks.3.attn.out_proj.comfy_quant": torch.tensor(list(cq.encode()), dtype=torch.uint8),
        "blocks.3.mlp.fc1.weight": qd,
        "blocks.3.mlp.fc1.weight_s_rel": s_rel,
        "blocks.3.mlp.fc1.weight_s_channel": s_ch,
        "blocks.3.mlp.fc1.weight_codebook": cb,
        "blocks.3.mlp.fc1.weight_correction": corr,
    }
    record = {"format": "asym_w4a8_int8", "group_size": g, "convrot": True, "convrot_groupsize": 256}
    path = tmp_path / "foreign.safetensors"
    save_file(tensors, str(path), metadata={"_quantization_metadata": json.dumps({"layers": {"blocks.3.mlp.fc1": record}})})
    with mx.SafeTensorSource(str(path)) as src:
        assert src.quantization_spec("blocks.3.mlp.fc1") == record
        a = mx.audit_quantized_layer(src, "blocks.3.attn.out_proj", (n, k))
        b = mx.audit_quantized_layer(src, "blocks.3.mlp.fc1", (n, k))
        assert (a.kind, a.ok, b.kind, b.ok) == ("int8", True, "w4a8", True), (a.issues, b.issues)
        l1 = mx.quant_linear(src, "blocks.3.attn.out_proj", device="cpu")
        l2 = mx.quant_linear(src, "blocks.3.mlp.fc1", device="cpu")
    assert l1.spec.convrot and l1.spec.convrot_groupsize == 64
    assert torch.equal(l1.qweight, w8) and torch.equal(l1.scale.reshape(-1), ws.reshape(-1))
    assert l2.spec.group_size == g and l2.spec.convrot_groupsize == 256
    assert torch.equal(l2.qdata, qd) and torch.equal(l2.s_rel, s_rel) and torch.equal(l2.s_channel, s_ch)
    assert torch.equal(l2.codebook, cb) and torch.equal(l2.correction, corr)
