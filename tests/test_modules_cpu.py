"""Module contract on the CPU (no kernel launches): the reference's checks and error classes of
ConvRotInt8Linear.prepare_output_slices (h3serve/native_engine/model/quantization.py:339-371),
in the reference's order, and the GEMM weight prepared once at construction."""

import json

import pytest
import torch


def _mx():
    import mx_qlinear

    return mx_qlinear


def _layer(k=1024, convrot=True, group=256, kernel=None):
    mx = _mx()
    spec = mx.ComfyQuantSpec.decode(json.dumps({"format": "int8_tensorwise", "convrot": convrot,
                                                "convrot_groupsize": group}))
    return mx.ConvRotInt8Linear(torch.zeros(64, k, dtype=torch.int8), torch.ones(64, 1), spec=spec, kernel=kernel)


def test_prepared_slices_need_the_library_kernel():
    layer = _layer(kernel=lambda *a: None)
    with pytest.raises(RuntimeError, match="audited"):
        layer.prepare_output_slices(torch.zeros(4, 1024, dtype=torch.bfloat16))


def test_prepared_slices_need_a_rank_two_gpu_activation():
    with pytest.raises(RuntimeError, match="rank-two GPU activation"):
        _layer().prepare_output_slices(torch.zeros(4, 1024, dtype=torch.bfloat16))


def test_prepared_slices_contract_on_a_gpu_like_input(monkeypatch):
    """The checks after the device check, in order, with a stand-in for a GPU tensor."""

    class FakeCuda:
        is_cuda = True
        ndim = 2

        def __init__(self, width):
            self.shape = (4, width)

    with pytest.raises(RuntimeError, match="group size 256"):
        _layer(convrot=False).prepare_output_slices(FakeCuda(1024))
    with pytest.raises(RuntimeError, match="group size 256"):
        _layer(group=64).prepare_output_slices(FakeCuda(1024))
    with pytest.raises(ValueError, match="input width"):
        _layer().prepare_output_slices(FakeCuda(512))
    with pytest.raises(RuntimeError, match="fused GPU contract"):
        _layer(k=32768).prepare_output_slices(FakeCuda(32768))


def test_int8_weight_stays_the_stored_tensor_when_no_padding_is_needed():
    w = torch.zeros(64, 1024, dtype=torch.int8)
    layer = _layer()
    assert layer.qweight.shape == w.shape and not hasattr(layer.qweight, "_mxq_gemm_weight")
