"""GPU parity of the ConvRot rotation + quantizer, SwiGLU, and the linears that use them,
against the oracle (bit-exact int8 and scales; bit-exact bf16 outputs)."""

import numpy as np
import pytest
import torch

from _util import activations, bf16_vec, bits, from_bits, gen, int8_weight, packed_int4
from oracle import convrot as cr
from oracle import eager_np
from oracle.bf16 import bf16_bits, bf16_to_f32

pytestmark = pytest.mark.gpu


def _mx():
    import mx_qlinear

    return mx_qlinear


@pytest.mark.parametrize("m,k,g", [(37, 5120, 256), (8, 1024, 256), (5, 1280, 256), (16, 3072, 1024),
                                   (9, 512, 64), (4, 256, 16), (3, 64, 4), (64, 16384, 256)])
def test_convrot_quantizer_matches_oracle(dev, m, k, g):
    print(f"convrot quant m={m} k={k} g={g}", flush=True)
    x = activations(m, k, 100 + k + g)
    q, s = _mx().quantize_int8_rowwise_convrot(x.to(dev), g)
    qr, sr, _ = cr.convrot_quantize_bf16(bits(x), g)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy(), sr)


@pytest.mark.parametrize("m,k,g", [(1, 5376, 256), (2, 4352, 64), (8, 6144, 256), (1, 6400, 256), (3, 8192, 16),
                                   (9, 5376, 256), (1, 4096, 64), (1, 256, 256)])
def test_convrot_quantizer_few_rows_matches_oracle(dev, m, k, g):
    """Launches of at most 8 rows take one unit (256 columns) per 16-lane group, in blocks of up to
    six waves (17-24 units), or the fewest units per group that fit four waves (25+ units); 9 rows
    take the throughput split. All bit-exact."""
    print(f"convrot quant few rows m={m} k={k} g={g}", flush=True)
    x = activations(m, k, 300 + m + k + g)
    q, s = _mx().quantize_int8_rowwise_convrot(x.to(dev), g)
    qr, sr, _ = cr.convrot_quantize_bf16(bits(x), g)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy(), sr)


@pytest.mark.parametrize("act", ["gelu_tanh", "swiglu"])
@pytest.mark.parametrize("g", [256, 0])
def test_convrot_quantizer_with_input_act(dev, act, g):
    m, k = 19, 2048
    width = 2 * k if act == "swiglu" else k
    x = activations(m, width, 7 + g, outlier_frac=0.0) * 2
    q, s = _mx().quantize_int8_rowwise_convrot(x.to(dev), g, act)
    qr, sr, _ = cr.convrot_quantize_bf16(bits(x), g, act)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy(), sr)


def test_convrot_quantizer_fp32_input(dev):
    x = activations(11, 2048, 3).float() * 1.37
    q, s = _mx().quantize_int8_rowwise_convrot(x.to(dev), 256)
    qr, sr, _ = cr.convrot_quantize_f32(x.numpy(), 256)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy(), sr)


def test_convrot_zero_and_constant_rows(dev):
    x = torch.zeros(3, 512, dtype=torch.bfloat16)
    x[1] = 1.0        # constant groups rotate to a single spike of 16 per group
    x[2, ::7] = -3.0
    q, s = _mx().quantize_int8_rowwise_convrot(x.to(dev), 256)
    qr, sr, _ = cr.convrot_quantize_bf16(bits(x), 256)
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().numpy(), sr)
    assert s[0].item() == np.float32(1e-30) and int(q[0].abs().max()) == 0


@pytest.mark.parametrize("k,g", [(512, 256), (512, 4), (1024, 64), (80, 16)])
def test_convrot_midpoint_rows(dev, k, g):
    """Rows whose rotated values land on bfloat16 midpoints in float32 while the exact value lies
    just above or below (1, 2^-8 and +-2^-30 in each group): the rounding must follow the exact
    value, not the float32 detour. K a multiple of 256 runs the unit form, K = 80 the window form."""
    x = np.zeros((6, k), np.float32)
    for r in range(6):
        for g0 in range(0, k, g):
            x[r, g0 + (r % 3)] = 1.0 * (1 + r)
            x[r, g0 + 1 + (r % 2)] = 2.0 ** -8 * (1 + r)
            x[r, g0 + 3] = (-1) ** r * 2.0 ** -30
    xb = torch.from_numpy(x).to(torch.bfloat16)
    rot = cr.fht_f64(x.astype(np.float64), g)
    f = rot.astype(np.float32).view(np.uint32)
    assert np.any(((f & 0xFFFF) == 0x8000) & (f.view(np.float32).astype(np.float64) != rot))  # the case arises
    q, s = _mx().quantize_int8_rowwise_convrot(xb.to(dev), g)
    qr, sr, yr = cr.convrot_quantize_bf16(bits(xb), g)
    assert np.array_equal(q.cpu().numpy(), qr) and np.array_equal(s.cpu().numpy(), sr)


def test_swiglu_all_gate_values(dev):
    """All 65,536 bf16 gate patterns against torch's silu(gate).mul_(up) via the oracle."""
    gate = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).reshape(64, 1024)
    up = activations(64, 1024, 9)
    x = torch.cat([gate, up], dim=1)
    y = _mx().apply_input_act(x.to(dev), "swiglu")
    assert np.array_equal(bits(y), cr.swiglu_bf16(bits(x)))


def test_int8_linear_convrot_matches_oracle(dev):
    m, k, n, g = 45, 2048, 384, 256
    x = activations(m, k, 51)
    w, ws = int8_weight(n, k, 52)
    b = bf16_vec(n, 53, 0.01)
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), b.to(dev), convrot=True, convrot_groupsize=g)
    q, s, _ = cr.convrot_quantize_bf16(bits(x), g)
    acc = eager_np.int8_matmul(q, w.numpy())
    ref = eager_np.dequant_epilogue(acc, s, ws.numpy(), bits(b), "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))


def test_int8_linear_swiglu_matches_oracle(dev):
    m, k, n = 21, 1024, 256
    x = activations(m, 2 * k, 61, outlier_frac=0.0)
    w, ws = int8_weight(n, k, 62)
    y = _mx().int8_linear(x.to(dev), w.to(dev), ws.to(dev), None, input_act="swiglu", convrot=True,
                          convrot_groupsize=256)
    q, s, _ = cr.convrot_quantize_bf16(bits(x), 256, "swiglu")
    ref = eager_np.dequant_epilogue(eager_np.int8_matmul(q, w.numpy()), s, ws.numpy(), None, "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))


def _convrot_layer(dev, n=320, k=1024, g=256, seed=70):
    mx = _mx()
    wf = (torch.randn(n, k, generator=gen(seed)) * 0.02).to(torch.bfloat16)
    q, s = cr.quantize_int8_convrot_weight(bf16_to_f32(bits(wf)), g)
    spec = {"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": g}
    state = {
        "l.weight": torch.from_numpy(q).to(dev),
        "l.weight_scale": torch.from_numpy(s).to(dev),
        "l.bias": bf16_vec(n, seed + 1, 0.01).to(dev),
        "l.comfy_quant": torch.tensor(list(__import__("json").dumps(spec).encode()), dtype=torch.uint8),
    }
    return mx.ConvRotInt8Linear.from_state_dict(state, "l"), wf


def test_convrot_module_forward_slices_and_prepared_inputs(dev):
    layer, wf = _convrot_layer(dev)
    x = activations(40, 1024, 71).to(dev)
    full = layer(x)
    # ConvRot is an orthogonal change of basis: the quantized layer approximates x @ W^T
    dense = (x.float() @ wf.float().to(dev).T) + layer.bias.float()
    rel = ((full.float() - dense).norm() / dense.norm()).item()
    assert rel < 0.05
    a = layer.forward_output_slice(x, 0, 128)
    b = layer.forward_output_slice(x, 128, 320)
    assert torch.equal(torch.cat([a, b], dim=1), full)
    prep = layer.prepare_output_slices(x)
    r = layer.forward_prepared_output_slice(x, prep, 3, 29, 64, 250)
    assert torch.equal(r, full[3:29, 64:250])


@pytest.mark.parametrize("source", ["random", "prepared"])
def test_w4a8_reference_format_with_convrot(dev, source):
    """Random storage, or storage that quantize_w4a8_int8_weight made from an N(0, 0.02) bf16
    weight in the uniform symmetric mode (no codebook)."""
    mx = _mx()
    n, k, gsz = 256, 1024, 16
    if source == "prepared":
        w = (torch.randn(n, k, generator=gen(85)) * 0.02).to(torch.bfloat16)
        qd, s_rel, s_ch, _, _ = mx.quantize_w4a8_int8_weight(w.to(dev), gsz, 256, codebook=False)
        qd, s_rel, s_ch = qd.cpu(), s_rel.cpu(), s_ch.cpu()
    else:
        qd = packed_int4(n, k, 81)
        s_rel = (torch.rand(n, k // gsz, generator=gen(82)) * 1.5 + 0.25).to(torch.float8_e4m3fn)
        s_ch = (torch.rand(n, generator=gen(83)) * 0.01 + 0.001)
    x = activations(33, k, 84)
    y = mx.w4a8_int8_linear(x.to(dev), qd.to(dev), s_rel.to(dev), s_ch.to(dev), group_size=gsz,
                            convrot_groupsize=256)
    w8 = eager_np.dequant_int4_grouped_to_int8(qd.numpy(), s_rel.view(torch.uint8).numpy(), None, gsz,
                                               s_rel_is_e4m3=True)
    q, s, _ = cr.convrot_quantize_bf16(bits(x), 256)
    ref = eager_np.dequant_epilogue(eager_np.int8_matmul(q, w8), s, s_ch.numpy(), None, "bf16")
    assert np.array_equal(bits(y), bf16_bits(ref))


def test_convrot_rejects_bad_group_sizes(dev):
    x = activations(2, 768, 1).to(dev)
    with pytest.raises(ValueError):
        _mx().quantize_int8_rowwise_convrot(x, 128)
    with pytest.raises(ValueError):
        _mx().quantize_int8_rowwise_convrot(x, 1024)  # does not divide 768
    w, ws = int8_weight(64, 768, 2)
    with pytest.raises(ValueError):
        _mx().int8_linear(x, w.to(dev), ws.to(dev), convrot=True, convrot_groupsize=32)


@pytest.mark.parametrize("g", [256, 0])
def test_convrot_nan_and_inf_rows_follow_the_oracle(dev, g):
    """NaN / inf inputs spread through the rotation group; the absmax propagates NaN (torch's
    amax), so such rows quantize to 0 with a NaN or inf scale."""
    x = activations(6, 1024, 41)
    x[1, 17] = float("nan")
    x[2, 5] = float("inf")
    x[3, 9] = -float("inf")
    x[3, 700] = float("inf")
    q, s = _mx().quantize_int8_rowwise_convrot(x.to(dev), g)
    with np.errstate(invalid="ignore"):
        qr, sr, _ = cr.convrot_quantize_bf16(bits(x), g)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy(), sr, equal_nan=True)
    xf = x.float() * 1.5
    xf[4, 3] = float("nan")
    q2, s2 = _mx().quantize_int8_rowwise_convrot(xf.to(dev), g or 256)
    with np.errstate(invalid="ignore"):
        qr2, sr2, _ = cr.convrot_quantize_f32(xf.numpy(), g or 256)
    assert np.array_equal(q2.cpu().numpy(), qr2)
    assert np.array_equal(s2.cpu().numpy(), sr2, equal_nan=True)
