"""GPU parity: the INT8 GEMMs' balanced tile queue.

With a workspace, the last eighth of each XCD's tiles is claimed at run time by whichever XCD's
workgroups get there first. Bar: every output (int32, fp32 / fp16 / bf16 dequant, GELU + row
absmax, SwiGLU, gated residual) equals the static-order launch (no workspace) bit for bit --
with the outputs pre-filled with a sentinel, so a tile that no workgroup took would show -- and
the oracle on sampled rows (first, last -- inside the partial edge tile -- and random ones);
the queue counters are back at zero after each call. Each case asserts from the launch plan
that it uses the queue.
"""

import ctypes

import numpy as np
import pytest
import torch

import mx_qlinear._lib as L
from _util import gen
from oracle import eager_np
from oracle.bf16 import bf16_bits

pytestmark = pytest.mark.gpu


def _ops():
    from mx_qlinear import ops

    return ops


def _i8(shape, seed):
    return torch.randint(-128, 128, shape, generator=gen(seed), dtype=torch.int8)


def _rows(m, seed, count=24):
    r = np.random.default_rng(seed).choice(m, size=count, replace=False)
    return np.unique(np.concatenate([[0, m - 1], r]))


def _exact_rows(a, w, rows):
    """int32 sums of the sampled rows; float64 products of int8 are exact at these K."""
    acc = a[rows].astype(np.float64) @ w.astype(np.float64).T
    return acc.astype(np.int64).astype(np.int32)


def _ws(dev, split):
    return _ops()._gemm_ws(dev) if split else (None, 0)


def _assert_queued(m, n, k, table=False):
    plan = L.gemm_plan(m, n, k, table)
    assert plan["pool"] > 0, plan
    return plan


def _counters_zero(dev):
    ptr, _ = _ops()._gemm_ws(dev)
    ws = _ops()._GEMM_WORKSPACES[(dev.index, torch.cuda.current_stream(dev).cuda_stream)]
    assert ws.data_ptr() == ptr.value
    assert int(ws.count_nonzero()) == 0


@pytest.mark.parametrize(
    "m,n,k",
    [(10496, 8192, 2048), (10459, 8144, 2000), (8187, 5120, 5120),
     (10496, 8408, 1040), (8060, 4990, 1024)],  # tile counts 1353 and 2457: XCD ranges of unequal length
)
def test_queue_i32_equals_static_order_and_oracle(dev, m, n, k):
    plan = _assert_queued(m, n, k)
    print(f"queue i32 m={m} n={n} k={k} plan={plan}", flush=True)
    a, w = _i8((m, k), m + 1), _i8((n, k), n + 2)
    ad, wd = a.to(dev), w.to(dev)
    got = {}
    for queued in (True, False):
        c = torch.full((m, n), -7, dtype=torch.int32, device=dev)
        L.call("mxq_int8_gemm_i32", _ops()._p(ad), _ops()._p(wd), _ops()._p(c), m, n, k, n, *_ws(dev, queued),
               _ops()._stream(dev))
        got[queued] = c.cpu().numpy()
    assert np.array_equal(got[True], got[False])
    rows = _rows(m, m)
    assert np.array_equal(got[True][rows], _exact_rows(a.numpy(), w.numpy(), rows))
    _counters_zero(dev)


@pytest.mark.parametrize("out_dtype,code", [(torch.bfloat16, 2), (torch.float16, 1), (torch.float32, 0)])
@pytest.mark.parametrize("m,n,k", [(10459, 8144, 2000), (8187, 5120, 5120), (8060, 4990, 2000)])
def test_queue_dequant_equals_static_order_and_oracle(dev, out_dtype, code, m, n, k):
    _assert_queued(m, n, k)
    print(f"queue dequant {out_dtype} m={m} n={n} k={k}", flush=True)
    a, w = _i8((m, k), 11), _i8((n, k), 12)
    xs = torch.rand(m, generator=gen(13)) * 0.01 + 1e-3
    ws = torch.rand(n, generator=gen(14)) * 0.01 + 1e-3
    bias = (torch.randn(n, generator=gen(15)) * 0.5).to(out_dtype)
    ops = _ops()
    dv = [t.to(dev) for t in (a, w, xs, ws, bias)]
    outs = {}
    for queued in (True, False):
        d = torch.full((m, n), float("nan"), dtype=out_dtype, device=dev)
        L.call("mxq_int8_gemm_dequant", *map(ops._p, dv[:4]), n, ops._p(dv[4]), ops._p(d), m, n, k, n, code,
               *_ws(dev, queued), ops._stream(dev))
        outs[queued] = d.cpu()
    assert torch.equal(outs[True].view(torch.uint8), outs[False].view(torch.uint8))
    rows = _rows(m, 7)
    acc = _exact_rows(a.numpy(), w.numpy(), rows)
    name = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[out_dtype]
    bias_np = bf16_bits(bias.float().numpy()) if out_dtype == torch.bfloat16 else bias.numpy()
    ref = eager_np.dequant_epilogue(acc, xs.numpy()[rows], ws.numpy(), bias_np, name, name)
    got = outs[True][rows]
    if out_dtype == torch.bfloat16:
        assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), bf16_bits(ref))
    else:
        assert np.array_equal(got.numpy(), ref.astype(got.numpy().dtype))


def test_queue_gelu_absmax_equals_static_order(dev):
    m, n, k = 8445, 8176, 1040
    _assert_queued(m, n, k, table=True)
    a, w = _i8((m, k), 21), _i8((n, k), 22)
    xs = torch.rand(m, generator=gen(23)) * 1e-3
    ws = torch.rand(n, generator=gen(24)) * 1e-2
    bias = (torch.randn(n, generator=gen(25)) * 0.5).to(torch.bfloat16)
    ops = _ops()
    dv = [t.to(dev) for t in (a, w, xs, ws, bias)]
    outs = {}
    for queued in (True, False):
        h = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=dev)
        amax = torch.zeros(m, dtype=torch.float32, device=dev)
        L.call("mxq_int8_gemm_dequant_gelu_absmax", *map(ops._p, dv[:4]), n, ops._p(dv[4]), ops._p(h), ops._p(amax),
               m, n, k, n, *_ws(dev, queued), ops._stream(dev))
        outs[queued] = (h.cpu(), amax.cpu())
    assert torch.equal(outs[True][0].view(torch.int16), outs[False][0].view(torch.int16))
    assert torch.equal(outs[True][1], outs[False][1])
    _counters_zero(dev)
    # sampled rows against the oracle's dequant -> GELU, and the row maxima of |h|
    rows = _rows(m, 3)
    acc = _exact_rows(a.numpy(), w.numpy(), rows)
    y = eager_np.dequant_epilogue(acc, xs.numpy()[rows], ws.numpy(), bf16_bits(bias.float().numpy()), "bf16")
    hb = eager_np.gelu_tanh_bf16(bf16_bits(y))
    got = outs[True][0][rows].view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, hb)
    amax_bits = (hb & np.uint16(0x7FFF)).max(axis=1).astype(np.uint32) << np.uint32(16)
    assert np.array_equal(outs[True][1].numpy()[rows].view(np.uint32), amax_bits)


def test_queue_swiglu_equals_static_order(dev):
    m, n, k = 8448, 8192, 1024
    _assert_queued(m, n, k, table=True)
    a, w = _i8((m, k), 31), _i8((n, k), 32)
    xs = torch.rand(m, generator=gen(33)) * 1e-3
    ws = torch.rand(n, generator=gen(34)) * 1e-2
    bias = (torch.randn(n, generator=gen(35)) * 0.5).to(torch.bfloat16)
    ops = _ops()
    dv = [t.to(dev) for t in (a, w, xs, ws, bias)]
    outs = {}
    for queued in (True, False):
        h = torch.full((m, n // 2), float("nan"), dtype=torch.bfloat16, device=dev)
        L.call("mxq_int8_gemm_dequant_swiglu", *map(ops._p, dv[:4]), n, ops._p(dv[4]), ops._p(h), m, n, k, n // 2,
               *_ws(dev, queued), ops._stream(dev))
        outs[queued] = h.cpu()
    assert torch.equal(outs[True].view(torch.int16), outs[False].view(torch.int16))


def test_queue_gated_residual_equals_static_order(dev):
    m, n, k = 10459, 8144, 2000
    _assert_queued(m, n, k)
    a, w = _i8((m, k), 41), _i8((n, k), 42)
    xs = torch.rand(m, generator=gen(43)) * 1e-3
    ws = torch.rand(n, generator=gen(44)) * 1e-2
    bias = (torch.randn(n, generator=gen(45)) * 0.5).to(torch.bfloat16)
    gate = (torch.randn(3, n, generator=gen(46))).to(torch.bfloat16)
    rows_map = torch.randint(0, 3, (m,), generator=gen(47), dtype=torch.int32)
    res0 = (torch.randn(m, n, generator=gen(48))).to(torch.bfloat16)
    ops = _ops()
    dv = [t.to(dev) for t in (a, w, xs, ws, bias, gate, rows_map)]
    outs = {}
    for queued in (True, False):
        res = res0.to(dev)
        L.call("mxq_int8_gemm_gated_residual", *map(ops._p, dv[:4]), n, ops._p(dv[4]), ops._p(res), n,
               ops._p(dv[5]), n, 3, ops._p(dv[6]), m, n, k, *_ws(dev, queued), ops._stream(dev))
        outs[queued] = res.cpu()
    assert torch.equal(outs[True].view(torch.int16), outs[False].view(torch.int16))


def test_queue_workspace_is_reused_and_per_stream(dev):
    """Back-to-back calls on one stream share its workspace (the counters return to zero); a
    second stream gets its own; the results of all of them agree."""
    m, n, k = 8187, 5120, 1024
    _assert_queued(m, n, k)
    a, w = _i8((m, k), 51).to(dev), _i8((n, k), 52).to(dev)
    ref = _ops().mm_int8(a, w.t())
    for _ in range(3):
        assert torch.equal(_ops().mm_int8(a, w.t()), ref)
    _counters_zero(dev)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        other = _ops().mm_int8(a, w.t())
        key = (dev.index, side.cuda_stream)
    torch.cuda.current_stream(dev).wait_stream(side)
    assert torch.equal(other, ref)
    ws_main = _ops()._GEMM_WORKSPACES[(dev.index, torch.cuda.current_stream(dev).cuda_stream)]
    assert _ops()._GEMM_WORKSPACES[key].data_ptr() != ws_main.data_ptr()
