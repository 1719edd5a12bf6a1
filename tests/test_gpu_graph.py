"""The path under HIP graph capture: a captured chain replays to the eager results.

Nothing in these chains records a hipMemsetAsync (the FFN's row-absmax buffer is cleared by a fill
kernel), so a captured graph can be replayed as a serving loop would. Each test replays several
times with eager work and synchronisations in between and checks every replay bit for bit against
the eager result.
"""

import pytest
import torch

from _util import activations, bf16_vec, gen, int8_weight

pytestmark = pytest.mark.gpu


def _mx():
    import mx_qlinear

    return mx_qlinear


def _replays_match(dev, fn, ref, replays=3):
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm up outside the capture (library handles, allocator)
        fn()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    noise = torch.randn(1 << 20, device=dev)
    for r in range(replays):
        (noise * 3).sum().item()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {r} differs from eager"
    del graph


def test_ffn_chain_in_a_graph(dev):
    m, k, hidden, n = 300, 512, 1024, 512
    x = activations(m, k, 1).to(dev)
    w1, s1 = int8_weight(hidden, k, 2)
    w2, s2 = int8_weight(n, hidden, 3)
    b1, b2 = bf16_vec(hidden, 4, 0.01).to(dev), bf16_vec(n, 5, 0.01).to(dev)
    w1, s1, w2, s2 = w1.to(dev), s1.to(dev), w2.to(dev), s2.to(dev)
    ws = _mx().FfnWorkspace(m, k, hidden, dev)
    ref = _mx().int8_ffn_gelu(x, w1, s1, b1, w2, s2, b2)
    _replays_match(dev, lambda: _mx().int8_ffn_gelu(x, w1, s1, b1, w2, s2, b2, workspace=ws), ref)


def test_h3_qkv_chain_in_a_graph(dev):
    """rms_adaln + ConvRot quant -> QKV GEMM, and the W4A8 group-128 GEMM on prepared weights."""
    m, d, n = 96, 512, 768
    x = activations(m, d, 11).to(dev)
    norm_w = (1 + 0.1 * torch.randn(d, generator=gen(12))).to(torch.bfloat16).to(dev)
    scale = (0.1 * torch.randn(2, d, generator=gen(13))).to(torch.bfloat16).to(dev)
    shift = (0.1 * torch.randn(2, d, generator=gen(14))).to(torch.bfloat16).to(dev)
    segs = ((0, 40, 1), (40, m, 0))
    w, s = int8_weight(n, d, 15)
    w, s = w.to(dev), s.to(dev)
    b = bf16_vec(n, 16, 0.01).to(dev)

    def qkv():
        q, xs = _mx().rms_adaln_quantize_int8(x, (norm_w, 1e-6), shift, scale, segs, convrot_groupsize=256)
        return _mx().int8_linear_prequantized(q, xs, w, s, b)

    _replays_match(dev, qkv, qkv())

    from _util import group_scales, packed_int4

    qd = _mx().prepare_w4a8_grouped(packed_int4(n, d, 17).to(dev))
    gs = group_scales(d, n, 128, 18).to(dev)
    _replays_match(dev, lambda: _mx().w4a8_grouped_linear(x, qd, gs, 128), _mx().w4a8_grouped_linear(x, qd, gs, 128))


def test_h3_mlp_chain_in_a_graph(dev):
    """rms_adaln + ConvRot quant -> fc1 with the SwiGLU epilogue (ping-pong kernel, compact SiLU
    table) -> ConvRot re-quant -> fc2 with the gated residual update, in place on a residual that
    the graph first restores from a saved copy."""
    m, d, f = 300, 512, 768
    w1, s1 = int8_weight(2 * f, d, 41)
    w2, s2 = int8_weight(d, f, 42)
    b1, b2 = bf16_vec(2 * f, 43, 0.02).to(dev), bf16_vec(d, 44, 0.02).to(dev)
    w1, s1, w2, s2 = w1.to(dev), s1.to(dev), w2.to(dev), s2.to(dev)
    norm_w = (1 + 0.1 * torch.randn(d, generator=gen(45))).to(torch.bfloat16).to(dev)
    scale, shift, gate = ((0.1 * torch.randn(3, d, generator=gen(46 + i))).to(torch.bfloat16).to(dev) for i in range(3))
    segs = ((0, 100, 0), (100, 200, 1), (200, 300, 2))
    fc1 = _mx().prepare_swiglu_fc1(w1, s1, b1)
    res0 = (activations(m, d, 49) * 2).to(dev)
    ref = res0.clone()
    _mx().h3_mlp_(ref, (norm_w, 1e-6), shift, scale, gate, segs, fc1, w2, s2, b2)
    res = torch.empty_like(res0)

    def chain():
        res.copy_(res0)
        return _mx().h3_mlp_(res, (norm_w, 1e-6), shift, scale, gate, segs, fc1, w2, s2, b2)

    _replays_match(dev, chain, ref)
