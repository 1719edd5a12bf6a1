"""GPU parity of the allocation-free W4A8 entry point (mxq_w4a8_codebook_gemm_noalloc) against
the entry point it varies (mxq_w4a8_codebook_gemm with a caller workspace), called through the
C ABI: two calls in a row, the second smaller, then a chunk too large for the static workspace;
two calls whose chunk GEMMs are large enough to claim tiles at run time (the workspace entry
with a per-stream tile-queue workspace, the allocation-free one with its static counters); and
two calls on two streams with no host wait between them (ordered by the entry point's event);
and a call captured in a HIP graph, replayed between eager calls of another problem.

Bar: outputs bit-identical to the workspace entry point's on every call.
"""

import pytest
import torch

from _util import activations, bf16_vec, gen, packed_int4

pytestmark = pytest.mark.gpu


def _problem(dev, m, n, k, g, e4m3, codebook, bias, seed):
    """Inputs of one W4A8 codebook GEMM as the C entry points take them."""
    import mx_qlinear
    from mx_qlinear import _lib

    x = activations(m, k, seed).to(dev)
    xq, xs = mx_qlinear.quantize_int8_rowwise(x)
    qd = packed_int4(n, k, seed + 1).to(dev)
    srel = torch.rand(n, k // g, generator=gen(seed + 2)) * 0.75 + 0.25
    if e4m3:
        sr, code = srel.to(torch.float8_e4m3fn).view(torch.uint8).to(dev), _lib.DTYPE_E4M3
    else:
        sr, code = srel.to(dev), _lib.DTYPE_F32
    cb = (torch.randn(16, generator=gen(seed + 3)) * 4).to(dev) if codebook else None
    sch = (torch.rand(n, generator=gen(seed + 4)) * 0.5 + 0.5).to(dev) * (0.06 / 127)
    b = bf16_vec(n, seed + 5, 0.01).to(dev) if bias else None
    return dict(m=m, n=n, k=k, g=g, xq=xq, xs=xs, qd=qd, sr=sr, code=code, cb=cb, sch=sch, b=b)


def _workspace_entry(dev, pb, chunk, queued, st):
    from mx_qlinear import _lib
    from mx_qlinear.ops import _gemm_ws, _p

    want = torch.full((pb["m"], pb["n"]), float("nan"), dtype=torch.bfloat16, device=dev)
    work = torch.empty((min(chunk, pb["n"]), pb["k"]), dtype=torch.int8, device=dev)
    gws = _gemm_ws(dev) if queued else (None, 0)
    _lib.call("mxq_w4a8_codebook_gemm", _p(pb["xq"]), _p(pb["qd"]), _p(pb["sr"]), pb["code"], _p(pb["cb"]),
              _p(pb["sch"]), _p(pb["xs"]), _p(pb["b"]), _p(work), _p(want), pb["m"], pb["n"], pb["k"], pb["g"], chunk,
              _lib.DTYPE_BF16, *gws, st)
    return want


def _noalloc_entry(dev, pb, chunk, st):
    from mx_qlinear import _lib
    from mx_qlinear.ops import _p

    got = torch.full((pb["m"], pb["n"]), float("nan"), dtype=torch.bfloat16, device=dev)
    _lib.call("mxq_w4a8_codebook_gemm_noalloc", _p(pb["xq"]), _p(pb["qd"]), _p(pb["sr"]), pb["code"], _p(pb["cb"]),
              _p(pb["sch"]), _p(pb["xs"]), _p(pb["b"]), _p(got), pb["m"], pb["n"], pb["k"], pb["g"], chunk,
              _lib.DTYPE_BF16, st)
    return got


def _call_pair(dev, m, n, k, g, e4m3, codebook, bias, chunk, seed, queued=False):
    from mx_qlinear import _lib
    from mx_qlinear.ops import _stream

    if queued:  # each chunk GEMM claims tiles at run time
        plan = _lib.gemm_plan(m, min(chunk, n), k)
        assert plan["pool"] > 0, plan

    print(f"no-alloc w4a8 m={m} n={n} k={k} g={g} e4m3={e4m3} codebook={codebook} chunk={chunk}", flush=True)
    pb = _problem(dev, m, n, k, g, e4m3, codebook, bias, seed)
    st = _stream(dev)
    want = _workspace_entry(dev, pb, chunk, queued, st)
    got = _noalloc_entry(dev, pb, chunk, st)
    torch.cuda.synchronize()
    assert not bool(torch.isnan(want).any())
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_matches_workspace_entry_two_calls(dev):
    # first call: several chunks, e4m3 scales, codebook, bias
    _call_pair(dev, 300, 5000, 1024, 16, True, True, True, 2048, 7001)
    # second call, smaller: one chunk, fp32 scales, no codebook, no bias; the array keeps the
    # first call's decode beyond this one's chunk, which must not leak into the result
    _call_pair(dev, 64, 700, 512, 16, False, False, False, 4096, 7002)


def test_noalloc_chunk_gemms_claim_tiles_like_the_workspace_entry(dev):
    # 8192 x 4096 chunks (512 tiles of 256) and 8000 x 4500 (576): the static counters must be
    # back at zero after the first call for the second to match
    _call_pair(dev, 8192, 8192, 1024, 16, True, True, True, 4096, 7101, queued=True)
    _call_pair(dev, 8000, 4500, 512, 16, False, True, False, 4500, 7102, queued=True)


def test_noalloc_rejects_a_chunk_beyond_the_static_workspace(dev):
    from mx_qlinear import _lib
    from mx_qlinear.ops import _p, _stream

    m, n, k, g = 8, 8192, 8192, 16
    xq = torch.zeros((m, k), dtype=torch.int8, device=dev)
    xs = torch.ones(m, dtype=torch.float32, device=dev)
    qd = torch.zeros((n, k // 2), dtype=torch.int8, device=dev)
    sr = torch.ones((n, k // g), dtype=torch.float32, device=dev)
    sch = torch.ones(n, dtype=torch.float32, device=dev)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    # 4096 x 8192 = 32 MiB fits; 4097 columns do not (the check runs before any launch)
    with pytest.raises(ValueError, match="static workspace"):
        _lib.call("mxq_w4a8_codebook_gemm_noalloc", _p(xq), _p(qd), _p(sr), _lib.DTYPE_F32, None, _p(sch), _p(xs),
                  None, _p(out), m, n, k, g, 4097, _lib.DTYPE_BF16, _stream(dev))


def test_noalloc_calls_on_two_streams_are_ordered(dev):
    """Two calls on two streams issued back to back with no host wait between them: the second
    call's stream waits for the first call (the entry point's order event), so neither call's
    decode overwrites the static array while the other's GEMMs read it. Both outputs equal the
    workspace entry's, computed beforehand on the current stream."""
    from mx_qlinear.ops import _stream

    print("no-alloc w4a8 two streams", flush=True)
    a = _problem(dev, 2048, 8192, 1024, 16, True, True, True, 7201)
    b = _problem(dev, 1024, 6000, 1024, 16, False, True, False, 7202)
    want_a = _workspace_entry(dev, a, 4096, False, _stream(dev))
    want_b = _workspace_entry(dev, b, 3000, False, _stream(dev))
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    got_a = torch.empty(0, device=dev)
    got_b = torch.empty(0, device=dev)
    for _ in range(3):
        with torch.cuda.stream(s1):
            got_a = _noalloc_entry(dev, a, 4096, s1.cuda_stream)
        with torch.cuda.stream(s2):
            got_b = _noalloc_entry(dev, b, 3000, s2.cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(got_a.view(torch.int16), want_a.view(torch.int16))
        assert torch.equal(got_b.view(torch.int16), want_b.view(torch.int16))


def test_noalloc_call_replays_in_a_graph(dev):
    """Captured in a HIP graph (where the entry point makes no order wait or record), the call
    replays to the workspace entry's result; between replays an eager call of another problem
    overwrites the static array, and the next replay decodes its own chunks again."""
    from mx_qlinear.ops import _stream

    print("no-alloc w4a8 graph replay", flush=True)
    a = _problem(dev, 1024, 6000, 1024, 16, True, True, True, 7301)
    other = _problem(dev, 512, 8192, 1024, 16, False, False, True, 7302)
    want = _workspace_entry(dev, a, 4096, False, _stream(dev))
    want_other = _workspace_entry(dev, other, 4096, False, _stream(dev))
    torch.cuda.synchronize()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # the first call per device looks up the arrays outside the capture
        _noalloc_entry(dev, a, 4096, side.cuda_stream)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = _noalloc_entry(dev, a, 4096, _stream(dev))
    for r in range(3):
        eager = _noalloc_entry(dev, other, 4096, _stream(dev))  # overwrites the static array
        torch.cuda.synchronize()
        assert torch.equal(eager.view(torch.int16), want_other.view(torch.int16))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {r} differs"
    del graph

