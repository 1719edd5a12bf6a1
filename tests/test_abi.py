"""The C ABI without a GPU: the library loads, exports every function the header declares
with the argument list the ctypes table uses, and rejects bad requests on the host before
any launch (the error paths of the reference's launchers and bindings, e.g.
CK/backends/cuda/ops/cutlass_gemm_int8.cu:613-665, w4a8_gemm.cu:93-164)."""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mx_qlinear.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"^(?:const char\*|int)\s+(mxq_\w+)\s*\(([^;]*)\)\s*;", text, re.M):
        args = [a.strip() for a in m.group(2).replace("\n", " ").split(",")]
        decls[m.group(1)] = [] if args == ["void"] else args
    return decls


@pytest.fixture(scope="module")
def lib():
    from mx_qlinear import _lib

    if not _lib.LIB_PATH.exists():
        from mx_qlinear import build

        build.build()
    return _lib.load()


def test_header_declares_the_ctypes_table():
    from mx_qlinear import _lib

    decls = _declared()
    assert set(_lib.SIGNATURES) | {"mxq_last_error", "mxq_abi_version"} == set(decls)
    for name, argtypes in _lib.SIGNATURES.items():
        assert len(argtypes) == len(decls[name]), name
        for ctype, decl in zip(argtypes, decls[name]):
            if ctype is ctypes.c_int64:
                assert decl.startswith("int64_t"), (name, decl)
            elif ctype is ctypes.c_int:
                assert decl.startswith("int "), (name, decl)
            elif ctype is ctypes.c_float:
                assert decl.startswith("float "), (name, decl)
            else:
                assert "*" in decl, (name, decl)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version_and_error_string(lib):
    from mx_qlinear import _lib

    assert lib.mxq_abi_version() == _lib.ABI_VERSION == 5
    lib.mxq_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.mxq_last_error(), bytes)
    # a rejected call leaves a message naming the problem
    rc = _lib.load().mxq_int8_gemm_i32(None, None, None, -1, 4, 16, 4, None, 0, None)
    assert rc == _lib.MXQ_ERR_INVALID
    assert b"negative" in lib.mxq_last_error()


@pytest.mark.parametrize(
    "args, code",
    [
        ((-1, 16, 16, 16), "INVALID"),   # negative M
        ((16, 16, 24, 16), "UNSUPPORTED"),  # K not a multiple of 16
        ((16, 16, 131072, 16), "UNSUPPORTED"),  # K beyond the int32 accumulator bound
        ((16, 32, 16, 16), "INVALID"),   # ldc < N
        ((16, 16, 0, 16), "UNSUPPORTED"),  # K == 0 with a non-empty output
    ],
)
def test_gemm_shape_checks(lib, args, code):
    from mx_qlinear import _lib

    m, n, k, ldc = args
    dummy = ctypes.c_void_p(16)  # never dereferenced: every case is rejected on the host
    rc = lib.mxq_int8_gemm_i32(dummy, dummy, dummy, m, n, k, ldc, None, 0, None)
    assert rc == getattr(_lib, "MXQ_ERR_" + code)


def test_empty_gemm_is_a_no_op(lib):
    from mx_qlinear import _lib

    assert lib.mxq_int8_gemm_i32(None, None, None, 0, 0, 16, 0, None, 0, None) == _lib.MXQ_OK


def test_dequant_rejects_bad_scale_count_and_dtype(lib):
    from mx_qlinear import _lib

    d = ctypes.c_void_p(256)
    rc = lib.mxq_int8_gemm_dequant(d, d, d, d, 3, None, d, 16, 16, 16, 16, _lib.DTYPE_BF16, None, 0, None)
    assert rc == _lib.MXQ_ERR_INVALID
    rc = lib.mxq_int8_gemm_dequant(d, d, d, d, 16, None, d, 16, 16, 16, 16, 7, None, 0, None)
    assert rc == _lib.MXQ_ERR_UNSUPPORTED


def test_gemm_rejects_a_misaligned_workspace(lib):
    from mx_qlinear import _lib

    d = ctypes.c_void_p(256)
    rc = lib.mxq_int8_gemm_i32(d, d, d, 16, 16, 16, 16, ctypes.c_void_p(4096 + 64), 1 << 20, None)
    assert rc == _lib.MXQ_ERR_INVALID
    assert b"256-byte aligned" in lib.mxq_last_error()


def test_gemm_workspace_size_matches_the_header():
    from mx_qlinear import _lib

    text = (ROOT / "include" / "mx_qlinear.h").read_text()
    assert "#define MXQ_GEMM_WORKSPACE_BYTES ((int64_t)4096)" in text
    assert _lib.GEMM_WORKSPACE_BYTES == 4096
    assert f"#define MXQ_ABI_VERSION {_lib.ABI_VERSION}" in text


def test_python_maps_codes_to_the_reference_exceptions(lib):
    from mx_qlinear import _lib

    with pytest.raises(ValueError):
        _lib.call("mxq_int8_gemm_i32", None, None, None, -1, 4, 16, 4, None, 0, None)
    with pytest.raises(RuntimeError):
        d = ctypes.c_void_p(16)
        _lib.call("mxq_int8_gemm_i32", d, d, d, 16, 16, 24, 16, None, 0, None)


@pytest.mark.parametrize(
    "m,n,k,table,tile,queued",
    [
        (75600, 5120, 20480, False, 256, True),   # FFN fc2 at 720p
        (75600, 20480, 5120, True, 256, True),    # FFN fc1 (planned as a GELU table epilogue)
        (75600, 28672, 5376, 2, 256, True),       # H3 fc1 with the SwiGLU epilogue (compact table)
        (75600, 15360, 5120, False, 256, True),   # QKV at 720p
        (8192, 5120, 5120, False, 128, True),     # 2.5 rounds of 128-tiles
        (1024, 3072, 3072, False, 128, False),    # under two rounds: static order
    ],
)
def test_gemm_plan_queues_large_problems(lib, m, n, k, table, tile, queued):
    from mx_qlinear import _lib

    plan = _lib.gemm_plan(m, n, k, table)
    assert plan["tile"] == tile
    tiles = -(-m // tile) * -(-n // plan["tile_n"])
    assert plan["tiles"] == tiles
    if queued:
        per = tiles // 8
        assert plan["pool"] == -(-per // 8)
        # 256-tiles without the GELU table epilogue: one looping workgroup per CU (this host has
        # no GPU, so the library plans for 256 CUs); otherwise one workgroup per tile plus claimers
        assert plan["persistent"] == (tile == 256 and table != 1)
        if plan["persistent"]:
            assert plan["wg_per_xcd"] == 256 // 8
        else:
            assert plan["wg_per_xcd"] == per + (tiles % 8 > 0) + plan["pool"]
        assert plan["grid"] == 8 * plan["wg_per_xcd"]
    else:
        assert plan["pool"] == 0 and plan["grid"] == tiles and not plan["persistent"]
    static = _lib.gemm_plan(m, n, k, table, workspace_bytes=0)
    assert static["pool"] == 0 and static["grid"] == tiles and not static["persistent"]


@pytest.mark.parametrize(
    "m,n,table,tile,tile_n,ahead",
    [
        (1024, 3072, False, 128, 96, 4),    # 192 tiles of 128 -> 256 of 128 x 96, one per CU, deep ring
        (1100, 1800, False, 128, 96, 4),    # 135 tiles of 128 -> 171 of 128 x 96, both edges partial
        (2048, 2048, False, 128, 128, 4),   # exactly 256 tiles of 128 (352 of 128 x 96 would not fit)
        (1100, 192, False, 128, 128, 4),    # 18 tiles either way: the square tiles stay
        (2050, 2056, False, 128, 128, 2),   # 289 tiles of 128: two workgroups per CU
        (75600, 5120, False, 256, 256, 2),
        (1024, 3072, True, 256, 256, 2),    # table epilogues always take 256-tiles
        (1024, 3072, 2, 256, 256, 2),
    ],
)
def test_gemm_plan_ring_depth(lib, m, n, table, tile, tile_n, ahead):
    from mx_qlinear import _lib

    plan = _lib.gemm_plan(m, n, 1024, table)
    assert (plan["tile"], plan["tile_n"], plan["ahead"]) == (tile, tile_n, ahead)
    assert plan["tiles"] == -(-m // tile) * -(-n // tile_n)


def _tile_walk(t, tiles_m, tiles_n, group_m):
    """Tile (row, column) at position t of the GEMM's tile order (gemm_i8.hip tile_walk): groups
    of group_m tile-rows, walked column by column."""
    group = group_m * tiles_n
    first_m = (t // group) * group_m
    gm = min(tiles_m - first_m, group_m)
    return first_m + (t % group) % gm, (t % group) // gm


@pytest.mark.parametrize("m,n,group_m", [(1024, 3072, 4), (2048, 2048, 4), (1100, 1800, None), (2050, 2056, 2),
                                         (300, 5000, None), (75600, 5120, 4), (8192, 5120, 2)])
def test_tile_order_visits_every_tile_once(lib, m, n, group_m):
    """Deep-ring problems (every tile on its own CU at once) group their tile order so that each
    XCD's range of tiles is nearly square (fewer operand panels per XCD); every order is a
    permutation of the tiles."""
    from mx_qlinear import _lib

    plan = _lib.gemm_plan(m, n, 1024)
    if group_m is not None:
        assert plan["group_m"] == group_m
    tm, tn = -(-m // plan["tile"]), -(-n // plan["tile_n"])
    seen = {_tile_walk(t, tm, tn, plan["group_m"]) for t in range(tm * tn)}
    assert seen == {(i, j) for i in range(tm) for j in range(tn)}
    if plan["ahead"] == 4:
        # each XCD's range spans no more panels than the two-row order would
        per = -(-tm * tn // 8)
        for x in range(8):
            cells = [_tile_walk(t, tm, tn, plan["group_m"]) for t in range(x * per, min((x + 1) * per, tm * tn))]
            two = [_tile_walk(t, tm, tn, 2) for t in range(x * per, min((x + 1) * per, tm * tn))]
            panels = lambda c: len({i for i, _ in c}) + len({j for _, j in c})
            assert panels(cells) <= panels(two) + 1


def _queue_cover(tiles, pool, wg_per_xcd, order):
    """Positions the balanced tile queue hands out, for workgroups arriving in `order`: the rule
    the GEMM kernel's pick_tile applies (XCD x = bid % 8 takes position start_x + bid / 8 of its
    range while that is below count_x - pool; later workgroups claim pool slots, their own XCD's
    first, then the others' in turn, and leave when all are gone)."""
    per, rem = tiles // 8, tiles % 8

    def rng(x):
        return x * per + min(x, rem), per + (1 if x < rem else 0)

    taken, claims = [], [0] * 8
    for bid in order:
        x, k = bid % 8, bid // 8
        start, count = rng(x)
        if k < count - pool:
            taken.append(start + k)
            continue
        for j in range(8):
            y = (x + j) % 8
            i = claims[y]
            claims[y] += 1
            if i < pool:
                ys, yc = rng(y)
                taken.append(ys + yc - pool + i)
                break
    return taken


def _persistent_cover(tiles, pool, wg_per_xcd, seed):
    """Positions the looping ping-pong workgroups take (gemm_i8.hip pp_tiles / pp_claim): workgroup
    (x = bid % 8, k = bid / 8) walks start_x + k, start_x + k + W, ... below start_x + count_x -
    pool, then claims pool slots (its own XCD's counter first, then the others in turn, skipping
    counters it found drained) until all are drained. Workgroups advance one tile at a time in a
    seeded random interleaving (seed None: round robin)."""
    import random

    per, rem = tiles // 8, tiles % 8

    def rng(x):
        return x * per + min(x, rem), per + (1 if x < rem else 0)

    grid = 8 * wg_per_xcd
    claims = [0] * 8
    state = {}
    for bid in range(grid):
        x, k = bid % 8, bid // 8
        start, count = rng(x)
        state[bid] = {"next": start + k, "end": start + count - pool, "j": 0}
    taken, live = [], list(range(grid))
    r = random.Random(seed)
    while live:
        bid = live[0] if seed is None else r.choice(live)
        if seed is None:
            live.append(live.pop(0))
        st, x = state[bid], bid % 8
        if st["next"] is not None and st["next"] < st["end"]:
            taken.append(st["next"])
            st["next"] += wg_per_xcd
            continue
        st["next"] = None
        got = None
        while st["j"] < 8:
            y = (x + st["j"]) % 8
            i = claims[y]
            claims[y] += 1
            if i < pool:
                ys, yc = rng(y)
                got = ys + yc - pool + i
                break
            st["j"] += 1
        if got is None:
            live.remove(bid)
        else:
            taken.append(got)
    return taken


@pytest.mark.parametrize("m,n,table", [(75600, 5120, False), (75600, 20480, True), (10496, 8408, False),
                                       (8060, 4990, False), (75600, 28672, True), (75600, 15360, False)])
def test_tile_queue_plan_covers_every_tile_once(lib, m, n, table):
    """With the launch plan's pool and grid, every tile is taken exactly once whatever order the
    workgroups arrive in (here: dispatch order, reversed, and seeded shuffles; for looping
    workgroups, round robin and seeded random interleavings of their steps)."""
    import random

    from mx_qlinear import _lib

    plan = _lib.gemm_plan(m, n, 1024, table)
    assert plan["pool"] > 0 and plan["grid"] == 8 * plan["wg_per_xcd"]
    if plan["persistent"]:
        for seed in (None, 0, 1, 2):
            got = _persistent_cover(plan["tiles"], plan["pool"], plan["wg_per_xcd"], seed)
            assert sorted(got) == list(range(plan["tiles"]))
        return
    orders = [list(range(plan["grid"])), list(range(plan["grid"]))[::-1]]
    for seed in range(3):
        o = list(range(plan["grid"]))
        random.Random(seed).shuffle(o)
        orders.append(o)
    for order in orders:
        assert sorted(_queue_cover(plan["tiles"], plan["pool"], plan["wg_per_xcd"], order)) == list(range(plan["tiles"]))


def test_bench_matches_kernel_instances_by_template_prefix():
    """bench.py's counter passes find the dominant kernel by its symbol; GEMM instances carry a
    trailing tile-configuration template argument that the symbol leaves out."""
    import importlib.util
    import pathlib

    spec = importlib.util.spec_from_file_location("bench", pathlib.Path(__file__).resolve().parents[1] / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    m = bench._symbol_matches
    assert m("gemm_i8_kernel<1, 2, 256>", "void mxq::gemm_i8_kernel<1, 2, 256, false>(mxq::GemmArgs)")
    assert m("gemm_i8_kernel<1, 2, 128>", "void mxq::gemm_i8_kernel<1, 2, 128, true>(mxq::GemmArgs)")
    assert not m("gemm_i8_kernel<1, 2, 128>", "void mxq::gemm_i8_kernel<1, 2, 256, false>(mxq::GemmArgs)")
    assert not m("gemm_i8_kernel<1, 2, 256>", "void mxq::gemm_i8_kernel<4, 2, 256, false>(mxq::GemmArgs)")
    assert m("w4a8_g128_kernel", "void mxq::w4a8_g128_kernel<128, 3>(mxq::G128Args)")
