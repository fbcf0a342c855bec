"""GPU test of wpcg_linear_gemm_noalloc, the batched GEMM that allocates
nothing: its workspace is the library's fixed per-GPU device array instead
of the linear's own. Called through the C ABI (ctypes on libwpcg.so) and
checked bit for bit against wpcg_linear_gemm, the entry point it is a
variant of (same kernels, same K-splits): two calls in a row, the second
with a smaller input (so stale workspace contents of the first would show),
then the other dtypes, more rows than one launch takes, the size limit,
and the first batched call on a fresh linear made inside a HIP graph
capture, replayed several times with other work between the replays.
"""
import ctypes as C

import numpy as np
import pytest

import wpcg
from wpcg import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = wpcg.Context(0)
    yield c
    c.close()


def bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _linear(ctx, scheme, rows, cols, seed):
    gen = synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks
    return wpcg.WpcLinear.from_blocks(ctx, scheme, gen(rows, cols, seed), rows, cols).set_mode(wpcg.MODE_FAST)


def _x(M, cols, dtype, seed):
    X = np.random.default_rng(seed).standard_normal((M, cols)).astype(np.float32)
    return bf16_bits(X) if dtype == wpcg.DTYPE_BF16 else X


def _noalloc(ctx, lin, xd, dtype, M, yd):
    return wpcg.lib.wpcg_linear_gemm_noalloc(lin.h, xd.ptr, dtype, M, yd.ptr, None)


def _both(ctx, lin, rows, cols, M, dtype, seed):
    """(noalloc result, wpcg_linear_gemm result) for the same X."""
    xd = ctx.upload(_x(M, cols, dtype, seed))
    ya, yb = ctx.alloc(4 * M * rows), ctx.alloc(4 * M * rows)
    rc = _noalloc(ctx, lin, xd, dtype, M, ya)
    assert rc == wpcg.OK, wpcg.last_error()
    ctx.sync()
    got = ya.read(np.float32, M * rows)
    lin.gemm_dev(xd, M, yb, dtype)
    ctx.sync()
    want = yb.read(np.float32, M * rows)
    for b in (xd, ya, yb):
        b.free()
    return got, want


def same_bits(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32),
                          np.ascontiguousarray(b, np.float32).view(np.uint32))


def test_two_calls_in_a_row_second_smaller(ctx):
    """A 2560x9728 v4 matrix with 48 bf16 rows (packed path, split K), then a
    1024x2560 v3 matrix with 5 fp32 rows (small path): each bit-identical
    to wpcg_linear_gemm on the same input."""
    print("[gpu] noalloc: two calls, second smaller", flush=True)
    a = _linear(ctx, 4, 2560, 9728, 1)
    b = _linear(ctx, 3, 1024, 2560, 2)
    got, want = _both(ctx, a, 2560, 9728, 48, wpcg.DTYPE_BF16, 3)
    assert np.all(np.isfinite(want)) and same_bits(got, want)
    got, want = _both(ctx, b, 1024, 2560, 5, wpcg.DTYPE_F32, 4)
    assert np.all(np.isfinite(want)) and same_bits(got, want)
    a.close()
    b.close()


@pytest.mark.parametrize("scheme,rows,cols,M,dtype", [
    (4, 2560, 9728, 100, wpcg.DTYPE_F32_SPLIT),  # four launches of 32 rows
    (4, 2560, 9728, 130, wpcg.DTYPE_BF16),       # three launches of <= 64 rows
    (3, 4096, 2560, 16, wpcg.DTYPE_BF16),        # the small kernel
    (4, 3840, 15360, 64, wpcg.DTYPE_BF16),       # Gemma-12B down_proj (config 4)
    (4, 4864, 896, 1, wpcg.DTYPE_F32),           # M = 1 fp32: the matvec
    (4, 37, 384, 7, wpcg.DTYPE_F32),             # ragged tile
])
def test_matches_wpcg_linear_gemm(ctx, scheme, rows, cols, M, dtype):
    print(f"[gpu] noalloc: v{scheme} {rows}x{cols} M={M} dtype={dtype}", flush=True)
    lin = _linear(ctx, scheme, rows, cols, rows + cols)
    got, want = _both(ctx, lin, rows, cols, M, dtype, M)
    assert np.all(np.isfinite(want)) and same_bits(got, want)
    lin.close()


def test_workspace_beyond_the_array_is_refused(ctx):
    """16 rows x 1025 blocks: the packed X alone (16 KiB per block) exceeds
    the 16 MiB array; the call is refused before any launch and says why."""
    lin = _linear(ctx, 4, 16, 1025 * 128, 9)
    xd, yd = ctx.alloc(2 * 20 * 1025 * 128), ctx.alloc(4 * 20 * 16)
    rc = _noalloc(ctx, lin, xd, wpcg.DTYPE_BF16, 20, yd)
    assert rc == wpcg.E_UNSUPPORTED
    assert "bytes of workspace" in wpcg.last_error()
    assert wpcg.lib.wpcg_linear_gemm_noalloc(None, xd.ptr, 1, 20, yd.ptr, None) == wpcg.E_ARG
    assert wpcg.lib.wpcg_linear_gemm_noalloc(lin.h, xd.ptr, 7, 20, yd.ptr, None) == wpcg.E_ARG
    lin.close()
    xd.free()
    yd.free()


def test_first_batched_call_inside_a_graph_capture(ctx):
    """On a linear that never made a batched workspace, the allocating entry
    point refuses to run under capture; this one is captured, and every
    replay (with eager work and synchronization between replays) equals the
    eager result."""
    print("[gpu] noalloc: graph capture", flush=True)
    rows, cols, M = 2560, 4096, 24
    lin = _linear(ctx, 3, rows, cols, 21)
    other = _linear(ctx, 4, 1024, 2560, 22)
    xd = ctx.upload(_x(M, cols, wpcg.DTYPE_BF16, 23))
    yd, ye = ctx.alloc(4 * M * rows), ctx.alloc(4 * M * rows)
    with pytest.raises(wpcg.WpcgError):
        ctx.capture(lambda: lin.gemm_dev(xd, M, ye, wpcg.DTYPE_BF16))
    g = ctx.capture(lambda: wpcg.check(_noalloc(ctx, lin, xd, wpcg.DTYPE_BF16, M, yd)))
    wpcg.check(_noalloc(ctx, lin, xd, wpcg.DTYPE_BF16, M, ye))  # eager, same scratch
    ctx.sync()
    want = ye.read(np.float32, M * rows)
    ox = ctx.upload(_x(9, 2560, wpcg.DTYPE_BF16, 24))
    oy = ctx.alloc(4 * 9 * 1024)
    for rep in range(4):
        yd.write(np.full(M * rows, np.nan, np.float32))
        g.launch()
        ctx.sync()
        assert same_bits(yd.read(np.float32, M * rows), want), f"replay {rep}"
        # other work on the same array between replays
        wpcg.check(_noalloc(ctx, other, ox, wpcg.DTYPE_BF16, 9, oy))
        ctx.sync()
    del g
    for b in (xd, yd, ye, ox, oy):
        b.free()
    lin.close()
    other.close()
