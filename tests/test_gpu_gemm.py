"""GPU tests of the batched dequant-GEMM (wpcg_linear_gemm): Y = X W^T for
M activations on the bf16 matrix cores. The reference has no batched path
(it runs one token at a time, README.md:174-180); the comparison is the
fp32 dequant-then-matmul the benchmark configuration names, evaluated here
in float64 as the truth:

  * X given in bf16: the codes and X are exact matrix-core operands, so the
    only error is fp32 accumulation (128 products per block, then one
    scale*D + zp*S per block). Bound per output:
        |y - y_true| <= 3e-5 * sum_k (|zp_k| + code_k*scale_k) * |x_k|
  * X given in fp32: X is rounded to bf16 (relative 2^-9 per value), so
        |y - y_true| <= (2^-9 + 3e-5) * sum_k (|zp_k| + code_k*scale_k) * |x_k|
    with y_true computed from the unrounded X.
  * X given in fp32 with DTYPE_F32_SPLIT: hi = bf16(x) and lo = bf16(x - hi)
    both go through the matrix cores (|x - hi - lo| <= 2^-18 |x|), so the
    bf16-input bound holds with 2^-17 added; and, against a plain rounding
    to bf16, the largest error stays under 2e-5 of the largest |y|, which
    rounding X to bf16 exceeds by ~50x on these inputs.

A wrong k-order, lane, column or block index moves outputs by ~1% of the
same sum, 300x above the first bound; the bf16-input cases catch that.
"""
import numpy as np
import pytest

import oracle as O
import wpcg
from wpcg import synth

pytestmark = pytest.mark.gpu

TOL_ACC = 3e-5
TOL_BF16 = 2.0 ** -9 + TOL_ACC
TOL_SPLIT = 2.0 ** -17 + TOL_ACC
SPLIT_REL = 2e-5  # max |y - y_true| / max |y_true|, split X


@pytest.fixture(scope="module")
def ctx():
    c = wpcg.Context(0)
    yield c
    c.close()


def parts64(scheme, blocks, rows, cols):
    """float64 zero points and code*scale in natural order, [rows, cols]."""
    bpb = 68 if scheme == 4 else 100
    b = blocks.reshape(-1, bpb)
    zp = b[:, 0:2].copy().view(np.float16).astype(np.float64)
    sc = b[:, 2:4].copy().view(np.float16).astype(np.float64)
    if scheme == 4:
        p = b[:, 4:]
        codes = np.concatenate([p & 15, p >> 4], axis=1)
    else:
        p = b[:, 4:].reshape(-1, 32, 3).astype(np.uint32)
        w = p[..., 0] | p[..., 1] << 8 | p[..., 2] << 16
        codes = np.stack([(w >> (6 * q)) & 63 for q in range(4)], axis=-1).reshape(-1, 128)
    zp_full = np.broadcast_to(zp, codes.shape).reshape(rows, cols)
    return zp_full, (codes.astype(np.float64) * sc).reshape(rows, cols)


def to_bf16_bits(x):
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def check(Y, X_true, scheme, blocks, rows, cols, tol, bias=None, what=""):
    zp, cs = parts64(scheme, blocks, rows, cols)
    X64 = X_true.astype(np.float64)
    truth = X64 @ (zp + cs).T
    if bias is not None:
        truth = truth + bias.astype(np.float64)
    mag = np.abs(X64) @ (np.abs(zp) + cs).T
    err = np.abs(Y.astype(np.float64) - truth)
    worst = float(np.max(err / (mag + 1e-30)))
    assert np.all(err <= tol * mag + 1e-30), f"{what}: worst error {worst:.3g} of the term sum (bound {tol:.3g})"
    return worst


def make(ctx, scheme, rows, cols, seed, bias=None):
    gen = synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks
    blocks = gen(rows, cols, seed)
    lin = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks, rows, cols, bias)
    return lin, blocks


@pytest.mark.parametrize("scheme", [4, 3])
@pytest.mark.parametrize("rows,cols", [(70, 256), (16, 128), (1, 384), (300, 1280)])
@pytest.mark.parametrize("M", [2, 5, 16, 17, 40, 64, 100])
def test_gemm_bounds_small(ctx, scheme, rows, cols, M):
    print(f"[gpu] gemm v{scheme} {rows}x{cols} M={M}", flush=True)
    rng = np.random.default_rng(rows * 1000 + cols + M + scheme)
    bias = rng.standard_normal(rows).astype(np.float32)
    lin, blocks = make(ctx, scheme, rows, cols, seed=rows + cols + M, bias=bias)
    X = rng.standard_normal((M, cols)).astype(np.float32)
    Xb = to_bf16_bits(X)
    check(lin.gemm(Xb, wpcg.DTYPE_BF16), bf16_to_f32(Xb), scheme, blocks, rows, cols, TOL_ACC, bias, "bf16 X")
    check(lin.gemm(X), X, scheme, blocks, rows, cols, TOL_BF16, bias, "fp32 X")
    lin.close()


@pytest.mark.parametrize("scheme", [4, 3])
@pytest.mark.parametrize("M", [5, 16, 33])
def test_gemm_every_ksplit_and_determinism(ctx, scheme, M):
    rows, cols = 200, 128 * 70
    lin, blocks = make(ctx, scheme, rows, cols, seed=9)
    rng = np.random.default_rng(4)
    Xb = to_bf16_bits(rng.standard_normal((M, cols)).astype(np.float32))
    for kg in (1, 2, 3, 5, 7, 40, 70, 0):
        lin.set_gemm_kslices(kg)
        print(f"[gpu] gemm v{scheme} M={M} kslices={kg} -> {lin.gemm_kslices()}", flush=True)
        Y = lin.gemm(Xb, wpcg.DTYPE_BF16)
        check(Y, bf16_to_f32(Xb), scheme, blocks, rows, cols, TOL_ACC, None, f"kg={kg}")
        assert np.array_equal(lin.gemm(Xb, wpcg.DTYPE_BF16), Y), f"kg={kg}: not deterministic"
    lin.close()


def test_gemm_m1_is_the_gemv(ctx):
    rows, cols = 300, 2560
    lin, blocks = make(ctx, 4, rows, cols, seed=3)
    x = synth.random_x(cols, 5)
    for mode in (wpcg.MODE_EXACT, wpcg.MODE_FAST):
        lin.set_mode(mode)
        assert np.array_equal(lin.gemm(x[None, :])[0], lin.matvec(x))
    # bf16 input with M == 1 runs the matrix-core kernel
    xb = to_bf16_bits(x)[None, :]
    check(lin.gemm(xb, wpcg.DTYPE_BF16), bf16_to_f32(xb), 4, blocks, rows, cols, TOL_ACC, None, "M=1 bf16")
    lin.close()


def test_gemm_matches_the_reference_per_token_path(ctx):
    """Against M separate calls of the reference's fused kernel (the oracle's
    restatement of matvec_v4_fused), at the fp32-input bound."""
    rows, cols, M = 256, 1024, 16
    lin, blocks = make(ctx, 4, rows, cols, seed=21)
    X = np.random.default_rng(8).standard_normal((M, cols)).astype(np.float32)
    ref = O.linear_matmul_v4(blocks, rows, cols, X)
    zp, cs = parts64(4, blocks, rows, cols)
    mag = np.abs(X.astype(np.float64)) @ (np.abs(zp) + cs).T
    Y = lin.gemm(X)
    assert np.all(np.abs(Y - ref) <= TOL_BF16 * mag + 1e-30)
    lin.close()


def test_gemm_graph_replays_match_eager(ctx):
    rows, cols, M = 512, 2048, 64
    lin, _ = make(ctx, 4, rows, cols, seed=31)
    rng = np.random.default_rng(2)
    X = rng.standard_normal((M, cols)).astype(np.float32)
    eager = lin.gemm(X)  # also makes the workspace, before capture
    xd, yd = ctx.upload(X), ctx.alloc(M * rows * 4)
    graph = ctx.capture(lambda: lin.gemm_dev(xd, M, yd))
    for rep in range(4):
        yd.write(np.full(M * rows, np.nan, np.float32))
        graph.launch()
        ctx.sync()
        assert np.array_equal(yd.read(np.float32, M * rows).reshape(M, rows), eager), rep
        assert np.array_equal(lin.gemm(X), eager), rep  # eager work between replays
    lin.close()


def test_gemm_first_call_under_capture_is_refused(ctx):
    lin, _ = make(ctx, 4, 64, 256, seed=1)
    xd, yd = ctx.upload(np.zeros((4, 256), np.float32)), ctx.alloc(4 * 64 * 4)
    with pytest.raises(wpcg.WpcgError) as e:
        ctx.capture(lambda: lin.gemm_dev(xd, 4, yd))
    assert e.value.code == wpcg.E_ARG and "before capturing" in str(e.value)
    lin.close()


@pytest.mark.parametrize("rows,cols", [(15360, 3840), (3840, 15360)])
def test_gemm_config4_shapes(ctx, rows, cols):
    """Gemma-12B gate/up and down, v4, M = 4, 16, 64 (the benchmark's shapes)."""
    print(f"[gpu] gemm config-4 shape {rows}x{cols}", flush=True)
    lin, blocks = make(ctx, 4, rows, cols, seed=rows // 128)
    rng = np.random.default_rng(12)
    for M in (4, 16, 64):
        X = rng.standard_normal((M, cols)).astype(np.float32)
        Xb = to_bf16_bits(X)
        w = check(lin.gemm(Xb, wpcg.DTYPE_BF16), bf16_to_f32(Xb), 4, blocks, rows, cols, TOL_ACC, None,
                  f"M={M} bf16")
        print(f"[gpu]   M={M}: worst bf16-input error {w:.2e} of the term sum", flush=True)
        check(lin.gemm(X), X, 4, blocks, rows, cols, TOL_BF16, None, f"M={M} fp32")
    lin.close()


def rel_to_max(Y, X, scheme, blocks, rows, cols, bias=None):
    zp, cs = parts64(scheme, blocks, rows, cols)
    truth = X.astype(np.float64) @ (zp + cs).T
    if bias is not None:
        truth = truth + bias.astype(np.float64)
    return float(np.max(np.abs(Y - truth)) / np.max(np.abs(truth)))


@pytest.mark.parametrize("scheme", [4, 3])
@pytest.mark.parametrize("rows,cols", [(70, 256), (300, 1280), (1000, 2560)])
@pytest.mark.parametrize("M", [1, 3, 8, 9, 16, 17, 32, 45, 70])
def test_gemm_split_fp32(ctx, scheme, rows, cols, M):
    """DTYPE_F32_SPLIT: the small kernel (M <= 8 per launch), the packed
    kernel with hi and lo tiles (9..32), several launches (> 32)."""
    print(f"[gpu] gemm split v{scheme} {rows}x{cols} M={M}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols + M + scheme)
    bias = rng.standard_normal(rows).astype(np.float32)
    lin, blocks = make(ctx, scheme, rows, cols, seed=rows + 3 * cols + M, bias=bias)
    X = rng.standard_normal((M, cols)).astype(np.float32)
    Y = lin.gemm(X, wpcg.DTYPE_F32_SPLIT)
    check(Y, X, scheme, blocks, rows, cols, TOL_SPLIT, bias, "split X")
    r = rel_to_max(Y, X, scheme, blocks, rows, cols, bias)
    assert r <= SPLIT_REL, f"split X: {r:.2e} of max |y|"
    if M > 1 and cols >= 1280:  # the bf16-rounded path really is coarser
        assert rel_to_max(lin.gemm(X), X, scheme, blocks, rows, cols, bias) > 5 * r
    assert np.array_equal(lin.gemm(X, wpcg.DTYPE_F32_SPLIT), Y), "not deterministic"
    lin.close()


@pytest.mark.parametrize("M", [4, 24])
def test_gemm_split_every_ksplit(ctx, M):
    rows, cols = 200, 128 * 70
    lin, blocks = make(ctx, 4, rows, cols, seed=19)
    X = np.random.default_rng(6).standard_normal((M, cols)).astype(np.float32)
    for kg in (1, 3, 7, 0):
        lin.set_gemm_kslices(kg)
        Y = lin.gemm(X, wpcg.DTYPE_F32_SPLIT)
        check(Y, X, 4, blocks, rows, cols, TOL_SPLIT, None, f"split kg={kg}")
        assert rel_to_max(Y, X, 4, blocks, rows, cols) <= SPLIT_REL
    lin.close()
