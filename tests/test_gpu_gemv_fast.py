"""GPU tests of FAST mode (matrix-core int8 dot products, split-K).

FAST mode is not bit-identical to the reference; it is held to two bounds,
both stated per row against the reference kernel's own result y_ref (the
oracle's restatement of matvec_v{3,4}_fused) and the float64 truth y_true:
  * |y - y_true| <= 1e-6 * sum_k (|zp_k| + code_k*scale_k) * |x_k|
    FAST evaluates each block as scale*sum(code*x) + zp*sum(x), so its
    rounding is relative to the two dequantisation components, not to
    w = zp + code*scale after their cancellation (a block whose weights are
    all exactly 0 still carries the fp32 rounding of 0.25*sum(x) twice). The
    reference's own v4 test normalises by term magnitude with 0.02
    (wpc-eval/src/fused_kernel.rs:676-682).
  * max over EVERY row of |y - y_true| / max(|y_true|, floor) < 1e-4, the
    reference's own test form (|got - exp| / max(|exp|, 1e-6) < 1e-4,
    wpc-eval/src/fused_kernel.rs:589-625) with the floor stated as 1% of the
    rms output. A floor scaled to the outputs is needed: below it a relative
    error measures fp32 summation order alone, and the reference kernel
    itself (the oracle's AVX2 restatement) is 1.45e-3 from float64 on the v3
    q_proj shape with the literal 1e-6 floor, 6.2e-4 with a floor of 0.1% of
    the rms output.
and against the reference kernel's own result y_ref (the oracle's AVX2
restatement, the same intrinsics in the same order), the north star's
"within 1e-4 max relative error with fp32 accumulation":
  * |y - y_ref| <= 2e-6 * the row's term magnitude: the first bound plus the
    reference kernel's own fp32 accumulation error (measured <= 3.4e-8 of
    the term magnitude over every shape below);
  * max over EVERY row of |y - y_ref| / max(|y_ref|, floor) < 1e-4 with the
    floor 5% of the rms output. Both kernels accumulate in fp32, in
    different orders; at a 1% floor the reference kernel is itself 2.0e-4
    from float64 on these shapes (2560x9728 v4), so no other summation
    order can be held within 1e-4 of it there. At 5% the reference's own
    distance from float64 is 4.3e-5, leaving FAST the rest.
A wrong code, lane or block index moves a row by ~1% of its term magnitude,
four orders of magnitude above the first bound.
"""
REL_TOL = 1e-4
FLOOR_OF_RMS = 1e-2
REF_FLOOR_OF_RMS = 5e-2
import numpy as np
import pytest

import oracle as O
import wpcg
from wpcg import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = wpcg.Context(0)
    yield c
    c.close()


def dequant_parts(scheme, blocks, rows, cols):
    """Natural-order zero points and code*scale, fp32, [rows, cols] each."""
    bpb = 68 if scheme == 4 else 100
    b = blocks.reshape(-1, bpb)
    zp = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    sc = b[:, 2:4].copy().view(np.float16).astype(np.float32)
    if scheme == 4:
        p = b[:, 4:]
        codes = np.concatenate([p & 15, p >> 4], axis=1)
    else:
        p = b[:, 4:].reshape(-1, 32, 3).astype(np.uint32)
        w = p[..., 0] | p[..., 1] << 8 | p[..., 2] << 16
        codes = np.stack([(w >> (6 * q)) & 63 for q in range(4)], axis=-1).reshape(-1, 128)
    zp_full = np.broadcast_to(zp, codes.shape).reshape(rows, cols)
    return zp_full, (codes.astype(np.float32) * sc).reshape(rows, cols)


def dequant_f32(scheme, blocks, rows, cols):
    """Natural-order fp32 weights zp + code*scale (two roundings)."""
    zp, cs = dequant_parts(scheme, blocks, rows, cols)
    return (zp + cs).astype(np.float32)


def check_fast(y, scheme, blocks, rows, cols, x, what, bias=None):
    zp, cs = dequant_parts(scheme, blocks, rows, cols)
    W = (zp + cs).astype(np.float32).astype(np.float64)
    x64 = x.astype(np.float64)
    y_true = W @ x64
    mag = (np.abs(zp.astype(np.float64)) + np.abs(cs.astype(np.float64))) @ np.abs(x64)
    if bias is not None:
        y_true = y_true + bias
    kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
    y_ref = O.linear_matvec(scheme, blocks, rows, cols, x, bias, kern, 8).astype(np.float64)
    err = np.abs(y.astype(np.float64) - y_true)
    worst = int(np.argmax(err / mag))
    assert np.all(err <= 1e-6 * mag), (
        f"{what}: row {worst} |y-y_true|={err[worst]:.3e} > 1e-6*{mag[worst]:.3e}")
    floor = FLOOR_OF_RMS * np.sqrt(np.mean(y_true ** 2))
    ref_floor = REF_FLOOR_OF_RMS * np.sqrt(np.mean(y_ref ** 2))
    yd = y.astype(np.float64)
    rel = float(np.max(err / np.maximum(np.abs(y_true), floor)))
    err_ref = np.abs(yd - y_ref)
    rel_ref = float(np.max(err_ref / np.maximum(np.abs(y_ref), ref_floor)))
    ref_own = float(np.max(np.abs(y_ref - y_true) / np.maximum(np.abs(y_true), ref_floor)))
    print(f"[gpu] {what}: max rel error over all {rows} rows: {rel:.2e} vs float64 (floor {floor:.2e}); "
          f"{rel_ref:.2e} vs the reference kernel (floor {ref_floor:.2e}; the reference's own vs float64 "
          f"{ref_own:.2e})", flush=True)
    assert rel < REL_TOL, f"{what}: max relative error {rel:.3e} vs float64 (floor {floor:.2e})"
    worst_r = int(np.argmax(err_ref / mag))
    assert np.all(err_ref <= 2e-6 * mag), (
        f"{what}: row {worst_r} |y-y_ref|={err_ref[worst_r]:.3e} > 2e-6*{mag[worst_r]:.3e}")
    assert rel_ref < REL_TOL, f"{what}: max relative error {rel_ref:.3e} vs the reference kernel"
    return rel, float((err / mag).max())


SHAPES = [
    (4, 4864, 896),    # config 0
    (4, 1024, 2560),   # k/v_proj
    (4, 2560, 9728),   # down_proj (split K)
    (4, 2560, 4096),   # o_proj
    (4, 768, 2048),    # MoE expert gate/up
    (4, 2048, 768),    # MoE expert down
    (4, 151, 128),     # one block, ragged tile
    (4, 33, 4224),     # 33 blocks, ragged rows
    (3, 4096, 2560),   # config 1 shapes, v3
    (3, 9728, 2560),
    (3, 2560, 9728),
    (3, 37, 640),
    (4, 8200, 640),    # 513 tiles of 5 blocks: two tiles per workgroup (one in the last)
    (4, 4864, 896),    # config 0: 304 tiles of 7 blocks, two tiles per workgroup
    (4, 4080, 896),    # 255 tiles of 7 blocks: four tiles per workgroup, three in the last
    (4, 488, 2560),    # 31 tiles: one tile per workgroup
    (4, 520, 4096),    # 33 tiles, 32 blocks: one tile per workgroup (two from 192 tiles)
    (3, 3056, 4096),   # 191 tiles, 32 blocks: one tile per workgroup
    (3, 3080, 4096),   # 193 tiles, 32 blocks: two tiles per workgroup, odd tile count
    (4, 2032, 9728),   # 127 tiles, 76 blocks: one tile per workgroup, 3 K-slices
    (4, 2056, 9728),   # 129 tiles, 76 blocks: two tiles per workgroup, 3 K-slices
    (3, 8195, 8320),   # two tiles per workgroup, 65 blocks: two K-slices
    (4, 32784, 2048),  # four tiles per workgroup, 2049 tiles (one in the last workgroup)
    (3, 33001, 1152),  # four tiles per workgroup, ragged last tile
    (4, 32784, 2176),  # 2049 tiles but 17 blocks: two tiles per workgroup
]


@pytest.mark.parametrize("scheme,rows,cols", SHAPES)
def test_fast_matches_reference_within_tolerance(ctx, scheme, rows, cols):
    print(f"[gpu] fast v{scheme} {rows}x{cols}", flush=True)
    gen = synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks
    blocks = gen(rows, cols, seed=rows + 3 * cols)
    x = synth.random_x(cols, seed=cols + 5)
    lin = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks, rows, cols).set_mode(wpcg.MODE_FAST)
    y = lin.matvec(x)
    check_fast(y, scheme, blocks, rows, cols, x, f"v{scheme} {rows}x{cols}")
    # split-K partials are added in slice order: repeated calls are identical
    y2 = lin.matvec(x)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("scheme,rows,cols", SHAPES)
def test_valu_kernel_matches_reference_within_tolerance(ctx, scheme, rows, cols):
    """WPCG_FAST_KERNEL_VALU: the same GEMVs on the vector-ALU kernel (fp32
    x, codes unpacked by shift/mask, fp32 FMAs in its own order), held to
    the same bounds against float64 and the reference kernel; deterministic
    run to run, K-split handoffs included."""
    print(f"[gpu] valu v{scheme} {rows}x{cols}", flush=True)
    gen = synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks
    blocks = gen(rows, cols, seed=rows + 3 * cols)
    x = synth.random_x(cols, seed=cols + 5)
    lin = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks, rows, cols).set_mode(wpcg.MODE_FAST)
    lin.set_fast_kernel(wpcg.FAST_KERNEL_VALU)
    y = lin.matvec(x)
    check_fast(y, scheme, blocks, rows, cols, x, f"valu v{scheme} {rows}x{cols}")
    y2 = lin.matvec(x)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def test_valu_kernel_bias_extremes_and_groups(ctx):
    """The vector-ALU kernel with a bias, the extreme inputs of the MFMA
    test, and grouped launches (q/k/v-shaped problems of one launch) equal to
    separate launches bit for bit."""
    rows, cols = 300, 1280
    blocks = synth.random_v4_blocks(rows, cols, 77)
    bias = synth.random_x(rows, 78)
    lin = wpcg.WpcLinear.from_blocks(ctx, 4, blocks, rows, cols, bias=bias).set_mode(wpcg.MODE_FAST)
    lin.set_fast_kernel(wpcg.FAST_KERNEL_VALU)
    rng = np.random.default_rng(79)
    x = rng.standard_normal(cols).astype(np.float32)
    x[:128] = 0.0
    x[128:256] = 1e-30
    x[256:384] *= 1e4
    x[400] = -7e5
    check_fast(lin.matvec(x), 4, blocks, rows, cols, x, "valu extremes", bias=bias.astype(np.float64))
    shapes = [(3, 4096, 2560), (3, 1024, 2560), (3, 1024, 2560)]
    lins = []
    for i, (sch, r, c) in enumerate(shapes):
        b = synth.random_v3_blocks(r, c, seed=900 + i)
        lins.append(wpcg.WpcLinear.from_blocks(ctx, sch, b, r, c).set_mode(wpcg.MODE_FAST)
                    .set_fast_kernel(wpcg.FAST_KERNEL_VALU))
    xg = synth.random_x(2560, seed=905)
    xd = ctx.upload(xg)
    ys = [ctx.alloc(4 * r) for _, r, _ in shapes]
    wpcg.matvec_multi(lins, [xd] * 3, ys)
    ctx.sync()
    for l, yb, (_, r, _) in zip(lins, ys, shapes):
        assert np.array_equal(yb.read(np.float32, r).view(np.uint32), l.matvec(xg).view(np.uint32))


def test_fast_with_bias_and_extreme_inputs(ctx):
    rows, cols = 300, 1280
    blocks = synth.random_v4_blocks(rows, cols, 77)
    bias = synth.random_x(rows, 78)
    lin = wpcg.WpcLinear.from_blocks(ctx, 4, blocks, rows, cols, bias=bias).set_mode(wpcg.MODE_FAST)
    rng = np.random.default_rng(79)
    x = rng.standard_normal(cols).astype(np.float32)
    x[:128] = 0.0                                # an all-zero block of x
    x[128:256] *= np.float32(1e-30)              # a block of tiny values
    x[256:384] *= np.float32(1e4)                # a block of large values
    x[400] = np.float32(-7e5)                    # one outlier in a block
    check_fast(lin.matvec(x), 4, blocks, rows, cols, x, "extremes", bias=bias.astype(np.float64))


def test_fast_every_code_value(ctx):
    x = (np.arange(256, dtype=np.float32) * np.float32(0.01) - np.float32(0.6)).astype(np.float32)
    for scheme, n in ((4, 16), (3, 64)):
        rows = []
        for v in range(n):
            for _ in range(2):
                blk = np.zeros(68 if scheme == 4 else 100, np.uint8)
                blk[0:2] = np.array([np.float16(-0.25)]).view(np.uint8)
                blk[2:4] = np.array([np.float16(0.03125)]).view(np.uint8)
                codes = np.full(128, v, np.uint8)
                blk[4:] = O.v4_pack(codes) if scheme == 4 else O.v3_pack(codes)
                rows.append(blk)
        blocks = np.concatenate(rows)
        lin = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks, n, 256).set_mode(wpcg.MODE_FAST)
        check_fast(lin.matvec(x), scheme, blocks, n, 256, x, f"every code v{scheme}")


def test_grouped_launch_equals_separate_launches(ctx):
    # q/k/v share x; gate/up share another x; plus one v3 member and one
    # EXACT member, which the group runs in launches of their own.
    specs = [(4, 4096, 2560, "f"), (4, 1024, 2560, "f"), (4, 1024, 2560, "f"),
             (4, 9728, 2560, "f"), (4, 9728, 2560, "f"), (3, 512, 2560, "f"), (4, 256, 2560, "e")]
    lins, xs, ys, refs = [], [], [], []
    x = synth.random_x(2560, 91)
    xb = ctx.upload(x)
    for i, (scheme, r, c, mode) in enumerate(specs):
        gen = synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks
        lin = wpcg.WpcLinear.from_blocks(ctx, scheme, gen(r, c, 200 + i), r, c)
        lin.set_mode(wpcg.MODE_FAST if mode == "f" else wpcg.MODE_EXACT)
        lins.append(lin)
        xs.append(xb)
        ys.append(ctx.alloc(4 * r))
        refs.append(lin.matvec(x))
    wpcg.matvec_multi(lins, xs, ys)
    ctx.sync()
    for lin, y, ref in zip(lins, ys, refs):
        got = y.read(np.float32, lin.out_features())
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_graph_replays_match_eager(ctx):
    # Split-K counters reset inside the kernel, so every replay of a captured
    # graph must give the eager result; eager work runs between replays.
    r1, r2, c = 2560, 1024, 9728
    a = wpcg.WpcLinear.from_blocks(ctx, 4, synth.random_v4_blocks(r1, c, 301), r1, c).set_mode(wpcg.MODE_FAST)
    b = wpcg.WpcLinear.from_blocks(ctx, 3, synth.random_v3_blocks(r2, c, 302), r2, c).set_mode(wpcg.MODE_FAST)
    x = synth.random_x(c, 303)
    xb, ya, yb = ctx.upload(x), ctx.alloc(4 * r1), ctx.alloc(4 * r2)
    ea, eb = a.matvec(x), b.matvec(x)

    def body():
        a.matvec_dev(xb, ya)
        b.matvec_dev(xb, yb)

    g = ctx.capture(body)
    for rep in range(4):
        ya.write(np.full(r1, np.nan, np.float32))
        g.launch()
        ctx.sync()
        assert np.array_equal(ya.read(np.float32, r1).view(np.uint32), ea.view(np.uint32)), rep
        assert np.array_equal(yb.read(np.float32, r2).view(np.uint32), eb.view(np.uint32)), rep
        assert np.array_equal(a.matvec(x).view(np.uint32), ea.view(np.uint32))


def test_clone_computes_the_same(ctx):
    rows, cols = 2560, 4096
    lin = wpcg.WpcLinear.from_blocks(ctx, 4, synth.random_v4_blocks(rows, cols, 400), rows, cols)
    x = synth.random_x(cols, 401)
    for mode in (wpcg.MODE_EXACT, wpcg.MODE_FAST):
        lin.set_mode(mode)
        c = lin.clone()
        assert np.array_equal(c.matvec(x).view(np.uint32), lin.matvec(x).view(np.uint32))
        c.close()


@pytest.mark.parametrize("scheme,rows,cols", [(4, 1024, 2560), (3, 96, 9728)])
def test_every_k_split_gives_the_same_rows(ctx, scheme, rows, cols):
    # Every split the library accepts, including requests that would leave an
    # empty trailing slice before normalisation (nb=20 with 6, 8, 12 slices).
    gen = synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks
    blocks = gen(rows, cols, seed=500 + cols)
    x = synth.random_x(cols, 501)
    lin = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks, rows, cols).set_mode(wpcg.MODE_FAST)
    nb = cols // 128
    seen = {}
    for req in range(1, nb + 1):
        lin.set_kslices(req)
        k = lin.kslices()
        assert k == wpcg.plan_kslices(rows, cols, req)
        print(f"[gpu] split request {req} -> {k}", flush=True)
        y = lin.matvec(x)
        if k not in seen:
            check_fast(y, scheme, blocks, rows, cols, x, f"kslices={k}")
            seen[k] = y
        assert np.array_equal(y.view(np.uint32), seen[k].view(np.uint32))
