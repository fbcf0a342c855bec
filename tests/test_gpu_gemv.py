"""GPU parity of the dequant-GEMV path against the CPU oracle.

EXACT mode must be bit-identical to the reference's AVX2 row kernels
(matvec_v4_fused / matvec_v3_fused, wpc-eval/src/fused_kernel.rs), i.e. to
the oracle's fused restatement, which tests/test_oracle_kernels.py pins
against the intrinsic sequence itself. Dequantization and the embedding
lookup are bit-exact in both rounding modes.
"""
import numpy as np
import pytest

import oracle as O
import wpcg
from wpcg import synth

pytestmark = pytest.mark.gpu

THREADS = 8


@pytest.fixture(scope="module")
def ctx():
    c = wpcg.Context(0)
    yield c
    c.close()


def oracle_y(scheme, blocks, rows, cols, x, bias=None):
    kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
    return O.linear_matvec(scheme, blocks, rows, cols, x, bias, kern, THREADS)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bit_equal(got, exp, what):
    d = np.flatnonzero(bits(got) != bits(exp))
    assert d.size == 0, (f"{what}: {d.size} of {exp.size} differ; first row {d[0]}: "
                         f"got {got[d[0]]!r} expected {exp[d[0]]!r}")


V4_SHAPES = [
    (4864, 896),    # config 0 (Qwen2.5-0.5B up_proj)
    (1, 128),       # one block
    (37, 256),      # rows not a multiple of a workgroup's 32
    (65, 4224),     # 33 blocks: crosses the 32-block LDS segment
    (1024, 2560),   # Qwen3 k/v_proj
    (2560, 9728),   # Qwen3 down_proj (76 blocks per row)
    (768, 2048),    # MoE expert gate/up
    (2048, 768),    # MoE expert down
]


@pytest.mark.parametrize("rows,cols", V4_SHAPES)
def test_v4_exact_is_bit_identical_to_the_reference_kernel(ctx, rows, cols):
    print(f"[gpu] v4 exact {rows}x{cols}", flush=True)
    blocks = synth.random_v4_blocks(rows, cols, seed=rows * 7 + cols)
    x = synth.random_x(cols, seed=cols)
    lin = wpcg.WpcLinear.from_blocks(ctx, 4, blocks, rows, cols)
    assert_bit_equal(lin.matvec(x), oracle_y(4, blocks, rows, cols, x), f"v4 {rows}x{cols}")
    lin.close()


V3_SHAPES = [
    (4096, 2560),   # q_proj      (config 1)
    (1024, 2560),   # k/v_proj
    (2560, 4096),   # o_proj
    (9728, 2560),   # gate/up_proj
    (2560, 9728),   # down_proj
    (3, 128),
    (45, 4224),
]


@pytest.mark.parametrize("rows,cols", V3_SHAPES)
def test_v3_exact_is_bit_identical_to_the_reference_kernel(ctx, rows, cols):
    print(f"[gpu] v3 exact {rows}x{cols}", flush=True)
    blocks = synth.random_v3_blocks(rows, cols, seed=rows * 11 + cols)
    x = synth.random_x(cols, seed=cols + 1)
    lin = wpcg.WpcLinear.from_blocks(ctx, 3, blocks, rows, cols)
    assert_bit_equal(lin.matvec(x), oracle_y(3, blocks, rows, cols, x), f"v3 {rows}x{cols}")
    lin.close()


@pytest.mark.parametrize("scheme", [3, 4])
def test_every_code_value(ctx, scheme):
    # fused_kernel.rs:631-650 through the GPU kernel: each row is one code
    # value in every position, with an f16-exact scale.
    n = 16 if scheme == 4 else 64
    x = (np.arange(256, dtype=np.float32) * np.float32(0.01) - np.float32(0.6)).astype(np.float32)
    rows = []
    for v in range(n):
        for b in range(2):
            blk = np.zeros(68 if scheme == 4 else 100, np.uint8)
            blk[0:2] = np.array([np.float16(-0.25)]).view(np.uint8)
            blk[2:4] = np.array([np.float16(0.03125)]).view(np.uint8)
            codes = np.full(128, v, np.uint8)
            blk[4:] = O.v4_pack(codes) if scheme == 4 else O.v3_pack(codes)
            rows.append(blk)
    blocks = np.concatenate(rows)
    lin = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks, n, 256)
    assert_bit_equal(lin.matvec(x), oracle_y(scheme, blocks, n, 256, x), "every code")


@pytest.mark.parametrize("scheme", [3, 4])
def test_bias_is_added_after_the_row_kernel(ctx, scheme):
    rows, cols = 300, 640
    blocks = (synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks)(rows, cols, 9)
    x = synth.random_x(cols, 10)
    bias = synth.random_x(rows, 11)
    lin = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks, rows, cols, bias=bias)
    assert_bit_equal(lin.matvec(x), oracle_y(scheme, blocks, rows, cols, x, bias), "bias")


def test_empty_inner_dimension_gives_zeros_plus_bias(ctx):
    bias = np.arange(5, dtype=np.float32)
    lin = wpcg.WpcLinear.from_blocks(ctx, 4, np.zeros(0, np.uint8), 5, 0, bias=bias)
    assert_bit_equal(lin.matvec(np.zeros(0, np.float32)), bias, "K=0")
    empty = wpcg.WpcLinear.from_blocks(ctx, 4, np.zeros(0, np.uint8), 0, 256)
    assert empty.matvec(np.zeros(256, np.float32)).size == 0


def test_device_and_host_matvec_agree(ctx):
    rows, cols = 777, 1536
    blocks = synth.random_v4_blocks(rows, cols, 21)
    x = synth.random_x(cols, 22)
    lin = wpcg.WpcLinear.from_blocks(ctx, 4, blocks, rows, cols)
    xb, yb = ctx.upload(x), ctx.alloc(rows * 4)
    lin.matvec_dev(xb, yb)
    ctx.sync()
    assert_bit_equal(yb.read(np.float32, rows), lin.matvec(x), "device vs host")


def _natural_codes(scheme, blocks):
    b = blocks.reshape(-1, 68 if scheme == 4 else 100)
    unpack = O.v4_unpack if scheme == 4 else O.v3_unpack
    return b, np.stack([unpack(r[4:]) for r in b])


@pytest.mark.parametrize("scheme", [3, 4])
def test_dequant_is_bit_exact_in_both_roundings(ctx, scheme):
    rows, cols = 64, 512
    blocks = (synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks)(rows, cols, 31)
    b, codes = _natural_codes(scheme, blocks)
    zp = b[:, 0:2].copy().view(np.float16).astype(np.float32)  # [nblk, 1]
    sc = b[:, 2:4].copy().view(np.float16).astype(np.float32)
    lin = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks, rows, cols)
    # two roundings: numpy float32 never fuses
    two = (zp + codes.astype(np.float32) * sc).astype(np.float32).reshape(rows, cols)
    # one rounding: code*scale + zp is exact in float64, then rounded once
    fma = (codes.astype(np.float64) * sc.astype(np.float64) + zp.astype(np.float64))
    fma = fma.astype(np.float32).reshape(rows, cols)
    assert_bit_equal(lin.dequant(wpcg.ROUND_TWO).ravel(), two.ravel(), "two-rounding dequant")
    assert_bit_equal(lin.dequant(wpcg.ROUND_FMA).ravel(), fma.ravel(), "fma dequant")


@pytest.mark.parametrize("scheme", [3, 4])
def test_embed_matches_row_decode(ctx, scheme):
    vocab, hidden = 1000, 2048
    blocks = (synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks)(vocab, hidden, 41)
    emb = wpcg.WpcLinear.from_blocks(ctx, scheme, blocks, vocab, hidden)
    for tok in (0, 1, 517, vocab - 1):
        assert_bit_equal(emb.embed(tok), O.embed(scheme, blocks, hidden, tok), f"embed {tok}")
    with pytest.raises(wpcg.WpcgError) as e:
        emb.embed(vocab)
    assert e.value.code == wpcg.E_ARG


def test_linear_from_artifact(ctx, tmp_path):
    up = synth.random_v4_blocks(320, 896, 51)
    down = synth.random_v4_blocks(896, 640, 52)
    synth.write_artifact(str(tmp_path), 4, [
        ("model.layers.0.mlp.down_proj.weight", [896, 640], down),
        ("model.layers.0.mlp.up_proj.weight", [320, 896], up)])
    data = wpcg.WpcModelDataV4.open(str(tmp_path))
    x = synth.random_x(896, 53)
    lin = wpcg.WpcLinearV4(ctx, data, "model.layers.0.mlp.up_proj.weight", 320, 896)
    assert (lin.in_features(), lin.out_features()) == (896, 320)
    assert_bit_equal(lin.matvec(x), oracle_y(4, up, 320, 896, x), "artifact up_proj")
    x2 = synth.random_x(640, 54)
    lin2 = wpcg.WpcLinearV4(ctx, data, "model.layers.0.mlp.down_proj.weight", 896, 640)
    assert_bit_equal(lin2.matvec(x2), oracle_y(4, down, 896, 640, x2), "artifact down_proj")
