"""Pins the oracle's row kernels (wpc-eval/src/fused_kernel.rs) and Linear.

The reference fixtures are restated from its tests; the reference
tolerances are kept. Independent checks: a float64 brute force of the
documented decode formula, and the reference's own AVX2 intrinsic sequence
(compiled from the oracle) which the lane-by-lane restatement must match
bit for bit.
"""
import numpy as np
import pytest

import oracle as O


def make_v4_blocks(codes_list, zps, scales):
    out = []
    for codes, zp, sc in zip(codes_list, zps, scales):
        blk = np.zeros(68, np.uint8)
        blk[0:2] = np.array([np.float16(zp)]).view(np.uint8)
        blk[2:4] = np.array([np.float16(sc)]).view(np.uint8)
        blk[4:] = O.v4_pack(codes)
        out.append(blk)
    return np.concatenate(out)


def multi_block_fixture_v4(n_blocks):
    # fused_kernel.rs:549-566
    i = np.arange(128)
    codes = [((i * 3 + bi * 5) % 16).astype(np.uint8) for bi in range(n_blocks)]
    zps = [np.float32(-0.4) + np.float32(bi) * np.float32(0.1) for bi in range(n_blocks)]
    scs = [np.float32(0.017) + np.float32(bi) * np.float32(0.003) for bi in range(n_blocks)]
    x = (np.sin(np.arange(n_blocks * 128, dtype=np.float32) * np.float32(0.013))
         + np.float32(0.5)).astype(np.float32)
    return make_v4_blocks(codes, zps, scs), x


def multi_block_fixture_v2(n_blocks):
    # fused_kernel.rs:433-452
    i = np.arange(128)
    out = []
    for bi in range(n_blocks):
        blk = np.zeros(132, np.uint8)
        blk[0:2] = np.array([np.float16(np.float32(-0.4) + np.float32(bi) * np.float32(0.1))]).view(np.uint8)
        blk[2:4] = np.array([np.float16(np.float32(0.017) + np.float32(bi) * np.float32(0.003))]).view(np.uint8)
        blk[4:] = ((i + bi * 13) % 64).astype(np.uint8)
        out.append(blk)
    x = (np.sin(np.arange(n_blocks * 128, dtype=np.float32) * np.float32(0.013))
         + np.float32(0.5)).astype(np.float32)
    return np.concatenate(out), x


def v2_to_v3(blocks_v2):
    # QuantBlockV3::from_v2 (wpc-format/src/lib.rs:281-288)
    b = blocks_v2.reshape(-1, 132)
    out = np.zeros((b.shape[0], 100), np.uint8)
    out[:, :4] = b[:, :4]
    for r in range(b.shape[0]):
        out[r, 4:] = O.v3_pack(b[r, 4:])
    return out.ravel()


def brute_dot(scheme, blocks, x):
    """float64 dot of the documented decode formula zp + code*scale."""
    bpb = {4: 68, 3: 100, 2: 132}[scheme]
    b = blocks.reshape(-1, bpb)
    acc = 0.0
    for bi in range(b.shape[0]):
        zp = float(O.f16_to_f32(b[bi, 0:2].view(np.uint16))[0])
        sc = float(O.f16_to_f32(b[bi, 2:4].view(np.uint16))[0])
        if scheme == 4:
            codes = O.v4_unpack(b[bi, 4:])
        elif scheme == 3:
            codes = O.v3_unpack(b[bi, 4:])
        else:
            codes = b[bi, 4:]
        w = zp + codes.astype(np.float64) * sc
        acc += float(np.dot(w, x[bi * 128:(bi + 1) * 128].astype(np.float64)))
    return acc


def rel(a, b):
    return abs(a - b) / max(abs(b), 1e-6)


# ------------------------------------------------------------------ v4
def test_scalar_v4_matches_the_reference_formula():
    # fused_kernel.rs:585-592
    blocks, x = multi_block_fixture_v4(5)
    assert rel(O.matvec_row(4, 0, blocks, x), brute_dot(4, blocks, x)) < 1e-4


def test_scalar_v4_walks_the_whole_row_not_just_the_first_block():
    # fused_kernel.rs:594-601
    blocks, x = multi_block_fixture_v4(7)
    assert rel(O.matvec_row(4, 0, blocks, x), brute_dot(4, blocks, x)) < 1e-4


def test_fused_v4_agrees_with_scalar_v4_over_many_blocks():
    # fused_kernel.rs:603-614
    blocks, x = multi_block_fixture_v4(13)
    s = O.matvec_row(4, 0, blocks, x)
    f = O.matvec_row(4, 1, blocks, x)
    assert rel(s, f) < 1e-4


def test_fused_v4_matches_the_reference_formula():
    # fused_kernel.rs:616-626
    blocks, x = multi_block_fixture_v4(9)
    assert rel(O.matvec_row(4, 1, blocks, x), brute_dot(4, blocks, x)) < 1e-4


def test_fused_v4_handles_every_code_value():
    # fused_kernel.rs:631-650
    x = (np.arange(128, dtype=np.float32) * np.float32(0.01) - np.float32(0.6)).astype(np.float32)
    for v in range(16):
        blk = make_v4_blocks([np.full(128, v, np.uint8)], [-0.25], [0.03125])
        assert rel(O.matvec_row(4, 1, blk, x), brute_dot(4, blk, x)) < 1e-4


def test_fused_v4_tracks_fused_v3_on_the_same_weights():
    # fused_kernel.rs:656-683 (error against term magnitude < 0.02)
    n = 11 * 128
    i = np.arange(n, dtype=np.float32)
    w = (np.sin(i * np.float32(0.011)) * np.float32(0.04)).astype(np.float32)
    x = np.cos(i * np.float32(0.019)).astype(np.float32)
    b3 = O.encode_tensor_v3(w)
    b4 = O.encode_tensor_v4(w)
    exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
    y4 = O.matvec_row(4, 1, b4, x)
    y3 = O.matvec_row(3, 1, b3, x)
    scale = float(np.sum(np.abs(w.astype(np.float64) * x)))
    assert abs(y4 - exact) / scale < 0.02
    assert abs(y3 - exact) / scale < 0.02


@pytest.mark.skipif(not O.have_avx2(), reason="CPU lacks AVX2+FMA")
@pytest.mark.parametrize("seed", range(6))
def test_fused_v4_restatement_is_bit_identical_to_the_avx2_intrinsics(seed):
    # The lane-by-lane fmaf restatement against the reference's own
    # intrinsic sequence (fused_kernel.rs:237-271, hsum_avx2 :8-19).
    rng = np.random.default_rng(seed)
    nb = int(rng.integers(1, 80))
    blocks = rng.integers(0, 256, nb * 68, dtype=np.uint8)
    hdr = blocks.reshape(nb, 68)
    hdr[:, 0:2] = np.float16(rng.normal(-0.03, 0.005, nb)).reshape(nb, 1).view(np.uint8)
    hdr[:, 2:4] = np.float16(rng.uniform(0.002, 0.006, nb)).reshape(nb, 1).view(np.uint8)
    x = rng.standard_normal(nb * 128).astype(np.float32)
    a = np.float32(O.matvec_row(4, 1, blocks, x))
    b = np.float32(O.matvec_row(4, 2, blocks, x))
    assert a.view(np.uint32) == b.view(np.uint32)


# ------------------------------------------------------------------ v3
def test_scalar_v3_matches_scalar_v2_on_the_same_weights():
    # fused_kernel.rs:488-498
    b2, x = multi_block_fixture_v2(9)
    b3 = v2_to_v3(b2)
    assert rel(O.matvec_row(3, 0, b3, x), O.matvec_row(2, 0, b2, x)) < 1e-5


def test_fused_v3_agrees_with_scalar_v3():
    # fused_kernel.rs:515-528
    b2, x = multi_block_fixture_v2(6)
    b3 = v2_to_v3(b2)
    assert rel(O.matvec_row(3, 0, b3, x), O.matvec_row(3, 1, b3, x)) < 1e-4


def test_scalar_v3_matches_the_reference_formula():
    # fused_kernel.rs:530-539
    b2, x = multi_block_fixture_v2(5)
    b3 = v2_to_v3(b2)
    assert rel(O.matvec_row(3, 0, b3, x), brute_dot(2, b2, x)) < 1e-4


def test_fused_v3_matches_float64_over_many_blocks():
    b2, x = multi_block_fixture_v2(13)
    b3 = v2_to_v3(b2)
    assert rel(O.matvec_row(3, 1, b3, x), brute_dot(3, b3, x)) < 1e-4


@pytest.mark.skipif(not O.have_avx2(), reason="CPU lacks AVX2+FMA")
@pytest.mark.parametrize("seed", range(6))
def test_fused_v3_restatement_is_bit_identical_to_the_avx2_intrinsics(seed):
    # fused_kernel.rs:163-189
    rng = np.random.default_rng(100 + seed)
    nb = int(rng.integers(1, 80))
    blocks = rng.integers(0, 256, nb * 100, dtype=np.uint8)
    hdr = blocks.reshape(nb, 100)
    hdr[:, 0:2] = np.float16(rng.normal(-0.03, 0.005, nb)).reshape(nb, 1).view(np.uint8)
    hdr[:, 2:4] = np.float16(rng.uniform(0.002, 0.006, nb)).reshape(nb, 1).view(np.uint8)
    x = rng.standard_normal(nb * 128).astype(np.float32)
    a = np.float32(O.matvec_row(3, 1, blocks, x))
    b = np.float32(O.matvec_row(3, 2, blocks, x))
    assert a.view(np.uint32) == b.view(np.uint32)


# ------------------------------------------------------------------ Linear
@pytest.mark.parametrize("scheme", [3, 4])
def test_linear_rows_are_independent_of_thread_count(scheme):
    # WpcLinearV4::matvec runs rows under rayon (wpc_weights_v4.rs:172-187);
    # each row is a separate kernel call, so threads cannot change results.
    rng = np.random.default_rng(scheme)
    rows, cols = 300, 384
    bpb = 68 if scheme == 4 else 100
    blocks = rng.integers(0, 256, rows * (cols // 128) * bpb, dtype=np.uint8)
    hdr = blocks.reshape(-1, bpb)
    hdr[:, 0:2] = np.float16(rng.normal(-0.03, 0.005, hdr.shape[0])).reshape(-1, 1).view(np.uint8)
    hdr[:, 2:4] = np.float16(rng.uniform(0.002, 0.006, hdr.shape[0])).reshape(-1, 1).view(np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    y1 = O.linear_matvec(scheme, blocks, rows, cols, x, bias, O.KERNEL_FUSED, 1)
    y8 = O.linear_matvec(scheme, blocks, rows, cols, x, bias, O.KERNEL_FUSED, 8)
    assert np.array_equal(y1.view(np.uint32), y8.view(np.uint32))
    y0 = O.linear_matvec(scheme, blocks, rows, cols, x, None, O.KERNEL_FUSED, 3)
    # bias is added after the row kernels (wpc_weights_v4.rs:188-192)
    assert np.array_equal((y0 + bias).view(np.uint32), y1.view(np.uint32))
    for r in range(0, rows, 37):
        assert y0[r] == np.float32(O.matvec_row(scheme, 1, hdr[r * (cols // 128):(r + 1) * (cols // 128)].ravel(), x))


def test_embed_v4_two_rounding_decode():
    # row_decode_into_v4 (wpc_weights_v4.rs:103-115): zp + code*scale, two
    # roundings, natural order. Independent check: numpy float32 arithmetic
    # never fuses, so zp + c*s in float32 numpy is the two-rounding value.
    rng = np.random.default_rng(5)
    vocab, hidden = 20, 256
    nb = vocab * hidden // 128
    blocks = rng.integers(0, 256, nb * 68, dtype=np.uint8)
    hdr = blocks.reshape(nb, 68)
    hdr[:, 0:2] = np.float16(rng.normal(-0.03, 0.005, nb)).reshape(nb, 1).view(np.uint8)
    hdr[:, 2:4] = np.float16(rng.uniform(0.002, 0.006, nb)).reshape(nb, 1).view(np.uint8)
    for tok in (0, 7, vocab - 1):
        got = O.embed(4, blocks, hidden, tok)
        exp = []
        for b in range(hidden // 128):
            blk = hdr[tok * (hidden // 128) + b]
            zp = blk[0:2].view(np.float16).astype(np.float32)[0]
            sc = blk[2:4].view(np.float16).astype(np.float32)[0]
            exp.append(zp + O.v4_unpack(blk[4:]).astype(np.float32) * sc)
        exp = np.concatenate(exp).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
