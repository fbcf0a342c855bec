"""Pins the oracle's binary16 conversion, block codecs and encoder.

Each test names the reference test or definition it restates
(paths relative to the reference repository) and, where the reference has
no test, the independent check used instead (numpy's float16, numpy bit
streams, brute force).
"""
import numpy as np
import pytest

import oracle as O


# --------------------------------------------------------------- binary16
def test_f16_to_f32_exhaustive_against_numpy():
    # half 2.7.1 f16::to_f32 is an exact widening; numpy's float16 is an
    # independent implementation of the same IEEE-754 binary16 decode.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32(h)
    exp = h.view(np.float16).astype(np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def _f16_rne_cases():
    rng = np.random.default_rng(1)
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = allh[np.isfinite(allh.view(np.float16))]
    vals = finite.view(np.float16).astype(np.float64)
    vals = np.unique(vals)
    mids = (vals[:-1] + vals[1:]) / 2.0  # exact ties in binary32
    mids32 = mids.astype(np.float32)
    up = np.nextafter(mids32, np.float32(np.inf))
    dn = np.nextafter(mids32, np.float32(-np.inf))
    rand_bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 1e-8,
                        5.96e-8, 2.98e-8, 2.9802322e-08, 1e-45, -1e-45, 6.1035156e-05,
                        6.1035156e-05 * 0.999], np.float32)
    return np.concatenate([vals.astype(np.float32), mids32, up, dn,
                           rand_bits.view(np.float32), special])


def test_f32_to_f16_rne_against_numpy():
    # half 2.7.1 f16::from_f32 rounds to nearest-even; the reference's own
    # tests only pin exact round trips (wpc-format/src/lib.rs:397-460), so the
    # inexact cases are pinned by numpy's independent binary16 rounding.
    f = _f16_rne_cases()
    got = O.f32_to_f16(f)
    with np.errstate(over="ignore", invalid="ignore"):
        exp = f.astype(np.float16).view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], exp[~nan])
    # NaN stays NaN (exponent all ones, mantissa nonzero)
    g = got[nan]
    assert np.all((g & 0x7C00) == 0x7C00) and np.all((g & 0x03FF) != 0)


# --------------------------------------------------------------- v4 codec
def test_v4_packing_round_trips_every_code_in_every_nibble():
    # wpc-format/src/lib.rs:462-486
    for v in range(16):
        uniform = np.full(128, v, np.uint8)
        assert np.array_equal(O.v4_unpack(O.v4_pack(uniform)), uniform)
    i = np.arange(128)
    codes = ((i * 5 + i // 16) % 16).astype(np.uint8)
    packed = O.v4_pack(codes)
    assert np.array_equal(O.v4_unpack(packed), codes)
    # the documented byte layout (lib.rs:481-485)
    assert np.array_equal(packed & 0x0F, codes[:64])
    assert np.array_equal(packed >> 4, codes[64:])


def test_v4_packing_mixed_pattern():
    # wpc-core/src/quant_encoder.rs:210-226
    i = np.arange(128)
    codes = ((i * 3 + i // 8) % 16).astype(np.uint8)
    assert np.array_equal(O.v4_unpack(O.v4_pack(codes)), codes)


def test_v4_pack_masks_out_of_range_codes():
    # pack_codes masks to 4 bits (lib.rs:344-353)
    codes = np.full(128, 0xF7, np.uint8)
    assert np.array_equal(O.v4_unpack(O.v4_pack(codes)), np.full(128, 7, np.uint8))


# --------------------------------------------------------------- v3 codec
def test_v3_packing_round_trips_every_code_value():
    # wpc-core/src/quant_encoder.rs:102-118
    i = np.arange(128)
    codes = ((i * 7 + i // 4) % 64).astype(np.uint8)
    assert np.array_equal(O.v3_unpack(O.v3_pack(codes)), codes)
    for v in range(64):
        u = np.full(128, v, np.uint8)
        assert np.array_equal(O.v3_unpack(O.v3_pack(u)), u)


def test_v3_packing_is_a_little_endian_6bit_stream():
    # The layout at wpc-format/src/lib.rs:190-194 (c0 in the low six bits of
    # byte 0, c1's low two bits above it, ...) is a little-endian bit stream
    # of 6-bit codes. numpy's packbits builds that stream independently.
    rng = np.random.default_rng(7)
    for _ in range(50):
        codes = rng.integers(0, 64, 128, dtype=np.uint8)
        bits = ((codes[:, None] >> np.arange(6)) & 1).astype(np.uint8).ravel()
        stream = np.packbits(bits, bitorder="little")
        assert np.array_equal(O.v3_pack(codes), stream)


def test_v3_two_plane_is_code_identical_to_the_reference_packing():
    # The two-plane device layout has no reference implementation; it must
    # decode to exactly the codes the reference's 4-in-3 unpack yields.
    rng = np.random.default_rng(3)
    cases = [rng.integers(0, 64, 128, dtype=np.uint8) for _ in range(200)]
    cases += [np.full(128, v, np.uint8) for v in range(64)]
    for codes in cases:
        ref_packed = O.v3_pack(codes)
        ref_codes = O.v3_unpack(ref_packed)
        lp, hp = O.v3tp_pack(ref_codes)
        assert np.array_equal(O.v3tp_unpack(lp, hp), ref_codes)
        # plane definitions, written as numpy expressions
        c = ref_codes.astype(np.uint16)
        assert np.array_equal(lp, ((c[:64] & 15) | ((c[64:] & 15) << 4)).astype(np.uint8))
        hi = (c >> 4) & 3
        exp_hp = hi[0:32] | (hi[32:64] << 2) | (hi[64:96] << 4) | (hi[96:128] << 6)
        assert np.array_equal(hp, exp_hp.astype(np.uint8))


# --------------------------------------------------------------- encoder
def _decode(block, scheme):
    zp = O.f16_to_f32(block[0:2].view(np.uint16))[0]
    sc = O.f16_to_f32(block[2:4].view(np.uint16))[0]
    codes = O.v4_unpack(block[4:68]) if scheme == 4 else O.v3_unpack(block[4:100])
    return zp, sc, codes


def _round_half_away(v):
    v = v.astype(np.float64)
    return np.where(v >= 0, np.floor(v + 0.5), np.ceil(v - 0.5))


@pytest.mark.parametrize("seed", range(5))
def test_v4_encoder_closed_form(seed):
    # affine_quant_block_v4 (wpc-core/src/quant_encoder.rs:66-85): fp32 min
    # and scale = (max-min)/15, codes round half away from zero, clamped;
    # zero_point and scale stored as f16 (numpy RNE).
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(128) * 0.02).astype(np.float32)
    blk = O.quant_block_v4(w)
    mn, mx = np.float32(w.min()), np.float32(w.max())
    scale = np.float32((mx - mn) / np.float32(15.0))
    q = np.float32(w - mn) / scale  # float32 arithmetic, as the reference
    codes = np.clip(_round_half_away(q.astype(np.float32)), 0, 15).astype(np.uint8)
    assert np.array_equal(O.v4_unpack(blk[4:68]), codes)
    assert blk[0:2].view(np.uint16)[0] == np.float16(mn).view(np.uint16)
    assert blk[2:4].view(np.uint16)[0] == np.float16(scale).view(np.uint16)


def test_v4_encoder_flat_block_uses_unit_scale():
    # `scale = 1.0` when max == min (quant_encoder.rs:74)
    blk = O.quant_block_v4(np.full(128, 0.25, np.float32))
    zp, sc, codes = _decode(blk, 4)
    assert zp == np.float32(0.25) and sc == 1.0 and not codes.any()


def test_v4_encoder_never_emits_a_code_above_fifteen():
    # quant_encoder.rs:228-241
    i = np.arange(128, dtype=np.float32)
    w = np.sin(i * np.float32(0.91)) * np.float32(12.5) - np.float32(3.0)
    _, _, codes = _decode(O.quant_block_v4(w), 4)
    assert codes.max() <= 15


def test_v4_reconstruction_error_stays_within_one_step():
    # quant_encoder.rs:243-269
    i = np.arange(128, dtype=np.float32)
    w = (np.sin(i * np.float32(0.37)) * np.float32(0.05)).astype(np.float32)
    zp, sc, codes = _decode(O.quant_block_v4(w), 4)
    dec = zp + codes.astype(np.float32) * sc
    assert np.all(np.abs(dec - w) <= sc * 0.5 + sc * 0.05 + 1e-6)


def test_v4_is_coarser_than_v3_but_still_close():
    # quant_encoder.rs:271-303
    i = np.arange(128, dtype=np.float32)
    w = (np.sin(i * np.float32(0.13)) * np.float32(0.04)
         + np.cos(i * np.float32(0.7)) * np.float32(0.01)).astype(np.float32)
    z3, s3, c3 = _decode(O.quant_block_v3(w), 3)
    z4, s4, c4 = _decode(O.quant_block_v4(w), 4)
    r3 = np.sqrt(np.mean((z3 + c3 * s3 - w) ** 2))
    r4 = np.sqrt(np.mean((z4 + c4 * s4 - w) ** 2))
    assert r3 <= r4 < r3 * 8.0


def test_v3_reconstructs_bit_identically_to_v2():
    # quant_encoder.rs:120-147
    i = np.arange(128, dtype=np.float32)
    w = (np.sin(i * np.float32(0.37)) * np.float32(0.05)).astype(np.float32)
    v2 = O.quant_block_v2(w)
    v3 = O.quant_block_v3(w)
    assert np.array_equal(v2[:4], v3[:4])
    assert np.array_equal(O.v3_unpack(v3[4:]), v2[4:])


def test_v2_affine_block_ramp_error():
    # quant_encoder.rs:167-197
    w = (np.arange(128, dtype=np.float32) * np.float32(0.05) - np.float32(3.2))
    b = O.quant_block_v2(w)
    zp = O.f16_to_f32(b[0:2].view(np.uint16))[0]
    sc = O.f16_to_f32(b[2:4].view(np.uint16))[0]
    dec = zp + b[4:].astype(np.float32) * sc
    rmse = np.sqrt(np.mean((dec - w) ** 2))
    ref = np.sqrt(np.mean(np.maximum(np.abs(w), 1e-6) ** 2))
    assert rmse / ref < 0.05


def test_block_disk_round_trip_sizes():
    # quant_encoder.rs:305-315 and lib.rs:440-445: 68-byte v4, 100-byte v3
    w = np.arange(128, dtype=np.float32) * np.float32(0.05) - np.float32(3.2)
    assert O.quant_block_v4(w).size == 68
    assert O.quant_block_v3(w).size == 100
    assert O.quant_block_v2(w).size == 132


def test_tensor_encode_matches_block_encode():
    # quant_encoder.rs:317-330
    i = np.arange(128 * 5, dtype=np.float32)
    data = (np.sin(i * np.float32(0.017)) * np.float32(0.3)).astype(np.float32)
    blocks = O.encode_tensor_v4(data).reshape(5, 68)
    for b in range(5):
        assert np.array_equal(blocks[b], O.quant_block_v4(data[b * 128:(b + 1) * 128]))
    b3 = O.encode_tensor_v3(data).reshape(5, 100)
    for b in range(5):
        assert np.array_equal(b3[b], O.quant_block_v3(data[b * 128:(b + 1) * 128]))
