"""The benchmark configurations' PRNG (wpcg.synth: xoshiro256++ seeded through
SplitMix64, rand 0.8.7's f32 draw, Box-Muller in f32 as the reference's
evaluator computes x, wpc-eval/src/main.rs:77-82).

The generators are pinned by their published test vectors: SplitMix64 from
state 0 (Steele, Lea and Flood's generator as Vigna publishes it) and
xoshiro256++ from the state words (1, 2, 3, 4), the vector rand_xoshiro 0.6.0's
own tests use. The rest are properties a wrong restatement breaks: the draw's
24-bit grid, one stream per matrix row (a matrix's first rows do not depend on
its row count), x as a prefix of one stream, parameter ranges, and Box-Muller
against float64.
"""
import numpy as np

from wpcg import synth


def test_splitmix64_published_vector():
    st = np.zeros(1, np.uint64)
    got = []
    for _ in range(4):
        st, z = synth.splitmix64_np(st)
        got.append(int(z[0]))
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]


def test_xoshiro256pp_published_vector():
    rng = synth.Xoshiro256pp(state=[[1], [2], [3], [4]])
    got = [int(rng.next_u64()[0]) for _ in range(10)]
    assert got == [41943041, 58720359, 3588806011781223, 3591011842654386, 9228616714210784205,
                   9973669472204895162, 14011001112246962877, 12406186145184390807,
                   15849039046786891736, 10450023813501588000]


def test_streams_are_independent_lanes():
    a = synth.Xoshiro256pp([5, 6, 7])
    b = synth.Xoshiro256pp([6])
    for _ in range(20):
        va, vb = a.next_u64(), b.next_u64()
        assert va[1] == vb[0]


def test_next_u32_is_the_upper_half_and_f32_the_24_bit_grid():
    a = synth.Xoshiro256pp([123])
    b = synth.Xoshiro256pp([123])
    for _ in range(50):
        assert int(a.next_u32()[0]) == int(b.next_u64()[0]) >> 32
    c = synth.Xoshiro256pp(np.arange(1000, dtype=np.uint64))
    d = synth.Xoshiro256pp(np.arange(1000, dtype=np.uint64))
    u = c.gen_f32()
    assert u.dtype == np.float32 and np.all(u >= 0) and np.all(u < 1)
    assert np.array_equal(u.astype(np.float64) * 2.0 ** 24, (d.next_u64() >> np.uint64(40)).astype(np.float64))


def test_box_muller_against_float64():
    rng = np.random.default_rng(3)
    u1 = rng.uniform(2.0 ** -24, 1.0, 4000).astype(np.float32)
    u2 = rng.uniform(0.0, 1.0, 4000).astype(np.float32)
    got = synth._box_muller_f32(u1, u2).astype(np.float64)
    two_pi = float(np.float32(2.0) * np.float32(np.pi))
    ang = (np.float32(two_pi) * u2).astype(np.float64)
    want = np.sqrt(-2.0 * np.log(u1.astype(np.float64))) * np.cos(ang)
    assert np.max(np.abs(got - want)) <= 4e-6 * np.max(np.abs(want))


def test_x_is_a_prefix_of_one_stream_and_standard_normal():
    x = synth.wpc_x(6000)
    assert np.array_equal(synth.wpc_x(100), x[:100])
    assert abs(float(x.mean())) < 0.05 and abs(float(x.std()) - 1.0) < 0.05
    assert np.isfinite(x).all()


def _unpack(scheme, blocks, rows, cols):
    nb = cols // 128
    b = blocks.reshape(rows * nb, synth.BPB[scheme])
    zp = b[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    sc = b[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    if scheme == 4:
        codes = np.concatenate([b[:, 4:] & 15, b[:, 4:] >> 4], axis=1)
    else:
        w = b[:, 4:].astype(np.uint32).reshape(-1, 32, 3)
        word = w[..., 0] | w[..., 1] << 8 | w[..., 2] << 16
        codes = np.stack([(word >> (6 * q)) & 63 for q in range(4)], axis=-1).reshape(-1, 128)
    return zp, sc, codes


def test_blocks_rows_do_not_depend_on_the_row_count():
    for scheme in (4, 3):
        a = synth.wpc_blocks(scheme, 12, 256, matrix_id=3)
        b = synth.wpc_blocks(scheme, 5, 256, matrix_id=3)
        assert np.array_equal(a[:b.size], b)
        c = synth.wpc_blocks(scheme, 5, 256, matrix_id=4)
        assert not np.array_equal(b, c)


def test_block_parameters_follow_the_configs():
    for scheme, top in ((4, 15), (3, 63)):
        rows, cols = 64, 1024
        zp, sc, codes = _unpack(scheme, synth.wpc_blocks(scheme, rows, cols, matrix_id=1), rows, cols)
        assert codes.min() == 0 and codes.max() == top
        # uniform codes: every value near its share
        counts = np.bincount(codes.ravel(), minlength=top + 1)
        assert counts.min() > 0.8 * codes.size / (top + 1)
        assert np.all(sc >= 0.002 - 1e-6) and np.all(sc <= 0.006 + 1e-6)
        assert abs(float(zp.mean()) + 0.03) < 0.002 and abs(float(zp.std()) - 0.005) < 0.001
