"""Pins the oracle's router, softmax, RMSNorm, RoPE, argmax and SiLU.

Known answers come from the reference's own tests; the rest is checked
against float64 numpy and brute-force selection.
"""
import math

import numpy as np
import pytest

import oracle as O


# ------------------------------------------------------------- route
def test_route_picks_the_highest_scores():
    # qwen3_moe_model.rs:602-610
    ids, _ = O.route([0.1, 0.5, 0.2, 0.9, 0.05], 2, False)
    assert list(ids) == [3, 1]


def test_route_renormalises_when_asked():
    # qwen3_moe_model.rs:612-621
    ids, w = O.route([0.1, 0.5, 0.2, 0.9, 0.05], 2, True)
    assert abs(float(w.sum()) - 1.0) < 1e-6
    assert abs(w[0] - 0.642857) < 1e-4


def test_route_leaves_weights_alone_when_not_asked():
    # qwen3_moe_model.rs:623-630
    _, w = O.route([0.1, 0.5, 0.2, 0.9, 0.05], 2, False)
    assert abs(w[0] - 0.9) < 1e-6 and abs(w[1] - 0.5) < 1e-6


def test_route_ties_go_to_the_lowest_index():
    # strict `>` scan (qwen3_moe_model.rs:382-386)
    ids, _ = O.route([0.3, 0.5, 0.5, 0.1, 0.5], 3, False)
    assert list(ids) == [1, 2, 4]


@pytest.mark.parametrize("seed", range(20))
def test_route_against_brute_force(seed):
    rng = np.random.default_rng(seed)
    s = rng.standard_normal(128).astype(np.float32)
    if seed % 3 == 0:  # inject exact ties
        s[rng.integers(0, 128, 10)] = s[5]
    p = O.softmax(s)
    ids, w = O.route(p, 8, True)
    order = sorted(range(128), key=lambda i: (-float(p[i]), i))[:8]
    assert list(ids) == order
    sel = p[order].astype(np.float32)
    tot = np.float32(0.0)
    for v in sel:  # sequential f32 sum, as the reference's iterator sum
        tot = np.float32(tot + v)
    assert np.array_equal(w, (sel / tot).astype(np.float32))


def test_route_skips_nan_scores():
    ids, _ = O.route([float("nan"), 0.2, 0.1], 2, False)
    assert list(ids) == [1, 2]


# ------------------------------------------------------------- softmax
def test_softmax_sums_to_one_and_is_monotonic():
    # norm.rs:73-80
    x = O.softmax([1.0, 2.0, 3.0])
    assert abs(float(x.sum()) - 1.0) < 1e-6 and x[0] < x[1] < x[2]


def test_softmax_uniform_for_equal_inputs():
    # norm.rs:82-89
    assert np.allclose(O.softmax([5.0] * 4), 0.25, atol=1e-6)


def test_softmax_matches_float64():
    rng = np.random.default_rng(0)
    s = (rng.standard_normal(128) * 3).astype(np.float32)
    e = np.exp(s.astype(np.float64) - s.max())
    assert np.allclose(O.softmax(s), e / e.sum(), rtol=1e-6, atol=1e-9)


# ------------------------------------------------------------- rms_norm
def test_rms_norm_unit_weight_normalizes_rms_to_one():
    # norm.rs:49-60
    out = O.rms_norm([3.0, 4.0, 0.0, 0.0], [1.0] * 4, 1e-6)
    assert np.allclose(out, [1.2, 1.6, 0, 0], atol=1e-4)


def test_rms_norm_applies_weight_scaling():
    # norm.rs:62-71
    out = O.rms_norm([1.0] * 4, [2.0, 0.5, 1.0, 1.0], 1e-6)
    assert abs(out[0] - 2.0) < 1e-5 and abs(out[1] - 0.5) < 1e-5


def test_rms_norm_matches_float64():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(2048).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 2048).astype(np.float32)
    x64 = x.astype(np.float64)
    exp = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
    assert np.allclose(O.rms_norm(x, w, 1e-6), exp, rtol=3e-6, atol=1e-7)


# ------------------------------------------------------------- rope
def test_rope_at_position_zero_is_identity():
    # rope.rs:136-145
    assert np.allclose(O.apply_rope([1.0, 2.0, 3.0, 4.0], 0, 1e6), [1, 2, 3, 4], atol=1e-6)


def test_rope_preserves_per_pair_norm():
    # rope.rs:147-162
    x = np.array([0.5, -1.3, 2.7, 0.1], np.float32)
    y = O.apply_rope(x, 5, 1e6)
    n0 = np.hypot(x[:2], x[2:])
    n1 = np.hypot(y[:2], y[2:])
    assert np.allclose(n0, n1, atol=1e-4)


def test_rope_matches_complex_rotation():
    # rotate_half convention: (x1 + i x2) * e^{i angle}, angle = pos*theta^(-2i/d)
    rng = np.random.default_rng(2)
    d, pos, theta = 128, 77, 1e6
    x = rng.standard_normal(d).astype(np.float32)
    i = np.arange(d // 2)
    ang = pos * theta ** (-(2.0 * i) / d)
    z = (x[: d // 2] + 1j * x[d // 2:]).astype(np.complex128) * np.exp(1j * ang)
    exp = np.concatenate([z.real, z.imag])
    assert np.allclose(O.apply_rope(x, pos, theta), exp, atol=2e-6)


# ------------------------------------------------------------- argmax / silu
def test_argmax_picks_the_largest_first_index():
    # sampling.rs:220-224
    assert O.argmax([0.1, 5.0, -2.0, 4.9]) == 1
    assert O.argmax([1.0, 3.0, 3.0]) == 1


def test_silu_matches_float64():
    for g in (-20.0, -3.5, -0.1, 0.0, 0.7, 4.0, 30.0):
        exp = g / (1.0 + math.exp(-g)) * 1.25
        assert abs(O.silu_mul(g, 1.25) - exp) <= 1e-6 * max(1.0, abs(exp))
