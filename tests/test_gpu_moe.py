"""GPU tests of the Qwen3-MoE sparse-MLP pieces against the oracle
(reference: wpc-runtime/src/weights.rs:59-78 DenseLinear::matvec,
norm.rs:28-43 softmax_inplace, qwen3_moe_model.rs:376-402 route and
:500-530 the expert loop). EXACT results must be bit-identical; FAST ones
are held to the bounds stated per test."""
import os

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


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.array_equal(bits(a), bits(b)) or bool(
        np.all((bits(a) == bits(b)) | (np.isnan(a) & np.isnan(b))))


@pytest.mark.parametrize("out_f,in_f", [(128, 2048), (5, 300), (70, 129), (1, 1)])
def test_dense_exact_bit_identical_and_fast_close(ctx, out_f, in_f):
    print(f"[gpu] dense {out_f}x{in_f}", flush=True)
    rng = np.random.default_rng(out_f * 7 + in_f)
    W = (rng.standard_normal((out_f, in_f)) * 0.02).astype(np.float32)
    x = rng.standard_normal(in_f).astype(np.float32)
    bias = rng.standard_normal(out_f).astype(np.float32)
    for b in (None, bias):
        d = wpcg.DenseLinear(ctx, W, b)
        ref = O.dense_matvec(W, x, b)
        assert same(d.matvec(x), ref)
        d.set_mode(wpcg.MODE_FAST)
        y = d.matvec(x).astype(np.float64)
        mag = np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64)) + (0 if b is None else np.abs(b))
        assert np.all(np.abs(y - ref) <= 1e-6 * mag + 1e-30)
        d.close()


@pytest.mark.parametrize("n", [1, 64, 128, 2048, 2560, 5000])
def test_rms_norm_bit_identical(ctx, n):
    # many scales, so the square root and the divisions see many exponents
    print(f"[gpu] rms_norm {n}", flush=True)
    rng = np.random.default_rng(n + 1)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    for rep in range(40):
        x = (rng.standard_normal(n) * np.float32(10.0 ** rng.uniform(-6, 4))).astype(np.float32)
        got = wpcg.rms_norm(ctx, x, w, 1e-6)
        assert same(got, O.rms_norm(x, w, 1e-6)), rep
        fast = wpcg.rms_norm(ctx, x, w, 1e-6, wpcg.MODE_FAST)
        assert np.allclose(fast, got, rtol=1e-5, atol=0), rep


@pytest.mark.parametrize("n", [1, 2, 128, 1000, 4097])
def test_softmax_bit_identical(ctx, n):
    print(f"[gpu] softmax {n}", flush=True)
    rng = np.random.default_rng(n)
    for scale in (0.1, 5.0, 80.0):
        x = (rng.standard_normal(n) * scale).astype(np.float32)
        if n > 3:
            x[1] = -np.inf
            x[2] = x[0]
        assert same(wpcg.softmax(ctx, x), O.softmax(x))


def test_silu_mul_bit_identical_over_the_float_range(ctx):
    # every exponent range of g, exp(-g) overflowing and underflowing,
    # subnormals, signed zeros; u random
    rng = np.random.default_rng(11)
    g = rng.integers(0, 2**32, 1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    g = g[np.isfinite(g)]
    g = np.concatenate([g, np.array([0.0, -0.0, 88.0, -88.0, 103.9, -103.9, 1e-40, -1e-40,
                                     np.inf, -np.inf, np.nan], np.float32)])
    u = rng.standard_normal(g.size).astype(np.float32)
    print(f"[gpu] silu_mul over {g.size} values", flush=True)
    assert same(wpcg.silu_mul(ctx, g, u), O.silu_mul_array(g, u))


@pytest.mark.parametrize("n,top_k", [(128, 8), (16, 4), (8, 8), (300, 16), (1, 1)])
def test_route_matches_the_reference_scan(ctx, n, top_k):
    print(f"[gpu] route n={n} top_k={top_k}", flush=True)
    rng = np.random.default_rng(n + top_k)
    for case in range(5):
        p = rng.random(n).astype(np.float32)
        if case == 1 and n > 4:     # ties: lowest index first
            p[:] = np.float32(0.25)
            p[n // 2] = np.float32(0.5)
        if case == 2 and n > 4:     # NaN and -inf are never chosen
            p[0] = np.nan
            p[3] = -np.inf
        if case == 3:
            p = O.softmax((rng.standard_normal(n) * 3).astype(np.float32))
        if case == 4:               # +0 and -0 tie: the lower index first
            p = np.where(rng.random(n) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
            if n > 2:
                p[n - 1] = np.float32(0.125)
        for norm in (True, False):
            ids, w = wpcg.route(ctx, p, top_k, norm)
            rid, rw = O.route(p, top_k, norm)
            got = rid.size
            assert np.array_equal(ids[:got], rid) and np.all(ids[got:] == -1), (case, norm)
            assert same(w[:got], rw) and np.all(w[got:] == 0), (case, norm)


def make_moe(ctx, n_exp, hidden, inter, top_k, seed):
    rng = np.random.default_rng(seed)
    router = (rng.standard_normal((n_exp, hidden)) * 0.02).astype(np.float32)
    experts = [(synth.random_v4_blocks(inter, hidden, seed * 1000 + 3 * e),
                synth.random_v4_blocks(inter, hidden, seed * 1000 + 3 * e + 1),
                synth.random_v4_blocks(hidden, inter, seed * 1000 + 3 * e + 2)) for e in range(n_exp)]
    moe = wpcg.MoeLayer(ctx, wpcg.SCHEME_V4, n_exp, hidden, inter, top_k).set_router(router)
    for e, (g, u, d) in enumerate(experts):
        moe.set_expert(e, g, u, d)
    return moe, router, experts


@pytest.mark.parametrize("n_exp,hidden,inter,top_k", [(16, 256, 128, 4), (128, 2048, 768, 8)])
def test_moe_layer_exact_and_fast(ctx, n_exp, hidden, inter, top_k):
    print(f"[gpu] moe n_exp={n_exp} hidden={hidden} inter={inter} top_k={top_k}", flush=True)
    moe, router, experts = make_moe(ctx, n_exp, hidden, inter, top_k, seed=hidden + n_exp)
    rng = np.random.default_rng(5)
    for rep in range(3):
        x = rng.standard_normal(hidden).astype(np.float32)
        ref, rid, rw = O.moe_ffn_v4(router, experts, x, top_k)
        moe.set_mode(wpcg.MODE_EXACT)
        out, ids, w = moe.forward(x)
        assert np.array_equal(ids, rid), rep
        assert same(w, rw), rep
        assert same(out, ref), rep
        moe.set_mode(wpcg.MODE_FAST)
        fout, fids, fw = moe.forward(x)
        # FAST router and GEMVs: same experts on these inputs (no near
        # ties), weights to fp32 rounding, outputs to 1e-5 of their scale
        assert np.array_equal(fids, rid), rep
        assert np.allclose(fw, rw, rtol=1e-5, atol=0), rep
        assert np.max(np.abs(fout - ref)) <= 1e-5 * np.max(np.abs(ref)), rep
    moe.close()


def test_moe_loads_experts_from_an_artifact(ctx, tmp_path):
    n_exp, hidden, inter, top_k, layer = 8, 256, 128, 2, 3
    moe, router, experts = make_moe(ctx, n_exp, hidden, inter, top_k, seed=77)
    tensors = []
    for e, (g, u, d) in enumerate(experts):
        p = f"model.layers.{layer}.mlp.experts.{e}"
        tensors += [(f"{p}.gate_proj.weight", [inter, hidden], g),
                    (f"{p}.up_proj.weight", [inter, hidden], u),
                    (f"{p}.down_proj.weight", [hidden, inter], d)]
    synth.write_artifact(str(tmp_path / "a"), 4, tensors)
    data = wpcg.WpcModelDataV4.open(str(tmp_path / "a"))
    moe2 = wpcg.MoeLayer(ctx, wpcg.SCHEME_V4, n_exp, hidden, inter, top_k).set_router(router)
    moe2.load_experts(data, layer)
    x = np.random.default_rng(1).standard_normal(hidden).astype(np.float32)
    a, b = moe.forward(x), moe2.forward(x)
    assert same(a[0], b[0]) and np.array_equal(a[1], b[1])
    with pytest.raises(wpcg.WpcgError) as e:  # another layer's experts are absent
        moe2.load_experts(data, layer + 1)
    assert e.value.code == wpcg.E_NOTFOUND
    moe.close()
    moe2.close()
    data.close()
