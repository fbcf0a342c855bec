"""The HIP path against the committed golden fixtures (tests/golden/):
EXACT GEMV, both dequantization roundings and the embedding decode must
reproduce the stored reference outputs bit for bit; FAST must stay within
1e-6 of each row's term magnitude sum(|w|*|x|) of them."""
import os

import numpy as np
import pytest

import wpcg

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name + ".npz")) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def ctx():
    c = wpcg.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("name", ["ref_multiblock_v4", "synth_v4_37x384", "synth_v3_45x384"])
def test_golden_gemv(ctx, name):
    print(f"[gpu] golden {name}", flush=True)
    f = load(name)
    scheme = 3 if "_v3_" in name else 4
    rows, cols = int(f["rows"]), int(f["cols"])
    lin = wpcg.WpcLinear.from_blocks(ctx, scheme, f["blocks"], rows, cols)
    assert np.array_equal(bits(lin.matvec(f["x"])), bits(f["y_fused"]))
    lin.set_mode(wpcg.MODE_FAST)
    y = lin.matvec(f["x"]).astype(np.float64)
    if "w_fma" in f:
        mag = np.abs(f["w_fma"].astype(np.float64)) @ np.abs(f["x"].astype(np.float64))
        assert np.all(np.abs(y - f["y_fused"]) <= 1e-6 * mag + 1e-30)
    else:
        assert abs(y[0] - float(f["y_fused"][0])) <= 1e-5 * abs(float(f["y_fused"][0]))
    lin.close()


@pytest.mark.parametrize("name", ["synth_v4_37x384", "synth_v3_45x384"])
def test_golden_dequant_and_embed(ctx, name):
    print(f"[gpu] golden dequant/embed {name}", flush=True)
    f = load(name)
    scheme = 3 if "_v3_" in name else 4
    rows, cols = int(f["rows"]), int(f["cols"])
    lin = wpcg.WpcLinear.from_blocks(ctx, scheme, f["blocks"], rows, cols)
    assert np.array_equal(bits(lin.dequant(wpcg.ROUND_FMA)), bits(f["w_fma"]))
    assert np.array_equal(bits(lin.dequant(wpcg.ROUND_TWO)), bits(f["w_two"]))
    for i, r in enumerate(f["embed_rows"]):
        assert np.array_equal(bits(lin.embed(int(r))), bits(f["embed"][i]))
    lin.close()
