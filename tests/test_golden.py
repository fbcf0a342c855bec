"""The committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py) against the oracle: every stored output is
recomputed and must match bit for bit, so a change in the oracle or in the
fixtures fails here. The reference's own multi-block fixture
(wpc-eval/src/fused_kernel.rs:549-566) is also checked against its
float64 value at the reference's tolerance (fused_kernel.rs:616-626)."""
import os

import numpy as np
import pytest

import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SYNTH = ["synth_v4_37x384", "synth_v3_45x384"]


def load(name):
    with np.load(os.path.join(HERE, name + ".npz")) as z:  # allow_pickle=False
        return {k: z[k] for k in z.files}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_reference_multiblock_fixture():
    f = load("ref_multiblock_v4")
    y_f = O.matvec_row(4, O.KERNEL_FUSED, f["blocks"], f["x"])
    y_s = O.matvec_row(4, O.KERNEL_SCALAR, f["blocks"], f["x"])
    assert bits(np.float32(y_f)) == bits(f["y_fused"])[0]
    assert bits(np.float32(y_s)) == bits(f["y_scalar"])[0]
    # float64 truth of the same weights
    b = f["blocks"].reshape(-1, 68)
    zp = O.f16_to_f32(b[:, 0:2].copy().view(np.uint16).ravel()).astype(np.float64)
    sc = O.f16_to_f32(b[:, 2:4].copy().view(np.uint16).ravel()).astype(np.float64)
    codes = np.stack([O.v4_unpack(r[4:]) for r in b]).astype(np.float64)
    w = (zp[:, None] + codes * sc[:, None]).ravel()
    truth = float(w @ f["x"].astype(np.float64))
    assert abs(y_f - truth) <= 1e-4 * max(1.0, abs(truth))


@pytest.mark.parametrize("name", SYNTH)
def test_synthetic_fixtures_match_the_oracle(name):
    f = load(name)
    scheme = 4 if "_v4_" in name else 3
    rows, cols = int(f["rows"]), int(f["cols"])
    y = O.linear_matvec(scheme, f["blocks"], rows, cols, f["x"], None, O.KERNEL_FUSED, 3)
    assert np.array_equal(bits(y), bits(f["y_fused"]))
    y = O.linear_matvec(scheme, f["blocks"], rows, cols, f["x"], None, O.KERNEL_SCALAR, 2)
    assert np.array_equal(bits(y), bits(f["y_scalar"]))
    if O.have_avx2():  # the intrinsics build gives the restatement's bits
        y = O.linear_matvec(scheme, f["blocks"], rows, cols, f["x"], None, O.KERNEL_AVX2, 4)
        assert np.array_equal(bits(y), bits(f["y_fused"]))
    for i, r in enumerate(f["embed_rows"]):
        assert np.array_equal(bits(O.embed(scheme, f["blocks"], cols, int(r))), bits(f["embed"][i]))
    # the two-rounding dequant is what embed decodes, row by row
    for i, r in enumerate(f["embed_rows"]):
        assert np.array_equal(bits(f["w_two"][int(r)]), bits(f["embed"][i]))
    # the FMA dequant differs from the two-rounding one by at most one rounding
    d = np.abs(f["w_fma"].astype(np.float64) - f["w_two"].astype(np.float64))
    assert np.all(d <= np.spacing(np.abs(f["w_two"])).astype(np.float64) * 1.0 + 1e-30)
