"""wpcg_encode (the product's host encoder) against the oracle's restatement
of encode_tensor_v4 / encode_tensor_v3 (wpc-core/src/quant_encoder.rs:49-96),
which tests/test_oracle_format.py pins: identical bytes on random weights and
on the edge cases (flat blocks, NaN, infinities, huge and tiny values)."""
import numpy as np
import pytest

import oracle as O
import wpcg


@pytest.mark.parametrize("scheme", [4, 3])
def test_encoder_matches_the_oracle(scheme):
    rng = np.random.default_rng(scheme)
    w = (rng.standard_normal(128 * 4096) * 0.02).astype(np.float32)
    w[:128] = 0.5                      # flat block
    w[128:256] = np.linspace(-1, 1, 128, dtype=np.float32)
    w[300] = np.nan
    w[600] = np.inf
    w[700] = -np.inf
    w[1024:1152] *= np.float32(1e30)   # scale overflows f16
    w[2048:2176] *= np.float32(1e-30)  # scale underflows f16
    ref = O.encode_tensor_v4(w) if scheme == 4 else O.encode_tensor_v3(w)
    got = wpcg.encode(scheme, w)
    assert got.dtype == np.uint8 and got.size == ref.size
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"first differing byte {bad[0]} (block {bad[0] // (68 if scheme == 4 else 100)})"


def test_encoder_rejects_partial_blocks():
    with pytest.raises(wpcg.WpcgError) as e:
        wpcg.encode(4, np.zeros(100, np.float32))
    assert e.value.code == wpcg.E_SHAPE
