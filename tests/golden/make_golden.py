"""Writes the golden fixtures in this directory (run from the repository
root: python tests/golden/make_golden.py).

The reference (Rust) cannot be built or run in this image, so its expected
outputs come from the oracle's restatement of the reference kernels
(oracle/wpc_oracle.c), itself pinned against the reference's own test
fixtures and known answers (tests/test_oracle_*.py). Freezing the outputs
here gives the GPU tests fixed vectors to meet bit for bit and turns any
later drift of the oracle into a test failure (tests/test_golden.py).

Fixtures (numpy .npz, no pickled objects):
  ref_multiblock_v4.npz  the reference's multi-block v4 fixture
                         (wpc-eval/src/fused_kernel.rs:549-566) as one
                         20-block row, with its fused (AVX2) and scalar
                         outputs
  synth_v4_37x384.npz    seeded synthetic v4 matrix (codes uniform 0..15,
  synth_v3_45x384.npz    zp f16(N(-0.03,0.005)), scale f16(U(0.002,0.006)),
                         x N(0,1)) and v3 twin: fused and scalar GEMV, the
                         dequantized matrix in both roundings, embed rows
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "wpc-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle as O  # noqa: E402
from wpcg import synth  # noqa: E402

EMBED_ROWS = (0, 5, -1)


def ref_multiblock_v4(n_blocks=20):
    # fused_kernel.rs:549-566: codes (i*3 + b*5) % 16, zp -0.4 + 0.1 b,
    # scale 0.017 + 0.003 b, x = sin(0.013 k) + 0.5
    i = np.arange(128)
    blocks = []
    for b in range(n_blocks):
        blk = np.zeros(68, np.uint8)
        blk[0:2] = np.array([np.float16(np.float32(-0.4) + np.float32(b) * np.float32(0.1))]).view(np.uint8)
        blk[2:4] = np.array([np.float16(np.float32(0.017) + np.float32(b) * np.float32(0.003))]).view(np.uint8)
        blk[4:] = O.v4_pack(((i * 3 + b * 5) % 16).astype(np.uint8))
        blocks.append(blk)
    x = (np.sin(np.arange(n_blocks * 128, dtype=np.float32) * np.float32(0.013))
         + np.float32(0.5)).astype(np.float32)
    return np.concatenate(blocks), x


def dequant(scheme, blocks, rows, cols, rounding):
    """Natural-order fp32 weights; rounding 'fma' = fma(code, scale, zp),
    'two' = zp + code*scale (row_decode_into_v4, wpc_weights_v4.rs:103-115)."""
    bpb = 68 if scheme == 4 else 100
    b = blocks.reshape(-1, bpb)
    zp = O.f16_to_f32(b[:, 0:2].copy().view(np.uint16).ravel())
    sc = O.f16_to_f32(b[:, 2:4].copy().view(np.uint16).ravel())
    codes = np.stack([O.v4_unpack(r[4:]) if scheme == 4 else O.v3_unpack(r[4:]) for r in b])
    c = codes.astype(np.float32)
    if rounding == "two":
        w = (zp[:, None] + (c * sc[:, None]).astype(np.float32)).astype(np.float32)
    else:  # one rounding: exact product + zp, rounded once (float64 holds it exactly)
        w = (c.astype(np.float64) * sc[:, None].astype(np.float64)
             + zp[:, None].astype(np.float64)).astype(np.float32)
    return w.reshape(rows, cols)


def synth_fixture(scheme, rows, cols, seed):
    gen = synth.random_v4_blocks if scheme == 4 else synth.random_v3_blocks
    blocks = gen(rows, cols, seed=seed)
    x = synth.random_x(cols, seed=seed + 1)
    return dict(
        blocks=blocks, x=x, rows=np.int64(rows), cols=np.int64(cols),
        y_fused=O.linear_matvec(scheme, blocks, rows, cols, x, None, O.KERNEL_FUSED, 1),
        y_scalar=O.linear_matvec(scheme, blocks, rows, cols, x, None, O.KERNEL_SCALAR, 1),
        w_fma=dequant(scheme, blocks, rows, cols, "fma"),
        w_two=dequant(scheme, blocks, rows, cols, "two"),
        embed_rows=np.array([r % rows for r in EMBED_ROWS], np.int64),
        embed=np.stack([O.embed(scheme, blocks, cols, r % rows) for r in EMBED_ROWS]),
    )


def build_all():
    blocks, x = ref_multiblock_v4()
    out = {
        "ref_multiblock_v4": dict(
            blocks=blocks, x=x, rows=np.int64(1), cols=np.int64(x.size),
            y_fused=np.array([O.matvec_row(4, O.KERNEL_FUSED, blocks, x)], np.float32),
            y_scalar=np.array([O.matvec_row(4, O.KERNEL_SCALAR, blocks, x)], np.float32)),
        "synth_v4_37x384": synth_fixture(4, 37, 384, 7001),
        "synth_v3_45x384": synth_fixture(3, 45, 384, 7003),
    }
    return out


if __name__ == "__main__":
    for name, arrays in build_all().items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
        print(f"wrote {name}.npz")
