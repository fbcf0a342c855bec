"""CPU tests of the C ABI boundary: the library loads and exports every
symbol include/wpcg.h declares, and every host-side failure the reference
turns into an error or a panic comes back as a status code. No GPU compute.

Forced failures and the reference behaviour they mirror (paths relative to
the reference repository):
  missing/unreadable meta or .wpc   WpcModelDataV4::open `?`   wpc_weights_v4.rs:46-60
  bad JSON / missing field          serde_json::from_str `?`    wpc_weights_v4.rs:49
  block_size != 128                 anyhow::ensure!             wpc_weights_v4.rs:51-56
  unknown tensor                    panic in tensor_range       wpc_weights_v4.rs:80-85
  size not a multiple of 68         assert in blocks_for        wpc_weights_v4.rs:95
  in_features % 128, block count    asserts in WpcLinearV4::new wpc_weights_v4.rs:134-147
  no GPU                            (none: CPU-only reference)  -> E_DEVICE
"""
import ctypes as C
import json
import os
import subprocess

import numpy as np
import pytest

import wpcg
from wpcg import synth


def test_library_exports_every_declared_symbol():
    declared = wpcg.declared_symbols()
    assert len(declared) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", wpcg.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    for s in declared:
        assert hasattr(wpcg.lib, s)


def test_version_string():
    assert b"gfx950" in wpcg.lib.wpcg_version()


def _no_gpu():
    return wpcg.device_count() == 0


@pytest.mark.skipif(not _no_gpu(), reason="a GPU is visible")
def test_no_device_is_a_status_code():
    with pytest.raises(wpcg.WpcgError) as e:
        wpcg.Context(0)
    assert e.value.code == wpcg.E_DEVICE
    n = C.c_int(-1)
    assert wpcg.lib.wpcg_device_count(C.byref(n)) == wpcg.E_DEVICE and n.value == 0


def test_null_arguments_are_rejected():
    h = C.c_void_p()
    assert wpcg.lib.wpcg_linear_matvec(None, None, None, None) == wpcg.E_ARG
    assert wpcg.lib.wpcg_artifact_open(None, 4, C.byref(h)) == wpcg.E_ARG
    assert wpcg.lib.wpcg_artifact_open(b"/tmp", 5, C.byref(h)) == wpcg.E_ARG
    assert wpcg.lib.wpcg_ctx_sync(None) == wpcg.E_ARG
    assert wpcg.lib.wpcg_linear_set_mode(None, 0) == wpcg.E_ARG


def test_shape_errors_match_wpclinear_new():
    blocks = synth.random_v4_blocks(4, 256, 0)
    with pytest.raises(wpcg.WpcgError) as e:  # in_features % 128
        wpcg.WpcLinear.from_blocks(None, 4, blocks, 4, 200)
    assert e.value.code == wpcg.E_SHAPE
    with pytest.raises(wpcg.WpcgError) as e:  # block count mismatch
        wpcg.WpcLinear.from_blocks(None, 4, blocks, 5, 256)
    assert e.value.code == wpcg.E_SHAPE
    with pytest.raises(wpcg.WpcgError) as e:  # not whole blocks
        wpcg.WpcLinear.from_blocks(None, 4, blocks[:-1], 4, 256)
    assert e.value.code == wpcg.E_FORMAT
    with pytest.raises(wpcg.WpcgError) as e:  # v3 sizes
        wpcg.WpcLinear.from_blocks(None, 3, synth.random_v3_blocks(4, 256, 0), 4, 384)
    assert e.value.code == wpcg.E_SHAPE


def _write(tmp_path, scheme=4, meta=None, wpc=b""):
    d = tmp_path / "art"
    d.mkdir(exist_ok=True)
    if meta is not None:
        (d / f"model_v{scheme}.meta").write_text(meta if isinstance(meta, str) else json.dumps(meta))
    if wpc is not None:
        (d / f"model_v{scheme}.wpc").write_bytes(wpc)
    return str(d)


def _open_rc(path, scheme=4):
    h = C.c_void_p()
    rc = wpcg.lib.wpcg_artifact_open(os.fsencode(path), scheme, C.byref(h))
    if rc == 0:
        wpcg.lib.wpcg_artifact_close(h)
    return rc


def test_artifact_open_errors(tmp_path):
    assert _open_rc(str(tmp_path / "nowhere")) == wpcg.E_IO
    d = _write(tmp_path, meta=None, wpc=b"x")
    assert _open_rc(d) == wpcg.E_IO  # meta missing
    d = _write(tmp_path, meta='{"layers": [], "block_size": 128', wpc=b"")
    assert _open_rc(d) == wpcg.E_FORMAT  # truncated JSON
    d = _write(tmp_path, meta={"layers": []}, wpc=b"")
    assert _open_rc(d) == wpcg.E_FORMAT  # missing block_size
    d = _write(tmp_path, meta={"layers": [], "block_size": 64}, wpc=b"")
    assert _open_rc(d) == wpcg.E_FORMAT  # block_size mismatch
    d = _write(tmp_path, meta={"layers": [{"name": "a", "offset_bytes": 0, "size_bytes": 0}],
                               "block_size": 128}, wpc=b"")
    assert _open_rc(d) == wpcg.E_FORMAT  # entry lacks shape (serde requires it)
    d = _write(tmp_path, meta={"layers": [], "block_size": 128.0}, wpc=b"")
    assert _open_rc(d) == wpcg.E_FORMAT  # not an integer
    d = _write(tmp_path, meta={"layers": [], "block_size": 128}, wpc=None)
    os.remove(os.path.join(d, "model_v4.wpc"))
    assert _open_rc(d) == wpcg.E_IO  # .wpc missing
    d = _write(tmp_path, meta={"layers": [], "block_size": 128, "extra": {"k": [1, 2]}}, wpc=b"")
    assert _open_rc(d) == wpcg.OK  # unknown keys ignored, as serde does


def test_artifact_tensor_lookup(tmp_path):
    b1 = synth.random_v4_blocks(3, 256, 1)
    b2 = synth.random_v4_blocks(2, 128, 2)
    meta = synth.write_artifact(str(tmp_path / "a"), 4,
                                [("model.layers.0.mlp.up_proj.weight", [3, 256], b1),
                                 ("model.embed_tokens.weight", [2, 128], b2)])
    # non-layer tensors sort first (tensor_sort_key)
    assert meta["layers"][0]["name"] == "model.embed_tokens.weight"
    data = wpcg.WpcModelDataV4.open(str(tmp_path / "a"))
    assert data.tensor_count() == 2
    assert np.array_equal(data.tensor_bytes("model.layers.0.mlp.up_proj.weight"), b1)
    assert np.array_equal(data.tensor_bytes("model.embed_tokens.weight"), b2)
    with pytest.raises(wpcg.WpcgError) as e:
        data.tensor_bytes("nope")
    assert e.value.code == wpcg.E_NOTFOUND
    # a shape that disagrees with the stored block count
    with pytest.raises(wpcg.WpcgError) as e:
        wpcg.WpcLinear.from_artifact(None, data, "model.embed_tokens.weight", 3, 128)
    assert e.value.code == wpcg.E_SHAPE
    data.close()


def test_artifact_bad_ranges(tmp_path):
    d = _write(tmp_path, meta={"layers": [
        {"name": "odd", "shape": [1, 128], "offset_bytes": 0, "size_bytes": 67},
        {"name": "past", "shape": [1, 128], "offset_bytes": 68, "size_bytes": 68}],
        "block_size": 128}, wpc=bytes(100))
    data = wpcg.WpcModelDataV4.open(d)
    for name in ("odd", "past"):
        with pytest.raises(wpcg.WpcgError) as e:
            data.tensor_bytes(name)
        assert e.value.code == wpcg.E_FORMAT


def test_synth_v3_packing_matches_the_oracle_codec():
    import oracle as O
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 64, (20, 128), dtype=np.uint8)
    packed = synth.pack_v3_codes(codes)
    for r in range(20):
        assert np.array_equal(packed[r], O.v3_pack(codes[r]))


def test_fast_split_plan_never_makes_an_empty_slice():
    # FAST mode splits each row's nb blocks into slices of ceil(nb/k) blocks;
    # every slice must start inside the row (an empty trailing slice would
    # address blocks past the end of the matrix) and fit the LDS stage: 64
    # blocks with one 16-row tile per workgroup, 32 with two, 16 with four.
    # Matrices of 32 tiles or more take four tiles when a row has at most 16
    # blocks; of 192 tiles or more, two when it has at most 32; of 128 tiles
    # or more, two when a row is longer than 64 blocks; of 512 tiles or
    # more, two tiles at least. Checked for every block count and requested
    # split.
    def most_of(rows, nb):
        tiles = -(-rows // 16)
        if tiles >= 32 and nb <= 16:
            return 16
        if tiles >= 192 and nb <= 32:
            return 32
        if tiles >= 128 and nb > 64:
            return 32
        return 32 if tiles >= 512 else 64
    for nb in range(1, 161):
        for req in [0] + list(range(1, nb + 3)):
            for rows in (16, 496, 497, 1024, 2032, 2048, 2560, 3056, 3072, 8176, 8177, 9728, 151936):
                most = most_of(rows, nb)
                k = wpcg.plan_kslices(rows, nb * 128, req)
                nbk = -(-nb // k)
                assert 1 <= k <= nb and nbk <= most, (nb, req, rows, k)
                assert (k - 1) * nbk < nb <= k * nbk, (nb, req, k, nbk)
                if req == 0:
                    # the default: the fewest slices that fit, or, when that
                    # is more than one, slices of at most 32 blocks
                    raw = -(-nb // most)
                    if raw > 1:
                        raw = -(-nb // min(most, 32))
                    nbk_raw = -(-nb // raw)
                    assert k == -(-nb // nbk_raw), (nb, rows, k)
    with pytest.raises(wpcg.WpcgError) as e:
        wpcg.plan_kslices(4, 100)
    assert e.value.code == wpcg.E_SHAPE


def test_model_create_refuses_a_head_the_reference_never_builds():
    """wpcg_model_create checks the head before it needs a device: `tied`
    must be 1 for a dense decoder (the reference's dense loader builds no
    lm_head and always calls embed.logits: qwen3_model.rs:187-206,
    model.rs:545) and 0 for Qwen3-MoE (lm_head always: qwen3_moe_model.rs:
    337-343). Either mismatch is E_UNSUPPORTED; the consistent configs pass
    that check and fail only on the missing context (E_ARG)."""
    base = dict(n_layers=1, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, inter=256, vocab=64,
                n_experts=0, top_k=0, moe_inter=0, norm_topk=1, tied=1, max_pos=16, eps=1e-6,
                rope_theta=1e6)
    moe = dict(base, inter=0, n_experts=4, top_k=2, moe_inter=128, tied=0)
    h = C.c_void_p()
    for cfg, want in ((base, wpcg.E_ARG), (dict(base, tied=0), wpcg.E_UNSUPPORTED),
                      (moe, wpcg.E_ARG), (dict(moe, tied=1), wpcg.E_UNSUPPORTED)):
        c = wpcg.ModelConfig(**cfg)
        rc = wpcg.lib.wpcg_model_create(None, 4, C.byref(c), C.byref(h))
        assert rc == want, (cfg["n_experts"], cfg["tied"], rc, wpcg.last_error())
        if want == wpcg.E_UNSUPPORTED:
            assert "logits" in wpcg.last_error()


def test_deferred_split_shape_check():
    """The FAST launcher refuses a deferred K-split (slices k >= 1 written to
    a vector each, added by the readers) of more than three slices: readers
    add at most two deferred vectors and a model's deferral buffer holds two,
    so a fourth slice would write past it. Compiled from the library's own
    internal header with the host compiler; no GPU."""
    import shutil
    import tempfile
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no host C++ compiler")
    src = r'''
#include "wpcg_internal.hpp"
#include <cstdio>
int main() {
    int bad = 0;
    for (int kg = 0; kg <= 8; kg++)
        for (int routed = 0; routed <= 1; routed++) {
            const bool want = kg >= 2 && kg <= 3 && !routed;
            if (wpcg::deferred_split_ok(kg, routed != 0) != want) { std::printf("kg %d routed %d\n", kg, routed); bad++; }
        }
    return bad;
}
'''
    csrc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "wpc-engine_amd", "csrc")
    with tempfile.TemporaryDirectory() as d:
        cpp, exe = os.path.join(d, "t.cpp"), os.path.join(d, "t")
        with open(cpp, "w") as f:
            f.write(src)
        r = subprocess.run([gxx, "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I", csrc,
                            cpp, "-o", exe], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        r = subprocess.run([exe], capture_output=True, text=True)
        assert r.returncode == 0, r.stdout
