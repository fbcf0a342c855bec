"""Seeded synthetic WPC blocks and artifacts in the reference's byte format.

random_v4_blocks / random_v3_blocks draw block parameters as the benchmark
configurations specify: codes uniform over the scheme's range, zero_point
f16(N(-0.03, 0.005)), scale f16(U(0.002, 0.006)), f16 by round-to-nearest-
even (numpy's float16 conversion, the same rounding as the reference's
half::f16::from_f32). numpy's PCG64 generator is used with the given seed.

write_artifact emits model_v{3,4}.meta + model_v{3,4}.wpc exactly as the
reference's compiler lays them out (wpc-compiler/src/main.rs:644-696): blocks
appended tensor after tensor, meta {"layers":[{name, shape, offset_bytes,
size_bytes}], "block_size":128}, with tensors in the compiler's locality
order (tensor_sort_key, wpc-compiler/src/main.rs:93-128).
"""
from __future__ import annotations

import json
import os
import re

import numpy as np

BPB = {3: 100, 4: 68}


def _params(rng, n):
    zp = rng.normal(-0.03, 0.005, n).astype(np.float32).astype(np.float16)
    sc = rng.uniform(0.002, 0.006, n).astype(np.float32).astype(np.float16)
    return zp.view(np.uint8).reshape(n, 2), sc.view(np.uint8).reshape(n, 2)


def random_v4_blocks(rows: int, cols: int, seed: int) -> np.ndarray:
    """rows*(cols/128) v4 blocks (68 bytes each), codes U{0..15}."""
    assert cols % 128 == 0
    n = rows * (cols // 128)
    rng = np.random.default_rng(seed)
    out = np.empty((n, 68), np.uint8)
    zp, sc = _params(rng, n)
    out[:, 0:2] = zp
    out[:, 2:4] = sc
    # packed byte j = code j | code j+64 << 4, both uniform: any byte value
    out[:, 4:] = rng.integers(0, 256, (n, 64), dtype=np.uint8)
    return out.ravel()


def pack_v3_codes(codes: np.ndarray) -> np.ndarray:
    """QuantBlockV3::pack_codes for an [n, 128] code array -> [n, 96]."""
    c = codes.astype(np.uint32).reshape(-1, 32, 4)
    word = c[..., 0] | c[..., 1] << 6 | c[..., 2] << 12 | c[..., 3] << 18
    out = np.empty(c.shape[:2] + (3,), np.uint8)
    out[..., 0] = word & 0xFF
    out[..., 1] = (word >> 8) & 0xFF
    out[..., 2] = (word >> 16) & 0xFF
    return out.reshape(-1, 96)


def random_v3_blocks(rows: int, cols: int, seed: int) -> np.ndarray:
    """rows*(cols/128) v3 blocks (100 bytes each), codes U{0..63}."""
    assert cols % 128 == 0
    n = rows * (cols // 128)
    rng = np.random.default_rng(seed)
    out = np.empty((n, 100), np.uint8)
    zp, sc = _params(rng, n)
    out[:, 0:2] = zp
    out[:, 2:4] = sc
    out[:, 4:] = pack_v3_codes(rng.integers(0, 64, (n, 128), dtype=np.uint8))
    return out.ravel()


def random_x(n: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


def tensor_sort_key(name: str):
    """(layer, section, expert, projection), wpc-compiler/src/main.rs:93-128."""
    m = re.search(r"layers\.(\d+)\.", name)
    layer = int(m.group(1)) + 1 if m else 0
    m = re.search(r"experts\.(\d+)\.", name)
    expert = int(m.group(1)) if m else None
    if "gate_proj" in name:
        proj = 0
    elif "up_proj" in name:
        proj = 1
    elif "down_proj" in name:
        proj = 2
    else:
        proj = 3
    if expert is not None:
        return (layer, 2, expert, proj)
    if "mlp.gate.weight" in name:
        return (layer, 1, 0, 0)
    return (layer, 0, 0, proj)


def write_artifact(out_dir: str, scheme: int, tensors, sort: bool = True) -> dict:
    """tensors: iterable of (name, shape, blocks_uint8). Returns the meta."""
    os.makedirs(out_dir, exist_ok=True)
    items = list(tensors)
    if sort:
        items = sorted(items, key=lambda t: tensor_sort_key(t[0]))  # stable
    meta = {"layers": [], "block_size": 128}
    off = 0
    with open(os.path.join(out_dir, f"model_v{scheme}.wpc"), "wb") as f:
        for name, shape, blocks in items:
            blocks = np.ascontiguousarray(blocks, np.uint8)
            assert blocks.size % BPB[scheme] == 0
            f.write(blocks.tobytes())
            meta["layers"].append({"name": name, "shape": list(shape),
                                   "offset_bytes": off, "size_bytes": int(blocks.size)})
            off += int(blocks.size)
    with open(os.path.join(out_dir, f"model_v{scheme}.meta"), "w") as f:
        json.dump(meta, f, indent=2)
    return meta


def model_tensors(cfg, scheme: int, seed: int, encode, std: float = 0.02, share_experts: bool = False):
    """Seeded synthetic weights of a dense Qwen3 / Qwen3-MoE decoder, by the
    reference's tensor names: every matrix ~N(0, std) then encoded with
    `encode(scheme, w)` (the artifact compiler's encoder), norms 1.0, the
    MoE router fp32 ~N(0, std). cfg: wpcg.ModelConfig or a dict of its fields.
    With share_experts, every layer gets the same expert blocks (distinct
    routers): one layer's worth of generation for a large model.
    Yields (name, array)."""
    c = cfg if isinstance(cfg, dict) else cfg.as_dict()
    rng = np.random.default_rng(seed)
    H, hd, V = c["hidden"], c["head_dim"], c["vocab"]
    qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd

    def mat(rows, cols):
        return encode(scheme, (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(std)))

    ones_h = np.ones(H, np.float32)
    yield "model.embed_tokens.weight", mat(V, H)
    if not c["tied"]:
        yield "lm_head.weight", mat(V, H)
    yield "model.norm.weight", ones_h
    shared = None
    for l in range(c["n_layers"]):
        p = f"model.layers.{l}."
        yield p + "input_layernorm.weight", ones_h
        yield p + "post_attention_layernorm.weight", ones_h
        yield p + "self_attn.q_norm.weight", np.ones(hd, np.float32)
        yield p + "self_attn.k_norm.weight", np.ones(hd, np.float32)
        yield p + "self_attn.q_proj.weight", mat(qd, H)
        yield p + "self_attn.k_proj.weight", mat(kvd, H)
        yield p + "self_attn.v_proj.weight", mat(kvd, H)
        yield p + "self_attn.o_proj.weight", mat(H, qd)
        if c["n_experts"] == 0:
            I = c["inter"]
            yield p + "mlp.gate_proj.weight", mat(I, H)
            yield p + "mlp.up_proj.weight", mat(I, H)
            yield p + "mlp.down_proj.weight", mat(H, I)
        else:
            I, E = c["moe_inter"], c["n_experts"]
            yield p + "mlp.gate.weight", (rng.standard_normal((E, H), dtype=np.float32) * np.float32(std))
            if shared is None or not share_experts:
                shared = [(mat(I, H), mat(I, H), mat(H, I)) for _ in range(E)]
            for e, (g, u, d) in enumerate(shared):
                yield p + f"mlp.experts.{e}.gate_proj.weight", g
                yield p + f"mlp.experts.{e}.up_proj.weight", u
                yield p + f"mlp.experts.{e}.down_proj.weight", d
