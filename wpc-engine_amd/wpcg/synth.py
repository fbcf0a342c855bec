"""Seeded synthetic WPC blocks and artifacts in the reference's byte format.

random_v4_blocks / random_v3_blocks draw block parameters as the benchmark
configurations specify: codes uniform over the scheme's range, zero_point
f16(N(-0.03, 0.005)), scale f16(U(0.002, 0.006)), f16 by round-to-nearest-
even (numpy's float16 conversion, the same rounding as the reference's
half::f16::from_f32). numpy's PCG64 generator is used with the given seed.
wpc_blocks / wpc_x draw the same parameters with the benchmark
configurations' own PRNG (xoshiro256++ seeded as the reference's evaluator
seeds it; see below), so a Rust caller can regenerate them.

write_artifact emits model_v{3,4}.meta + model_v{3,4}.wpc exactly as the
reference's compiler lays them out (wpc-compiler/src/main.rs:644-696): blocks
appended tensor after tensor, meta {"layers":[{name, shape, offset_bytes,
size_bytes}], "block_size":128}, with tensors in the compiler's locality
order (tensor_sort_key, wpc-compiler/src/main.rs:93-128).

safetensors_bytes writes the dense checkpoint format the reference reads
its fp32 tensors from (an 8-byte little-endian header length, the JSON
header, the data); write_checkpoint lays out a whole model directory
(config.json, one or several safetensors files with an index) beside its
artifact.
"""
from __future__ import annotations

import json
import os

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


# ---- the benchmark configurations' PRNG -------------------------------------
# Configs 0 and 1 draw their inputs with xoshiro256++ and Box-Muller as the
# reference's evaluator does (wpc-eval/src/main.rs:77-82: seed 0x1234_5678,
# `rng.gen::<f32>()` twice per value, `(-2 ln u1).sqrt() * (2 pi u2).cos()` in
# f32), with crates pinned in the reference's Cargo.lock (rand 0.8.7,
# rand_xoshiro 0.6.0). Restated from their published algorithms:
# - xoshiro256++ 1.0 (Blackman and Vigna): result = rotl(s0 + s3, 23) + s0,
#   then t = s1 << 17, s2 ^= s0, s3 ^= s1, s1 ^= s2, s0 ^= s3, s2 ^= t,
#   s3 = rotl(s3, 45);
# - `seed_from_u64(seed)`: the four state words are the first four outputs of
#   SplitMix64 started at `seed` (x += 0x9e3779b97f4a7c15; z = x;
#   z = (z ^ z>>30) * 0xbf58476d1ce4e5b9; z = (z ^ z>>27) * 0x94d049bb133111eb;
#   z ^ z>>31);
# - `next_u32` is the upper half of `next_u64`; `gen::<f32>()` is
#   (next_u32 >> 8) * 2^-24;
# - ln and cos are the host libm's logf and cosf (what Rust's f32::ln/cos call
#   on Linux), sqrt is correctly rounded, every other step one f32 rounding.
# The weights of a matrix use one stream per row r, seeded
# WPC_SEED + ((matrix_id + 1) << 32) + r, and per block in order: u1, u2 (a
# normal n by the same Box-Muller), u, then 128 codes `next_u32 >> (32 - bits)`;
# zp = f16(-0.03 + 0.005 n), scale = f16(0.002 + 0.004 u) (round to nearest
# even, as half::f16::from_f32). x of length n is the first n values of the
# stream seeded WPC_SEED.
WPC_SEED = 0x12345678
_M64 = (1 << 64) - 1


def _rotl_np(x, k):
    return (x << np.uint64(k)) | (x >> np.uint64(64 - k))


def splitmix64_np(state):
    """One SplitMix64 step over a uint64 array: (new state, output)."""
    state = state + np.uint64(0x9E3779B97F4A7C15)
    z = (state ^ (state >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return state, z ^ (z >> np.uint64(31))


class Xoshiro256pp:
    """Independent xoshiro256++ streams, one per seed, advanced together
    (numpy uint64 arithmetic wraps modulo 2^64). `state` may be given
    instead of seeds: a (4, S) array of the four state words."""

    def __init__(self, seeds=None, state=None):
        if state is not None:
            self.s = [np.asarray(w, np.uint64).copy() for w in state]
            return
        st = np.atleast_1d(np.asarray(seeds, dtype=np.uint64)).copy()
        self.s = []
        for _ in range(4):
            st, z = splitmix64_np(st)
            self.s.append(z)

    def next_u64(self) -> np.ndarray:
        s0, s1, s2, s3 = self.s
        result = _rotl_np(s0 + s3, 23) + s0
        t = s1 << np.uint64(17)
        s2 = s2 ^ s0
        s3 = s3 ^ s1
        s1 = s1 ^ s2
        s0 = s0 ^ s3
        s2 = s2 ^ t
        s3 = _rotl_np(s3, 45)
        self.s = [s0, s1, s2, s3]
        return result

    def next_u32(self) -> np.ndarray:
        return (self.next_u64() >> np.uint64(32)).astype(np.uint32)

    def gen_f32(self) -> np.ndarray:
        return (self.next_u32() >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)


_libm = None


def _box_muller_f32(u1: np.ndarray, u2: np.ndarray) -> np.ndarray:
    """sqrt(-2 ln u1) * cos(2 pi u2), in f32 with the host libm's logf and cosf."""
    global _libm
    import ctypes
    if _libm is None:
        _libm = ctypes.CDLL("libm.so.6")
        for fn in (_libm.logf, _libm.cosf):
            fn.restype = ctypes.c_float
            fn.argtypes = [ctypes.c_float]
    two_pi = np.float32(2.0) * np.float32(np.pi)  # Rust's 2.0f32 * f32::consts::PI
    lg = np.array([_libm.logf(float(v)) for v in u1], np.float32)
    ang = (two_pi * u2.astype(np.float32)).astype(np.float32)
    cs = np.array([_libm.cosf(float(v)) for v in ang], np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        return (np.sqrt(np.float32(-2.0) * lg) * cs).astype(np.float32)


def wpc_x(n: int, seed: int = WPC_SEED) -> np.ndarray:
    """x of length n drawn as the reference's evaluator draws it (one stream,
    two uniforms per value, Box-Muller in f32)."""
    rng = Xoshiro256pp([seed])
    u = np.empty(2 * n, np.float32)
    for i in range(2 * n):
        u[i] = rng.gen_f32()[0]
    return _box_muller_f32(u[0::2], u[1::2])


def wpc_blocks(scheme: int, rows: int, cols: int, matrix_id: int, seed: int = WPC_SEED) -> np.ndarray:
    """rows*(cols/128) v4 or v3 blocks with the configs' parameters, drawn
    per row as described above."""
    assert cols % 128 == 0 and scheme in (3, 4)
    nb, bits = cols // 128, (4 if scheme == 4 else 6)
    seeds = np.uint64(seed) + (np.uint64(matrix_id + 1) << np.uint64(32)) + np.arange(rows, dtype=np.uint64)
    rng = Xoshiro256pp(seeds)
    u1 = np.empty((nb, rows), np.float32)
    u2 = np.empty((nb, rows), np.float32)
    uu = np.empty((nb, rows), np.float32)
    codes = np.empty((nb, 128, rows), np.uint8)
    shift = np.uint32(32 - bits)
    for b in range(nb):
        u1[b] = rng.gen_f32()
        u2[b] = rng.gen_f32()
        uu[b] = rng.gen_f32()
        for k in range(128):
            codes[b, k] = (rng.next_u32() >> shift).astype(np.uint8)
    n = _box_muller_f32(u1.ravel(), u2.ravel()).reshape(nb, rows)
    zp = (np.float32(-0.03) + (np.float32(0.005) * n).astype(np.float32)).astype(np.float32)
    sc = (np.float32(0.002) + (np.float32(0.004) * uu).astype(np.float32)).astype(np.float32)
    zp16 = zp.T.reshape(-1).astype(np.float16)  # [row][block] order
    sc16 = sc.T.reshape(-1).astype(np.float16)
    c = codes.transpose(2, 0, 1).reshape(rows * nb, 128)  # [row][block][k]
    out = np.empty((rows * nb, BPB[scheme]), np.uint8)
    out[:, 0:2] = zp16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = sc16.view(np.uint8).reshape(-1, 2)
    if scheme == 4:
        out[:, 4:] = (c[:, :64] & 15) | ((c[:, 64:] & 15) << 4)
    else:
        out[:, 4:] = pack_v3_codes(c)
    return out.ravel()


def _rust_usize(s: str):
    """`s.parse::<usize>().ok()`: an optional '+', then one or more ASCII
    digits, at most 2^64 - 1; anything else is None."""
    if s.startswith("+"):
        s = s[1:]
    if not s or not all("0" <= ch <= "9" for ch in s):
        return None
    v = int(s)
    return v if v < 2 ** 64 else None


def _field_after(name: str, marker: str):
    """`name.split(marker).nth(1).and_then(|r| r.split('.').next())` parsed as
    usize: the text between the first and second occurrence of `marker` (or
    the end), cut at its first '.'."""
    parts = name.split(marker)
    if len(parts) < 2:
        return None
    return _rust_usize(parts[1].split(".")[0])


def tensor_sort_key(name: str):
    """(layer, section, expert, projection), wpc-compiler/src/main.rs:93-128:
    layer is 0 for non-layer tensors, else the layer index + 1; section 0
    for the layer's other matrices, 1 for the router (`mlp.gate.weight`), 2
    for experts, which sort by numeric index, each one's gate/up/down
    adjacent. Sorting by it is stable (Rust's sort_by_key)."""
    layer = _field_after(name, "layers.")
    layer = layer + 1 if layer is not None else 0
    expert = _field_after(name, "experts.")
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


def permute_rows(blocks, rows: int, cols: int, scheme: int, perm) -> np.ndarray:
    """The block rows of a [rows, cols] matrix (reference layout, one row =
    cols/128 consecutive blocks) in the order `perm`."""
    row_bytes = (cols // 128) * BPB[scheme]
    return np.ascontiguousarray(np.asarray(blocks, np.uint8).reshape(rows, row_bytes)[perm]).ravel()


def model_tensors(cfg, scheme: int, seed: int, encode, std: float = 0.02, derive_layers: bool = False,
                  lm_head: bool | None = None):
    """Seeded synthetic weights of a dense Qwen3 / Qwen3-MoE decoder, by the
    reference's tensor names: every matrix ~N(0, std) then encoded with
    `encode(scheme, w)` (the artifact compiler's encoder), norms 1.0, the
    MoE router fp32 ~N(0, std). cfg: wpcg.ModelConfig or a dict of its fields.
    With derive_layers, only layer 0's matrices are encoded from fresh draws;
    every later layer's quantized matrices are seeded random row permutations
    of layer 0's (one permutation per layer and matrix), so each layer holds
    distinct weights of the same distribution without encoding every layer
    on the host (15 GB of experts for the Qwen3-30B-A3B shape). Routers are
    drawn fresh for every layer. lm_head.weight is yielded for a MoE model
    (its head) and, with lm_head=True, for a dense one too (a tensor an
    untied dense checkpoint holds and the reference's dense loader never
    reads).
    Yields (name, array)."""
    c = cfg if isinstance(cfg, dict) else cfg.as_dict()
    rng = np.random.default_rng(seed)
    H, hd, V = c["hidden"], c["head_dim"], c["vocab"]
    qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd

    def mat(rows, cols):
        return encode(scheme, (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(std)))

    ones_h = np.ones(H, np.float32)
    yield "model.embed_tokens.weight", mat(V, H)
    if c["n_experts"] if lm_head is None else lm_head:
        yield "lm_head.weight", mat(V, H)
    yield "model.norm.weight", ones_h
    E = c["n_experts"]
    I = c["moe_inter"] if E else c["inter"]
    # (suffix, rows, cols) of every quantized matrix of a layer
    shapes = [("self_attn.q_proj.weight", qd, H), ("self_attn.k_proj.weight", kvd, H),
              ("self_attn.v_proj.weight", kvd, H), ("self_attn.o_proj.weight", H, qd)]
    if E == 0:
        shapes += [("mlp.gate_proj.weight", I, H), ("mlp.up_proj.weight", I, H), ("mlp.down_proj.weight", H, I)]
    else:
        for e in range(E):
            shapes += [(f"mlp.experts.{e}.gate_proj.weight", I, H), (f"mlp.experts.{e}.up_proj.weight", I, H),
                       (f"mlp.experts.{e}.down_proj.weight", H, I)]
    first = None
    for l in range(c["n_layers"]):
        p = f"model.layers.{l}."
        yield p + "input_layernorm.weight", ones_h
        yield p + "post_attention_layernorm.weight", ones_h
        yield p + "self_attn.q_norm.weight", np.ones(hd, np.float32)
        yield p + "self_attn.k_norm.weight", np.ones(hd, np.float32)
        if E:
            yield p + "mlp.gate.weight", (rng.standard_normal((E, H), dtype=np.float32) * np.float32(std))
        if first is None or not derive_layers:
            mats = [mat(r, k) for _, r, k in shapes]
            if derive_layers:
                first = mats
        else:
            prng = np.random.default_rng((seed, l))
            mats = [permute_rows(b, r, k, scheme, prng.permutation(r)) for b, (_, r, k) in zip(first, shapes)]
        for (suffix, _, _), b in zip(shapes, mats):
            yield p + suffix, b


# dtype name -> (numpy dtype of the stored element, bytes per element); BF16
# is stored as the upper 16 bits of a float32.
ST_DTYPES = {"F32": ("<f4", 4), "F16": ("<f2", 2), "BF16": ("<u2", 2), "F64": ("<f8", 8),
             "I32": ("<i4", 4), "I64": ("<i8", 8), "U8": ("u1", 1), "I8": ("i1", 1),
             "BOOL": ("u1", 1), "I16": ("<i2", 2), "U16": ("<u2", 2), "U32": ("<u4", 4),
             "U64": ("<u8", 8), "F8_E5M2": ("u1", 1), "F8_E4M3": ("u1", 1)}


def to_bf16_bits(a) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (NaN kept a NaN)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.ascontiguousarray(a, np.float32))
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def safetensors_bytes(tensors, metadata=None) -> bytes:
    """A .safetensors file: tensors is an iterable of (name, dtype, shape,
    raw bytes) laid out in that order; metadata an optional str->str map."""
    header, chunks, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dtype, shape, raw in tensors:
        raw = bytes(raw)
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        chunks.append(raw)
        off += len(raw)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)  # the writer's alignment padding
    return len(h).to_bytes(8, "little") + h + b"".join(chunks)


def encode_st(name: str, dtype: str, a) -> tuple:
    """(name, dtype, shape, raw) for a float array stored as F32/F16/BF16."""
    a = np.asarray(a, np.float32)
    if dtype == "F32":
        raw = a.astype("<f4").tobytes()
    elif dtype == "F16":
        raw = a.astype("<f2").tobytes()
    elif dtype == "BF16":
        raw = to_bf16_bits(a).astype("<u2").tobytes()
    else:
        raise ValueError(dtype)
    return name, dtype, a.shape, raw


def widened(dtype: str, a) -> np.ndarray:
    """The float32 values a reader of `dtype` storage sees."""
    a = np.asarray(a, np.float32)
    if dtype == "F16":
        return a.astype(np.float16).astype(np.float32)
    if dtype == "BF16":
        return (to_bf16_bits(a).astype(np.uint32) << 16).view(np.float32).reshape(a.shape)
    return a.copy()


def config_json(cfg, tie_word_embeddings="auto") -> dict:
    """config.json fields of a wpcg.ModelConfig (or dict of its fields), in
    the Hugging Face names the reference's Config reads.
    tie_word_embeddings: "auto" writes what checkpoints of the kind declare
    (dense Qwen3-4B true, Qwen3-MoE false), True/False that value, None
    leaves the key out. It never changes the head the reference's loaders
    take (the embedding table for dense, lm_head for MoE)."""
    c = cfg if isinstance(cfg, dict) else cfg.as_dict()
    j = {"model_type": "qwen3_moe" if c["n_experts"] else "qwen3",
         "vocab_size": c["vocab"], "hidden_size": c["hidden"], "num_hidden_layers": c["n_layers"],
         "num_attention_heads": c["n_heads"], "num_key_value_heads": c["n_kv_heads"],
         "intermediate_size": c["inter"] or 6144, "head_dim": c["head_dim"],
         "rope_theta": float(c["rope_theta"]), "rms_norm_eps": float(c["eps"])}
    if tie_word_embeddings == "auto":
        j["tie_word_embeddings"] = not c["n_experts"]
    elif tie_word_embeddings is not None:
        j["tie_word_embeddings"] = bool(tie_word_embeddings)
    if c["n_experts"]:
        j.update(num_experts=c["n_experts"], num_experts_per_tok=c["top_k"],
                 moe_intermediate_size=c["moe_inter"], norm_topk_prob=bool(c["norm_topk"]))
    return j


def write_checkpoint(model_dir: str, wpc_dir: str, cfg, scheme: int, seed: int, encode,
                     dtype: str = "BF16", shards: int = 1, tie_word_embeddings="auto",
                     lm_head: bool | None = None) -> dict:
    """A model directory as the reference loads it: config.json plus the fp32
    tensors (norms ~1 + N(0, 0.1), routers ~N(0, 0.02)) in safetensors of
    `dtype`, one model.safetensors or `shards` files with an index; and the
    quantized matrices in a WPC artifact under wpc_dir. tie_word_embeddings
    goes to config.json as config_json writes it; lm_head as model_tensors
    takes it. Returns every tensor as the decoder sees it (fp32 tensors
    widened from their storage)."""
    os.makedirs(model_dir, exist_ok=True)
    with open(os.path.join(model_dir, "config.json"), "w") as f:
        json.dump(config_json(cfg, tie_word_embeddings), f, indent=2)
    rng = np.random.default_rng(seed + 7)
    tensors, dense, quant = {}, [], []
    for name, arr in model_tensors(cfg, scheme, seed, encode, lm_head=lm_head):
        if arr.dtype == np.uint8:
            quant.append((name, None, arr))
            tensors[name] = arr
            continue
        if name.endswith("mlp.gate.weight"):
            v = arr
        else:
            v = (1.0 + 0.1 * rng.standard_normal(arr.shape)).astype(np.float32)
        dense.append(encode_st(name, dtype, v))
        tensors[name] = widened(dtype, v).reshape(-1)
    c = cfg if isinstance(cfg, dict) else cfg.as_dict()
    write_artifact(wpc_dir, scheme, [(n, _quant_shape(n, c), b) for n, _, b in quant])
    if shards <= 1:
        with open(os.path.join(model_dir, "model.safetensors"), "wb") as f:
            f.write(safetensors_bytes(dense, {"format": "pt"}))
    else:
        weight_map = {}
        for s in range(shards):
            fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            part = dense[s::shards]
            with open(os.path.join(model_dir, fname), "wb") as f:
                f.write(safetensors_bytes(part, {"format": "pt"}))
            for t in part:
                weight_map[t[0]] = fname
        with open(os.path.join(model_dir, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {"total_size": sum(len(t[3]) for t in dense)},
                       "weight_map": weight_map}, f, indent=2)
    return tensors


def _quant_shape(name: str, c) -> list:
    """[out, in] of a quantized matrix by its name."""
    H, hd = c["hidden"], c["head_dim"]
    qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd
    I = c["moe_inter"] if c["n_experts"] else c["inter"]
    if "embed_tokens" in name or name.startswith("lm_head"):
        return [c["vocab"], H]
    if "q_proj" in name:
        return [qd, H]
    if "k_proj" in name or "v_proj" in name:
        return [kvd, H]
    if "o_proj" in name:
        return [H, qd]
    if "down_proj" in name:
        return [H, I]
    return [I, H]
