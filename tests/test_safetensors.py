"""CPU tests of the checkpoint readers behind the C ABI: safetensors files
(SafetensorsFile, wpc-runtime/src/weights.rs:125-178), sharded checkpoints
(ShardedSafetensors, weights.rs:180-264) and config.json (Config,
wpc-runtime/src/config.rs; moe_dims, qwen3_moe_model.rs:121-135).

What pins them:
  - dtype decoding against numpy's own conversions (every one of the 65536
    f16 patterns; bf16 as float32 with the low 16 bits cleared) and, for
    f16 NaNs, the half crate's published rule (payload kept, quiet bit set);
  - the file-format checks of the safetensors crate 0.4.5 (header length
    and start, offsets tiling the data, sizes against shape x dtype), each
    one broken in turn on an otherwise valid file;
  - the reference's own config tests (config.rs:104-170 and
    qwen3_moe_model.rs:549-640), with their JSON fixtures.
Where the reference panics (invalid file, missing tensor, unsupported
dtype) the readers return E_FORMAT / E_NOTFOUND / E_UNSUPPORTED.
"""
import json
import os

import numpy as np
import pytest

import wpcg
from wpcg import synth


def write(path, tensors, metadata=None):
    with open(path, "wb") as f:
        f.write(synth.safetensors_bytes(tensors, metadata))
    return path


def rc_of(fn, *args):
    with pytest.raises(wpcg.WpcgError) as e:
        fn(*args)
    return e.value.code


def f32_bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------- dtypes
def test_f32_f16_bf16_round_trip(tmp_path):
    rng = np.random.default_rng(1)
    a = rng.standard_normal((3, 5)).astype(np.float32)
    p = write(tmp_path / "m.safetensors",
              [synth.encode_st("a32", "F32", a), synth.encode_st("a16", "F16", a),
               synth.encode_st("abf", "BF16", a)], {"format": "pt"})
    st = wpcg.SafetensorsFile.open(p)
    assert st.names() == ["a32", "a16", "abf"]
    for n, dt in (("a32", "F32"), ("a16", "F16"), ("abf", "BF16")):
        assert st.shape(n) == [3, 5]
        assert st.dtype(n) == dt
    assert np.array_equal(f32_bits(st.read_f32("a32")), f32_bits(a.reshape(-1)))
    assert np.array_equal(f32_bits(st.read_f32("a16")), f32_bits(a.astype(np.float16).astype(np.float32).reshape(-1)))
    # bf16 = the upper half of the float32 pattern, widened by a 16-bit shift
    want = (synth.to_bf16_bits(a).astype(np.uint32) << 16).reshape(-1)
    assert np.array_equal(f32_bits(st.read_f32("abf")), want)
    st.close()


def test_every_f16_pattern(tmp_path):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    p = write(tmp_path / "h.safetensors", [("h", "F16", [65536], h.astype("<u2").tobytes())])
    got = f32_bits(wpcg.SafetensorsFile.open(p).read_f32("h"))
    want = f32_bits(h.view(np.float16).astype(np.float32))
    nan = ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
    assert np.array_equal(got[~nan], want[~nan])  # zeros, subnormals, normals, infinities
    # NaN: sign, all-ones exponent, payload << 13 with the quiet bit set
    hn = h[nan].astype(np.uint32)
    want_nan = ((hn & 0x8000) << 16) | 0x7FC00000 | ((hn & 0x3FF) << 13)
    assert np.array_equal(got[nan], want_nan)
    assert got[0x7C01] == 0x7FC02000 and got[0xFE00] == 0xFFC00000
    assert got[0x0001] == f32_bits(np.float32(2.0 ** -24))  # smallest subnormal


def test_bf16_special_values(tmp_path):
    bits = np.array([0x0000, 0x8000, 0x3F80, 0xBF80, 0x7F80, 0xFF80, 0x7FC0, 0x0001, 0x7F7F], np.uint16)
    p = write(tmp_path / "b.safetensors", [("b", "BF16", [bits.size], bits.astype("<u2").tobytes())])
    got = f32_bits(wpcg.SafetensorsFile.open(p).read_f32("b"))
    assert np.array_equal(got, bits.astype(np.uint32) << 16)
    v = got.view(np.float32)
    assert v[2] == 1.0 and v[3] == -1.0 and np.isinf(v[4]) and np.isnan(v[6])


def test_unsupported_dtype_and_wrong_count(tmp_path):
    p = write(tmp_path / "i.safetensors",
              [("i", "I32", [4], np.arange(4, dtype="<i4").tobytes()),
               ("f", "F32", [2, 2], np.ones(4, "<f4").tobytes())])
    st = wpcg.SafetensorsFile.open(p)
    assert st.shape("i") == [4] and st.dtype("i") == "I32"
    assert rc_of(st.read_f32, "i") == wpcg.E_UNSUPPORTED
    out = np.empty(3, np.float32)
    rc = wpcg.lib.wpcg_safetensors_read_f32(st.h, b"f", out.ctypes.data, 3)
    assert rc == wpcg.E_SHAPE
    assert rc_of(st.read_f32, "nope") == wpcg.E_NOTFOUND
    assert rc_of(st.shape, "nope") == wpcg.E_NOTFOUND


def test_scalar_and_empty_tensors(tmp_path):
    p = write(tmp_path / "s.safetensors",
              [("empty", "F32", [0, 4], b""), ("scalar", "F32", [], np.float32(2.5).tobytes())])
    st = wpcg.SafetensorsFile.open(p)
    assert st.shape("scalar") == [] and st.read_f32("scalar").tolist() == [2.5]
    assert st.shape("empty") == [0, 4] and st.read_f32("empty").size == 0


def test_all_format_dtypes_validate(tmp_path):
    """Every dtype of the 0.4.5 format is accepted at open (sizes 1/2/4/8)."""
    ts = []
    for name, (npdt, size) in synth.ST_DTYPES.items():
        ts.append((name, name, [3], bytes(3 * size)))
    st = wpcg.SafetensorsFile.open(write(tmp_path / "all.safetensors", ts))
    assert sorted(st.names()) == sorted(synth.ST_DTYPES)


# ------------------------------------------------------- format validation
def _valid(tmp_path):
    return synth.safetensors_bytes([synth.encode_st("a", "F32", np.ones(4)),
                                    synth.encode_st("b", "BF16", np.ones((2, 3)))])


def _with_header(header: dict, data: bytes, pad=True) -> bytes:
    h = json.dumps(header).encode()
    if pad:
        h += b" " * (-len(h) % 8)
    return len(h).to_bytes(8, "little") + h + data


@pytest.mark.parametrize("case", ["too_small", "too_large", "past_end", "no_brace", "bad_json",
                                  "gap", "overlap", "size_mismatch", "trailing", "short",
                                  "unknown_dtype", "bad_offsets", "bad_metadata", "negative_dim"])
def test_invalid_files_are_rejected(tmp_path, case):
    data = np.ones(4, "<f4").tobytes()
    hdr = {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}
    if case == "too_small":
        blob = b"\x01\x00\x00"
    elif case == "too_large":
        blob = (100000001).to_bytes(8, "little") + b"{}"
    elif case == "past_end":
        blob = (64).to_bytes(8, "little") + b"{}"
    elif case == "no_brace":
        blob = _with_header(hdr, data)
        blob = blob[:8] + b"[" + blob[9:]
    elif case == "bad_json":
        h = b'{"a": {"dtype": "F32",'
        blob = len(h).to_bytes(8, "little") + h + data
    elif case == "gap":
        blob = _with_header({"a": {"dtype": "F32", "shape": [4], "data_offsets": [4, 20]}}, bytes(4) + data)
    elif case == "overlap":
        blob = _with_header({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]},
                             "b": {"dtype": "F32", "shape": [2], "data_offsets": [8, 16]}}, data)
    elif case == "size_mismatch":
        blob = _with_header({"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, data)
    elif case == "trailing":
        blob = _with_header(hdr, data + b"\0\0\0\0")
    elif case == "short":
        blob = _with_header(hdr, data[:12])
    elif case == "unknown_dtype":
        blob = _with_header({"a": {"dtype": "F128", "shape": [1], "data_offsets": [0, 16]}}, data)
    elif case == "bad_offsets":
        blob = _with_header({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0]}}, data)
    elif case == "bad_metadata":
        blob = _with_header({"__metadata__": {"k": 1}, **hdr}, data)
    elif case == "negative_dim":
        blob = _with_header({"a": {"dtype": "F32", "shape": [-4], "data_offsets": [0, 16]}}, data)
    p = tmp_path / "bad.safetensors"
    p.write_bytes(blob)
    assert rc_of(wpcg.SafetensorsFile.open, p) == wpcg.E_FORMAT
    assert "invalid safetensors file" in wpcg.last_error()


def test_valid_variants_are_accepted(tmp_path):
    data = np.arange(4, dtype="<f4").tobytes()
    # offsets listed out of order, no padding, null metadata, a header whose
    # keys are not in data order: all valid
    hdr = {"__metadata__": None,
           "b": {"dtype": "F32", "shape": [2], "data_offsets": [8, 16]},
           "a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    p = tmp_path / "v.safetensors"
    p.write_bytes(_with_header(hdr, data, pad=False))
    st = wpcg.SafetensorsFile.open(p)
    assert st.read_f32("a").tolist() == [0.0, 1.0] and st.read_f32("b").tolist() == [2.0, 3.0]
    assert rc_of(wpcg.SafetensorsFile.open, tmp_path / "absent.safetensors") == wpcg.E_IO


# ------------------------------------------------------------ sharding
def test_sharded_checkpoint(tmp_path):
    rng = np.random.default_rng(5)
    a, b, c = (rng.standard_normal(n).astype(np.float32) for n in (8, 16, 4))
    write(tmp_path / "model-00001-of-00002.safetensors", [synth.encode_st("x.a", "BF16", a),
                                                          synth.encode_st("x.c", "F32", c)])
    write(tmp_path / "model-00002-of-00002.safetensors", [synth.encode_st("y.b", "F16", b)])
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({
        "metadata": {"total_size": 0},
        "weight_map": {"x.a": "model-00001-of-00002.safetensors", "x.c": "model-00001-of-00002.safetensors",
                       "y.b": "model-00002-of-00002.safetensors"}}))
    st = wpcg.ShardedSafetensors.open(tmp_path)
    assert np.array_equal(st.read_f32("x.a"), synth.widened("BF16", a))
    assert np.array_equal(st.read_f32("y.b"), synth.widened("F16", b))
    assert np.array_equal(st.read_f32("x.c"), c)
    assert st.shape("y.b") == [16]
    assert sorted(st.names()) == ["x.a", "x.c", "y.b"]
    # a name the index does not list is missing, even where a shard holds it
    assert rc_of(st.read_f32, "z") == wpcg.E_NOTFOUND
    assert "not in safetensors index" in wpcg.last_error()
    st.close()


def test_index_naming_a_tensor_its_shard_lacks(tmp_path):
    write(tmp_path / "s1.safetensors", [synth.encode_st("a", "F32", np.ones(2))])
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {"a": "s1.safetensors", "b": "s1.safetensors", "n": 3}}))
    st = wpcg.ShardedSafetensors.open(tmp_path)  # a non-string entry is skipped
    assert st.read_f32("a").tolist() == [1.0, 1.0]
    assert rc_of(st.read_f32, "b") == wpcg.E_NOTFOUND
    assert rc_of(st.read_f32, "n") == wpcg.E_NOTFOUND


def test_single_file_wins_over_index(tmp_path):
    write(tmp_path / "model.safetensors", [synth.encode_st("a", "F32", np.full(2, 7.0))])
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"a": "missing.st"}}))
    st = wpcg.ShardedSafetensors.open(tmp_path)
    assert st.read_f32("a").tolist() == [7.0, 7.0]


def test_directory_errors(tmp_path):
    assert rc_of(wpcg.ShardedSafetensors.open, tmp_path) == wpcg.E_IO
    assert "neither model.safetensors nor model.safetensors.index.json" in wpcg.last_error()
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}}))
    assert rc_of(wpcg.ShardedSafetensors.open, tmp_path) == wpcg.E_FORMAT
    assert "weight_map" in wpcg.last_error()
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"a": "gone.safetensors"}}))
    assert rc_of(wpcg.ShardedSafetensors.open, tmp_path) == wpcg.E_IO
    (tmp_path / "model.safetensors.index.json").write_text("{not json")
    assert rc_of(wpcg.ShardedSafetensors.open, tmp_path) == wpcg.E_FORMAT


# -------------------------------------------------------------- config.json
# The reference's own fixtures (config.rs:104-136; qwen3_moe_model.rs:549-600)
QWEN2_JSON = """{
    "model_type": "qwen2",
    "vocab_size": 151936,
    "hidden_size": 1536,
    "num_hidden_layers": 28,
    "num_attention_heads": 12,
    "num_key_value_heads": 2,
    "intermediate_size": 8960,
    "rope_theta": 1000000.0,
    "rms_norm_eps": 1e-06,
    "tie_word_embeddings": true
}"""
QWEN3_JSON = """{
    "model_type": "qwen3",
    "vocab_size": 151936,
    "hidden_size": 2560,
    "num_hidden_layers": 36,
    "num_attention_heads": 32,
    "num_key_value_heads": 8,
    "intermediate_size": 9728,
    "head_dim": 128,
    "attention_bias": false,
    "rope_theta": 5000000.0,
    "rms_norm_eps": 1e-06,
    "tie_word_embeddings": true
}"""
DENSE_JSON = """{
    "model_type": "qwen3", "vocab_size": 10, "hidden_size": 8,
    "num_hidden_layers": 1, "num_attention_heads": 2,
    "num_key_value_heads": 1, "intermediate_size": 16,
    "rope_theta": 10000.0, "rms_norm_eps": 1e-6
}"""


def cfg_with(n_exp, top_k, norm):
    return f"""{{
        "model_type": "qwen3_moe",
        "vocab_size": 100, "hidden_size": 8,
        "num_hidden_layers": 1, "num_attention_heads": 2,
        "num_key_value_heads": 1, "intermediate_size": 16,
        "rope_theta": 10000.0, "rms_norm_eps": 1e-6,
        "num_experts": {n_exp}, "num_experts_per_tok": {top_k},
        "moe_intermediate_size": 4, "norm_topk_prob": {"true" if norm else "false"}
    }}"""


def test_qwen2_derives_head_dim_from_hidden_size():
    c = wpcg.config_from_json_str(QWEN2_JSON, 64)
    assert c.head_dim == 1536 // 12 == 128
    assert c.n_experts == 0 and c.tied == 1 and c.max_pos == 64


def test_qwen3_reads_head_dim_from_the_file():
    c = wpcg.config_from_json_str(QWEN3_JSON, 4096)
    assert c.head_dim == 128 != c.hidden // c.n_heads
    assert c.n_heads * c.head_dim == 4096
    # unknown keys (attention_bias) are ignored
    assert (c.n_layers, c.hidden, c.n_kv_heads, c.inter, c.vocab) == (36, 2560, 8, 9728, 151936)
    assert c.rope_theta == 5000000.0 and c.eps == np.float32(1e-6)


def test_moe_config_fields_parse():
    c = wpcg.config_from_json_str(cfg_with(128, 8, True), 32)
    assert (c.n_experts, c.top_k, c.moe_inter, c.norm_topk) == (128, 8, 4, 1)
    c = wpcg.config_from_json_str(cfg_with(5, 2, False), 32)
    assert (c.n_experts, c.top_k, c.norm_topk) == (5, 2, 0)


def test_dense_config_has_no_moe_fields():
    c = wpcg.config_from_json_str(DENSE_JSON, 32)
    assert c.n_experts == 0 and c.top_k == 0 and c.norm_topk == 1
    assert c.tied == 1  # default_true


@pytest.mark.parametrize("flag", [True, False, None])
def test_head_follows_the_model_kind_not_tie_word_embeddings(flag):
    """The reference's loaders never read tie_word_embeddings for the head:
    dense load_wpc_v4 builds no lm_head and Model::forward_token always calls
    embed.logits (qwen3_model.rs:187-206, model.rs:545); Qwen3-MoE always
    loads lm_head.weight (qwen3_moe_model.rs:337-343). So `tied` is 1 for
    every dense config and 0 for every MoE config, with the key true, false
    or absent (serde's default_true)."""
    for text, tied in ((DENSE_JSON, 1), (QWEN3_JSON, 1), (cfg_with(8, 2, True), 0)):
        j = json.loads(text)
        j.pop("tie_word_embeddings", None)
        if flag is not None:
            j["tie_word_embeddings"] = flag
        assert wpcg.config_from_json_str(json.dumps(j), 8).tied == tied, (j.get("model_type"), flag)


def test_top_k_beyond_expert_count_is_rejected():
    with pytest.raises(wpcg.WpcgError) as e:
        wpcg.config_from_json_str(cfg_with(4, 8, True), 32)
    assert e.value.code == wpcg.E_FORMAT and "is not in 1..=4" in str(e.value)
    with pytest.raises(wpcg.WpcgError):
        wpcg.config_from_json_str(cfg_with(4, 0, True), 32)


def test_moe_fields_required_and_defaults():
    j = json.loads(cfg_with(8, 2, True))
    del j["norm_topk_prob"]
    assert wpcg.config_from_json_str(json.dumps(j), 8).norm_topk == 1  # unwrap_or(true)
    for key in ("num_experts", "num_experts_per_tok", "moe_intermediate_size"):
        jj = dict(j)
        del jj[key]
        with pytest.raises(wpcg.WpcgError) as e:
            wpcg.config_from_json_str(json.dumps(jj), 8)
        assert key in str(e.value)


def test_config_errors_and_load(tmp_path):
    j = json.loads(QWEN3_JSON)
    for key in ("vocab_size", "hidden_size", "num_hidden_layers", "num_attention_heads",
                "num_key_value_heads", "intermediate_size", "rope_theta", "rms_norm_eps"):
        jj = dict(j)
        del jj[key]
        with pytest.raises(wpcg.WpcgError) as e:
            wpcg.config_from_json_str(json.dumps(jj), 8)
        assert e.value.code == wpcg.E_FORMAT and key in str(e.value)
    for key, bad in (("hidden_size", -1), ("hidden_size", 2.5), ("rope_theta", "x"),
                     ("tie_word_embeddings", 1), ("head_dim", "128")):
        jj = dict(j, **{key: bad})
        with pytest.raises(wpcg.WpcgError):
            wpcg.config_from_json_str(json.dumps(jj), 8)
    jj = dict(j, tie_word_embeddings=False, head_dim=None, rope_theta=10000)  # an integer is a valid f64
    c = wpcg.config_from_json_str(json.dumps(jj), 8)
    assert c.head_dim == 2560 // 32 and c.rope_theta == 10000.0
    assert c.tied == 1  # dense: the embedding table is the head whatever the flag says
    p = tmp_path / "config.json"
    p.write_text(QWEN3_JSON)
    assert wpcg.config_load(p, 16).as_dict() == wpcg.config_from_json_str(QWEN3_JSON, 16).as_dict()
    with pytest.raises(wpcg.WpcgError) as e:
        wpcg.config_load(tmp_path / "none.json", 16)
    assert e.value.code == wpcg.E_IO


def test_checkpoint_writer_round_trip(tmp_path):
    """synth.write_checkpoint's config.json and safetensors read back as the
    config and tensors it returns (single file and three shards)."""
    cfg = dict(n_layers=2, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, inter=0, vocab=256,
               n_experts=4, top_k=2, moe_inter=128, norm_topk=1, tied=0, max_pos=16, eps=1e-6,
               rope_theta=1e6)
    for shards in (1, 3):
        d = tmp_path / f"m{shards}"
        tensors = synth.write_checkpoint(str(d), str(d / "wpc"), cfg, 4, 11, wpcg.encode, "BF16", shards)
        c = wpcg.config_load(d / "config.json", 16).as_dict()
        for k, v in cfg.items():
            if k != "inter":
                assert c[k] == pytest.approx(v, rel=1e-7), k
        st = wpcg.ShardedSafetensors.open(d)
        fp = [n for n, a in tensors.items() if a.dtype == np.float32]
        assert sorted(st.names()) == sorted(fp)
        for n in fp:
            assert np.array_equal(st.read_f32(n), tensors[n])
        st.close()
        art = wpcg.WpcModelDataV4.open(str(d / "wpc"))
        assert art.tensor_count() == len(tensors) - len(fp)
        art.close()


def test_json_edge_cases():
    """The JSON reader behind both formats: escapes, unicode, nesting limit,
    trailing garbage, duplicate keys (the last one wins, as serde_json's map)."""
    base = json.loads(QWEN3_JSON)
    txt = json.dumps(base)
    # duplicate key: the later value is the one used
    dup = txt[:-1] + ', "hidden_size": 4096}'
    assert wpcg.config_from_json_str(dup, 8).hidden == 4096
    # escapes and non-ASCII text are read, whitespace anywhere
    odd = json.dumps(dict(base, model_type="qwen3", note="tab\\t \\u00e9 \\ud83d\\ude00 \"q\""), indent=3)
    assert wpcg.config_from_json_str(odd, 8).hidden == 2560
    for bad in (txt + " x", txt[:-1], '{"a": [1, 2,]}', '{"a": "\\q"}', '{"a": 01}', "[" * 200 + "]" * 200,
                '{"vocab_size": 1e400}'):
        with pytest.raises(wpcg.WpcgError) as e:
            wpcg.config_from_json_str(bad, 8)
        assert e.value.code == wpcg.E_FORMAT, bad[:30]


def test_deeply_nested_header_is_rejected(tmp_path):
    h = ('{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}, "__metadata__": '
         + '{"x": ' * 300 + '"y"' + "}" * 300 + "}").encode()
    p = tmp_path / "deep.safetensors"
    p.write_bytes(len(h).to_bytes(8, "little") + h + bytes(4))
    assert rc_of(wpcg.SafetensorsFile.open, p) == wpcg.E_FORMAT
