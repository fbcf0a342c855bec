"""Row a15: the artifact's expert-contiguous tensor order.

The reference compiler sorts every tensor by tensor_sort_key before writing
(wpc-compiler/src/main.rs:93-128, applied at :367): a stable sort on
(layer, section, expert, projection), so non-layer tensors come first in
their original order; within a layer the attention matrices (and, for a
dense model, the MLP), then the router `mlp.gate.weight`, then experts in
numeric order with each expert's gate, up, down adjacent.

The expected orders here are built by explicit loops over layers and
experts, not by the key, and the inputs are given in the order a
safetensors header lists them (names sorted as strings, so experts.10
precedes experts.2) or shuffled.
"""
import json
import os
import random

import numpy as np

from wpcg import synth

ATTN = ["self_attn.k_proj.weight", "self_attn.o_proj.weight", "self_attn.q_proj.weight",
        "self_attn.v_proj.weight"]


def _moe_names(n_layers, n_experts, with_router=True):
    names = ["lm_head.weight", "model.embed_tokens.weight"]
    for l in range(n_layers):
        p = f"model.layers.{l}."
        names += [p + a for a in ATTN]
        if with_router:
            names.append(p + "mlp.gate.weight")
        for e in range(n_experts):
            for proj in ("down_proj", "gate_proj", "up_proj"):
                names.append(p + f"mlp.experts.{e}.{proj}.weight")
    return names


def _expected_moe(n_layers, n_experts, source_order, with_router=True):
    """The compiler's output order, written out loop by loop."""
    out = [n for n in source_order if "layers." not in n]  # non-layer, original order
    for l in range(n_layers):
        p = f"model.layers.{l}."
        out += [n for n in source_order if n.startswith(p) and n[len(p):] in ATTN]
        if with_router:
            out.append(p + "mlp.gate.weight")
        for e in range(n_experts):
            for proj in ("gate_proj", "up_proj", "down_proj"):
                out.append(p + f"mlp.experts.{e}.{proj}.weight")
    return out


def test_full_qwen3_moe_layer_order():
    """A Qwen3-30B-A3B layer (128 experts) over 3 layers, from header order."""
    src = sorted(_moe_names(3, 128))  # string order: layers.10 < layers.2, experts.10 < experts.2
    got = sorted(src, key=synth.tensor_sort_key)
    assert got == _expected_moe(3, 128, src)


def test_order_is_stable_for_equal_keys_and_independent_of_input_shuffle():
    names = _moe_names(12, 16)
    for seed in range(5):
        src = names[:]
        random.Random(seed).shuffle(src)
        got = sorted(src, key=synth.tensor_sort_key)
        exp = _expected_moe(12, 16, src)
        assert got == exp
        # equal keys (attention matrices, non-layer tensors) keep input order
        att = [n for n in src if "layers.4." in n and "self_attn" in n]
        assert [n for n in got if "layers.4." in n and "self_attn" in n] == att


def test_dense_layer_mlp_sorts_before_attention():
    """Without experts the key's section is 0 for every matrix and the
    projection index decides: gate_proj 0, up_proj 1, down_proj 2, and
    everything else 3, so a dense layer's MLP precedes its attention."""
    p = "model.layers.0."
    src = [p + "self_attn.q_proj.weight", p + "mlp.down_proj.weight", p + "self_attn.k_proj.weight",
           p + "mlp.up_proj.weight", p + "mlp.gate_proj.weight", "model.embed_tokens.weight"]
    got = sorted(src, key=synth.tensor_sort_key)
    assert got == ["model.embed_tokens.weight", p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight",
                   p + "mlp.down_proj.weight", p + "self_attn.q_proj.weight",
                   p + "self_attn.k_proj.weight"]


def test_key_parses_numbers_as_rust_does():
    k = synth.tensor_sort_key
    # usize::from_str accepts a leading '+', not '-', and needs a digit
    assert k("model.layers.+3.x")[0] == 4
    assert k("model.layers.-3.x")[0] == 0
    assert k("model.layers..x")[0] == 0
    # the field is the text after the FIRST "layers." up to its first '.'
    assert k("a.layers.7")[0] == 8
    assert k("a.layers.x.layers.3.q")[0] == 0
    assert k("a.layers.12layers.3")[0] == 13
    assert k("model.layers.18446744073709551615.q")[0] == 2 ** 64
    assert k("model.layers.18446744073709551616.q")[0] == 0  # overflow: None
    # experts.N without a layer still sorts into section 2
    assert k("mlp.experts.5.down_proj.weight") == (0, 2, 5, 2)
    assert k("model.layers.2.mlp.gate.weight") == (3, 1, 0, 0)
    # "gate_proj" is tested before "up_proj"; "gate_up_proj" holds only "up_proj"
    assert k("model.layers.0.mlp.experts.1.gate_proj.up_proj.weight") == (1, 2, 1, 0)
    assert k("model.layers.0.mlp.experts.1.gate_up_proj.weight") == (1, 2, 1, 1)


def test_written_artifact_makes_each_expert_one_contiguous_run(tmp_path):
    n_exp = 12
    blocks = {}
    tensors = []
    for n in sorted(_moe_names(2, n_exp, with_router=False)):
        rows = 2 if "experts" in n else 1
        b = synth.random_v4_blocks(rows, 128, len(tensors))
        blocks[n] = b
        tensors.append((n, [rows, 128], b))
    meta = synth.write_artifact(str(tmp_path), 4, tensors)
    names = [t["name"] for t in meta["layers"]]
    assert names == _expected_moe(2, n_exp, [t[0] for t in tensors], with_router=False)
    with open(os.path.join(tmp_path, "model_v4.meta")) as f:
        assert json.load(f) == meta
    raw = np.fromfile(os.path.join(tmp_path, "model_v4.wpc"), np.uint8)
    off = 0
    for t in meta["layers"]:
        assert t["offset_bytes"] == off
        assert np.array_equal(raw[off:off + t["size_bytes"]], blocks[t["name"]])
        off += t["size_bytes"]
    assert off == raw.size
    # expert e of layer l: gate, up, down at consecutive offsets
    by = {t["name"]: t for t in meta["layers"]}
    for l in range(2):
        for e in range(n_exp):
            p = f"model.layers.{l}.mlp.experts.{e}."
            g, u, d = (by[p + f"{q}_proj.weight"] for q in ("gate", "up", "down"))
            assert u["offset_bytes"] == g["offset_bytes"] + g["size_bytes"]
            assert d["offset_bytes"] == u["offset_bytes"] + u["size_bytes"]
