"""Independent pin of the oracle's decode-step composition: HF transformers.

The oracle's or_forward_token_v4 (dense Qwen3 and Qwen3-MoE), or_moe_ffn_v4
and or_dense_matvec compose functions that other tests pin one by one
(f16, codecs, GEMV kernels, RMSNorm, RoPE, softmax, route, SiLU). This file
checks the composition itself against a second, unrelated implementation of
the same models: transformers' Qwen3ForCausalLM / Qwen3MoeForCausalLM, the
implementation the reference validates its engine against
(wpc-runtime/scripts/hf_reference.py:26-58: HF greedy decode, token for
token). The models are built offline from a config (no checkpoint), in
float64, and given the oracle's weights dequantized from the v4 blocks
(w = zp + code*scale: the product is exact in fp32 for 4-bit codes and f16
scales, so the GEMV's fma dequant and the embedding's two-rounding dequant
give the same fp32 weight). Norm weights are random and non-unit, so a norm
weight dropped or applied in the wrong place fails.

What is asserted (semantics: model.rs:419-547, qwen3_moe_model.rs:406-542):
  - teacher-forced logits of every step (prompt + 64 greedy steps) within
    LOGIT_TOL of the logit range of HF's float64 logits;
  - the oracle's greedy ids equal HF's argmax at every one of the 64 steps,
    i.e. HF's greedy decode from the same prompt yields the same 64 ids, and
    the top-2 margin of each step is reported against the tolerance;
  - or_moe_ffn_v4 against HF's Qwen3MoeSparseMoeBlock: the same experts in the
    same (descending) order, and the output within a stated bound;
  - or_dense_matvec against float64 (error within gamma_K * sum|w x|) and
    against numpy's strictly sequential float32 accumulate (bit for bit: the
    reference sums in index order, product and sum rounded separately,
    weights.rs:59-78).

transformers computes RMSNorm and the router softmax in float32 even in a
float64 model (Qwen3RMSNorm, Qwen3MoeTopKRouter); the tolerances cover that.
torch and transformers are imported inside the tests (skipped when absent),
so collecting this file in a GPU session loads no second HIP runtime.
"""
import numpy as np
import pytest

import oracle as O
from wpcg import synth

# |oracle - HF| <= LOGIT_TOL * (max - min of HF's logits) at every step.
# Measured worst: 3.3e-7 (dense), 3.8e-7 (MoE):
# the oracle is fp32 throughout.
LOGIT_TOL = 1e-5

DENSE = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=384, vocab=512,
             n_experts=0, top_k=0, moe_inter=0, norm_topk=1, tied=1, eps=1e-6, rope_theta=1e6)
MOE = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=0, vocab=512,
           n_experts=16, top_k=4, moe_inter=128, norm_topk=1, tied=0, eps=1e-6, rope_theta=1e6)


def _hf():
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    return torch, transformers


def dequant_v4(blocks, rows, cols):
    """Reference v4 blocks -> fp32 [rows, cols]: byte j of a block holds
    code j (low nibble) and code j + 64 (high nibble); w = zp + code*scale."""
    b = np.asarray(blocks, np.uint8).reshape(rows * (cols // 128), 68)
    zp = b[:, 0:2].copy().view(np.float16).astype(np.float64)
    sc = b[:, 2:4].copy().view(np.float16).astype(np.float64)
    codes = np.concatenate([b[:, 4:] & 15, b[:, 4:] >> 4], axis=1).astype(np.float64)
    return (zp + codes * sc).astype(np.float32).reshape(rows, cols)


def _tensors(cfg, seed, lm_head=None):
    """The synthetic model's tensors, with random non-unit norm weights
    (lm_head: as synth.model_tensors takes it)."""
    t = dict(synth.model_tensors(cfg, 4, seed, lambda s, w: O.encode_tensor_v4(w), lm_head=lm_head))
    rng = np.random.default_rng(seed + 1)
    for n in list(t):
        if n.endswith("norm.weight") or n.endswith("layernorm.weight"):
            t[n] = (1.0 + 0.25 * rng.standard_normal(t[n].size)).astype(np.float32)
    return t


def _shape(cfg, name):
    H, hd = cfg["hidden"], cfg["head_dim"]
    qd, kvd = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    inter = cfg["moe_inter"] if "experts." in name else cfg["inter"]
    for key, shp in (("embed_tokens", (cfg["vocab"], H)), ("lm_head", (cfg["vocab"], H)),
                     ("q_proj", (qd, H)), ("k_proj", (kvd, H)), ("v_proj", (kvd, H)),
                     ("o_proj", (H, qd)), ("gate_proj", (inter, H)), ("up_proj", (inter, H)),
                     ("down_proj", (H, inter))):
        if key in name:
            return shp
    raise KeyError(name)


def hf_model(cfg, tensors):
    """A float64 transformers model holding the oracle's weights, with the
    head the reference's loaders take: tied to the embedding for a dense
    model (an lm_head.weight among the tensors is not loaded, as
    qwen3_model.rs:187-206 never reads it), its own lm_head for MoE."""
    torch, tf = _hf()
    tie = not cfg["n_experts"]
    common = dict(vocab_size=cfg["vocab"], hidden_size=cfg["hidden"],
                  num_hidden_layers=cfg["n_layers"], num_attention_heads=cfg["n_heads"],
                  num_key_value_heads=cfg["n_kv_heads"], head_dim=cfg["head_dim"],
                  rope_theta=cfg["rope_theta"], rms_norm_eps=cfg["eps"],
                  tie_word_embeddings=tie, max_position_embeddings=4096,
                  attention_bias=False, hidden_act="silu", attn_implementation="eager")
    if cfg["n_experts"]:
        hc = tf.Qwen3MoeConfig(intermediate_size=cfg["moe_inter"], moe_intermediate_size=cfg["moe_inter"],
                               num_experts=cfg["n_experts"], num_experts_per_tok=cfg["top_k"],
                               norm_topk_prob=bool(cfg["norm_topk"]), decoder_sparse_step=1,
                               mlp_only_layers=[], experts_implementation="eager", **common)
        model = tf.Qwen3MoeForCausalLM(hc)
    else:
        hc = tf.Qwen3Config(intermediate_size=cfg["inter"], **common)
        model = tf.Qwen3ForCausalLM(hc)
    assert float(model.config.rope_parameters["rope_theta"]) == cfg["rope_theta"]
    model = model.double().eval()
    sd = {}
    for name, a in tensors.items():
        if a.dtype == np.uint8:
            sd[name] = dequant_v4(a, *_shape(cfg, name))
        else:
            sd[name] = np.asarray(a, np.float32).reshape(-1)
    if cfg["n_experts"]:
        E = cfg["n_experts"]
        for l in range(cfg["n_layers"]):
            p = f"model.layers.{l}.mlp."
            gu = [np.concatenate([sd.pop(p + f"experts.{e}.gate_proj.weight"),
                                  sd.pop(p + f"experts.{e}.up_proj.weight")]) for e in range(E)]
            sd[p + "experts.gate_up_proj"] = np.stack(gu)
            sd[p + "experts.down_proj"] = np.stack([sd.pop(p + f"experts.{e}.down_proj.weight")
                                                    for e in range(E)])
            sd[p + "gate.weight"] = sd[p + "gate.weight"].reshape(E, cfg["hidden"])
    params = dict(model.named_parameters())
    with torch.no_grad():
        for name, a in sd.items():
            if name == "lm_head.weight" and tie:
                continue
            p = params[name]
            p.copy_(torch.from_numpy(np.asarray(a, np.float64).reshape(tuple(p.shape))))
        loaded = set(sd) | ({"lm_head.weight"} if tie else set())
        missing = [n for n in params if n not in loaded]
        assert not missing, missing
    return model


def _greedy_oracle(cfg, tensors, prompt, n_new):
    kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
    ref = O.Model(cfg, tensors, len(prompt) + n_new + 1, kern, 8)
    seq, logits = list(prompt), []
    for i in range(len(prompt) + n_new - 1):
        r = ref.forward_token(seq[i])
        logits.append(r)
        if i + 1 >= len(prompt):
            seq.append(O.argmax(r))
    ref.close()
    return seq, np.stack(logits)


@pytest.mark.parametrize("name,cfg,seed,lm_head", [("dense", DENSE, 41, None), ("moe", MOE, 42, None),
                                                   ("dense-with-lm_head", DENSE, 43, True)])
def test_forward_token_matches_transformers(name, cfg, seed, lm_head):
    """dense-with-lm_head: the tensors also hold an lm_head.weight (an untied
    dense checkpoint such as Qwen3-8B); the reference's dense decoder still
    takes its logits from the embedding (model.rs:545), and so must the
    oracle: HF is built tied, so an oracle that read lm_head would differ at
    the first step."""
    torch, _ = _hf()
    tensors = _tensors(cfg, seed, lm_head)
    model = hf_model(cfg, tensors)
    n_prompt, n_new = 8, 64
    prompt = [int(t) for t in np.random.default_rng(seed).integers(0, cfg["vocab"], n_prompt)]
    seq, ours = _greedy_oracle(cfg, tensors, prompt, n_new)
    assert len(seq) == n_prompt + n_new
    with torch.no_grad():
        hf = model(input_ids=torch.tensor([seq[:-1]]), use_cache=False).logits[0].numpy()
    assert hf.shape == ours.shape
    worst, min_margin = 0.0, np.inf
    for step in range(len(seq) - 1):
        span = float(hf[step].max() - hf[step].min())
        err = float(np.max(np.abs(ours[step].astype(np.float64) - hf[step]))) / span
        worst = max(worst, err)
        assert err <= LOGIT_TOL, f"{name}: step {step} differs by {err:.2e} of the logit range"
        if step + 1 >= n_prompt:
            top2 = np.sort(hf[step])[-2:]
            min_margin = min(min_margin, float(top2[1] - top2[0]) / span)
            assert int(np.argmax(hf[step])) == seq[step + 1], f"{name}: greedy id differs at step {step}"
    print(f"[hf] {name}: {len(seq) - 1} steps, worst logit error {worst:.2e} of the range; "
          f"64 greedy ids identical, smallest top-2 margin {min_margin:.2e} of the range")
    # HF's own greedy loop, step by step with its KV cache, gives the same ids
    with torch.no_grad():
        out = model.generate(input_ids=torch.tensor([prompt]), max_new_tokens=n_new, do_sample=False,
                             num_beams=1, use_cache=True, pad_token_id=0)
    assert out[0].tolist() == seq


def test_moe_ffn_matches_sparse_moe_block():
    torch, tf = _hf()
    E, H, I, k = 32, 256, 128, 6
    rng = np.random.default_rng(7)
    router = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    experts = [tuple(O.encode_tensor_v4((rng.standard_normal(r * c) * 0.02).astype(np.float32))
                     for r, c in ((I, H), (I, H), (H, I))) for _ in range(E)]
    hc = tf.Qwen3MoeConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E,
                           num_experts_per_tok=k, norm_topk_prob=True, hidden_act="silu",
                           experts_implementation="eager")
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock
    blk = Qwen3MoeSparseMoeBlock(hc).double().eval()
    with torch.no_grad():
        blk.gate.weight.copy_(torch.from_numpy(router.astype(np.float64)))
        for e, (g, u, d) in enumerate(experts):
            blk.experts.gate_up_proj[e].copy_(torch.from_numpy(
                np.concatenate([dequant_v4(g, I, H), dequant_v4(u, I, H)]).astype(np.float64)))
            blk.experts.down_proj[e].copy_(torch.from_numpy(dequant_v4(d, H, I).astype(np.float64)))
    worst = 0.0
    for trial in range(16):
        x = rng.standard_normal(H).astype(np.float32)
        out, ids, w = O.moe_ffn_v4(router, experts, x, k, True)
        with torch.no_grad():
            xt = torch.from_numpy(x.astype(np.float64)).view(1, 1, H)
            _, hw, hidx = blk.gate(xt.view(1, H))
            y = blk(xt).view(H).numpy()
        assert hidx[0].tolist() == ids.tolist(), f"trial {trial}: experts {ids} vs HF {hidx[0].tolist()}"
        assert np.allclose(w, hw[0].numpy(), rtol=1e-6, atol=0)
        scale = float(np.max(np.abs(y)))
        err = float(np.max(np.abs(out - y))) / scale
        worst = max(worst, err)
        assert err <= 1e-5, f"trial {trial}: moe output off by {err:.2e}"
    print(f"[hf] moe block: 16 inputs, same experts and order, worst error {worst:.2e} of max|y|")


def test_dense_matvec_against_float64_and_sequential_sum():
    rng = np.random.default_rng(11)
    for out_f, in_f in ((128, 2048), (7, 5), (33, 1000)):
        W = rng.standard_normal((out_f, in_f)).astype(np.float32)
        x = rng.standard_normal(in_f).astype(np.float32)
        b = rng.standard_normal(out_f).astype(np.float32)
        y = O.dense_matvec(W, x)
        exact = W.astype(np.float64) @ x.astype(np.float64)
        u = 2.0 ** -24
        gamma = in_f * u / (1 - in_f * u)
        bound = gamma * (np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64)))
        assert np.all(np.abs(y - exact) <= bound)
        # index order, each product rounded to fp32 before it is added
        seq = np.add.accumulate((W * x[None, :]).astype(np.float32), axis=1, dtype=np.float32)[:, -1]
        assert np.array_equal(y.view(np.uint32), seq.view(np.uint32))
        # bias added after the sum
        yb = O.dense_matvec(W, x, b)
        assert np.array_equal(yb.view(np.uint32), (seq + b).astype(np.float32).view(np.uint32))
    # a transposed operand fails the float64 check
    Wsq = rng.standard_normal((64, 64)).astype(np.float32)
    xs = rng.standard_normal(64).astype(np.float32)
    wrong = O.dense_matvec(np.ascontiguousarray(Wsq.T), xs)
    assert not np.allclose(wrong, Wsq.astype(np.float64) @ xs, rtol=1e-3)


def test_dequant_matches_the_oracle_embedding():
    """The dequant used to load HF equals the oracle's embedding rows (two
    roundings) bit for bit, so both models hold the same weights."""
    blocks = synth.random_v4_blocks(40, 512, 5)
    W = dequant_v4(blocks, 40, 512)
    for r in range(40):
        assert np.array_equal(W[r].view(np.uint32), O.embed(4, blocks, 512, r).view(np.uint32))
