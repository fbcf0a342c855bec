"""GPU tests of the device-resident decode step against the oracle's
restatement of Model::forward_token (model.rs:419-547) and
Qwen3MoeModel::forward_token (qwen3_moe_model.rs:406-542) with greedy
argmax (sampling.rs:3-14), on seeded synthetic v4 models (weights
~N(0, 0.02) encoded as the artifact compiler does, norms 1.0).

EXACT mode: the logits of every step are bit-identical to the oracle's, and
greedy generation gives the same token ids for 64 steps. FAST mode (the mode
the throughput figures use): every step's logits within FAST_TOL of the
oracle's logit range, and its 64 greedy ids identical to EXACT's (and so to
the oracle's).

Shapes: small dense and MoE models; two layers of the Qwen3-30B-A3B shape
(config 3) and of the dense Qwen3-4B shape (config 2: hidden 2560, 32q/8kv
heads of 128, intermediate 9728, tied vocabulary of 151936); and a model whose
o_proj input is an odd number of blocks (6 heads of 64 = 3 blocks), which
exercises the FAST attention merge on a half-filled pair of blocks."""

# FAST logits: |fast - oracle| <= FAST_TOL * (max - min of the oracle's
# logits) at every step. FAST carries x to 28 bits per 128-block with exact
# integer dot products and sums in a fixed order other than the reference's;
# the measured worst is about 1.1e-6 of the range.
FAST_TOL = 1e-5
import numpy as np
import pytest

import oracle as O
import wpcg
from wpcg import synth

pytestmark = pytest.mark.gpu

DENSE = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=512, vocab=1000,
             n_experts=0, top_k=0, moe_inter=0, norm_topk=1, tied=1, max_pos=96, eps=1e-6,
             rope_theta=1e6)
MOE = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=0, vocab=1000,
           n_experts=16, top_k=4, moe_inter=128, norm_topk=1, tied=0, max_pos=96, eps=1e-6,
           rope_theta=1e6)
# Qwen3-30B-A3B shapes (config 3) with two of the 48 layers
QWEN3_MOE_2L = dict(n_layers=2, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=128, inter=0,
                    vocab=151936, n_experts=128, top_k=8, moe_inter=768, norm_topk=1, tied=0,
                    max_pos=80, eps=1e-6, rope_theta=1e6)
# Qwen3-4B shapes (config 2) with two of the 36 layers
QWEN3_4B_2L = dict(n_layers=2, hidden=2560, n_heads=32, n_kv_heads=8, head_dim=128, inter=9728,
                   vocab=151936, n_experts=0, top_k=0, moe_inter=0, norm_topk=1, tied=1,
                   max_pos=96, eps=1e-6, rope_theta=1e6)
# o_proj reads 6 x 64 = 384 values: 3 blocks, an odd count
ODD_OPROJ = dict(n_layers=2, hidden=256, n_heads=6, n_kv_heads=2, head_dim=64, inter=384, vocab=1000,
                 n_experts=0, top_k=0, moe_inter=0, norm_topk=1, tied=1, max_pos=96, eps=1e-6,
                 rope_theta=1e6)
# Long contexts: past 16 x 32 = 512 positions each FAST attention chunk holds
# a second block of 32 positions, past 1024 a third. LONG: head_dim 64 with
# 2 query heads per key head (the 512-thread attention); LONG_REP8: head_dim
# 128 with 8 query heads per key head (the 256-thread attention, as in the
# Qwen3-30B-A3B shape).
LONG = dict(DENSE, max_pos=1100)
LONG_REP8 = dict(n_layers=1, hidden=512, n_heads=16, n_kv_heads=2, head_dim=128, inter=512, vocab=1000,
                 n_experts=0, top_k=0, moe_inter=0, norm_topk=1, tied=1, max_pos=1100, eps=1e-6,
                 rope_theta=1e6)


@pytest.fixture(scope="module")
def ctx():
    c = wpcg.Context(0)
    yield c
    c.close()


def build(ctx, cfg, seed):
    tensors = dict(synth.model_tensors(cfg, 4, seed, wpcg.encode))
    m = wpcg.Model(ctx, 4, wpcg.ModelConfig(**cfg))
    for name, arr in tensors.items():
        m.set_tensor(name, arr)
    kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
    ref = O.Model(cfg, tensors, cfg["max_pos"], kern, 16)
    return m, ref


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name,cfg,n_prompt,n_new,seed", [("dense", DENSE, 8, 64, 101),
                                                          ("moe", MOE, 8, 64, 202),
                                                          ("qwen3-moe-2L", QWEN3_MOE_2L, 12, 64, 303),
                                                          ("qwen3-4b-2L", QWEN3_4B_2L, 12, 64, 404),
                                                          ("odd-oproj", ODD_OPROJ, 8, 64, 505)])
def test_exact_decode_is_bit_identical(ctx, name, cfg, n_prompt, n_new, seed):
    print(f"[gpu] decode {name}: building", flush=True)
    m, ref = build(ctx, cfg, seed)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, cfg["vocab"], n_prompt).astype(np.uint32)
    # step by step, feeding the oracle's own greedy choice back in
    print(f"[gpu] decode {name}: {n_prompt} prompt + {n_new} greedy steps", flush=True)
    ids = []
    tok = int(prompt[0])
    for step in range(n_prompt + n_new - 1):
        r = ref.forward_token(tok)
        g, a = m.forward_token(tok)
        assert np.array_equal(bits(g), bits(r)), f"{name}: logits differ at step {step}"
        assert a == int(np.argmax(r)) or r[a] == r.max()
        nxt = O.argmax(r)
        assert a == nxt, f"{name}: argmax {a} vs {nxt} at step {step}"
        if step + 1 < n_prompt:
            tok = int(prompt[step + 1])
        else:
            ids.append(nxt)
            tok = nxt
    assert m.position() == n_prompt + n_new - 1
    # the same greedy run entirely on the device
    out, _ = m.generate(prompt, n_new)
    assert list(out[: len(ids)]) == ids, f"{name}: generate() diverges from the stepwise run"
    print(f"[gpu] decode {name}: {n_new} greedy ids identical, e.g. {ids[:8]}", flush=True)

    # FAST mode: the first prompt step's logits close to EXACT's, and the same
    # 64 greedy ids from the same prompt (generate: batched prompt in FAST)
    m.set_mode(wpcg.MODE_FAST).reset()
    g, _ = m.forward_token(int(prompt[0]))
    m.reset()
    m.set_mode(wpcg.MODE_EXACT)
    e, _ = m.forward_token(int(prompt[0]))
    span = float(e.max() - e.min())
    err = float(np.max(np.abs(g - e))) / span
    assert err <= FAST_TOL, f"{name}: FAST logits {err:.2e} of the range from EXACT"
    m.set_mode(wpcg.MODE_FAST)
    for prefill in (True, False):
        m.set_prefill(prefill)
        fout, _ = m.generate(prompt, n_new)
        same = int(np.argmax(np.concatenate([fout != out, [True]])))
        print(f"[gpu] decode {name}: FAST ({'batched' if prefill else 'stepwise'} prompt) greedy ids "
              f"match EXACT for {same} of {n_new} steps", flush=True)
        assert list(fout) == list(out), f"{name}: FAST greedy ids part from EXACT at step {same}"
    m.close()
    ref.close()


@pytest.mark.parametrize("name,cfg,n_steps,seed", [("dense", DENSE, 90, 111), ("moe", MOE, 90, 212),
                                                    ("qwen3-moe-2L", QWEN3_MOE_2L, 78, 313),
                                                    ("qwen3-4b-2L", QWEN3_4B_2L, 90, 414),
                                                    ("odd-oproj", ODD_OPROJ, 90, 515),
                                                    ("long", LONG, 1060, 616),
                                                    ("long-rep8", LONG_REP8, 1060, 717)])
def test_fast_decode_tracks_the_reference(ctx, name, cfg, n_steps, seed):
    """FAST mode step by step on the oracle's greedy tokens: every step's
    logits within FAST_TOL of the logit range of the oracle's, and the same
    argmax. The FAST attention splits the positions into blocks of 32, chunk
    c holding blocks c, c + 16, ...; the steps cross many block boundaries
    (and, in the long cases, the second and third rounds of blocks), so the
    chunk merge, empty chunks and the key/value appends of every chunk are
    exercised."""
    print(f"[gpu] fast decode {name}: building", flush=True)
    m, ref = build(ctx, cfg, seed)
    m.set_mode(wpcg.MODE_FAST)
    tok = int(np.random.default_rng(5).integers(0, cfg["vocab"]))
    worst = 0.0
    ties = 0
    for step in range(n_steps):
        r = ref.forward_token(tok)
        g, a = m.forward_token(tok)
        span = float(r.max() - r.min())
        err = float(np.max(np.abs(g - r))) / span
        worst = max(worst, err)
        assert err <= FAST_TOL, f"{name}: step {step} logits off by {err:.2e} of the range"
        tok = O.argmax(r)
        if a != tok:
            # only a near-tie may differ: the oracle's top two logits closer
            # than the two-sided tolerance band (the next step still takes
            # the oracle's token)
            top2 = np.sort(r)[-2:]
            assert float(top2[1] - top2[0]) <= 2 * FAST_TOL * span, \
                f"{name}: step {step} argmax {a} vs the oracle's {tok}"
            ties += 1
    print(f"[gpu] fast decode {name}: {n_steps} steps, worst logit error {worst:.2e} of the range, "
          f"{ties} near-tie argmax differences", flush=True)
    m.close()
    ref.close()


@pytest.mark.parametrize("factor,nan_rows,answers", [(2.0, (3,), (0, 70)), (0.5, (0, 3), (1, 70))])
def test_fast_argmax_ties_and_nan(ctx, factor, nan_rows, answers):
    """The FAST head leaves one argmax key per workgroup and the argmax
    reduces the keys; it must still return the first index of the largest
    logit and never a NaN one, as the reference's argmax (sampling.rs:3-14)
    scans. The tied embedding here holds one base row everywhere, that row
    with its zero points and scales times `factor` (every logit exactly
    scaled, in the oracle and on the GPU) at rows 70 and 900, in different
    workgroups of the head, and NaN scales at `nan_rows`. So the largest
    logit ties exactly, either between rows 70 and 900 or among every base
    row, and the answer is 70 or the first base row that is not NaN."""
    cfg = dict(DENSE)
    tensors = dict(synth.model_tensors(cfg, 4, 818, wpcg.encode))
    name = "model.embed_tokens.weight"
    emb = tensors[name].reshape(cfg["vocab"], -1, 68).copy()
    emb[:] = emb[1]
    params = emb[70, :, 0:4].copy().view(np.float16) * np.float16(factor)
    emb[70, :, 0:4] = emb[900, :, 0:4] = params.view(np.uint8)
    for r in nan_rows:
        emb[r, :, 2:4] = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)
    tensors[name] = emb.reshape(-1)
    m = wpcg.Model(ctx, 4, wpcg.ModelConfig(**cfg))
    for k, arr in tensors.items():
        m.set_tensor(k, arr)
    kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
    ref = O.Model(cfg, tensors, cfg["max_pos"], kern, 16)
    m.set_mode(wpcg.MODE_FAST)
    tok, seen = 2, set()
    for step in range(20):
        r = ref.forward_token(tok)
        g, a = m.forward_token(tok)
        assert all(np.isnan(r[i]) and np.isnan(g[i]) for i in nan_rows), step
        tok = O.argmax(r)
        assert tok in answers, f"step {step}: the oracle's argmax {tok}"
        assert a == tok, f"step {step}: FAST argmax {a} vs the oracle's {tok}"
        seen.add(tok)
    print(f"[gpu] argmax keys (x{factor}): 20 steps equal to the oracle's, answers {sorted(seen)}", flush=True)
    m.close()
    ref.close()


def test_decode_errors(ctx):
    cfg = dict(DENSE)
    m = wpcg.Model(ctx, 4, wpcg.ModelConfig(**cfg))
    with pytest.raises(wpcg.WpcgError) as e:  # nothing loaded yet
        m.forward_token(1)
    assert e.value.code == wpcg.E_ARG and "model.embed_tokens.weight" in wpcg.last_error()
    with pytest.raises(wpcg.WpcgError) as e:
        m.set_tensor("model.layers.9.self_attn.q_proj.weight", np.zeros(68, np.uint8))
    assert e.value.code == wpcg.E_NOTFOUND
    with pytest.raises(wpcg.WpcgError) as e:
        m.set_tensor("model.norm.weight", np.ones(3, np.float32))
    assert e.value.code == wpcg.E_SHAPE
    m.close()


@pytest.mark.parametrize("name,cfg,scheme,dtype,shards,seed,tie,lm_head", [
    ("dense-v4-bf16", DENSE, 4, "BF16", 1, 121, "auto", None),
    ("dense-v3-bf16-sharded", DENSE, 3, "BF16", 2, 131, "auto", None),
    ("moe-v4-f16-sharded", MOE, 4, "F16", 3, 222, "auto", None),
    ("dense-v4-untied-with-lm_head", DENSE, 4, "BF16", 1, 141, False, True),
    ("moe-v4-no-tie-key", MOE, 4, "F32", 1, 242, None, None),
    ("moe-v4-tie-true", MOE, 4, "BF16", 2, 252, True, None)])
def test_model_loads_from_checkpoint(ctx, tmp_path, name, cfg, scheme, dtype, shards, seed, tie, lm_head):
    """load_wpc_v{3,4} end to end: config.json, the norms and routers from
    safetensors (non-unit norms stored in `dtype`), the matrices from the
    artifact. v4: EXACT logits bit-identical to the oracle's decode step on
    the tensors as the checkpoint holds them. v3 (the oracle's decode step
    is v4 only): bit-identical to the same model given every tensor through
    set_tensor, i.e. the loader places every tensor where set_tensor does.
    The head is the reference's whatever config.json's tie_word_embeddings
    says: a dense checkpoint declaring itself untied and holding an
    lm_head.weight still decodes through the embedding table
    (qwen3_model.rs:187-206, model.rs:545), and a MoE config with the key
    absent (serde's default true) or true still uses lm_head.weight
    (qwen3_moe_model.rs:337-343); the oracle chooses the same way, pinned
    against transformers on the CPU."""
    print(f"[gpu] checkpoint load {name}", flush=True)
    tensors = synth.write_checkpoint(str(tmp_path / "model"), str(tmp_path / "wpc"), cfg, scheme, seed,
                                     wpcg.encode, dtype, shards, tie_word_embeddings=tie, lm_head=lm_head)
    if lm_head and not cfg["n_experts"]:
        assert "lm_head.weight" in tensors  # in the artifact, never read
    import json
    with open(tmp_path / "model" / "config.json") as f:
        declared = json.load(f).get("tie_word_embeddings")
    assert declared == (None if tie is None else (not cfg["n_experts"]) if tie == "auto" else tie)
    m = wpcg.Model.load_wpc(ctx, scheme, tmp_path / "model", tmp_path / "wpc", cfg["max_pos"])
    assert m.cfg.as_dict()["n_experts"] == cfg["n_experts"]
    if scheme == 4:
        kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
        ref = O.Model(cfg, tensors, cfg["max_pos"], kern, 16)
        step_ref = ref.forward_token
    else:
        ref = wpcg.Model(ctx, scheme, wpcg.ModelConfig(**cfg))
        for n, a in tensors.items():
            ref.set_tensor(n, a)
        step_ref = lambda t: ref.forward_token(t)[0]  # noqa: E731
    tok = 5
    for step in range(12):
        r = step_ref(tok)
        g, a = m.forward_token(tok)
        assert np.all(np.isfinite(r))
        assert np.array_equal(bits(g), bits(r)), f"{name}: logits differ at step {step}"
        tok = O.argmax(r)
        assert a == tok
    print(f"[gpu] checkpoint load {name}: 12 steps bit-identical", flush=True)
    m.close()
    ref.close()
