"""GPU tests of the batched prefill (wpcg_model_prefill) against the same
model run token by token (forward_token; the reference's prompt loop,
wpc-runtime/src/main.rs:259-262), on seeded synthetic v4 models.

The reference has no batched forward pass, so its semantics are those n
steps. EXACT mode runs exactly them: bit-identical. FAST mode batches the
tokens (matrix-core GEMMs with X carried as two bf16 terms, causal attention
over the cache, experts grouped by the pairs routed to them), so it is held
to a tolerance against the oracle's steps (the CPU restatement of
forward_token) and against the step-by-step FAST run:
  * logits of the last token within TOL of the oracle's logit range;
  * every key and value written to the cache within TOL of the cache's
    largest magnitude (against the FAST steps: the oracle's cache is internal);
  * greedy decoding continued from the prefilled state gives the oracle's ids,
    every one of 24.
Speculative verification is held to the same bars against the oracle's
steps. Cases cover one pass, several passes (more tokens than a pass holds),
a prefill after decode steps (a non-zero start position), dense and MoE.
"""
import numpy as np
import pytest

import oracle as O
import wpcg
from wpcg import synth

pytestmark = pytest.mark.gpu

DENSE = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=512, vocab=1000,
             n_experts=0, top_k=0, moe_inter=0, norm_topk=1, tied=1, max_pos=352, eps=1e-6,
             rope_theta=1e6)
MOE = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=0, vocab=1000,
           n_experts=16, top_k=4, moe_inter=128, norm_topk=1, tied=0, max_pos=352, eps=1e-6,
           rope_theta=1e6)
# Qwen3-30B-A3B shapes (config 3) with two of the 48 layers
QWEN3_MOE_2L = dict(n_layers=2, hidden=2048, n_heads=32, n_kv_heads=4, head_dim=128, inter=0,
                    vocab=151936, n_experts=128, top_k=8, moe_inter=768, norm_topk=1, tied=0,
                    max_pos=320, eps=1e-6, rope_theta=1e6)
# Qwen3-4B shapes (config 2) with two of the 36 layers: 128-wide heads (the
# attention writes o_proj's packed input), o_proj and down in K-slices
QWEN3_DENSE_2L = dict(n_layers=2, hidden=2560, n_heads=32, n_kv_heads=8, head_dim=128, inter=9728,
                      vocab=151936, n_experts=0, top_k=0, moe_inter=0, norm_topk=1, tied=1,
                      max_pos=192, eps=1e-6, rope_theta=1e6)
# measured: 3e-6 of the logit range, 9e-6 of the cache magnitude
TOL = 5e-5


@pytest.fixture(scope="module")
def ctx():
    c = wpcg.Context(0)
    yield c
    c.close()


def build(ctx, cfg, seed, mode, with_oracle=False):
    tensors = dict(synth.model_tensors(cfg, 4, seed, wpcg.encode))
    m = wpcg.Model(ctx, 4, wpcg.ModelConfig(**cfg))
    for name, arr in tensors.items():
        m.set_tensor(name, arr)
    m.set_mode(mode)
    if not with_oracle:
        return m
    kern = O.KERNEL_AVX2 if O.have_avx2() else O.KERNEL_FUSED
    return m, O.Model(cfg, tensors, cfg["max_pos"], kern, 16)


def oracle_run(ref, toks, n_greedy):
    """The oracle's steps over toks, then n_greedy greedy steps: (logits
    after the last of toks, its argmax, the greedy ids, each greedy step's
    logits)."""
    for t in toks:
        last = ref.forward_token(int(t))
    first = O.argmax(last)
    ids, lgs, tok = [], [], first
    for _ in range(n_greedy):
        lg = ref.forward_token(tok)
        tok = O.argmax(lg)
        ids.append(tok)
        lgs.append(lg)
    return last, first, ids, lgs


def cache(m, cfg, n):
    """Keys and values of positions < n, [layer][kv_head][n][head_dim]."""
    L, kv, mp, hd = cfg["n_layers"], cfg["n_kv_heads"], cfg["max_pos"], cfg["head_dim"]
    size = L * kv * mp * hd
    k = m.debug_read(9, size).reshape(L, kv, mp, hd)[:, :, :n]
    v = m.debug_read(10, size).reshape(L, kv, mp, hd)[:, :, :n]
    return k, v


def greedy(m, first, steps):
    ids, tok = [], first
    for _ in range(steps):
        _, tok = m.forward_token(tok, want_logits=False)
        ids.append(tok)
    return ids


@pytest.mark.parametrize("name,cfg,n_pre,n,seed", [
    ("dense-one-pass", DENSE, 0, 100, 11),
    ("dense-two-passes", DENSE, 0, 300, 12),
    ("dense-after-steps", DENSE, 7, 90, 13),
    ("moe-one-pass", MOE, 0, 200, 21),
    ("moe-two-passes", MOE, 3, 290, 22),
    ("qwen3-moe-2L", QWEN3_MOE_2L, 0, 256, 31),
    ("qwen3-dense-2L", QWEN3_DENSE_2L, 5, 128, 32),
    # a ragged batch at a non-zero start: the q/k/v epilogue's partial
    # column group and rotation offsets, the expert GEMM's small items
    ("qwen3-moe-2L-ragged", QWEN3_MOE_2L, 3, 77, 34),
])
def test_fast_prefill_matches_steps(ctx, name, cfg, n_pre, n, seed):
    print(f"[gpu] prefill {name}: {n_pre} steps then {n} tokens", flush=True)
    m, ref = build(ctx, cfg, seed, wpcg.MODE_FAST, with_oracle=True)
    rng = np.random.default_rng(seed)
    toks = rng.integers(0, cfg["vocab"], n_pre + n).astype(np.uint32)
    o_last, o_id, o_ids, _ = oracle_run(ref, toks, 24)
    ref.close()
    # token by token (FAST steps): the cache to compare with
    for t in toks:
        m.forward_token(int(t), want_logits=False)
    kr, vr = cache(m, cfg, n_pre + n)
    # the same tokens, the last n batched
    m.reset()
    for t in toks[:n_pre]:
        m.forward_token(int(t), want_logits=False)
    got, got_id = m.prefill(toks[n_pre:])
    assert m.position() == n_pre + n
    kg, vg = cache(m, cfg, n_pre + n)
    ids = greedy(m, got_id, 24)
    span = float(o_last.max() - o_last.min())
    err = float(np.max(np.abs(got - o_last))) / span
    kerr = max(float(np.max(np.abs(kg - kr))) / float(np.max(np.abs(kr))),
               float(np.max(np.abs(vg - vr))) / float(np.max(np.abs(vr))))
    same = int(np.argmax(np.concatenate([np.array(ids) != np.array(o_ids), [True]])))
    print(f"[gpu] prefill {name}: logits {err:.2e} of the oracle's range, cache {kerr:.2e} of FAST "
          f"steps', argmax {got_id} vs {o_id}, greedy ids equal the oracle's for {same} of 24", flush=True)
    assert err <= TOL, f"{name}: last logits {err:.2e} of the range"
    assert kerr <= TOL, f"{name}: cache {kerr:.2e}"
    assert got_id == o_id
    assert ids == o_ids, f"{name}: greedy continuation parts from the oracle at step {same}"
    m.close()


@pytest.mark.parametrize("name,cfg,n,seed", [("moe-v3", MOE, 200, 24),
                                             ("qwen3-moe-2L-v3", QWEN3_MOE_2L, 256, 33)])
def test_fast_prefill_v3_matches_steps(ctx, name, cfg, n, seed):
    """v3 weights (6-bit codes; the grouped expert GEMM's second code plane):
    the reference's model loaders read v4 only, so the oracle has no v3
    model; the batched prefill is held to the FAST steps of the same model
    instead: last logits within TOL of their range, every cached key and
    value within TOL of the cache's largest magnitude, the same argmax."""
    print(f"[gpu] prefill {name}: {n} tokens", flush=True)
    tensors = dict(synth.model_tensors(cfg, 3, seed, wpcg.encode))
    m = wpcg.Model(ctx, 3, wpcg.ModelConfig(**cfg))
    for nm, arr in tensors.items():
        m.set_tensor(nm, arr)
    m.set_mode(wpcg.MODE_FAST)
    toks = np.random.default_rng(seed).integers(0, cfg["vocab"], n).astype(np.uint32)
    for t in toks:
        ref, ref_id = m.forward_token(int(t))
    kr, vr = cache(m, cfg, n)
    m.reset()
    got, got_id = m.prefill(toks)
    kg, vg = cache(m, cfg, n)
    span = float(ref.max() - ref.min())
    err = float(np.max(np.abs(got - ref))) / span
    kerr = max(float(np.max(np.abs(kg - kr))) / float(np.max(np.abs(kr))),
               float(np.max(np.abs(vg - vr))) / float(np.max(np.abs(vr))))
    print(f"[gpu] prefill {name}: logits {err:.2e} of the steps' range, cache {kerr:.2e}, argmax {got_id} vs "
          f"{ref_id}", flush=True)
    assert err <= TOL and kerr <= TOL and got_id == ref_id
    m.close()


def test_exact_prefill_is_the_steps(ctx):
    cfg = MOE
    m = build(ctx, cfg, 41, wpcg.MODE_EXACT)
    toks = np.random.default_rng(4).integers(0, cfg["vocab"], 20).astype(np.uint32)
    for t in toks:
        ref, ref_id = m.forward_token(int(t))
    kr, vr = cache(m, cfg, 20)
    m.reset()
    got, got_id = m.prefill(toks)
    kg, vg = cache(m, cfg, 20)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)) and got_id == ref_id
    assert np.array_equal(kg, kr) and np.array_equal(vg, vr)
    m.close()


@pytest.mark.parametrize("name,cfg,seed", [("dense", DENSE, 51), ("moe", MOE, 52)])
def test_generate_with_prefill(ctx, name, cfg, seed):
    """FAST generate, batched prompt and step-by-step prompt: the oracle's
    32 greedy ids, every one."""
    m, ref = build(ctx, cfg, seed, wpcg.MODE_FAST, with_oracle=True)
    prompt = np.random.default_rng(seed).integers(0, cfg["vocab"], 64).astype(np.uint32)
    _, o_first, o_ids, _ = oracle_run(ref, prompt, 31)
    ref.close()
    want = [o_first] + o_ids
    a, _ = m.generate(prompt, 32)
    m.set_prefill(False)
    b, _ = m.generate(prompt, 32)
    for what, got in (("batched", a), ("stepwise", b)):
        same = int(np.argmax(np.concatenate([np.array(got) != np.array(want), [True]])))
        print(f"[gpu] generate {name} ({what} prompt): ids equal the oracle's for {same} of 32", flush=True)
        assert list(got) == want, f"{name}: {what} prompt parts from the oracle at step {same}"
    m.close()


def test_prefill_errors(ctx):
    cfg = dict(DENSE, max_pos=40)
    m = build(ctx, cfg, 61, wpcg.MODE_FAST)
    with pytest.raises(wpcg.WpcgError) as e:
        m.prefill(np.zeros(41, np.uint32))
    assert e.value.code == wpcg.E_ARG
    with pytest.raises(wpcg.WpcgError) as e:
        m.prefill(np.array([5, cfg["vocab"]], np.uint32))
    assert e.value.code == wpcg.E_ARG
    m.prefill(np.arange(30, dtype=np.uint32))
    with pytest.raises(wpcg.WpcgError):  # 30 + 11 > 40
        m.prefill(np.arange(11, dtype=np.uint32))
    m.prefill(np.arange(10, dtype=np.uint32))  # exactly full
    assert m.position() == 40
    m.close()


@pytest.mark.parametrize("name,cfg,mode,seed", [("moe-fast", MOE, wpcg.MODE_FAST, 71),
                                                ("qwen3-moe-2L-fast", QWEN3_MOE_2L, wpcg.MODE_FAST, 72),
                                                ("dense-exact", DENSE, wpcg.MODE_EXACT, 73)])
def test_speculative_verify(ctx, name, cfg, mode, seed):
    """verify([a0, g1 .. g7]) against the greedy steps a0 -> g1 -> ... -> g8:
    argmax[i] == g[i+1]; a wrong draft changes only what follows it; a
    rewind to an accepted prefix continues exactly as the steps did."""
    print(f"[gpu] verify {name}", flush=True)
    m, ref = build(ctx, cfg, seed, mode, with_oracle=True)
    prompt = np.random.default_rng(seed).integers(0, cfg["vocab"], 40).astype(np.uint32)
    # the oracle's steps: a0 after the prompt, then g1..g8 greedily
    _, o_a0, o_g, o_lg = oracle_run(ref, prompt, 8)
    ref.close()
    _, a0 = m.prefill(prompt)
    assert a0 == o_a0
    n = len(prompt)
    g, step_logits, tok = [], [], a0
    for _ in range(8):
        lg, tok = m.forward_token(tok)
        g.append(tok)
        step_logits.append(lg)
    assert g == o_g, f"{name}: the GPU's steps {g} vs the oracle's {o_g}"
    m.set_position(n)
    drafts = np.array([a0] + g[:7], np.uint32)
    ids, lg = m.verify(drafts, want_logits=True)
    assert m.position() == n + 8
    assert list(ids) == g, f"{name}: {list(ids)} vs {g}"
    span = float(np.max(o_lg) - np.min(o_lg))
    err = float(np.max(np.abs(lg - np.array(o_lg)))) / span
    print(f"[gpu] verify {name}: 8 argmaxes equal the oracle's steps, logits {err:.2e} of range", flush=True)
    if mode == wpcg.MODE_EXACT:
        assert np.array_equal(lg.view(np.uint32), np.array(o_lg).view(np.uint32))
    else:
        assert err <= TOL
    # a wrong third draft: the first two verdicts stand
    m.set_position(n)
    bad = drafts.copy()
    bad[2] = (int(g[1]) + 1) % cfg["vocab"]
    ids2, _ = m.verify(bad)
    assert list(ids2[:2]) == g[:2]
    # keep positions n (a0) and n + 1 (g[0]), drop the rest: position n + 2
    # takes g[1] again, after which the greedy token is g[2]
    m.set_position(n + 2)
    _, nxt = m.forward_token(int(g[1]))
    assert nxt == g[2]
    with pytest.raises(wpcg.WpcgError):
        m.set_position(n + 10)  # only backwards
    m.close()
