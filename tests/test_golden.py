"""The oracle against the golden fixtures (brute-force float64, tests/golden/make_fixtures.py)."""
import os

import numpy as np

from oracle import numpy_ref as ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def tiny_gpt():
    z = load("gpt_tiny.npz")
    cfg = {k[4:]: (z[k].item() if z[k].ndim == 0 else z[k]) for k in z.files if k.startswith("cfg_")}
    cfg["act"] = str(cfg["act"])
    params = {k[2:]: z[k] for k in z.files if k.startswith("p_")}
    return z, cfg, params


def test_oracle_gpt_tiny_matches_golden():
    z, cfg, params = tiny_gpt()
    probs, logits = ref.gpt_forward(z["ids"], params, cfg, return_logits=True)
    assert ref.max_rel(logits, z["logits"]) < 1e-5
    assert ref.max_rel(probs, z["probs"]) < 1e-5
    assert np.array_equal(ref.argmax(logits), np.argmax(z["logits"], -1))


def test_oracle_gpt_params_match_fixture_seeding():
    z, cfg, params = tiny_gpt()
    regen = ref.gpt_params(cfg, seed=7, scale=0.5)
    for k, v in params.items():
        assert np.array_equal(regen[k], v), k


def test_oracle_layernorm_matches_golden():
    z = load("layernorm_small.npz")
    assert ref.max_rel(ref.layernorm(z["x"], z["gamma"], z["beta"]), z["y"]) < 1e-6


def test_oracle_causal_softmax_matches_golden():
    z = load("softmax_causal_small.npz")
    s = z["scores"]
    T = s.shape[-1]
    p = ref.softmax(s + ref.causal_mask(T))
    assert ref.max_rel(p, z["probs"]) < 1e-6
    assert np.all(p[:, np.triu_indices(T, 1)[0], np.triu_indices(T, 1)[1]] == 0)


def tiny_vit():
    z = load("vit_tiny.npz")
    cfg = {k[4:]: z[k] for k in z.files if k.startswith("cfg_")}
    cfg = {k: (tuple(int(a) for a in v) if v.ndim else (str(v) if v.dtype.kind == "U" else int(v)))
           for k, v in cfg.items()}
    params = {k[2:]: z[k] for k in z.files if k.startswith("p_")}
    return z, cfg, params


def test_oracle_vit_tiny_matches_golden():
    """The oracle's ViT composition (patch order, projector, unmasked blocks, LayerNorm,
    VitMLPHead, SiLU, Dense, softmax) against brute-force float64 loops."""
    z, cfg, params = tiny_vit()
    probs, logits = ref.vit_forward(z["images"], params, cfg, return_logits=True)
    assert ref.max_rel(logits, z["logits"]) < 1e-5
    assert ref.max_rel(probs, z["probs"]) < 1e-5
    # the head output before SiLU, from the pinned pieces
    x = ref.vit_projector(z["images"], params["proj"], params["cls"], params["pos"], cfg["patch"])
    for l in range(cfg["layers"]):
        p = [params[f"b{l}.{k}"] for k in ("g1", "be1", "wqkv", "bqkv", "wo", "bo", "g2", "be2",
                                          "w1", "bb1", "w2", "bb2")]
        x = ref.block(x, p, cfg["heads"], cfg["act"], False, None)
    x = ref.layernorm(x, params["lnf.g"], params["lnf.be"])
    assert ref.max_rel(ref.vit_head(x, params["head.w"], params["head.b"]), z["head"]) < 1e-5


def test_oracle_vit_param_order_matches_fixture():
    z, cfg, params = tiny_vit()
    assert [n for n, _ in ref.vit_param_shapes(cfg)] == [str(n) for n in z["param_order"]]
    regen = ref.vit_params(cfg, seed=11, scale=0.5)
    for k, v in params.items():
        assert np.array_equal(regen[k], v), k


def tiny_gemma():
    z = load("gemma_tiny.npz")
    cfg = {k[4:]: z[k].item() for k in z.files if k.startswith("cfg_")}
    params = {k[2:]: z[k] for k in z.files if k.startswith("p_")}
    return z, cfg, params


def test_oracle_gemma_tiny_matches_golden():
    """The oracle's Gemma-style composition (sqrt(C)-scaled gather, (1 + gain) RMSNorms with
    eps 1e-6, 4 query heads on one key/value head with rotate-half RoPE on queries and keys
    at absolute positions, GeGLU, both residuals, final norm, tied head) against brute-force
    float64 loops written independently of it."""
    z, cfg, params = tiny_gemma()
    logits = ref.gemma_forward(z["ids"], params, cfg)
    assert ref.max_rel(logits, z["logits"]) < 1e-5
    assert np.array_equal(ref.argmax(logits), np.argmax(z["logits"], -1))


def test_oracle_gemma_tiny_cached_calls_match_golden():
    """Prefill 7 positions into the cache, then one token at position 7 and four at 8..11:
    each call's logits equal the fixture's rows at those absolute positions."""
    z, cfg, params = tiny_gemma()
    ids, cache = z["ids"], {}
    parts = [ref.gemma_forward(ids[:, :7], params, cfg, cache=cache),
             ref.gemma_forward(ids[:, 7:8], params, cfg, pos0=7, cache=cache),
             ref.gemma_forward(ids[:, 8:], params, cfg, pos0=8, cache=cache)]
    assert ref.max_rel(np.concatenate(parts, 1), z["logits"]) < 1e-5


def test_oracle_gemma_param_order_matches_fixture():
    z, cfg, params = tiny_gemma()
    assert [n for n, _ in ref.gemma_param_shapes(cfg)] == [str(n) for n in z["param_order"]]
    regen = ref.gemma_params(cfg, seed=13, scale=0.3)
    for k, v in params.items():
        assert np.array_equal(regen[k], v), k


def _gemma_variant(ids, P, cfg, drop_attn_residual=False, drop_ffn_residual=False,
                   gain_offset=1.0, embed_scale=True):
    """The decoder composed from the oracle's pinned pieces, with switches that plant one
    plausible composition mistake each (CPU only; with no switch set it must equal
    ref.gemma_forward)."""
    C = cfg["d"]
    x = P["table"][ids] * (np.sqrt(np.float32(C)) if embed_scale else np.float32(1))
    for l in range(cfg["layers"]):
        h, _, _ = ref.mqa(ref.rmsnorm(x, P[f"b{l}.g1"], np.float32(1e-6), gain_offset),
                          P[f"b{l}.wqkv"], P[f"b{l}.wo"], cfg["heads"], cfg["kv_heads"],
                          cfg["head_dim"], 0, cfg["rope_base"])
        y = h if drop_attn_residual else x + h
        f = ref.geglu_ffn(ref.rmsnorm(y, P[f"b{l}.g2"], np.float32(1e-6), gain_offset),
                          P[f"b{l}.wg"], P[f"b{l}.wu"], P[f"b{l}.wd"])
        x = f if drop_ffn_residual else y + f
    x = ref.rmsnorm(x, P["normf.g"], np.float32(1e-6), gain_offset)
    return ref.embed_back(x, P["table"])


def test_gemma_fixture_catches_planted_composition_mistakes(monkeypatch):
    """Each mistake planted on the CPU moves the logits far past the 1e-5 bar against the
    fixture: a dropped attention or FFN residual, a gain used without its 1 + offset, the
    sqrt(C) embedding scale left out, RoPE on the queries only, and a cached call whose
    rotation restarts at position 0 instead of its absolute position."""
    z, cfg, params = tiny_gemma()
    ids = z["ids"]
    assert ref.max_rel(_gemma_variant(ids, params, cfg), ref.gemma_forward(ids, params, cfg)) == 0
    for kw in (dict(drop_attn_residual=True), dict(drop_ffn_residual=True),
               dict(gain_offset=0.0), dict(embed_scale=False)):
        assert ref.max_rel(_gemma_variant(ids, params, cfg, **kw), z["logits"]) > 1e-2, kw
    orig_rope, orig_table = ref.rope, ref.rope_table
    calls = []

    def rope_queries_only(a, cos, sin):  # mqa rotates q, then k
        calls.append(1)
        return orig_rope(a, cos, sin) if len(calls) % 2 == 1 else np.asarray(a, np.float32)
    with monkeypatch.context() as m:
        m.setattr(ref, "rope", rope_queries_only)
        bad = ref.gemma_forward(ids, params, cfg)
    assert len(calls) == 2 * cfg["layers"]
    assert ref.max_rel(bad, z["logits"]) > 1e-2
    cache = {}
    ref.gemma_forward(ids[:, :7], params, cfg, cache=cache)
    with monkeypatch.context() as m:
        m.setattr(ref, "rope_table", lambda T, D, base=10000.0, pos0=0: orig_table(T, D, base, 0))
        bad = ref.gemma_forward(ids[:, 7:], params, cfg, pos0=7, cache=cache)
    assert ref.max_rel(bad, z["logits"][:, 7:]) > 1e-2


def test_oracle_mqa_invariant_to_a_common_position_shift(monkeypatch):
    """RoPE makes q_m . k_n depend on m - n only, so an uncached call whose every position
    (queries and keys alike) is shifted by the same offset gives the same output. RoPE on
    the queries only, or on the values, would not."""
    rng = np.random.default_rng(37)
    B, T, C, Hq, D = 2, 9, 32, 4, 16
    x = rng.standard_normal((B, T, C)).astype(np.float32)
    w = rng.standard_normal((C, (Hq + 2) * D)).astype(np.float32) * np.float32(0.4)
    wo = rng.standard_normal((Hq * D, C)).astype(np.float32) * np.float32(0.4)
    base, _, _ = ref.mqa(x, w, wo, Hq, 1, D)
    orig_table = ref.rope_table
    for shift in (1, 37, 1000):
        with monkeypatch.context() as m:
            m.setattr(ref, "rope_table", lambda T_, D_, b=10000.0, pos0=0, s=shift:
                      orig_table(T_, D_, b, pos0 + s))
            moved, _, _ = ref.mqa(x, w, wo, Hq, 1, D)
        assert ref.max_rel(moved, base) < 1e-5, shift
    # planted on the CPU: RoPE on the queries only is not shift invariant
    orig_rope = ref.rope
    calls = []

    def q_only(a, cos, sin):
        calls.append(1)
        return orig_rope(a, cos, sin) if len(calls) % 2 == 1 else np.asarray(a, np.float32)
    with monkeypatch.context() as m:
        m.setattr(ref, "rope", q_only)
        a0, _, _ = ref.mqa(x, w, wo, Hq, 1, D)
        m.setattr(ref, "rope_table", lambda T_, D_, b=10000.0, pos0=0:
                  orig_table(T_, D_, b, pos0 + 37))
        a1, _, _ = ref.mqa(x, w, wo, Hq, 1, D)
    assert ref.max_rel(a1, a0) > 1e-3
