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
