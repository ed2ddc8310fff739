"""Weight files on the device: a GPT saved and loaded into a differently seeded model of the
same shape gives bit-identical parameters (bf16 bits included) and predictions."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_gpt_save_load_round_trip(tmp_path, dt):
    import tl_hip
    import checkpoint
    import gpt
    tl_hip.ctx()
    cfg = dict(vocab=65, ctx=32, layers=2, d=64, heads=4, act="gelu")
    ids = np.random.default_rng(0).integers(0, cfg["vocab"], (2, 32))
    a, _ = gpt.build_gpt(cfg, dtype=dt)
    gpt.seed_parameters(a, 0)
    want = a.predict(ids).get()
    path = str(tmp_path / "gpt.npz")
    checkpoint.save_weights(a, path)
    b, _ = gpt.build_gpt(cfg, dtype=dt)
    gpt.seed_parameters(b, 1)
    assert not np.array_equal(b.predict(ids).get(), want)
    checkpoint.load_weights(b, path)
    for la, lb in zip(a.layers, b.layers):
        for pa, pb in zip(getattr(la, "parameters", []), getattr(lb, "parameters", [])):
            assert np.array_equal(pa.get_raw(), pb.get_raw())
    assert np.array_equal(b.predict(ids).get(), want)


def _notebook_gpt_records(P, cfg):
    """The notebook GPT's layer list (reference demo.ipynb:1473-1501: GPTEmbedFront, Dropout,
    L TransformerBlocks, LayerNorm, GPTEmbedBack, SoftMax) with each layer's parameters in
    its `parameters` order (GPTEmbedFront [pos, table], transformer_adapters.py:138, 143;
    TransformerBlock layers.py:458 with 275-279, 362-366), filled from oracle parameters."""
    recs = [("GPTEmbedFront", [P["pos"], P["table"]]), ("Dropout", [])]
    for l in range(cfg["layers"]):
        recs.append(("TransformerBlock", [P[f"b{l}.{k}"] for k in (
            "g1", "be1", "wqkv", "bqkv", "wo", "bo", "g2", "be2", "w1", "bb1", "w2", "bb2")]))
    recs += [("LayerNorm", [P["lnf.g"], P["lnf.be"]]), ("GPTEmbedBack", []), ("SoftMax", [])]
    return recs


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("fmt", ["npz", "notebook-pickle"])
def test_gpt_loaded_from_oracle_parameters_matches_oracle(tmp_path, dt, fmt):
    """A weight file written on the host from the oracle's parameters (not from a device
    model) in the notebook's per-layer order, loaded into a freshly built, differently seeded
    device GPT: logits and probabilities match the oracle's forward on those parameters."""
    import json
    import pickle
    import tl_hip
    import checkpoint
    import gpt
    from oracle import numpy_ref as ref
    tl_hip.ctx()
    cfg = dict(vocab=97, ctx=64, layers=3, d=64, heads=4, act="gelu")
    P = ref.gpt_params(cfg, 17, scale=0.1)
    recs = _notebook_gpt_records(P, cfg)
    path = str(tmp_path / ("w.npz" if fmt == "npz" else "w.pkl"))
    if fmt == "npz":
        arrays = {f"L{i:04d}.P{j:02d}": a for i, (_, ps) in enumerate(recs) for j, a in enumerate(ps)}
        meta = {"format": checkpoint.FORMAT,
                "layers": [{"name": n, "shapes": [list(a.shape) for a in ps]} for n, ps in recs]}
        arrays["__layout__"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
        np.savez(path, **arrays)
    else:
        with open(path, "wb") as f:
            pickle.dump([{"name": n, "parameters": ps} for n, ps in recs], f)
    net, _ = gpt.build_gpt(cfg, dtype=dt)
    gpt.seed_parameters(net, 3)
    (checkpoint.load_weights if fmt == "npz" else checkpoint.load_notebook_weights)(net, path)
    ids = np.random.default_rng(18).integers(0, cfg["vocab"], (2, 50))
    probs = net.predict(ids).get()
    logits = net.layers[-2].output.get()
    bf16 = dt == "bf16"
    Pw = {k: ref.round_bf16(v) for k, v in P.items()} if bf16 else P
    want_p, want_l = ref.gpt_forward(ids, Pw, cfg, bf16=bf16, return_logits=True)
    tol = 2e-2 if bf16 else 1e-5
    assert ref.max_rel(logits, want_l) <= tol
    assert ref.max_rel(probs, want_p) <= tol
