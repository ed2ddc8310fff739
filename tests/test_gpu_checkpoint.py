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
