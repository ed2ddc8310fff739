"""ViT front end and classifier on the MI355X against the NumPy oracle: the patch gather,
VitProjector (projection, class/register rows, positions), encoder attention at a token
count that is not a multiple of 8, a tiny notebook-style ViT end to end (fp32, 1e-5), and
BASELINE config 4 at full size (bf16, 2e-2 on sampled images, class ids bit-exact against
np.argmax of the downloaded probabilities)."""
import numpy as np
import pytest

from oracle import numpy_ref as ref

pytestmark = pytest.mark.gpu
F32 = np.float32


@pytest.fixture(scope="module")
def tl():
    import tl_hip
    tl_hip.ctx()
    import backend
    import layers
    import transformer_adapters
    import vit
    return dict(xp=tl_hip, backend=backend, layers=layers, ta=transformer_adapters, vit=vit)


@pytest.mark.parametrize("dts", [("fp32", "fp32"), ("fp32", "bf16"), ("bf16", "bf16"), ("bf16", "fp32")])
@pytest.mark.parametrize("shape", [(2, 3, 32, 32, 4, 4), (3, 3, 32, 32, 2, 2), (1, 1, 6, 4, 3, 2),
                                   (5, 4, 8, 12, 4, 3)])
def test_patchify_matches_reference_order(tl, dts, shape):
    xp = tl["xp"]
    B, C, H, W, p0, p1 = shape
    x = np.random.default_rng(B * H + p1).standard_normal((B, C, H, W)).astype(F32)
    if dts[0] == "bf16":
        x = ref.round_bf16(x)
    got = xp.patchify(xp.array(x, dtype=dts[0]), (p0, p1), dtype=dts[1]).get()
    want = ref.patchify(x, (p0, p1))
    if dts[1] == "bf16":
        want = ref.round_bf16(want)
    assert np.array_equal(got, want)


def test_patchify_rejects_partial_patches(tl):
    xp = tl["xp"]
    with pytest.raises(ValueError):
        xp.patchify(xp.zeros((1, 3, 10, 8)), (4, 4))
    lib, h = xp.lib(), xp.ctx().handle
    x, y = xp.zeros((1, 3, 10, 8)), xp.zeros((1, 240))
    assert lib.tl_patchify(h, x.ptr, y.ptr, 1, 3, 10, 8, 4, 4, 0, 0) == 1  # TL_ERR_INVALID


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("registers", [0, 4])
def test_vit_projector_layer(tl, dt, registers):
    tl["backend"].set_float_type(dt)
    layer = tl["ta"].VitProjector((3, 32, 32), (4, 4), 384, num_registers=registers)
    rng = np.random.default_rng(registers + 1)
    P = []
    for p in layer.parameters:
        a = rng.standard_normal(p.shape).astype(F32) * F32(0.5)
        a = ref.round_bf16(a) if dt == "bf16" else a
        p.set(a)
        P.append(a)
    x = rng.standard_normal((6, 3, 32, 32)).astype(F32)
    if dt == "bf16":
        x = ref.round_bf16(x)
    y = layer.forward(tl["xp"].array(x, dtype=dt)).get()
    want = ref.vit_projector(x, *P, (4, 4))
    assert y.shape == (6, 1 + registers + 64, 384)
    assert ref.max_rel(y, want) <= (1e-5 if dt == "fp32" else 2e-2)
    # host arrays are accepted like the reference's xp arrays
    y2 = layer.forward(x).get()
    assert ref.max_rel(y2, want) <= (1e-5 if dt == "fp32" else 2e-2)


@pytest.mark.parametrize("cfg", [((3, 32, 32), (4, 4), 384, 0, 7), ((3, 32, 32), (4, 4), 384, 1, 3),
                                 ((3, 32, 32), (4, 4), 384, 4, 2), ((1, 16, 16), (4, 4), 96, 2, 5),
                                 ((3, 16, 8), (4, 2), 192, 1, 3), ((2, 32, 32), (4, 4), 288, 1, 2),
                                 ((2, 16, 16), (2, 4), 480, 1, 3)])
def test_vit_projector_fused_equals_three_launches(tl, cfg):
    """tl_vit_project (one launch per forward) against the patch gather + batched GEMM +
    class-row gather composition, bit for bit: K = 16 .. 48 features, 16 / 32 / 64 patches,
    dim 96 .. 480 (one to five 96-column groups, so a wave may take two), 0 .. 4
    class/register rows."""
    xp = tl["xp"]
    tl["backend"].set_float_type("bf16")
    (C, H, W), patch, E, regs, B = cfg
    layer = tl["ta"].VitProjector((C, H, W), patch, E, num_registers=regs)
    rng = np.random.default_rng(E + regs + B)
    for p in layer.parameters:
        p.set(ref.round_bf16(rng.standard_normal(p.shape).astype(F32)))
    x = xp.array(ref.round_bf16(rng.standard_normal((B, C, H, W)).astype(F32)), dtype="bf16")
    assert xp.vit_project_ok(x, patch, E, 1 + regs)
    layer.fused = True
    got = layer.forward(x).get().view(np.uint16).copy()
    layer.fused = False
    want = layer.forward(x).get().view(np.uint16)
    assert np.array_equal(got, want), cfg


def test_vit_project_unsupported_shape_falls_back(tl):
    """Patches of more than 64 features are outside tl_vit_project (TL_ERR_UNSUPPORTED at
    the C ABI); the projector then composes the three launches and still matches the
    oracle."""
    xp = tl["xp"]
    tl["backend"].set_float_type("bf16")
    layer = tl["ta"].VitProjector((3, 32, 32), (8, 8), 192)  # K = 192
    rng = np.random.default_rng(11)
    P = []
    for p in layer.parameters:
        a = ref.round_bf16(rng.standard_normal(p.shape).astype(F32) * F32(0.5))
        p.set(a)
        P.append(a)
    x = ref.round_bf16(rng.standard_normal((2, 3, 32, 32)).astype(F32))
    dx = xp.array(x, dtype="bf16")
    assert not xp.vit_project_ok(dx, (8, 8), 192, 1)
    out = xp.empty((2, 17, 192), "bf16")
    pos = layer.positional_embeddings
    w = xp.empty((192, 192), "bf16")
    rc = xp.lib().tl_vit_project(xp.ctx().handle, dx.ptr, w.ptr, layer.cls_reg_tokens.ptr, pos.ptr,
                                 out.ptr, 2, 3, 32, 32, 8, 8, 192, 1, 1)
    assert rc == xp.TL_ERR_UNSUPPORTED
    y = layer.forward(dx).get()
    assert ref.max_rel(y, ref.vit_projector(x, *P, (8, 8))) <= 2e-2


def test_vit_projector_rejects_wrong_image_shape(tl):
    tl["backend"].set_float_type("fp32")
    layer = tl["ta"].VitProjector((3, 32, 32), (4, 4), 64)
    with pytest.raises(ValueError):
        layer.forward(np.zeros((2, 3, 28, 28), F32))


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_encoder_attention_at_65_tokens(tl, dt):
    """Config 4's token count (64 patches + CLS) is not a multiple of 8: the fused kernel
    runs with padded key capacity; the padding is never read as values."""
    B, T, C, H = 4, 65, 384, 6
    tl["backend"].set_float_type(dt)
    mha = tl["layers"].MultiHeadAttention(C, 0, H, decoder=False)
    rng = np.random.default_rng(65)
    P = [rng.standard_normal(p.shape).astype(F32) * F32(0.1) for p in mha.parameters]
    P = [ref.round_bf16(p) if dt == "bf16" else p for p in P]
    for p, a in zip(mha.parameters, P):
        p.set(a)
    x = rng.standard_normal((B, T, C)).astype(F32)
    if dt == "bf16":
        x = ref.round_bf16(x)
    y = mha.forward(tl["xp"].array(x, dtype=dt)).get()
    want = ref.mha(x, *P, H, False, None, rnd=ref.round_bf16 if dt == "bf16" else None)
    assert ref.max_rel(y, want) <= (1e-5 if dt == "fp32" else 2e-2)
    if dt == "bf16":
        assert mha.softmax is None  # the fused kernel ran


def test_tiny_notebook_vit_fp32(tl):
    """The notebook composition (registers, SiLU hidden head, Dropout in eval) at a small
    size, end to end against the oracle."""
    cfg = dict(image=(3, 16, 16), patch=(2, 2), d=32, heads=4, layers=2, act="silu",
               registers=4, classes=10, head_hidden=16, dropout=0.1)
    net = tl["vit"].build_vit(cfg, "fp32")
    tl["vit"].seed_vit(net, 3, 0.2)
    x = np.random.default_rng(4).standard_normal((5, 3, 16, 16)).astype(F32)
    probs = net.predict(x)
    want = ref.vit_forward(x, ref.vit_params(cfg, 3, 0.2), cfg)
    got = probs.get()
    assert ref.max_rel(got, want) <= 1e-5
    assert np.array_equal(tl["xp"].argmax(probs).get(), np.argmax(got, -1))


def test_vit_golden_fixture_fp32(tl):
    """The notebook ViT composition against tests/golden/vit_tiny.npz (brute-force float64
    loops, independent of the oracle): non-square patches of a non-square image, a register
    token, SiLU blocks, a hidden SiLU head. Head output, class scores and probabilities."""
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vit_tiny.npz"))
    cfg = {k[4:]: z[k] for k in z.files if k.startswith("cfg_")}
    cfg = {k: (tuple(int(a) for a in v) if v.ndim else (str(v) if v.dtype.kind == "U" else int(v)))
           for k, v in cfg.items()}
    net = tl["vit"].build_vit(cfg, "fp32")
    params = [p for layer in net.layers for p in layer.parameters]
    names = [str(n) for n in z["param_order"]]
    assert len(params) == len(names)
    for p, n in zip(params, names):
        p.set(z["p_" + n])
    probs = net.predict(z["images"])
    head = net.layers[-5].output.get()   # VitMLPHead
    logits = net.layers[-2].output.get()  # Dense
    assert ref.max_rel(head, z["head"]) <= 1e-5
    assert ref.max_rel(logits, z["logits"]) <= 1e-5
    assert ref.max_rel(probs.get(), z["probs"]) <= 1e-5
    assert np.array_equal(tl["xp"].argmax(probs).get(), np.argmax(z["probs"], -1))


def _cifar_like(rng, n):
    """Pixels uniform in [0, 1], normalised per channel as (x - 0.5) / sqrt(1/12)."""
    x = rng.random((n, 3, 32, 32), dtype=F32)
    return ((x - F32(0.5)) / F32(np.sqrt(1.0 / 12.0))).astype(F32)


def test_vit_config4_full_shape_bf16(tl):
    """BASELINE config 4 at its full size (B=512, 65 tokens, d 384, 6 heads, 8 layers,
    10 classes, bf16): rows are probability vectors, images are independent of the rest of
    the batch, and sampled images (first, middle and last) match the oracle on the head's
    class scores (before the softmax, which would compress their error) and on the
    probabilities."""
    cfg = tl["vit"].VIT_S4
    net = tl["vit"].build_vit(cfg, "bf16")
    tl["vit"].seed_vit(net, 5, 0.02)
    x = ref.round_bf16(_cifar_like(np.random.default_rng(6), 512))
    xp = tl["xp"]
    probs_dev = net.predict(xp.array(x, dtype="bf16"))
    probs = probs_dev.get()
    scores = net.layers[-2].output.get()  # VitMLPHead output, [512, 10]
    assert probs.shape == (512, 10) and scores.shape == (512, 10)
    assert np.array_equal(xp.argmax(probs_dev).get(), np.argmax(probs, -1))
    np.testing.assert_allclose(probs.astype(np.float64).sum(-1), 1.0, rtol=2e-2)
    P = ref.vit_params(cfg, 5, 0.02, bf16=True)
    idx = [0, 1, 255, 510, 511]
    want_p, want_s = ref.vit_forward(x[idx], P, cfg, bf16=True, return_logits=True)
    assert ref.max_rel(scores[idx], want_s) <= 2e-2
    assert ref.max_rel(probs[idx], want_p) <= 2e-2
    sub = net.predict(xp.array(x[idx], dtype="bf16")).get()
    assert ref.max_rel(sub, probs[idx]) <= 1e-2  # other tile shapes at 5 images
    assert ref.max_rel(net.layers[-2].output.get(), scores[idx]) <= 2e-2
