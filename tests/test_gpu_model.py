"""Model-level parity on the MI355X: the Layer interface (layers.py, transformer_adapters.py,
network.py) on XP_RUNTIME=MI355X against the NumPy oracle on identical seeded weights and
token ids. fp32: max_rel <= 1e-5; bf16: max_rel <= 2e-2 on logits; argmax ids bit-exact
against np.argmax of the downloaded logits."""
import os

import numpy as np
import pytest

from oracle import numpy_ref as ref

pytestmark = pytest.mark.gpu
F32 = np.float32
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def tl():
    import tl_hip
    tl_hip.ctx()
    import backend
    import gpt
    import layers
    import transformer_adapters
    return dict(xp=tl_hip, backend=backend, gpt=gpt, layers=layers, ta=transformer_adapters)


def run_gpt(tl, cfg, ids, dt, seed, scale=0.02):
    net, _ = tl["gpt"].build_gpt(cfg, dtype=dt)
    tl["gpt"].seed_parameters(net, seed, scale)
    probs = net.predict(ids)
    logits = net.layers[-2].output
    return net, probs, logits


def test_char_gpt_fp32_end_to_end(tl):
    """vocab 65, ctx 128, 4 layers, d 128, 4 heads, GeLU, batch 4."""
    cfg = dict(vocab=65, ctx=128, layers=4, d=128, heads=4, act="gelu")
    ids = np.random.default_rng(1).integers(0, 65, (4, 128))
    net, probs, logits = run_gpt(tl, cfg, ids, "fp32", seed=0)
    want_p, want_l = ref.gpt_forward(ids, ref.gpt_params(cfg, 0), cfg, return_logits=True)
    got_l = logits.get()
    assert ref.max_rel(got_l, want_l) <= 1e-5
    assert ref.max_rel(probs.get(), want_p) <= 1e-5
    ids_dev = tl["xp"].argmax(logits).get()
    assert np.array_equal(ids_dev, np.argmax(got_l, -1))
    assert np.array_equal(tl["xp"].argmax(probs).get(), np.argmax(probs.get(), -1))


def test_gpt_fp32_on_the_fp32_matrix_cores(tl):
    """An fp32 GPT large enough that its FFN, LM-head and batched attention products take the
    fp32 MFMA kernel (>= 128 output tiles of 128x128; weights packed [N, K]) and its smaller
    ones the VALU kernel: logits and probabilities within 1e-5 of the oracle, device argmax
    ids equal to NumPy's on the same logits."""
    cfg = dict(vocab=1030, ctx=512, layers=2, d=256, heads=4, act="gelu")
    ids = np.random.default_rng(21).integers(0, cfg["vocab"], (4, 512))
    net, probs, logits = run_gpt(tl, cfg, ids, "fp32", seed=2)
    want_p, want_l = ref.gpt_forward(ids, ref.gpt_params(cfg, 2), cfg, return_logits=True)
    got_l = logits.get()
    assert ref.max_rel(got_l, want_l) <= 1e-5
    assert ref.max_rel(probs.get(), want_p) <= 1e-5
    assert np.array_equal(tl["xp"].argmax(logits).get(), np.argmax(got_l, -1))


def test_char_gpt_uint8_ids_like_the_notebook(tl):
    cfg = dict(vocab=65, ctx=128, layers=1, d=128, heads=4, act="silu")
    ids = np.random.default_rng(2).integers(0, 65, (2, 50)).astype(np.uint8)
    net, probs, logits = run_gpt(tl, cfg, ids, "fp32", seed=3)
    want = ref.gpt_forward(ids, ref.gpt_params(cfg, 3), cfg)
    assert ref.max_rel(probs.get(), want) <= 1e-5


def test_tiny_gpt_golden(tl):
    z = np.load(os.path.join(GOLDEN, "gpt_tiny.npz"))
    cfg = {k[4:]: (z[k].item() if z[k].ndim == 0 else z[k]) for k in z.files if k.startswith("cfg_")}
    cfg["act"] = str(cfg["act"])
    net, probs, logits = run_gpt(tl, cfg, z["ids"], "fp32", seed=7, scale=0.5)
    assert ref.max_rel(logits.get(), z["logits"]) <= 1e-5
    assert ref.max_rel(probs.get(), z["probs"]) <= 1e-5
    assert np.array_equal(tl["xp"].argmax(logits).get(), np.argmax(z["logits"], -1))


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("decoder", [True, False])
@pytest.mark.parametrize("shape", [(2, 16, 64, 4), (1, 100, 96, 3), (2, 256, 768, 12)])
def test_multihead_attention_layer(tl, dt, decoder, shape):
    B, T, C, H = shape
    tl["backend"].set_float_type(dt)
    mha = tl["layers"].MultiHeadAttention(C, T + 4, H, decoder=decoder)
    rng = np.random.default_rng(B * T + C)
    P = [rng.standard_normal(p.shape).astype(F32) * F32(0.3 / np.sqrt(C) * 4) for p in mha.parameters]
    P = [ref.round_bf16(p) if dt == "bf16" else p for p in P]
    for p, a in zip(mha.parameters, P):
        p.set(a)
    x = rng.standard_normal((B, T, C)).astype(F32)
    if dt == "bf16":
        x = ref.round_bf16(x)
    y = mha.forward(tl["xp"].array(x, dtype=dt)).get()
    want = ref.mha(x, *P, H, decoder, T + 4, rnd=ref.round_bf16 if dt == "bf16" else None)
    tol = 1e-5 if dt == "fp32" else 2e-2
    assert ref.max_rel(y, want) <= tol, (dt, decoder, shape)


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_block_sublayer_taps_like_the_reference(tl, dt):
    """TransformerBlock with fuse_residual = False (reference layers.py:463-467): attn_block
    .output is MHA(LN1 x) and ffn.output is FFN(LN2 y), each against the oracle's sublayer
    (not the residual stream), and the block output equals both the oracle's block and the
    fused-residual path's."""
    tl["backend"].set_float_type(dt)
    B, T, C, H = 2, 40, 64, 4
    import activations
    blk = tl["layers"].TransformerBlock(C, T, H, activations.GeLU, decoder=True)
    rng = np.random.default_rng(29)
    P = [rng.standard_normal(p.shape).astype(F32) * F32(0.2) for p in blk.parameters]
    P[0] = 1 + P[0]  # LN1 gamma around 1
    P[6] = 1 + P[6]  # LN2 gamma around 1
    rnd = ref.round_bf16 if dt == "bf16" else None
    P = [rnd(p) if rnd else p for p in P]
    for p, a in zip(blk.parameters, P):
        p.set(a)
    x = rng.standard_normal((B, T, C)).astype(F32)
    x = rnd(x) if rnd else x
    xd = tl["xp"].array(x, dtype=dt)
    fused = blk.forward(xd).get()
    blk.fuse_residual = False
    try:
        out = blk.forward(xd).get()
        attn_tap = blk.attn_block.output.get()
        ffn_tap = blk.ffn.output.get()
    finally:
        del blk.fuse_residual
    g1, be1, wqkv, bqkv, wo, bo, g2, be2, w1, bb1, w2, bb2 = P
    r = rnd or (lambda a: a)
    want_attn = ref.mha(r(ref.layernorm(x, g1, be1)), wqkv, bqkv, wo, bo, H, True, T, rnd)
    y = r(x + r(want_attn))
    want_ffn = ref.ffn(r(ref.layernorm(y, g2, be2)), w1, bb1, w2, bb2, "gelu", rnd)
    tol = 1e-5 if dt == "fp32" else 2e-2
    assert ref.max_rel(attn_tap, want_attn) <= tol
    assert ref.max_rel(ffn_tap, want_ffn) <= tol
    assert ref.max_rel(out, ref.block(x, P, H, "gelu", True, T, rnd)) <= tol
    assert ref.max_rel(out, fused) <= (1e-6 if dt == "fp32" else 2e-2)
    # the default path keeps the residual stream in the taps
    blk.forward(xd)
    assert ref.max_rel(blk.ffn.output.get(), fused) == 0.0


@pytest.mark.parametrize("dt", ["bf16", "fp32"])
@pytest.mark.parametrize("decoder", [True, False])
def test_attention_fused_matches_unfused_layer(tl, decoder, dt):
    """The same layer through the fused kernel and through QK^T / softmax / P.V."""
    tl["backend"].set_float_type(dt)
    B, T, C, H = 2, 128, 256, 4
    mha = tl["layers"].MultiHeadAttention(C, T, H, decoder=decoder)
    rng = np.random.default_rng(17)
    for p in mha.parameters:
        p.set(rng.standard_normal(p.shape).astype(F32) * F32(0.1))
    x = tl["xp"].array(rng.standard_normal((B, T, C)).astype(F32), dtype=dt)
    fused = mha.forward(x).get()
    assert mha.softmax is None
    mha.fused = False
    unfused = mha.forward(x).get()
    assert mha.softmax is not None
    assert ref.max_rel(fused, unfused) <= (2e-2 if dt == "bf16" else 1e-5)


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_dense_and_vit_head(tl, dt):
    tl["backend"].set_float_type(dt)
    rng = np.random.default_rng(9)
    d = tl["layers"].Dense(48, 10)
    head = tl["ta"].VitMLPHead(384, 10)
    for layer in (d, head):
        for p in layer.parameters:
            p.set(rng.standard_normal(p.shape).astype(F32) * F32(0.1))
    rnd = ref.round_bf16 if dt == "bf16" else (lambda a: a)
    x = rnd(rng.standard_normal((5, 7, 48)).astype(F32))
    y = d.forward(tl["xp"].array(x, dtype=dt)).get()
    w, b = [rnd(p.get()) for p in d.parameters]
    tol = 1e-5 if dt == "fp32" else 2e-2
    assert ref.max_rel(y, ref.dense(x, w, b)) <= tol
    xv = rnd(rng.standard_normal((6, 65, 384)).astype(F32))
    yv = head.forward(tl["xp"].array(xv, dtype=dt)).get()
    w, b = [p.get() for p in head.parameters]
    assert ref.max_rel(yv, ref.vit_head(xv, w, b)) <= tol


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_weight_written_through_a_view_is_repacked(tl, dt):
    """The GEMM reads a packed [N, K] copy of a weight for large products (fp32 with >= 128
    tiles of 128x128, bf16 always). Writing the weight through another view of its buffer,
    or as a kernel's output operand, must make the next forward use the new values."""
    xp = tl["xp"]
    tl["backend"].set_float_type(dt)
    rnd = ref.round_bf16 if dt == "bf16" else (lambda a: a)
    tol = 1e-5 if dt == "fp32" else 2e-2
    d = tl["layers"].Dense(256, 512)
    rng = np.random.default_rng(77)
    d.bias.set(np.zeros(512, F32))
    x = rnd(rng.standard_normal((4096, 256)).astype(F32))
    xd = xp.array(x, dtype=dt)
    w0 = rnd(rng.standard_normal((256, 512)).astype(F32) * F32(0.1))
    d.weights.set(w0)
    assert ref.max_rel(d.forward(xd).get(), x @ w0) <= tol
    w1 = rnd(rng.standard_normal((256, 512)).astype(F32) * F32(0.1))
    d.weights.reshape(-1).set(w1.reshape(-1))  # a different DeviceTensor over the same buffer
    assert ref.max_rel(d.forward(xd).get(), x @ w1) <= tol
    w2t = rnd(rng.standard_normal((512, 256)).astype(F32) * F32(0.1))
    xp.transpose2d(xp.array(w2t, dtype=dt), out=d.weights, out_offset=0, ldy=512)
    assert ref.max_rel(d.forward(xd).get(), x @ w2t.T) <= tol


def test_gpt2_small_shape_bf16_short(tl):
    """BASELINE config 3 model (vocab 50257, 12 layers, d 768, 12 heads) at B=2, T=128."""
    cfg = dict(vocab=50257, ctx=1024, layers=12, d=768, heads=12, act="gelu")
    ids = np.random.default_rng(5).integers(0, 50257, (2, 128))
    net, probs, logits = run_gpt(tl, cfg, ids, "bf16", seed=0)
    want_p, want_l = ref.gpt_forward(ids, ref.gpt_params(cfg, 0, bf16=True), cfg, bf16=True,
                                     return_logits=True)
    got_l = logits.get()
    assert ref.max_rel(got_l, want_l) <= 2e-2
    assert ref.max_rel(probs.get(), want_p) <= 2e-2
    assert np.array_equal(tl["xp"].argmax(logits).get(), np.argmax(got_l, -1))


def test_gpt2_small_full_shape_bf16(tl):
    """BASELINE config 3 at its full size, B=8, T=1024: size-independent properties over the
    whole batch, oracle parity on sequences 0 and 7 (causal rows of one sequence depend only
    on that sequence, so the first and last batch entries pin the batch strides), and every
    sequence run alone equals its row of the batched run."""
    cfg = dict(vocab=50257, ctx=1024, layers=12, d=768, heads=12, act="gelu")
    ids = np.random.default_rng(6).integers(0, 50257, (8, 1024))
    net, probs, logits = run_gpt(tl, cfg, ids, "bf16", seed=1)
    xp = tl["xp"]
    ids_logits = xp.argmax(logits).get()
    ids_probs = xp.argmax(probs).get()
    p_last = probs.get()[:, -1, :]
    np.testing.assert_allclose(p_last.astype(np.float64).sum(-1), 1.0, rtol=2e-2)
    # softmax is monotone: the most likely token is the largest logit (up to bf16 ties)
    agree = np.mean(ids_logits == ids_probs)
    assert agree > 0.99, agree
    full = logits.get()
    assert np.array_equal(ids_logits, np.argmax(full, -1))  # device argmax, bit-exact
    want_p, want_l = ref.gpt_forward(ids[[0, 7]], ref.gpt_params(cfg, 1, bf16=True), cfg,
                                     bf16=True, return_logits=True)
    assert ref.max_rel(full[0], want_l[0]) <= 2e-2
    assert ref.max_rel(full[7], want_l[1]) <= 2e-2
    for b in range(8):
        net.predict(ids[b:b + 1])
        alone = net.layers[-2].output.get()[0]
        assert ref.max_rel(alone, full[b]) <= 1e-6, b


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_embed_front_sinusoidal_positions(tl, dt):
    """GPTEmbedFront's sinusoidal branch (reference transformer_adapters.py:128-135, 148-153):
    table[ids] + the closed-form position table, one rounding of the sum in bf16, bit-exact."""
    tl["backend"].set_float_type(dt)
    V, ctx, C = 37, 50, 24
    table = tl["ta"].GPTEmbeddingTable(V, C)
    front = tl["ta"].GPTEmbedFront(table, ctx, positional_embedding="sinusoidal")
    assert front.parameters == [table.table]  # no trainable positions in this branch
    rng = np.random.default_rng(31)
    tab = rng.standard_normal((V, C)).astype(F32)
    tab = ref.round_bf16(tab) if dt == "bf16" else tab
    table.table.set(tab)
    ids = rng.integers(0, V, (3, 41))
    got = front.forward(ids).get()
    pos = ref.sinusoidal_positions(ctx, C)
    if dt == "bf16":
        want = ref.round_bf16(ref.embed_front(ids, tab, ref.round_bf16(pos)))
    else:
        want = ref.embed_front(ids, tab, pos)
    assert np.array_equal(got, want)


def test_sequence_longer_than_context_is_rejected(tl):
    cfg = dict(vocab=11, ctx=8, layers=1, d=16, heads=2, act="gelu")
    net, _ = tl["gpt"].build_gpt(cfg, dtype="fp32")
    with pytest.raises(ValueError):
        net.predict(np.zeros((1, 9), np.int64))


def test_out_of_range_token_raises_index_error(tl):
    cfg = dict(vocab=11, ctx=8, layers=1, d=16, heads=2, act="gelu")
    net, _ = tl["gpt"].build_gpt(cfg, dtype="fp32")
    with pytest.raises(IndexError):
        net.predict(np.array([[1, 11]])).get()
    tl["xp"].synchronize()
