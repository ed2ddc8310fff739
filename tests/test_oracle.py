"""Pins the NumPy oracle (oracle/numpy_ref.py) against closed forms, brute force and
invariants, so that a dropped term, wrong sign, transposed operand or wrong index in the
oracle fails here before it can vouch for a kernel."""
import math

import numpy as np
import pytest

from oracle import numpy_ref as ref

F32 = np.float32


# ---- bf16 rounding ------------------------------------------------------------------------
def test_bf16_rounding_bit_patterns():
    vals = np.array([1.0, -2.0, 0.0, np.inf, -np.inf], dtype=F32)
    assert ref.bf16_bits(vals).tolist() == [0x3F80, 0xC000, 0x0000, 0x7F80, 0xFF80]
    # ties to even: 0x3F808000 is halfway between 0x3F80 and 0x3F81 -> even 0x3F80
    u = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF], dtype=np.uint32)
    assert ref.bf16_bits(u.view(F32)).tolist() == [0x3F80, 0x3F82, 0x3F81, 0x3F80]
    nan = ref.bf16_bits(np.array([np.nan], dtype=F32))
    assert (int(nan[0]) & 0x7F80) == 0x7F80 and (int(nan[0]) & 0x7F) != 0
    assert np.array_equal(ref.round_bf16(np.array([3.0], F32)), np.array([3.0], F32))


def test_max_rel_metric():
    assert ref.max_rel([1.0, 2.0], [1.0, 2.0]) == 0.0
    assert math.isclose(ref.max_rel([1.0, 2.5], [1.0, 2.0]), 0.25)


# ---- activations ----------------------------------------------------------------------
def test_gelu_closed_form_and_identities():
    x = np.linspace(-8, 8, 2001, dtype=F32)
    x64 = x.astype(np.float64)
    exact = 0.5 * x64 * (1 + np.tanh(math.sqrt(2 / math.pi) * (x64 + 0.044715 * x64 ** 3)))
    assert np.max(np.abs(ref.gelu(x) - exact)) < 1e-5
    assert ref.gelu(np.zeros(3, F32)).tolist() == [0, 0, 0]
    # odd-part identity: gelu(x) - gelu(-x) = x (because tanh is odd)
    np.testing.assert_allclose(ref.gelu(x) - ref.gelu(-x), x, atol=1e-5)
    assert abs(float(ref.gelu(np.array([1.0], F32))[0]) - 0.8411920) < 1e-6


def test_silu_matches_sigmoid_form():
    x = np.linspace(-20, 20, 4001, dtype=F32)
    sig = 1 / (1 + np.exp(-x.astype(np.float64)))  # independent formula
    np.testing.assert_allclose(ref.silu(x), x * sig, atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(ref.silu(x) - ref.silu(-x), x, atol=1e-5)


def test_softmax_properties():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((7, 33)).astype(F32) * 4
    p = ref.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max(-1, keepdims=True))
    np.testing.assert_allclose(p, e / e.sum(-1, keepdims=True), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-5)
    np.testing.assert_allclose(ref.softmax(x + F32(3.0)), p, rtol=1e-5, atol=1e-7)
    assert ref.softmax(np.array([[5.0]], F32)).tolist() == [[1.0]]
    # temperature divides the shifted logits
    e2 = np.exp((x.astype(np.float64) - x.max(-1, keepdims=True)) / 2.0)
    np.testing.assert_allclose(ref.softmax(x, F32(2.0)), e2 / e2.sum(-1, keepdims=True), rtol=1e-5)


# ---- normalisation ----------------------------------------------------------------------
def _ln_brute(x, g, b, eps):
    out = np.zeros_like(x, dtype=np.float64)
    for r in range(x.shape[0]):
        row = [float(v) for v in x[r]]
        n = len(row)
        mu = sum(row) / n
        var = sum((v - mu) ** 2 for v in row) / n
        for c in range(n):
            out[r, c] = (row[c] - mu) / math.sqrt(var + eps) * float(g[c]) + float(b[c])
    return out


def test_layernorm_brute_force_and_invariants():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 37)).astype(F32) * 3 + 1
    g = rng.standard_normal(37).astype(F32)
    b = rng.standard_normal(37).astype(F32)
    np.testing.assert_allclose(ref.layernorm(x, g, b), _ln_brute(x, g, b, 1e-5), rtol=1e-5, atol=1e-5)
    y = ref.layernorm(x, np.ones(37, F32), np.zeros(37, F32))
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-6)
    np.testing.assert_allclose(y.std(-1), np.sqrt(x.var(-1) / (x.var(-1) + 1e-5)), rtol=1e-5)


def test_rmsnorm_brute_force_and_scale_invariance():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 19)).astype(F32)
    g = rng.standard_normal(19).astype(F32)
    brute = np.zeros((4, 19))
    for r in range(4):
        ms = sum(float(v) ** 2 for v in x[r]) / 19
        for c in range(19):
            brute[r, c] = float(x[r, c]) / math.sqrt(ms + 1e-6) * (1.0 + float(g[c]))
    np.testing.assert_allclose(ref.rmsnorm(x, g, 1e-6, 1.0), brute, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ref.rmsnorm(x * F32(7.0), g, 0.0), ref.rmsnorm(x, g, 0.0), rtol=1e-5, atol=1e-6)


# ---- RoPE ---------------------------------------------------------------------------------
def test_rope_against_complex_form_and_invariants():
    rng = np.random.default_rng(3)
    T, D = 9, 8
    x = rng.standard_normal((2, T, D)).astype(F32)
    cos, sin = ref.rope_table(T, D, 10000.0)
    y = ref.rope(x, cos, sin)
    half = D // 2
    z = x[..., :half].astype(np.float64) + 1j * x[..., half:]
    theta = 10000.0 ** (-np.arange(half) * 2.0 / D)
    rot = z * np.exp(1j * np.arange(T)[:, None] * theta[None, :])
    np.testing.assert_allclose(y[..., :half], rot.real, atol=1e-5)
    np.testing.assert_allclose(y[..., half:], rot.imag, atol=1e-5)
    np.testing.assert_allclose(y[:, 0], x[:, 0], atol=0)  # position 0 is the identity
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)
    # relative position: <R_m q, R_n k> depends only on m - n
    q, k = x[0, 0], x[1, 0]
    def dot_at(m, n):
        c, s = ref.rope_table(1, D, 10000.0, m)
        c2, s2 = ref.rope_table(1, D, 10000.0, n)
        return float(ref.rope(q[None], c, s)[0] @ ref.rope(k[None], c2, s2)[0])
    assert abs(dot_at(5, 2) - dot_at(13, 10)) < 1e-4


# ---- attention / blocks -------------------------------------------------------------------
def _mha_brute(x, wqkv, bqkv, wo, bo, H, decoder):
    B, T, C = x.shape
    D = C // H
    x64 = x.astype(np.float64)
    qkv = x64 @ wqkv + bqkv
    out = np.zeros((B, T, C))
    for b in range(B):
        heads = np.zeros((T, C))
        for h in range(H):
            q = qkv[b, :, h * D:(h + 1) * D]
            k = qkv[b, :, C + h * D:C + (h + 1) * D]
            v = qkv[b, :, 2 * C + h * D:2 * C + (h + 1) * D]
            for i in range(T):
                s = [sum(q[i, d] * k[j, d] for d in range(D)) / math.sqrt(D) for j in range(T)]
                lim = i + 1 if decoder else T
                m = max(s[:lim])
                e = [math.exp(s[j] - m) if j < lim else 0.0 for j in range(T)]
                tot = sum(e)
                for d in range(D):
                    heads[i, h * D + d] = sum(e[j] / tot * v[j, d] for j in range(T))
        out[b] = heads @ wo + bo
    return out


@pytest.mark.parametrize("decoder", [True, False])
def test_mha_brute_force(decoder):
    rng = np.random.default_rng(4)
    B, T, C, H = 2, 5, 8, 2
    x = rng.standard_normal((B, T, C)).astype(F32)
    wqkv = rng.standard_normal((C, 3 * C)).astype(F32) * F32(0.3)
    bqkv = rng.standard_normal(3 * C).astype(F32) * F32(0.1)
    wo = rng.standard_normal((C, C)).astype(F32) * F32(0.3)
    bo = rng.standard_normal(C).astype(F32) * F32(0.1)
    got = ref.mha(x, wqkv, bqkv, wo, bo, H, decoder, context_length=T + 3)
    np.testing.assert_allclose(got, _mha_brute(x, wqkv, bqkv, wo, bo, H, decoder), rtol=1e-4, atol=1e-5)


def test_mha_head_order_with_permutation_weights():
    """Q = K = 0 makes attention uniform (causal: mean over the prefix); with V = x and an
    identity output projection the result is the running mean of x, whatever H is. Swapping
    head blocks in V and Wo together must leave the output unchanged; swapping only V must
    permute it, pinning the split/merge order."""
    rng = np.random.default_rng(5)
    B, T, C, H = 1, 4, 6, 3
    x = rng.standard_normal((B, T, C)).astype(F32)
    wqkv = np.zeros((C, 3 * C), F32)
    wqkv[:, 2 * C:] = np.eye(C, dtype=F32)
    y = ref.mha(x, wqkv, np.zeros(3 * C, F32), np.eye(C, dtype=F32), np.zeros(C, F32), H, True)
    running = np.cumsum(x, axis=1) / np.arange(1, T + 1)[None, :, None]
    np.testing.assert_allclose(y, running, rtol=1e-5, atol=1e-6)
    perm = np.array([2, 3, 0, 1, 4, 5])  # swap head 0 and head 1 (D=2)
    w2 = wqkv.copy()
    w2[:, 2 * C:] = np.eye(C, dtype=F32)[:, perm]
    y2 = ref.mha(x, w2, np.zeros(3 * C, F32), np.eye(C, dtype=F32), np.zeros(C, F32), H, True)
    np.testing.assert_allclose(y2, running[..., perm], rtol=1e-5, atol=1e-6)


def test_causal_mask_values():
    m = ref.causal_mask(3)
    assert m.dtype == F32
    assert m.tolist() == [[0, -1e9, -1e9], [0, 0, -1e9], [0, 0, 0]]


def test_embed_front_and_back_brute_force():
    rng = np.random.default_rng(6)
    table = rng.standard_normal((11, 4)).astype(F32)
    pos = rng.standard_normal((6, 4)).astype(F32)
    ids = np.array([[3, 0, 10], [1, 1, 7]])
    y = ref.embed_front(ids, table, pos)
    for b in range(2):
        for t in range(3):
            assert np.array_equal(y[b, t], table[ids[b, t]] + pos[t])
    logits = ref.embed_back(y, table)
    for b in range(2):
        for t in range(3):
            for v in range(11):
                assert abs(logits[b, t, v] - float(np.dot(y[b, t].astype(np.float64), table[v]))) < 1e-4


def test_sinusoidal_positions_closed_form():
    tab = ref.sinusoidal_positions(7, 6)
    for p in range(7):
        for i in range(6):
            ang = p / 10000 ** (2 * (i // 2) / 6)
            want = math.sin(ang) if i % 2 == 0 else math.cos(ang)
            assert abs(tab[p, i] - want) < 1e-6


def test_argmax_semantics():
    x = np.array([[1, 3, 3, 0], [np.nan, 1, np.nan, 2], [-1, -1, -1, -1]], dtype=F32)
    assert ref.argmax(x).tolist() == [1, 0, 0]


def test_gpt_param_order_matches_layer_order():
    cfg = dict(vocab=7, ctx=4, layers=2, d=4, heads=2)
    names = [n for n, _ in ref.gpt_param_shapes(cfg)]
    assert names[:2] == ["pos", "table"]
    assert names[2:14] == [f"b0.{k}" for k in ("g1", "be1", "wqkv", "bqkv", "wo", "bo", "g2",
                                               "be2", "w1", "bb1", "w2", "bb2")]
    assert names[-2:] == ["lnf.g", "lnf.be"]
    p = ref.gpt_params(cfg, 0)
    assert abs(float(p["b0.g1"].mean()) - 1.0) < 0.05 and abs(float(p["b0.be1"].mean())) < 0.05


# ---- Gemma-style pieces -------------------------------------------------------------------
def test_geglu_brute_force():
    rng = np.random.default_rng(31)
    x = rng.standard_normal((2, 3, 5)).astype(F32)
    wg, wu = rng.standard_normal((2, 5, 4)).astype(F32)
    wd = rng.standard_normal((4, 5)).astype(F32)
    want = np.zeros((2, 3, 5))
    for b in range(2):
        for t in range(3):
            h = []
            for f in range(4):
                g = sum(float(x[b, t, c]) * float(wg[c, f]) for c in range(5))
                u = sum(float(x[b, t, c]) * float(wu[c, f]) for c in range(5))
                gl = 0.5 * g * (1 + math.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)))
                h.append(gl * u)
            for c in range(5):
                want[b, t, c] = sum(h[f] * float(wd[f, c]) for f in range(4))
    assert ref.max_rel(ref.geglu_ffn(x, wg, wu, wd), want) < 1e-5
    # SwiGLU variant: silu(g) = g * sigmoid(g)
    g, u = x @ wg, x @ wu
    sw = (g / (1 + np.exp(-g.astype(np.float64)))) * u
    assert ref.max_rel(ref.geglu_ffn(x, wg, wu, wd, "silu"), sw @ wd) < 1e-5


def test_mqa_without_rope_equals_mha_when_heads_match():
    rng = np.random.default_rng(32)
    B, T, H, D = 2, 6, 3, 4
    C = H * D
    x = rng.standard_normal((B, T, C)).astype(F32)
    wqkv = rng.standard_normal((C, 3 * C)).astype(F32) * F32(0.3)
    wo = rng.standard_normal((C, C)).astype(F32) * F32(0.3)
    got, _, _ = ref.mqa(x, wqkv, wo, H, H, D, use_rope=False)
    want = ref.mha(x, wqkv, np.zeros(3 * C, F32), wo, np.zeros(C, F32), H, decoder=True)
    assert ref.max_rel(got, want) < 1e-5


def test_mqa_shared_kv_head_equals_replicated_weights():
    """Hkv = 1 must equal Hkv = Hq with the key/value columns copied to every head: pins
    the query-head -> kv-head map and the [Q | K | V] column split."""
    rng = np.random.default_rng(33)
    B, T, Hq, D = 2, 5, 4, 8
    C = 16
    x = rng.standard_normal((B, T, C)).astype(F32)
    wq = rng.standard_normal((C, Hq * D)).astype(F32) * F32(0.4)
    wk = rng.standard_normal((C, D)).astype(F32) * F32(0.4)
    wv = rng.standard_normal((C, D)).astype(F32) * F32(0.4)
    wo = rng.standard_normal((Hq * D, C)).astype(F32) * F32(0.4)
    got, k1, _ = ref.mqa(x, np.concatenate([wq, wk, wv], 1), wo, Hq, 1, D)
    rep = np.concatenate([wq, np.tile(wk, (1, Hq)), np.tile(wv, (1, Hq))], 1)
    want, kq, _ = ref.mqa(x, rep, wo, Hq, Hq, D)
    assert ref.max_rel(got, want) < 1e-6
    assert k1.shape == (B, 1, T, D) and np.array_equal(kq[:, 2], k1[:, 0])
    # grouped: Hq = 4, Hkv = 2 -> heads 0,1 read kv head 0 and heads 2,3 read kv head 1
    wk2 = rng.standard_normal((C, 2 * D)).astype(F32) * F32(0.4)
    wv2 = rng.standard_normal((C, 2 * D)).astype(F32) * F32(0.4)
    got2, _, _ = ref.mqa(x, np.concatenate([wq, wk2, wv2], 1), wo, Hq, 2, D)
    rep2 = np.concatenate([wq, wk2[:, :D], wk2[:, :D], wk2[:, D:], wk2[:, D:],
                           wv2[:, :D], wv2[:, :D], wv2[:, D:], wv2[:, D:]], 1)
    want2, _, _ = ref.mqa(x, rep2, wo, Hq, Hq, D)
    assert ref.max_rel(got2, want2) < 1e-6


def test_mqa_rope_identity_at_position_zero():
    """A single token at position 0 is not rotated, so RoPE on and off agree; at later
    positions they differ (the rotation is applied)."""
    rng = np.random.default_rng(34)
    x = rng.standard_normal((1, 5, 16)).astype(F32)
    w = rng.standard_normal((16, 6 * 8)).astype(F32) * F32(0.4)
    wo = rng.standard_normal((32, 16)).astype(F32) * F32(0.4)
    one, _, _ = ref.mqa(x[:, :1], w, wo, 4, 1, 8)
    none, _, _ = ref.mqa(x[:, :1], w, wo, 4, 1, 8, use_rope=False)
    assert ref.max_rel(one, none) < 1e-6
    a, _, _ = ref.mqa(x, w, wo, 4, 1, 8)
    b, _, _ = ref.mqa(x, w, wo, 4, 1, 8, use_rope=False)
    assert ref.max_rel(a, b) > 1e-3


def test_mqa_cached_calls_equal_one_call():
    rng = np.random.default_rng(35)
    x = rng.standard_normal((2, 9, 16)).astype(F32)
    w = rng.standard_normal((16, 6 * 8)).astype(F32) * F32(0.4)
    wo = rng.standard_normal((32, 16)).astype(F32) * F32(0.4)
    full, kf, vf = ref.mqa(x, w, wo, 4, 1, 8)
    a, k, v = ref.mqa(x[:, :6], w, wo, 4, 1, 8)
    b, k2, v2 = ref.mqa(x[:, 6:], w, wo, 4, 1, 8, pos0=6, past_k=k, past_v=v)
    assert ref.max_rel(np.concatenate([a, b], 1), full) < 1e-6
    assert ref.max_rel(k2, kf) == 0 and ref.max_rel(v2, vf) == 0


GEMMA_TINY = dict(vocab=40, ctx=32, layers=2, d=32, heads=4, kv_heads=1, head_dim=16, ffn=48)


def test_gemma_param_order():
    shapes = ref.gemma_param_shapes(GEMMA_TINY)
    assert shapes[0] == ("table", (40, 32))
    assert [n for n, _ in shapes[1:8]] == ["b0.g1", "b0.wqkv", "b0.wo", "b0.g2", "b0.wg",
                                          "b0.wu", "b0.wd"]
    assert dict(shapes)["b1.wqkv"] == (32, 6 * 16)
    assert shapes[-1] == ("normf.g", (32,))


def test_gemma_cached_forward_and_greedy_consistency():
    P = ref.gemma_params(GEMMA_TINY, 3, 0.3)
    ids = np.random.default_rng(36).integers(0, 40, (2, 7))
    full = ref.gemma_forward(ids, P, GEMMA_TINY)
    cache = {}
    a = ref.gemma_forward(ids[:, :4], P, GEMMA_TINY, cache=cache)
    b = ref.gemma_forward(ids[:, 4:], P, GEMMA_TINY, pos0=4, cache=cache)
    assert ref.max_rel(np.concatenate([a, b], 1), full) < 1e-5
    new, rows = ref.gemma_greedy(ids, P, GEMMA_TINY, 3)
    assert np.array_equal(new, np.argmax(rows, -1).T)
    seq = np.concatenate([ids, new[:, :2]], 1)
    assert ref.max_rel(ref.gemma_forward(seq, P, GEMMA_TINY)[:, -1], rows[2]) == 0
    # embedding scale: the first layer sees table[ids] * sqrt(d)
    x0 = P["table"][ids] * np.sqrt(F32(32))
    assert np.allclose(np.sqrt(np.mean(x0 ** 2)), np.sqrt(np.mean(P["table"] ** 2)) * np.sqrt(32), rtol=0.3)


# ---- Philox / normal draws ----------------------------------------------------------------
def test_philox_known_answer_vectors():
    """Random123's known-answer vectors for philox4x32-10."""
    cases = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in cases:
        got = ref.philox4x32_10(np.array(ctr, np.uint32), key)
        assert [int(v) for v in got] == want


def test_random_normal_moments_and_structure():
    z = ref.random_normal(1_000_003, seed=1234, stream=7).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 5e-3
    assert abs(np.mean(z ** 3)) < 2e-2 and abs(np.mean(z ** 4) - 3) < 3e-2
    # pairs share a radius: z0^2 + z1^2 = -2 ln u1 from word 0 of the same counter
    w = ref.philox4x32_10(np.array([[0, 0, 7, 0]], np.uint32), (1234, 0))[0]
    u1 = ((int(w[0]) >> 8) + 1) * 2.0 ** -24
    assert math.isclose(z[0] ** 2 + z[1] ** 2, -2 * math.log(u1), rel_tol=1e-5)
    # seed and stream select different draws; mean/std are affine
    assert not np.allclose(ref.random_normal(16, 1, 0), ref.random_normal(16, 2, 0))
    assert not np.allclose(ref.random_normal(16, 1, 0), ref.random_normal(16, 1, 1))
    np.testing.assert_allclose(ref.random_normal(10, 5, 3, 1.0, 0.02),
                               1.0 + 0.02 * ref.random_normal(10, 5, 3), rtol=1e-6)


def test_sample_uniforms_grid_and_moments():
    u = ref.sample_uniforms(400_000, seed=99, stream=3)
    assert u.min() >= 0 and u.max() < 1
    assert np.all(u * 2 ** 24 == np.floor(u * 2 ** 24))  # the 2^-24 grid of (w0 >> 8)
    assert abs(u.mean() - 0.5) < 2e-3 and abs(u.var() - 1 / 12) < 1e-3
    w = ref.philox4x32_10(np.array([[5, 0, 3, 0]], np.uint32), (99, 0))[0]
    assert u[5] == (int(w[0]) >> 8) * 2.0 ** -24
    assert not np.array_equal(ref.sample_uniforms(8, 99, 3), ref.sample_uniforms(8, 99, 4))


def test_sample_categorical_brute_force_and_frequencies():
    rng = np.random.default_rng(51)
    for n in (1, 2, 5, 17):
        p = rng.random(n).astype(F32)
        p[rng.random(n) < 0.3] = 0
        if p.sum() == 0:
            p[-1] = 1
        u = rng.random(64)
        got, x, _ = ref.sample_categorical(p, u)
        for j in range(64):  # first index whose running sum exceeds u * total
            run, want = 0.0, n - 1
            for i in range(n):
                run += float(p[i])
                if run > x[j]:
                    want = i
                    break
            assert got[j] == want and p[got[j]] > 0
    onehot = np.zeros(9, F32)
    onehot[4] = 1
    assert set(ref.sample_categorical(onehot, rng.random(100))[0]) == {4}
    p = np.array([0, 0.25, 0, 0.5, 0.25, 0], F32)
    assert ref.sample_categorical(p, [0.0])[0][0] == 1
    assert ref.sample_categorical(p, [1 - 2 ** -24])[0][0] == 4
    # frequencies of 200000 draws against p (chi-square, 9 degrees of freedom)
    p = rng.random(10).astype(F32)
    idx = ref.sample_categorical(p, ref.sample_uniforms(200_000, seed=7))[0]
    cnt = np.bincount(idx, minlength=10)
    e = 200_000 * p / p.sum()
    assert np.sum((cnt - e) ** 2 / e) < 30


# ---- ViT ------------------------------------------------------------------------------------
def test_patchify_brute_force():
    rng = np.random.default_rng(40)
    B, C, H, W, p0, p1 = 2, 3, 6, 4, 3, 2
    x = rng.standard_normal((B, C, H, W)).astype(F32)
    got = ref.patchify(x, (p0, p1))
    ph, pw = H // p0, W // p1
    assert got.shape == (B, ph * pw, p0 * p1 * C)
    for b in range(B):
        for i in range(ph):
            for j in range(pw):
                for a in range(p0):
                    for c2 in range(p1):
                        for ch in range(C):
                            assert got[b, i * pw + j, (a * p1 + c2) * C + ch] == x[b, ch, i * p0 + a, j * p1 + c2]


def test_vit_projector_brute_force():
    rng = np.random.default_rng(41)
    B, C, H, W, p, E, R = 2, 2, 4, 4, 2, 5, 3
    x = rng.standard_normal((B, C, H, W)).astype(F32)
    proj = rng.standard_normal((p * p * C, E)).astype(F32)
    cls = rng.standard_normal((R, E)).astype(F32)
    L = (H // p) * (W // p)
    pos = rng.standard_normal((R + L, E)).astype(F32)
    got = ref.vit_projector(x, proj, cls, pos, (p, p))
    want = np.zeros((B, R + L, E))
    for b in range(B):
        for r in range(R):
            want[b, r] = cls[r] + pos[r]
        for l in range(L):
            i, j = divmod(l, W // p)
            tok = [x[b, ch, i * p + a, j * p + c2] for a in range(p) for c2 in range(p) for ch in range(C)]
            want[b, R + l] = np.array(tok, np.float64) @ proj + pos[R + l]
    assert ref.max_rel(got, want) < 1e-5


def test_vit_forward_images_are_independent():
    cfg = dict(image=(3, 8, 8), patch=(4, 4), d=16, heads=2, layers=2, act="gelu", registers=1,
               classes=5, head_hidden=8)
    P = ref.vit_params(cfg, 0, 0.3)
    x = np.random.default_rng(42).standard_normal((3, 3, 8, 8)).astype(F32)
    full = ref.vit_forward(x, P, cfg)
    assert full.shape == (3, 5)
    np.testing.assert_allclose(full.sum(-1), 1.0, rtol=1e-5)
    assert ref.max_rel(ref.vit_forward(x[1:2], P, cfg), full[1:2]) < 1e-5
    names = [n for n, _ in ref.vit_param_shapes(cfg)]
    assert names[:3] == ["proj", "cls", "pos"] and names[-4:] == ["head.w", "head.b", "dense.w", "dense.b"]


def test_dense_brute_force():
    """reference layers.py:206-209: y = x @ W + b over the last axis of any leading shape."""
    rng = np.random.default_rng(43)
    x = rng.standard_normal((2, 3, 5)).astype(F32)
    w = rng.standard_normal((5, 4)).astype(F32)
    b = rng.standard_normal(4).astype(F32) * 3  # a bias large enough that dropping it fails
    got = ref.dense(x, w, b)
    assert got.shape == (2, 3, 4)
    for i in range(2):
        for j in range(3):
            for o in range(4):
                want = sum(float(x[i, j, k]) * float(w[k, o]) for k in range(5)) + float(b[o])
                assert abs(float(got[i, j, o]) - want) < 1e-5 * (1 + abs(want))


def test_vit_head_brute_force():
    """reference transformer_adapters.py:89-95: the class token (token 0) @ W + b."""
    rng = np.random.default_rng(44)
    x = rng.standard_normal((3, 4, 5)).astype(F32)
    w = rng.standard_normal((5, 2)).astype(F32)
    b = rng.standard_normal(2).astype(F32) * 3
    got = ref.vit_head(x, w, b)
    assert got.shape == (3, 2)
    for n in range(3):
        for o in range(2):
            want = sum(float(x[n, 0, k]) * float(w[k, o]) for k in range(5)) + float(b[o])
            assert abs(float(got[n, o]) - want) < 1e-5 * (1 + abs(want))
            other = sum(float(x[n, 1, k]) * float(w[k, o]) for k in range(5)) + float(b[o])
            assert abs(float(got[n, o]) - other) > 1e-3  # a wrong token index would fail


def test_sampler_stream_with_the_largest_uniform():
    """Philox stream 1205178 under key 0 gives draw 0 the largest uniform the sampler can
    draw, 1 - 2^-24 (the GPU test of the sampler's zero-probability fallback uses it)."""
    assert ref.sample_uniforms(1, 0, 1205178)[0] == 1.0 - 2.0 ** -24
    assert ref.sample_uniforms(1, 0, 1205177)[0] < 1.0 - 2.0 ** -24
