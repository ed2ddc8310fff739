"""CPU oracle: a NumPy restatement of torchless-nn's transformer forward.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import this module, and only as the checker (or, for the baseline, as the timed
CPU path). The product path (torchless-nn_amd/) never imports it.

Each function follows the reference op for op (file:line under luke-skynet/torchless-nn),
in float32 as the reference's CPU runtime does (backend.py:24). Functions with no reference
counterpart (RMSNorm, RoPE, GeGLU) restate the published definitions named in their
docstrings.

Pinning (how each function is checked, in tests/test_oracle.py and tests/golden/):
  gelu, silu       closed forms in float64 (silu against x*sigmoid(x), an independent
                   formula), odd-part identity f(x) - f(-x) = x, f(0) = 0
  softmax          float64 closed form, rows sum to 1, shift invariance, masked entries
                   exactly 0, single-column rows equal 1
  layernorm        brute-force float64 loops; per-row mean -> beta and std -> gamma
  rmsnorm          brute-force float64 loops; invariance to positive row scaling
  rope             complex-multiplication form, identity at position 0, pair norms
                   preserved, <R_m q, R_n k> depends only on m - n
  geglu_ffn        brute-force float64 scalar loops at a tiny shape
  mqa              without RoPE and with Hkv = Hq equals mha (zero biases, [Q|K|V]
                   columns), itself pinned; Hkv = 1 equals Hkv = Hq with the key/value
                   weights replicated per head (pins the head -> kv-head map); a cached
                   two-call run equals one call over the whole sequence; an uncached call
                   with every position shifted by the same offset gives the same output
                   (RoPE on queries and keys alike), which RoPE on the queries only fails
  gemma_forward    golden fixture tests/golden/gemma_tiny.npz: brute-force float64 loops of
                   the whole decoder (sqrt(C)-scaled gather, (1 + gain) RMSNorms with eps
                   1e-6, 4 query heads on one key/value head with rotate-half RoPE on
                   queries and keys at absolute positions, GeGLU, both residuals, final
                   norm, tied head) written independently of this module, whole-sequence
                   and as cached calls at positions 0, 7 and 8; planted mistakes (a dropped
                   residual, a gain without its 1 + offset, no sqrt(C) scale, RoPE on the
                   queries only, a cached call rotated from position 0) each fail it;
                   gemma_greedy ids are argmax of its own rows
  patchify         brute-force index loops (token i*(W/p1)+j, feature (a*p1+c2)*C+ch)
  vit_projector    brute-force loops over the same formula at a tiny shape
  vit_forward      golden fixture tests/golden/vit_tiny.npz: brute-force float64 loops of
                   the whole notebook ViT (patch order, projector, class/register rows,
                   positions, unmasked blocks, LayerNorm, VitMLPHead on token 0, SiLU,
                   Dense, softmax) written independently of this module; class scores and
                   probabilities both compared; images are independent (batch split)
  dense            brute-force float64 loops at a tiny shape with a non-zero bias
  vit_head         brute-force loops reading token 0 (not another token) plus the bias
  mha              brute-force per-head loops in float64 (golden fixture); permutation
                   weights pin the head split/merge order
  embed_front      brute-force gather + add
  argmax           NumPy semantics (first maximum, first NaN) on hand-made ties
  gpt_forward      brute-force float64 composition of the above at a tiny shape (golden
                   fixture)
  bf16 rounding    hand-computed bit patterns (ties to even, NaN, inf)
  philox4x32_10    the published known-answer vectors of Random123 (zero, all-ones and
                   pi-digit counters/keys)
  random_normal    moments of a large draw; Box-Muller radius/angle identities
  sample_uniforms  range [0, 1) on a 2^-24 grid; mean/variance of a large draw; word 0
                   of the KAT-pinned Philox (a wrong word or shift fails the grid check)
  sample_categorical  brute-force linear scan of the running sum at tiny sizes; one-hot
                   and zero-probability rows; empirical frequencies of 200000 draws match
                   p (chi-square); u = 0 and u just below 1 hit the first and last
                   nonzero entries
The reference itself was not imported or run: its files are pure Python over CuPy/NumPy
with no golden vectors, and every function above is pinned by the checks listed.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


# ---- bf16 (round to nearest even) -----------------------------------------------------
def bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even, NaN kept quiet."""
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + (0x7FFF + ((u >> 16) & 1))) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def from_bf16_bits(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def round_bf16(x) -> np.ndarray:
    """Value of float32 `x` after a round trip through bf16."""
    x = np.asarray(x, dtype=F32)
    return from_bf16_bits(bf16_bits(x)).reshape(x.shape)


def max_rel(got, ref) -> float:
    """Parity metric: max |got - ref| / max |ref| over the whole tensor."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.max(np.abs(ref)) if ref.size else 0.0
    if denom == 0:
        return float(np.max(np.abs(got - ref))) if ref.size else 0.0
    return float(np.max(np.abs(got - ref)) / denom)


# ---- activations (reference activations.py) -------------------------------------------
def gelu(x):
    """activations.py:24-28: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x**3)))."""
    x = np.asarray(x, dtype=F32)
    t = np.tanh((2 / np.pi) ** 0.5 * (x + 0.044715 * x ** 3))
    return 0.5 * x * (1 + t)


def silu(x):
    """activations.py:41-45: x * (1 + tanh(x/2)) / 2."""
    x = np.asarray(x, dtype=F32)
    return x * ((1 + np.tanh(x / 2)) / 2)


def softmax(x, temperature=F32(1.0)):
    """activations.py:57-64: exp((x - max)/T) / sum over the last axis."""
    x = np.asarray(x, dtype=F32)
    normalization = np.max(x, axis=-1, keepdims=True)
    exponent = np.exp((x - normalization) / temperature)
    return exponent / np.sum(exponent, axis=-1, keepdims=True)


def act(x, name):
    return {"gelu": gelu, "silu": silu}[name](x)


# ---- normalisation ---------------------------------------------------------------------
def layernorm(x, gamma, beta, eps=F32(1e-5)):
    """layers.py:415-428: population mean/var, std = (var + eps)**0.5, gamma*norm + beta."""
    x = np.asarray(x, dtype=F32)
    mean = np.mean(x, axis=-1, keepdims=True)
    var = np.var(x, axis=-1, keepdims=True)
    centered = x - mean
    std = (var + eps) ** F32(0.5)
    normed = centered / std
    return gamma * normed + beta


def rmsnorm(x, gamma, eps=F32(1e-6), gamma_offset=0.0):
    """RMSNorm (Zhang & Sennrich 2019): x / sqrt(mean(x^2) + eps) * (offset + gamma).
    No reference counterpart (layers.py:394 is a TODO); offset 1 is Gemma's convention."""
    x = np.asarray(x, dtype=F32)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return (x / np.sqrt(ms + F32(eps))) * (F32(gamma_offset) + gamma)


# ---- RoPE (Su et al. 2021, rotate-half pairing as in GPT-NeoX/Gemma) -------------------
def rope_table(seq_len, head_dim, base=10000.0, pos0=0):
    """cos/sin of (pos0 + t) * base^(-2i/D), evaluated in float64, stored as float32."""
    half = head_dim // 2
    i = np.arange(half, dtype=np.float64)
    inv_freq = base ** (-(2 * i) / head_dim)
    ang = (pos0 + np.arange(seq_len, dtype=np.float64))[:, None] * inv_freq[None, :]
    return np.cos(ang).astype(F32), np.sin(ang).astype(F32)


def rope(x, cos, sin):
    """x [..., T, D]: y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin, halves of the last axis."""
    x = np.asarray(x, dtype=F32)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1)


# ---- layers (reference layers.py) -------------------------------------------------------
def dense(x, w, b):
    """layers.py:206-209: x @ W + b."""
    return np.asarray(x, dtype=F32) @ w + b


def causal_mask(context_length):
    """layers.py:254-256: tril -> 0 on/below the diagonal, -1e9 above (float32)."""
    mask = np.tril(np.ones((context_length, context_length)))
    return np.where(mask == 0, -1e9, 0.0).astype(F32, copy=False)


def mha(x, wqkv, bqkv, wo, bo, num_heads, decoder=False, context_length=None, rnd=None):
    """layers.py:281-307 (dropout is the identity at inference, layers.py:231-232).
    `rnd` (optional) rounds the tensors the device materialises (bf16 pipeline)."""
    r = rnd or (lambda a: a)
    x = np.asarray(x, dtype=F32)
    B, T, C = x.shape
    D = C // num_heads
    qkv = r(x @ wqkv + bqkv)
    query, key_t, value = np.split(qkv, 3, axis=2)
    query = query.reshape((B, T, num_heads, D)).transpose(0, 2, 1, 3)
    key_t = key_t.reshape((B, T, num_heads, D)).transpose(0, 2, 3, 1)
    value = value.reshape((B, T, num_heads, D)).transpose(0, 2, 1, 3)
    attends = r((query @ key_t) / F32(D ** 0.5))
    if decoder:
        attends = attends + causal_mask(context_length or T)[:T, :T]
    normalization = np.max(attends, axis=-1, keepdims=True)
    exponent = np.exp(attends - normalization)
    probs = r(exponent / np.sum(exponent, axis=-1, keepdims=True))
    heads = r(probs @ value)
    heads = heads.transpose(0, 2, 1, 3).reshape(B, T, C)
    return heads @ wo + bo


def ffn(x, w1, b1, w2, b2, activation="gelu", rnd=None):
    """layers.py:369-375: act(x W1 + b1) W2 + b2."""
    r = rnd or (lambda a: a)
    h = r(act(np.asarray(x, dtype=F32) @ w1 + b1, activation))
    return h @ w2 + b2


def block(x, p, num_heads, activation="gelu", decoder=True, context_length=None, rnd=None):
    """layers.py:463-467: y = x + MHA(LN1 x); z = y + FFN(LN2 y).
    p = [g1, b1, Wqkv, bqkv, Wo, bo, g2, b2, W1, bb1, W2, bb2] (layers.py:458 order)."""
    r = rnd or (lambda a: a)
    g1, be1, wqkv, bqkv, wo, bo, g2, be2, w1, bb1, w2, bb2 = p
    y = r(x + mha(r(layernorm(x, g1, be1)), wqkv, bqkv, wo, bo, num_heads, decoder,
                  context_length, rnd))
    z = r(y + ffn(r(layernorm(y, g2, be2)), w1, bb1, w2, bb2, activation, rnd))
    return z


# ---- GPT adapters (reference transformer_adapters.py) ---------------------------------
def embed_front(ids, table, pos):
    """transformer_adapters.py:148-153: table[ids] + pos[:T]."""
    ids = np.asarray(ids)
    return table[ids] + pos[: ids.shape[1], :]


def sinusoidal_positions(context_length, embed_size):
    """transformer_adapters.py:128-135."""
    pos = np.arange(context_length)[:, None]
    i = np.arange(embed_size)[None, :]
    tab = pos / 10000 ** (2 * (i // 2) / embed_size)
    tab[:, 0::2] = np.sin(tab[:, 0::2])
    tab[:, 1::2] = np.cos(tab[:, 1::2])
    return tab.astype(F32, copy=False)


def embed_back(x, table):
    """transformer_adapters.py:174-177: logits = x @ table^T."""
    return np.asarray(x, dtype=F32) @ table.transpose()


def argmax(x):
    """network.py:135, 158: xp.argmax(y_hat, axis=-1) (NumPy: first max, first NaN)."""
    return np.argmax(x, axis=-1)


def vit_head(x, w, b):
    """transformer_adapters.py:89-95: x[:, 0, :] @ W + b."""
    return np.asarray(x, dtype=F32)[:, 0, :] @ w + b


# ---- GPT composition (reference demo.ipynb:1473-1501) ---------------------------------
def gpt_param_shapes(cfg):
    """Parameter shapes in `layer.parameters` order for the notebook GPT composition:
    GPTEmbedFront [pos, table] (transformer_adapters.py:138, 143), each TransformerBlock
    (layers.py:458 with 275-279, 362-366), the final LayerNorm [gamma, beta]."""
    V, T, C, L = cfg["vocab"], cfg["ctx"], cfg["d"], cfg["layers"]
    shapes = [("pos", (T, C)), ("table", (V, C))]
    for l in range(L):
        shapes += [(f"b{l}.g1", (C,)), (f"b{l}.be1", (C,)), (f"b{l}.wqkv", (C, 3 * C)),
                   (f"b{l}.bqkv", (3 * C,)), (f"b{l}.wo", (C, C)), (f"b{l}.bo", (C,)),
                   (f"b{l}.g2", (C,)), (f"b{l}.be2", (C,)), (f"b{l}.w1", (C, 4 * C)),
                   (f"b{l}.bb1", (4 * C,)), (f"b{l}.w2", (4 * C, C)), (f"b{l}.bb2", (C,))]
    shapes += [("lnf.g", (C,)), ("lnf.be", (C,))]
    return shapes


def gpt_params(cfg, seed, scale=0.02, bf16=False):
    """Seeded fill: N(0,1)*scale in parameter order from default_rng(seed); LayerNorm
    gammas get +1 so the affine part is exercised around the identity."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in gpt_param_shapes(cfg):
        a = rng.standard_normal(shape, dtype=F32) * F32(scale)
        if name.endswith(".g1") or name.endswith(".g2") or name == "lnf.g":
            a = a + F32(1.0)
        out[name] = round_bf16(a) if bf16 else a
    return out


def gpt_forward(ids, params, cfg, bf16=False, return_logits=False):
    """demo.ipynb:1473-1501: embed -> dropout(identity) -> L blocks -> LN -> tied head ->
    SoftMax. With bf16=True every tensor the device materialises is rounded to bf16."""
    rnd = round_bf16 if bf16 else None
    r = rnd or (lambda a: a)
    H, L = cfg["heads"], cfg["layers"]
    x = r(embed_front(ids, params["table"], params["pos"]))
    for l in range(L):
        p = [params[f"b{l}.{k}"] for k in ("g1", "be1", "wqkv", "bqkv", "wo", "bo", "g2", "be2",
                                          "w1", "bb1", "w2", "bb2")]
        x = block(x, p, H, cfg.get("act", "gelu"), True, cfg["ctx"], rnd)
    x = r(layernorm(x, params["lnf.g"], params["lnf.be"]))
    logits = r(embed_back(x, params["table"]))
    probs = r(softmax(logits))
    return (probs, logits) if return_logits else probs


# ---- Gemma-style decoder pieces (no reference counterpart) ------------------------------
def geglu_ffn(x, wg, wu, wd, activation="gelu", rnd=None):
    """Gated FFN (Shazeer 2020): (act(x Wg) * (x Wu)) Wd, no biases; act is the tanh GeLU
    of activations.py:24-28 (GeGLU) or SiLU (SwiGLU)."""
    r = rnd or (lambda a: a)
    x = np.asarray(x, dtype=F32)
    h = r(act(x @ wg, activation) * (x @ wu))
    return h @ wd


def mqa(x, wqkv, wo, num_heads, num_kv_heads, head_dim, pos0=0, rope_base=10000.0,
        past_k=None, past_v=None, rnd=None, use_rope=True):
    """Multi-/grouped-query causal attention with rotate-half RoPE (Shazeer 2019; Ainslie
    et al. 2023; Su et al. 2021). wqkv [C, (Hq + 2 Hkv) D] with columns [Q | K | V]; query
    head h reads key/value head h // (Hq / Hkv). x holds positions pos0 .. pos0 + T - 1;
    past_k/past_v [B, Hkv, pos0, D] are the rotated keys and values of earlier positions.
    Returns (y, k_all, v_all) with k_all/v_all [B, Hkv, pos0 + T, D]."""
    r = rnd or (lambda a: a)
    x = np.asarray(x, dtype=F32)
    B, T, C = x.shape
    Hq, Hkv, D = num_heads, num_kv_heads, head_dim
    if (past_k.shape[2] if past_k is not None else 0) != pos0:
        raise ValueError("pos0 must equal the number of cached positions")
    qkv = r(x @ wqkv)
    q = qkv[..., : Hq * D].reshape(B, T, Hq, D).transpose(0, 2, 1, 3)
    k = qkv[..., Hq * D: (Hq + Hkv) * D].reshape(B, T, Hkv, D).transpose(0, 2, 1, 3)
    v = qkv[..., (Hq + Hkv) * D:].reshape(B, T, Hkv, D).transpose(0, 2, 1, 3)
    if use_rope:
        cos, sin = rope_table(T, D, rope_base, pos0)
        q, k = r(rope(q, cos, sin)), r(rope(k, cos, sin))
    if past_k is not None:
        k = np.concatenate([past_k, k], axis=2)
        v = np.concatenate([past_v, v], axis=2)
    Tk = pos0 + T
    g = Hq // Hkv
    kk = np.repeat(k, g, axis=1)
    vv = np.repeat(v, g, axis=1)
    s = (q @ kk.transpose(0, 1, 3, 2)) / F32(D ** 0.5)
    qpos = pos0 + np.arange(T)[:, None]
    s = np.where(np.arange(Tk)[None, :] <= qpos, s, F32(-1e9)).astype(F32)
    s = s - np.max(s, axis=-1, keepdims=True)
    e = np.exp(s)
    p = e / np.sum(e, axis=-1, keepdims=True)
    heads = r(p @ vv).transpose(0, 2, 1, 3).reshape(B, T, Hq * D)
    return heads @ wo, k, v


def gemma_param_shapes(cfg):
    """Parameter shapes in GemmaDecoder layer order: table, then per block [attn-norm
    gamma, Wqkv, Wo, ffn-norm gamma, Wgate, Wup, Wdown], then the final-norm gamma."""
    V, C, L = cfg["vocab"], cfg["d"], cfg["layers"]
    Hq, Hkv, D, F = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["ffn"]
    shapes = [("table", (V, C))]
    for l in range(L):
        shapes += [(f"b{l}.g1", (C,)), (f"b{l}.wqkv", (C, (Hq + 2 * Hkv) * D)),
                   (f"b{l}.wo", (Hq * D, C)), (f"b{l}.g2", (C,)), (f"b{l}.wg", (C, F)),
                   (f"b{l}.wu", (C, F)), (f"b{l}.wd", (F, C))]
    shapes += [("normf.g", (C,))]
    return shapes


def gemma_params(cfg, seed, scale=0.02, bf16=False):
    """Seeded N(0,1)*scale in parameter order from default_rng(seed) (gammas included:
    RMSNorm scales by 1 + gamma)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in gemma_param_shapes(cfg):
        a = rng.standard_normal(shape, dtype=F32) * F32(scale)
        out[name] = round_bf16(a) if bf16 else a
    return out


def gemma_forward(ids, params, cfg, bf16=False, pos0=0, cache=None):
    """Logits [B, T, V] of the Gemma-style decoder for ids at positions pos0.. . `cache`
    (a dict filled in place, layer -> (k, v)) carries rotated keys/values between calls;
    None recomputes from scratch with pos0 = 0."""
    rnd = round_bf16 if bf16 else None
    r = rnd or (lambda a: a)
    ids = np.asarray(ids)
    C = cfg["d"]
    x = r(params["table"][ids] * np.sqrt(F32(C)))
    for l in range(cfg["layers"]):
        past = cache.get(l) if cache is not None else None
        h, k, v = mqa(r(rmsnorm(x, params[f"b{l}.g1"], F32(1e-6), 1.0)), params[f"b{l}.wqkv"],
                      params[f"b{l}.wo"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"], pos0,
                      cfg.get("rope_base", 10000.0), *(past or (None, None)), rnd=rnd)
        if cache is not None:
            cache[l] = (k, v)
        y = r(x + h)
        x = r(y + geglu_ffn(r(rmsnorm(y, params[f"b{l}.g2"], F32(1e-6), 1.0)), params[f"b{l}.wg"],
                            params[f"b{l}.wu"], params[f"b{l}.wd"], "gelu", rnd))
    x = r(rmsnorm(x, params["normf.g"], F32(1e-6), 1.0))
    return r(embed_back(x, params["table"]))


def gemma_greedy(ids, params, cfg, n_new, bf16=False):
    """Greedy decoding by recomputation (the reference's generate loop, demo.ipynb:1526-1533,
    with argmax in place of sampling): each step reruns the whole sequence and appends
    argmax of the last logits row. Returns (new ids [B, n_new], last-row logits
    [n_new, B, V])."""
    seq = np.asarray(ids)
    new, rows = [], []
    for _ in range(n_new):
        logits = gemma_forward(seq, params, cfg, bf16)
        last = logits[:, -1, :]
        nxt = argmax(last)
        new.append(nxt)
        rows.append(last)
        seq = np.concatenate([seq, nxt[:, None]], axis=1)
    return np.stack(new, axis=1), np.stack(rows)


# ---- device random numbers (Philox4x32-10 + Box-Muller) --------------------------------
def philox4x32_10(ctr, key):
    """Philox4x32-10 (Salmon et al., SC 2011). ctr uint32 [..., 4], key uint32 [2] ->
    uint32 [..., 4]. Each round: (lo0, hi0) = M0 * c0, (lo1, hi1) = M1 * c2,
    c = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0); then the key is bumped by the Weyl
    constants."""
    mask = np.uint64(0xFFFFFFFF)
    ctr = np.asarray(ctr, dtype=np.uint64)
    c = [ctr[..., i] for i in range(4)]
    k0, k1 = np.uint64(int(key[0])), np.uint64(int(key[1]))
    m0, m1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
    for _ in range(10):
        p0, p1 = m0 * c[0], m1 * c[2]
        c = [((p1 >> np.uint64(32)) ^ c[1] ^ k0) & mask, p1 & mask,
             ((p0 >> np.uint64(32)) ^ c[3] ^ k1) & mask, p0 & mask]
        k0 = (k0 + np.uint64(0x9E3779B9)) & mask
        k1 = (k1 + np.uint64(0xBB67AE85)) & mask
    return np.stack(c, axis=-1).astype(np.uint32)


def random_normal(n, seed, stream=0, mean=0.0, std=1.0):
    """Element e: Philox counter (e // 4 as two words, stream as two words), key = seed;
    Box-Muller on output words (0, 1) and (2, 3) with 24-bit uniforms
    u1 = (w >> 8 + 1) 2^-24, u2 = (w >> 8) 2^-24. Evaluated in float64, returned float32."""
    g = np.arange((n + 3) // 4, dtype=np.uint64)
    ctr = np.stack([g & np.uint64(0xFFFFFFFF), g >> np.uint64(32),
                    np.full_like(g, stream & 0xFFFFFFFF), np.full_like(g, stream >> 32)], -1)
    w = philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32)).astype(np.float64)
    out = np.empty((g.size, 4))
    for a, b in ((0, 1), (2, 3)):
        u1 = (np.floor(w[:, a] / 256) + 1) * 2.0 ** -24
        u2 = np.floor(w[:, b] / 256) * 2.0 ** -24
        r = np.sqrt(-2 * np.log(u1))
        out[:, a] = r * np.cos(2 * np.pi * u2)
        out[:, b] = r * np.sin(2 * np.pi * u2)
    return (mean + std * out.reshape(-1)[:n]).astype(F32)


def sample_uniforms(n, seed, stream=0):
    """The uniforms of tl_sample: draw j takes u = (w0 >> 8) 2^-24 in [0, 1) from Philox
    counter (j, 0, stream) under key seed. Evaluated in float64."""
    j = np.arange(n, dtype=np.uint64)
    ctr = np.stack([j & np.uint64(0xFFFFFFFF), j >> np.uint64(32),
                    np.full_like(j, stream & 0xFFFFFFFF), np.full_like(j, stream >> 32)], -1)
    w = philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))
    return np.floor(w[:, 0].astype(np.float64) / 256) * 2.0 ** -24


def sample_categorical(p, u):
    """xp.random.choice(a, p=p) (reference demo.ipynb:1531). The reference's runtime is CuPy
    (backend.py:12-18, no version pinned in the repository), whose documented choice draws
    a uniform u in [0, 1) per sample and returns cdf.searchsorted(u, side='right') for
    cdf = cumsum(p) / sum(p). Same rule here with the caller's uniforms (the device's Philox
    stream, sample_uniforms): index = number of running sums <= u * sum(p), clamped to the
    last index; float64 sums. Returns (indices, u * sum(p), cdf) so a test can tell
    draws that land within rounding of a boundary."""
    cdf = np.cumsum(np.asarray(p, dtype=np.float64))
    x = np.asarray(u, dtype=np.float64) * cdf[-1]
    idx = np.minimum(np.searchsorted(cdf, x, side="right"), cdf.size - 1)
    return idx.astype(np.int64), x, cdf


# ---- ViT (reference transformer_adapters.py:6-95, demo.ipynb cell 8) ----------------
def patchify(x, patch):
    """transformer_adapters.py:39-47: [B, C, H, W] -> reshape [B, C, H/p0, p0, W/p1, p1],
    transpose (0, 2, 4, 3, 5, 1), reshape [B, L, p0 p1 C]."""
    x = np.asarray(x)
    B, C, H, W = x.shape
    p0, p1 = patch
    r = x.reshape(B, C, H // p0, p0, W // p1, p1).transpose(0, 2, 4, 3, 5, 1)
    return r.reshape(B, (H // p0) * (W // p1), p0 * p1 * C)


def vit_projector(x, proj, cls_reg, pos, patch):
    """transformer_adapters.py:49-55: tokens @ projection (no bias), class/register tokens
    tiled over the batch and prepended, plus the positional table."""
    tokens = patchify(np.asarray(x, dtype=F32), patch)
    emb = tokens @ proj
    B = emb.shape[0]
    cls = np.broadcast_to(cls_reg, (B,) + cls_reg.shape)
    return np.concatenate([cls, emb], axis=1) + pos


def vit_param_shapes(cfg):
    """Parameter shapes in layer order: VitProjector [projection, cls_reg_tokens, positions]
    (transformer_adapters.py:29-31), the encoder blocks, the final LayerNorm, the head
    (VitMLPHead [W, b], then Dense [W, b] when the head has a hidden layer)."""
    C, H, W = cfg["image"]
    p0, p1 = cfg["patch"]
    d, R = cfg["d"], 1 + cfg.get("registers", 0)
    L = (H // p0) * (W // p1)
    shapes = [("proj", (p0 * p1 * C, d)), ("cls", (R, d)), ("pos", (R + L, d))]
    for l in range(cfg["layers"]):
        shapes += [(f"b{l}.g1", (d,)), (f"b{l}.be1", (d,)), (f"b{l}.wqkv", (d, 3 * d)),
                   (f"b{l}.bqkv", (3 * d,)), (f"b{l}.wo", (d, d)), (f"b{l}.bo", (d,)),
                   (f"b{l}.g2", (d,)), (f"b{l}.be2", (d,)), (f"b{l}.w1", (d, 4 * d)),
                   (f"b{l}.bb1", (4 * d,)), (f"b{l}.w2", (4 * d, d)), (f"b{l}.bb2", (d,))]
    shapes += [("lnf.g", (d,)), ("lnf.be", (d,))]
    hidden = cfg.get("head_hidden")
    if hidden:
        shapes += [("head.w", (d, hidden)), ("head.b", (hidden,)),
                   ("dense.w", (hidden, cfg["classes"])), ("dense.b", (cfg["classes"],))]
    else:
        shapes += [("head.w", (d, cfg["classes"])), ("head.b", (cfg["classes"],))]
    return shapes


def vit_params(cfg, seed, scale=0.02, bf16=False):
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in vit_param_shapes(cfg):
        a = rng.standard_normal(shape, dtype=F32) * F32(scale)
        if name.endswith(".g1") or name.endswith(".g2") or name == "lnf.g":
            a = a + F32(1.0)
        out[name] = round_bf16(a) if bf16 else a
    return out


def vit_forward(x, params, cfg, bf16=False, return_logits=False):
    """demo.ipynb cell 8 composition: projector -> encoder blocks (no mask) -> LayerNorm ->
    class-token head (-> SiLU -> Dense when the head has a hidden layer) -> SoftMax. With
    return_logits, also the class scores the SoftMax reads."""
    rnd = round_bf16 if bf16 else None
    r = rnd or (lambda a: a)
    x = r(np.asarray(x, dtype=F32))
    h = r(vit_projector(x, params["proj"], params["cls"], params["pos"], cfg["patch"]))
    for l in range(cfg["layers"]):
        p = [params[f"b{l}.{k}"] for k in ("g1", "be1", "wqkv", "bqkv", "wo", "bo", "g2", "be2",
                                          "w1", "bb1", "w2", "bb2")]
        h = block(h, p, cfg["heads"], cfg.get("act", "gelu"), False, None, rnd)
    h = r(layernorm(h, params["lnf.g"], params["lnf.be"]))
    y = r(vit_head(h, params["head.w"], params["head.b"]))
    if cfg.get("head_hidden"):
        y = r(silu(y))
        y = r(dense(y, params["dense.w"], params["dense.b"]))
    probs = r(softmax(y))
    return (probs, y) if return_logits else probs
