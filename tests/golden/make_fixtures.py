"""Writes the golden fixtures in this directory.

The expected outputs come from brute-force float64 loops written here from the reference's
definitions (cited per function), independently of oracle/numpy_ref.py, so the fixtures pin
both the oracle (CPU tests) and the HIP path (GPU tests). Inputs are seeded. The reference
itself is not imported. Run from the repository root:

    python tests/golden/make_fixtures.py
"""
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32 = np.float32


def ln_rows(x, g, b, eps=1e-5):
    """reference layers.py:419-427 (population variance, eps inside the square root)."""
    out = []
    for row in x:
        n = len(row)
        mu = sum(row) / n
        var = sum((v - mu) ** 2 for v in row) / n
        out.append([(row[c] - mu) / math.sqrt(var + eps) * g[c] + b[c] for c in range(n)])
    return out


def gelu(v):
    """reference activations.py:24-28."""
    return 0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))


def matvec(row, w, bias=None):
    """row (len K) times w (K x N nested lists) plus bias."""
    n = len(w[0])
    out = [sum(row[k] * w[k][j] for k in range(len(row))) for j in range(n)]
    if bias is not None:
        out = [out[j] + bias[j] for j in range(n)]
    return out


def silu(v):
    """reference activations.py:41-45, x (1 + tanh(x/2)) / 2, written here in its logistic
    form x / (1 + exp(-x)) (the same function: (1 + tanh(x/2)) / 2 = 1 / (1 + exp(-x)))."""
    if v < -700:
        return 0.0
    return v / (1.0 + math.exp(-v))


def softmax_row(s, lim=None):
    lim = len(s) if lim is None else lim
    m = max(s[:lim])
    e = [math.exp(s[j] - m) if j < lim else 0.0 for j in range(len(s))]
    t = sum(e)
    return [v / t for v in e]


def attention(x, wqkv, bqkv, wo, bo, H, causal=True):
    """reference layers.py:286-306; with `causal` the decoder mask (layers.py:254-256, 296),
    without it every query attends to every key (the ViT encoder, decoder=False)."""
    T, C = len(x), len(x[0])
    D = C // H
    qkv = [matvec(x[t], wqkv, bqkv) for t in range(T)]
    heads = [[0.0] * C for _ in range(T)]
    for h in range(H):
        for i in range(T):
            s = [sum(qkv[i][h * D + d] * qkv[j][C + h * D + d] for d in range(D)) / math.sqrt(D)
                 for j in range(T)]
            p = softmax_row(s, i + 1 if causal else T)
            for d in range(D):
                heads[i][h * D + d] = sum(p[j] * qkv[j][2 * C + h * D + d] for j in range(T))
    return [matvec(heads[t], wo, bo) for t in range(T)]


def gpt_brute(ids, P, cfg):
    """demo.ipynb:1473-1501 composition: embed + positions, L pre-LN blocks, LN, tied head,
    softmax."""
    C, H, L = cfg["d"], cfg["heads"], cfg["layers"]
    logits_all, probs_all = [], []
    for seq in ids:
        x = [[P["table"][tok][c] + P["pos"][t][c] for c in range(C)] for t, tok in enumerate(seq)]
        for l in range(L):
            g = lambda k: P[f"b{l}.{k}"]
            a = attention(ln_rows(x, g("g1"), g("be1")), g("wqkv"), g("bqkv"), g("wo"), g("bo"), H)
            y = [[x[t][c] + a[t][c] for c in range(C)] for t in range(len(x))]
            h = [[gelu(v) for v in matvec(r, g("w1"), g("bb1"))] for r in ln_rows(y, g("g2"), g("be2"))]
            f = [matvec(r, g("w2"), g("bb2")) for r in h]
            x = [[y[t][c] + f[t][c] for c in range(C)] for t in range(len(y))]
        x = ln_rows(x, P["lnf.g"], P["lnf.be"])
        lg = [[sum(r[c] * P["table"][v][c] for c in range(C)) for v in range(cfg["vocab"])] for r in x]
        logits_all.append(lg)
        probs_all.append([softmax_row(r) for r in lg])
    return np.array(logits_all), np.array(probs_all)


def gpt_params(cfg, seed, scale=0.02):
    """Seeded fill in layer.parameters order (reference transformer_adapters.py:138, 143;
    layers.py:458): N(0,1)*scale, +1 on LayerNorm gammas."""
    V, T, C, L = cfg["vocab"], cfg["ctx"], cfg["d"], cfg["layers"]
    shapes = [("pos", (T, C)), ("table", (V, C))]
    for l in range(L):
        shapes += [(f"b{l}.g1", (C,)), (f"b{l}.be1", (C,)), (f"b{l}.wqkv", (C, 3 * C)),
                   (f"b{l}.bqkv", (3 * C,)), (f"b{l}.wo", (C, C)), (f"b{l}.bo", (C,)),
                   (f"b{l}.g2", (C,)), (f"b{l}.be2", (C,)), (f"b{l}.w1", (C, 4 * C)),
                   (f"b{l}.bb1", (4 * C,)), (f"b{l}.w2", (4 * C, C)), (f"b{l}.bb2", (C,))]
    shapes += [("lnf.g", (C,)), ("lnf.be", (C,))]
    rng = np.random.default_rng(seed)
    P = {}
    for name, shape in shapes:
        a = rng.standard_normal(shape, dtype=F32) * F32(scale)
        if name.endswith(".g1") or name.endswith(".g2") or name == "lnf.g":
            a = a + F32(1.0)
        P[name] = a
    return P


VIT_BLOCK_KEYS = ("g1", "be1", "wqkv", "bqkv", "wo", "bo", "g2", "be2", "w1", "bb1", "w2", "bb2")


def vit_params(cfg, seed, scale):
    """Seeded fill in layer.parameters order: VitProjector [projection, cls_reg_tokens,
    positional_embeddings] (reference transformer_adapters.py:25-31), the encoder blocks
    (layers.py:458), the final LayerNorm, VitMLPHead [W, b] (transformer_adapters.py:80-86)
    and the head's Dense [W, b] (layers.py:200-204). N(0,1)*scale, +1 on LayerNorm gammas.
    Returns the names in order and the arrays."""
    C, H, W = cfg["image"]
    p0, p1 = cfg["patch"]
    d, R, F = cfg["d"], 1 + cfg["registers"], cfg["head_hidden"]
    L = (H // p0) * (W // p1)
    shapes = [("proj", (p0 * p1 * C, d)), ("cls", (R, d)), ("pos", (R + L, d))]
    for l in range(cfg["layers"]):
        shapes += [(f"b{l}.{k}", s) for k, s in zip(VIT_BLOCK_KEYS, [
            (d,), (d,), (d, 3 * d), (3 * d,), (d, d), (d,), (d,), (d,), (d, 4 * d), (4 * d,),
            (4 * d, d), (d,)])]
    shapes += [("lnf.g", (d,)), ("lnf.be", (d,)), ("head.w", (d, F)), ("head.b", (F,)),
               ("dense.w", (F, cfg["classes"])), ("dense.b", (cfg["classes"],))]
    rng = np.random.default_rng(seed)
    P = {}
    for name, shape in shapes:
        a = rng.standard_normal(shape, dtype=F32) * F32(scale)
        if name.endswith(".g1") or name.endswith(".g2") or name == "lnf.g":
            a = a + F32(1.0)
        P[name] = a
    return [n for n, _ in shapes], P


def vit_brute(images, P, cfg):
    """The notebook ViT classifier (demo.ipynb cell 8) in float64 loops: patch tokens in the
    order of reference transformer_adapters.py:39-47 (token i * (W/p1) + j, feature
    (row in patch * p1 + column in patch) * C + channel), projection without bias (:49),
    class/register rows first (:51-52), positions added (:54), encoder blocks without a
    mask (layers.py:463-467), final LayerNorm, VitMLPHead on token 0 (:89-95), SiLU, Dense
    (layers.py:206-209), softmax. Returns (head output, class logits, probabilities)."""
    C, H, W = cfg["image"]
    p0, p1 = cfg["patch"]
    nh, nw = H // p0, W // p1
    R, heads = 1 + cfg["registers"], cfg["heads"]
    head_all, logits_all, probs_all = [], [], []
    for img in images:
        toks = []
        for i in range(nh):
            for j in range(nw):
                toks.append([img[ch][i * p0 + a][j * p1 + b]
                             for a in range(p0) for b in range(p1) for ch in range(C)])
        rows = [list(P["cls"][r]) for r in range(R)] + [matvec(t, P["proj"]) for t in toks]
        x = [[v + P["pos"][t][c] for c, v in enumerate(row)] for t, row in enumerate(rows)]
        for l in range(cfg["layers"]):
            g = lambda k: P[f"b{l}.{k}"]
            a = attention(ln_rows(x, g("g1"), g("be1")), g("wqkv"), g("bqkv"), g("wo"), g("bo"),
                          heads, causal=False)
            y = [[x[t][c] + a[t][c] for c in range(len(x[0]))] for t in range(len(x))]
            h = [[silu(v) for v in matvec(r, g("w1"), g("bb1"))] for r in ln_rows(y, g("g2"), g("be2"))]
            f = [matvec(r, g("w2"), g("bb2")) for r in h]
            x = [[y[t][c] + f[t][c] for c in range(len(y[0]))] for t in range(len(y))]
        x = ln_rows(x, P["lnf.g"], P["lnf.be"])
        hd = matvec(x[0], P["head.w"], P["head.b"])
        lg = matvec([silu(v) for v in hd], P["dense.w"], P["dense.b"])
        head_all.append(hd)
        logits_all.append(lg)
        probs_all.append(softmax_row(lg))
    return np.array(head_all), np.array(logits_all), np.array(probs_all)


# ---- Gemma-style decoder (BASELINE config 5's architecture; no reference counterpart) ----
GEMMA_BLOCK_KEYS = ("g1", "wqkv", "wo", "g2", "wg", "wu", "wd")


def rms_rows(x, g, eps=1e-6):
    """RMSNorm (Zhang & Sennrich 2019) with Gemma's (1 + gamma) gain and eps 1e-6:
    x / sqrt(mean(x^2) + eps) * (1 + gamma[c])."""
    out = []
    for row in x:
        inv = 1.0 / math.sqrt(sum(v * v for v in row) / len(row) + eps)
        out.append([row[c] * inv * (1.0 + g[c]) for c in range(len(row))])
    return out


def rope_vec(v, pos, base):
    """Rotary position embedding, rotate-half pairing (Su et al. 2021, as Gemma pairs it):
    element i and element i + D/2 form one 2-vector, rotated by the angle
    pos * base^(-2i/D)."""
    D = len(v)
    h = D // 2
    out = list(v)
    for i in range(h):
        ang = pos * base ** (-2.0 * i / D)
        c, s = math.cos(ang), math.sin(ang)
        out[i] = v[i] * c - v[i + h] * s
        out[i + h] = v[i + h] * c + v[i] * s
    return out


def gemma_params(cfg, seed, scale):
    """Seeded fill in the decoder's layer order: the tied table [V, C], then per block [norm-1
    gain [C], Wqkv [C, (Hq + 2 Hkv) D] with columns [Q | K | V], Wo [Hq D, C], norm-2 gain
    [C], Wgate [C, F], Wup [C, F], Wdown [F, C]], then the final-norm gain [C]. N(0,1)*scale
    for every tensor, gains included (they scale by 1 + gain)."""
    V, C, L, F = cfg["vocab"], cfg["d"], cfg["layers"], cfg["ffn"]
    Hq, Hkv, D = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    shapes = [("table", (V, C))]
    for l in range(L):
        shapes += [(f"b{l}.{k}", s) for k, s in zip(GEMMA_BLOCK_KEYS, [
            (C,), (C, (Hq + 2 * Hkv) * D), (Hq * D, C), (C,), (C, F), (C, F), (F, C)])]
    shapes += [("normf.g", (C,))]
    rng = np.random.default_rng(seed)
    P = {n: rng.standard_normal(s, dtype=F32) * F32(scale) for n, s in shapes}
    return [n for n, _ in shapes], P


def gemma_brute(ids, P, cfg):
    """The Gemma-style decoder in float64 loops, per sequence: embedding row times sqrt(C);
    L pre-norm blocks, each x + Wo(attention(RoPE(q), RoPE(k), v) of RMSNorm(x)) then
    y + Wdown(gelu(RMSNorm(y) Wgate) * (RMSNorm(y) Wup)); query head h reads key/value head
    h // (Hq / Hkv); queries AND keys rotated at their absolute positions 0..T-1; causal
    softmax of q.k / sqrt(D); no biases; final RMSNorm; tied head logits = x . table[v].
    The GeLU is the reference's tanh form (activations.py:24-28); the causal rows are those
    of layers.py:293-304."""
    C, Hq, Hkv, D, L = cfg["d"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["layers"]
    base, grp = cfg["rope_base"], Hq // Hkv
    out = []
    for seq in ids:
        T = len(seq)
        x = [[P["table"][tok][c] * math.sqrt(C) for c in range(C)] for tok in seq]
        for l in range(L):
            g = lambda k: P[f"b{l}.{k}"]
            qkv = [matvec(r, g("wqkv")) for r in rms_rows(x, g("g1"))]
            q = [[rope_vec(qkv[t][h * D:(h + 1) * D], t, base) for h in range(Hq)]
                 for t in range(T)]
            k = [[rope_vec(qkv[t][(Hq + j) * D:(Hq + j + 1) * D], t, base) for j in range(Hkv)]
                 for t in range(T)]
            v = [[qkv[t][(Hq + Hkv + j) * D:(Hq + Hkv + j + 1) * D] for j in range(Hkv)]
                 for t in range(T)]
            heads = [[0.0] * (Hq * D) for _ in range(T)]
            for h in range(Hq):
                j = h // grp
                for i in range(T):
                    s = [sum(q[i][h][d] * k[t][j][d] for d in range(D)) / math.sqrt(D)
                         for t in range(i + 1)]
                    p = softmax_row(s)
                    for d in range(D):
                        heads[i][h * D + d] = sum(p[t] * v[t][j][d] for t in range(i + 1))
            a = [matvec(r, g("wo")) for r in heads]
            y = [[x[t][c] + a[t][c] for c in range(C)] for t in range(T)]
            yn = rms_rows(y, g("g2"))
            hid = [[gelu(gv) * uv for gv, uv in zip(matvec(r, g("wg")), matvec(r, g("wu")))]
                   for r in yn]
            f = [matvec(r, g("wd")) for r in hid]
            x = [[y[t][c] + f[t][c] for c in range(C)] for t in range(T)]
        x = rms_rows(x, P["normf.g"])
        out.append([[sum(r[c] * P["table"][w][c] for c in range(C)) for w in range(cfg["vocab"])]
                    for r in x])
    return np.array(out)


def main():
    # tiny GPT: scale 0.5 so that attention and GeLU are far from linear
    cfg = dict(vocab=11, ctx=6, layers=2, d=8, heads=2, act="gelu")
    P = gpt_params(cfg, seed=7, scale=0.5)
    ids = np.random.default_rng(8).integers(0, cfg["vocab"], (2, 5))
    Pl = {k: v.astype(np.float64).tolist() for k, v in P.items()}
    logits, probs = gpt_brute(ids.tolist(), Pl, cfg)
    np.savez(os.path.join(HERE, "gpt_tiny.npz"), ids=ids.astype(np.int64),
             logits=logits, probs=probs, **{"cfg_" + k: np.array(v) for k, v in cfg.items()},
             **{"p_" + k: v for k, v in P.items()})

    # LayerNorm rows with a non-trivial affine part
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((6, 40)) * 3 + 2).astype(F32)
    g = rng.standard_normal(40).astype(F32)
    b = rng.standard_normal(40).astype(F32)
    y = np.array(ln_rows(x.astype(np.float64).tolist(), g.tolist(), b.tolist()))
    np.savez(os.path.join(HERE, "layernorm_small.npz"), x=x, gamma=g, beta=b, y=y)

    # causal softmax of a [2, 7, 7] score block (rows attend to columns <= row index)
    s = (rng.standard_normal((2, 7, 7)) * 3).astype(F32)
    p = np.array([[softmax_row(row.tolist(), i + 1) for i, row in enumerate(blk)]
                  for blk in s.astype(np.float64)])
    np.savez(os.path.join(HERE, "softmax_causal_small.npz"), scores=s, probs=p)

    # tiny notebook-style ViT: non-square patches of a non-square image (so a transposed
    # patch order fails), one register token, SiLU encoder, hidden SiLU head
    vcfg = dict(image=(3, 4, 6), patch=(2, 3), d=8, heads=2, layers=2, act="silu",
                registers=1, classes=5, head_hidden=6)
    names, VP = vit_params(vcfg, seed=11, scale=0.5)
    imgs = np.random.default_rng(12).standard_normal((3,) + vcfg["image"]).astype(F32)
    head, logits, probs = vit_brute(imgs.astype(np.float64).tolist(),
                                    {k: v.astype(np.float64).tolist() for k, v in VP.items()}, vcfg)
    np.savez(os.path.join(HERE, "vit_tiny.npz"), images=imgs, head=head, logits=logits,
             probs=probs, param_order=np.array(names),
             **{"cfg_" + k: np.array(v) for k, v in vcfg.items()},
             **{"p_" + k: v for k, v in VP.items()})
    # tiny Gemma-style decoder: 4 query heads sharing one key/value head, head width 32,
    # GeGLU, (1 + gain) RMSNorms; scale 0.3 so that the gains, RoPE and GeGLU all matter;
    # 12 positions, so a cached run (prefill 7, then 1, then 4 at positions 7.. and 8..)
    # reads its rows from the same logits
    gcfg = dict(vocab=97, ctx=64, layers=2, d=64, heads=4, kv_heads=1, head_dim=32, ffn=96,
                rope_base=10000.0)
    gnames, GP = gemma_params(gcfg, seed=13, scale=0.3)
    gids = np.random.default_rng(14).integers(0, gcfg["vocab"], (2, 12))
    glogits = gemma_brute(gids.tolist(), {k: v.astype(np.float64).tolist() for k, v in GP.items()},
                          gcfg)
    np.savez(os.path.join(HERE, "gemma_tiny.npz"), ids=gids.astype(np.int64), logits=glogits,
             param_order=np.array(gnames), **{"cfg_" + k: np.array(v) for k, v in gcfg.items()},
             **{"p_" + k: v for k, v in GP.items()})
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
