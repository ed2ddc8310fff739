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


def softmax_row(s, lim=None):
    lim = len(s) if lim is None else lim
    m = max(s[:lim])
    e = [math.exp(s[j] - m) if j < lim else 0.0 for j in range(len(s))]
    t = sum(e)
    return [v / t for v in e]


def attention(x, wqkv, bqkv, wo, bo, H):
    """reference layers.py:286-306 with the decoder mask (layers.py:254-256, 296)."""
    T, C = len(x), len(x[0])
    D = C // H
    qkv = [matvec(x[t], wqkv, bqkv) for t in range(T)]
    heads = [[0.0] * C for _ in range(T)]
    for h in range(H):
        for i in range(T):
            s = [sum(qkv[i][h * D + d] * qkv[j][C + h * D + d] for d in range(D)) / math.sqrt(D)
                 for j in range(T)]
            p = softmax_row(s, i + 1)
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
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
