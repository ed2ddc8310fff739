"""The notebook GPT composition (reference demo.ipynb:1473-1501) and seeded weights.

build_gpt() assembles the same layer list as the reference's `GPT` class -- embedding
front, embedding dropout, L decoder TransformerBlocks, final LayerNorm, tied GPTEmbedBack,
SoftMax -- as a Network on the MI355X runtime. seed_parameters() overwrites every parameter,
in `layer.parameters` order, with N(0,1)*scale from default_rng(seed) (LayerNorm gammas get
+1), so runs are reproducible (the reference's own initialisation is unseeded,
backend.py:28).
"""
import numpy as np

import backend
import tl_hip as xp
from activations import GeLU, SiLU, SoftMax
from layers import Dropout, LayerNorm, TransformerBlock
from network import Network
from transformer_adapters import GPTEmbeddingTable, GPTEmbedFront, GPTEmbedBack

__all__ = ["build_gpt", "seed_parameters", "GPT_SMALL", "CHAR_GPT"]

# BASELINE configurations (model shapes only; batch and sequence length are inputs)
CHAR_GPT = dict(vocab=65, ctx=128, layers=4, d=128, heads=4, act="gelu")
GPT_SMALL = dict(vocab=50257, ctx=1024, layers=12, d=768, heads=12, act="gelu")

_ACTS = {"gelu": GeLU, "silu": SiLU}


def build_gpt(cfg, dtype=None):
    """Returns (network, embedding_table) for cfg = dict(vocab, ctx, layers, d, heads, act)."""
    if dtype is not None:
        backend.set_float_type(dtype)
    table = GPTEmbeddingTable(cfg["vocab"], cfg["d"])
    layers = [GPTEmbedFront(table, cfg["ctx"]), Dropout(0.0)]
    for _ in range(cfg["layers"]):
        layers.append(TransformerBlock(cfg["d"], cfg["ctx"], cfg["heads"], _ACTS[cfg.get("act", "gelu")],
                                       decoder=True))
    layers += [LayerNorm(cfg["d"]), GPTEmbedBack(table), SoftMax()]
    net = Network(layers)
    net.set_eval(True)
    return net, table


def seed_parameters(net, seed, scale=0.02):
    """Overwrite all parameters in order with seeded N(0,1)*scale (+1 on LayerNorm gamma)."""
    rng = np.random.default_rng(seed)
    for layer in net.layers:
        gammas = set()
        subs = [layer]
        if isinstance(layer, TransformerBlock):
            subs = [layer.pre_attn_norm, layer.pre_ffn_norm]
        for s in subs:
            if isinstance(s, LayerNorm):
                gammas.add(id(s.gamma))
        for p in layer.parameters:
            a = rng.standard_normal(p.shape, dtype=np.float32) * np.float32(scale)
            if id(p) in gammas:
                a = a + np.float32(1.0)
            p.set(a)
    return net
