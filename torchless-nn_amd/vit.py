"""ViT classifier compositions (reference demo.ipynb cell 8, demo.ipynb:1183-1216) and
seeded weights.

build_vit() assembles VitProjector, encoder TransformerBlocks (no causal mask), a final
LayerNorm and the class-token head as a Network on the MI355X runtime. With `head_hidden`
the head is the notebook's VitMLPHead(d, hidden) -> SiLU -> Dropout -> Dense(hidden,
classes); without it, VitMLPHead(d, classes) directly (the BASELINE config 4 head). A
SoftMax ends both. seed_vit() overwrites every parameter in `layer.parameters` order with
N(0,1)*scale from default_rng(seed) (LayerNorm gammas get +1), as gpt.seed_parameters does.
"""
import numpy as np

import backend
from activations import GeLU, SiLU, SoftMax
from layers import Dense, Dropout, LayerNorm, TransformerBlock
from network import Network
from transformer_adapters import VitMLPHead, VitProjector

__all__ = ["VIT_S4", "NOTEBOOK_VIT", "build_vit", "seed_vit"]

# ViT-S/4 on 32x32x3 images, 64 patches + CLS, 8 layers, d 384, 6 heads,
# MLP 1536 GeLU, 10 classes
VIT_S4 = dict(image=(3, 32, 32), patch=(4, 4), d=384, heads=6, layers=8, act="gelu",
              registers=0, classes=10, head_hidden=None, dropout=0.0)
# the notebook's CIFAR-10 model (demo.ipynb cell 8): patch 2, 4 register tokens, 12 blocks
NOTEBOOK_VIT = dict(image=(3, 32, 32), patch=(2, 2), d=256, heads=4, layers=12, act="silu",
                    registers=4, classes=10, head_hidden=256, dropout=0.1)

_ACTS = {"gelu": GeLU, "silu": SiLU}


def build_vit(cfg, dtype=None):
    if dtype is not None:
        backend.set_float_type(dtype)
    d, rate = cfg["d"], cfg.get("dropout", 0.0)
    layers = [VitProjector(tuple(cfg["image"]), tuple(cfg["patch"]), d,
                           num_registers=cfg.get("registers", 0))]
    for _ in range(cfg["layers"]):
        layers.append(TransformerBlock(d, 0, cfg["heads"], _ACTS[cfg.get("act", "gelu")],
                                       decoder=False, attn_dropout_rate=rate,
                                       res_dropout_rate=rate))
    layers.append(LayerNorm(d))
    hidden = cfg.get("head_hidden")
    if hidden:
        layers += [VitMLPHead(d, hidden), SiLU(), Dropout(rate), Dense(hidden, cfg["classes"])]
    else:
        layers.append(VitMLPHead(d, cfg["classes"]))
    layers.append(SoftMax())
    net = Network(layers)
    net.set_eval(True)
    return net


def seed_vit(net, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    for layer in net.layers:
        subs = [layer.pre_attn_norm, layer.pre_ffn_norm] if isinstance(layer, TransformerBlock) else [layer]
        gammas = {id(s.gamma) for s in subs if isinstance(s, LayerNorm)}
        for p in layer.parameters:
            a = rng.standard_normal(p.shape, dtype=np.float32) * np.float32(scale)
            if id(p) in gammas:
                a = a + np.float32(1.0)
            p.set(a)
    return net
