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
from layers import Dropout, KVCache, LayerNorm, TransformerBlock
from network import Network
from transformer_adapters import GPTEmbeddingTable, GPTEmbedFront, GPTEmbedBack

__all__ = ["build_gpt", "seed_parameters", "GPT_SMALL", "CHAR_GPT", "new_cache",
           "forward_cached", "generate", "generate_window"]

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


# ---- generation -----------------------------------------------------------------------
def _blocks(net):
    return [layer for layer in net.layers if isinstance(layer, TransformerBlock)]


def new_cache(net, batch, capacity):
    """A KV cache for every decoder block of `net` (keys/values of `capacity` positions)."""
    blocks = _blocks(net)
    attn = blocks[0].attn_block
    return KVCache(len(blocks), batch, attn.num_heads, capacity, attn.heads_dim,
                   net.layers[0].embedding_table.table.dtype)


def forward_cached(net, ids, cache, pos0, last_only=False):
    """The network's layers over ids [B, T] sitting at positions pos0 .. pos0 + T - 1, with
    each block's keys and values kept in `cache` (earlier positions are read from it).
    Returns the last layer's output (the SoftMax probabilities) [B, T, V], or with last_only
    [B, 1, V] for each sequence's last position (the layers after the last block run on B
    rows: what a generation step needs)."""
    n_blocks = sum(isinstance(layer, TransformerBlock) for layer in net.layers)
    x, i = ids, 0
    for layer in net.layers:
        if isinstance(layer, GPTEmbedFront):
            x = layer.forward(x, pos0=pos0)
        elif isinstance(layer, TransformerBlock):
            x = layer.forward(x, cache, i, pos0)
            i += 1
            if last_only and i == n_blocks and x.shape[1] > 1:
                B, T, C = x.shape
                x = xp.DeviceTensor((B, 1, C), x.dtype, pitch=T * x.pitch, buf=x.buf,
                                    offset=x.offset + (T - 1) * x.pitch * x.dtype.itemsize)
        else:
            x = layer.forward(x)
    return x


def _last_rows(probs):
    B, T, V = probs.shape
    es = probs.dtype.itemsize
    return xp.DeviceTensor((B, V), probs.dtype, pitch=T * probs.pitch, buf=probs.buf,
                           offset=probs.offset + (T - 1) * probs.pitch * es)


def generate(net, ids, n_new, sample=True, cache=None):
    """Autoregressive generation with a KV cache: one pass over the prompt ids [B, T], then
    one position per step. Each step's token is drawn from the last row's probabilities
    with xp.random.choice (sample=True, the notebook's rule, demo.ipynb:1531) or taken as
    their argmax (greedy). The learned positions limit T + n_new - 1 to the context length
    (generate_window slides the window beyond it). Returns the new ids [B, n_new] (host)."""
    if not isinstance(ids, xp.DeviceTensor):
        ids = xp.array(np.asarray(ids))
    B, T = ids.shape
    ctx_len = net.layers[0].context_length
    if T + n_new - 1 > ctx_len:
        raise ValueError(f"{T} + {n_new} tokens exceed the context length {ctx_len}; use "
                         f"generate_window")
    if n_new <= 0:
        return np.zeros((B, 0), np.int64)
    if cache is None:
        cache = new_cache(net, B, T + n_new)
    probs = forward_cached(net, ids, cache, 0, last_only=True)
    V = probs.shape[-1]
    steps = []
    for t in range(n_new):
        last = _last_rows(probs)
        if sample:
            nxt = xp.concatenate([xp.random.choice(V, size=(1, 1), p=last[b]) for b in range(B)],
                                 axis=0)
        else:
            nxt = xp.argmax(last).reshape(B, 1)
        steps.append(nxt)
        if t + 1 < n_new:
            probs = forward_cached(net, nxt, cache, T + t)
    return np.concatenate([s.get().reshape(B, 1) for s in steps], axis=1).astype(np.int64)


def generate_window(net, tokens, length, context_length, vocab_size, on_token=None):
    """The notebook's generation loop (reference demo.ipynb:1520-1537) on the device: keep
    the last context_length tokens, take the probabilities of the last position, draw the
    next token with xp.random.choice over xp.arange(vocab_size) and append it with
    xp.concatenate. tokens: a [1, T] uint8 device tensor (or host ids). `on_token(int)` sees
    each new token (the notebook prints it). Returns the grown token tensor."""
    if not isinstance(tokens, xp.DeviceTensor):
        tokens = xp.array(np.asarray(tokens, dtype=np.uint8).reshape(1, -1), dtype=xp.uint8)
    cand = xp.arange(0, vocab_size, dtype=xp.uint8)
    for _ in range(length):
        tokens = tokens[:, max(0, len(tokens[0]) - context_length):]
        probs = net.predict(tokens)[0, -1]
        out = xp.random.choice(cand, size=(1, 1), p=probs)
        tokens = xp.concatenate((tokens, out), axis=1)
        if on_token is not None:
            on_token(int(out[0, 0].get()))
    return tokens
