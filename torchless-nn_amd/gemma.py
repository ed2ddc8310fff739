"""Gemma-style decoder on the MI355X runtime: scaled tied embedding, pre-norm blocks with
RMSNorm ((1 + gamma), eps 1e-6), multi-query rotary attention and GeGLU FFN, final RMSNorm,
tied LM head; prefill into a KV cache, then greedy decoding that keeps every step on the
device (argmax output feeds the next embedding gather without a host round trip).

The reference generates by recomputing the whole window each step (demo.ipynb:1520-1537);
the layers and the decode loop here are new components built on the same Layer protocol.
"""
import numpy as np

import backend
import tl_hip as xp
from layers import DevicePosition, GemmaBlock, KVCache, RMSNorm
from transformer_adapters import GPTEmbeddingTable, GPTEmbedBack, ScaledEmbedFront

__all__ = ["GEMMA_2B", "GemmaDecoder", "build_gemma", "seed_gemma"]

# BASELINE config 5 model shape (vocab 256000, 18 layers, d 2048, 8 query heads sharing one
# key/value head of width 256, FFN 16384); ctx is the positional range the cache may span.
GEMMA_2B = dict(vocab=256000, ctx=8192, layers=18, d=2048, heads=8, kv_heads=1, head_dim=256,
                ffn=16384, rope_base=10000.0)


class GemmaDecoder:
    """Layer list [ScaledEmbedFront, GemmaBlock x L, RMSNorm, GPTEmbedBack] over one tied
    table. forward(ids, cache, pos0) -> logits [B, T, V] (row pitch a multiple of 8)."""

    def __init__(self, cfg):
        self.cfg = dict(cfg)
        d = cfg["d"]
        self.table = GPTEmbeddingTable(cfg["vocab"], d)
        self.front = ScaledEmbedFront(self.table, np.sqrt(np.float32(d)))
        self.blocks = [GemmaBlock(d, cfg["ctx"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                                  cfg["ffn"], cfg.get("rope_base", 10000.0))
                       for _ in range(cfg["layers"])]
        self.final_norm = RMSNorm(d, eps=1e-6, gamma_offset=1.0)
        self.back = GPTEmbedBack(self.table)
        self.layers = [self.front, *self.blocks, self.final_norm, self.back]
        self.dtype = self.table.table.dtype

    def new_cache(self, batch, capacity):
        c = self.cfg
        return KVCache(c["layers"], batch, c["kv_heads"], capacity, c["head_dim"], self.dtype)

    def forward(self, ids, cache=None, pos0=0, last_only=False):
        """Logits [B, T, V]; with last_only, [B, 1, V] for each sequence's last position
        only (what a generation step needs: the final norm and the LM head run on B rows
        instead of B x T, the weight-streaming decode product instead of a 4 GB logits
        write at config 5)."""
        x = self.front.forward(ids)
        c = self.cfg
        T, start = x.shape[1], pos0
        if (cache is not None and (c["heads"] // c["kv_heads"]) * T <= 16 and
                pos0 + T <= min(cache.capacity, c["ctx"]) and
                xp.attention_decode_dev_supported(self.dtype, c["head_dim"], cache.capacity)):
            # a decode step: one device copy of the position (and one RoPE table) serves
            # every block, and the blocks run the kernels a replayed step runs
            pos0 = DevicePosition.at(pos0, T, c["head_dim"], c.get("rope_base", 10000.0))
        for i, blk in enumerate(self.blocks):
            x = blk.forward(x, cache, i, pos0)
        if last_only and T > 1:
            B, _, C = x.shape
            es = x.dtype.itemsize
            x = xp.DeviceTensor((B, 1, C), x.dtype, pitch=T * x.pitch, buf=x.buf,
                                offset=x.offset + (T - 1) * x.pitch * es)
        logits = self.back.forward(self.final_norm.forward(x))
        if cache is not None:
            cache.length = start + T
        return logits

    @staticmethod
    def last_rows(logits):
        """View of logits[:, -1, :] as a [B, V] tensor (no copy)."""
        B, T, V = logits.shape
        es = logits.dtype.itemsize
        return xp.DeviceTensor((B, V), logits.dtype, pitch=T * logits.pitch, buf=logits.buf,
                               offset=logits.offset + (T - 1) * logits.pitch * es)

    def decode_step(self, tok, cache, dpos):
        """One greedy step at the device position dpos: the tokens tok [B] (int64, on the
        device) sit at position *dpos.pos; their keys and values go into the cache there and
        tok is overwritten with the argmax of the next-token logits, which are returned
        [B, 1, V]. Makes no host round trip, so it can be captured in a graph."""
        B = tok.size
        dpos.refresh()
        x = self.front.forward(tok.reshape(B, 1))
        for i, blk in enumerate(self.blocks):
            x = blk.forward(x, cache, i, dpos)
        logits = self.back.forward(self.final_norm.forward(x))
        xp.argmax(self.last_rows(logits), out=tok)
        return logits

    def generate_greedy(self, ids, n_new, cache=None, return_logits=False, graph=True):
        """Prefill `ids` [B, T] into a KV cache, then take `n_new` greedy steps, each feeding
        the device argmax of the last logits row back as the next token. Returns the new
        token ids [B, n_new] as a host int64 array (and, if asked, the per-step last-row
        logits [n_new, B, V] as float32: step 0 from the prefill).

        With graph=True (no logits asked for, and a model the fused attention kernel takes:
        bf16) the first decode step runs eagerly at a device position, the next is captured
        as one HIP graph (position advance and token record included) and replayed for the
        rest, so each step is one host call; the ids are the same as without."""
        if not isinstance(ids, xp.DeviceTensor):
            ids = xp.array(np.asarray(ids))
        B, T = ids.shape
        if cache is None:
            cache = self.new_cache(B, T + n_new)
        if (graph and not return_logits and n_new >= 2
                and xp.attention_decode_dev_supported(self.dtype, self.cfg["head_dim"],
                                                      cache.capacity)):
            return self._generate_graph(ids, n_new, cache)
        logits = self.forward(ids, cache, 0, last_only=True)
        steps, kept = [], []
        for t in range(n_new):
            last = self.last_rows(logits)
            if return_logits:
                kept.append(last.get())
            nxt = xp.argmax(last)  # [B] int64 on the device
            steps.append(nxt)
            if t + 1 < n_new:
                logits = self.forward(nxt.reshape(B, 1), cache, T + t)
        out = np.stack([s.get() for s in steps], axis=1) if steps else np.zeros((B, 0), np.int64)
        return (out, np.stack(kept)) if return_logits else out

    def _generate_graph(self, ids, n_new, cache):
        B, T = ids.shape
        if T + n_new - 1 > cache.capacity:
            raise ValueError("KV cache too small")
        c = self.cfg
        logits = self.forward(ids, cache, 0, last_only=True)
        tok = xp.empty((B,), xp.int64)
        xp.argmax(self.last_rows(logits), out=tok)
        del logits
        hist = xp.empty((B, n_new), xp.int64)  # column j: the token at position T + j
        dpos = DevicePosition(T, 1, c["head_dim"], c.get("rope_base", 10000.0))
        xp.ids_append(tok, hist, dpos.pos, T)

        def step():
            self.decode_step(tok, cache, dpos)
            dpos.advance(1)
            xp.ids_append(tok, hist, dpos.pos, T)

        step()  # eager: creates what later steps reuse (packed weights, workspace)
        if n_new > 2:
            with xp.capture() as g:
                step()
            try:
                for _ in range(n_new - 2):
                    g.launch()
            finally:
                g.destroy()
        cache.length = T + n_new - 1
        return hist.get()


def build_gemma(cfg, dtype=None):
    if dtype is not None:
        backend.set_float_type(dtype)
    return GemmaDecoder(cfg)


def seed_gemma(model, seed, scale=0.02, device=False):
    """Overwrite all parameters, in layer order, with seeded N(0,1)*scale (the RMSNorm
    gammas too: they scale by 1 + gamma). device=False draws on the host from
    numpy default_rng(seed) (what the parity tests mirror); device=True draws on the GPU
    with Philox keyed by seed, stream = the parameter's index (seconds for 2.5B weights)."""
    params = [p for layer in model.layers for p in layer.parameters]
    if device:
        for i, p in enumerate(params):
            xp.random_normal(p.shape, seed, stream=i, std=scale, out=p)
        return model
    rng = np.random.default_rng(seed)
    for p in params:
        p.set(rng.standard_normal(p.shape, dtype=np.float32) * np.float32(scale))
    return model
