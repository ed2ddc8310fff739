"""GPT embedding and prediction layers (reference transformer_adapters.py:108-181) and the
ViT classifier head (reference transformer_adapters.py:76-95) on the MI355X runtime."""
import numpy as np

import backend
import tl_hip as xp
from utils import Layer
from layers import linear

__all__ = ["GPTEmbeddingTable", "GPTEmbedFront", "GPTEmbedBack", "VitMLPHead",
           "ScaledEmbedFront"]


def _round_up(n, m):
    return (n + m - 1) // m * m


class GPTEmbeddingTable:
    """Tied token table [V, C] shared by GPTEmbedFront and GPTEmbedBack (reference
    transformer_adapters.py:108-116; no gradient or AdamW copies at inference)."""

    def __init__(self, vocab_size, embed_size):
        self.vocab_size = vocab_size
        self.embed_size = embed_size
        self.table = backend.init_random_tensor((vocab_size, embed_size))


class GPTEmbedFront(Layer):
    """table[ids] + positions[:T] (reference transformer_adapters.py:119-153) in one
    gather kernel. Ids may be a host array (uploaded here) or a device int tensor; an id
    outside [0, vocab) raises BadInputError (an IndexError) at the next synchronisation."""

    def __init__(self, embedding_table, context_length, positional_embedding="learned"):
        super(GPTEmbedFront, self).__init__()
        assert positional_embedding == "learned" or positional_embedding == "sinusoidal"
        self.positional_embedding = positional_embedding
        self.context_length = context_length
        C = embedding_table.embed_size
        if positional_embedding == "sinusoidal":
            # reference transformer_adapters.py:128-135, evaluated once at construction
            pos = np.arange(context_length)[:, None]
            i = np.arange(C)[None, :]
            tab = pos / 10000 ** (2 * (i // 2) / C)
            tab[:, 0::2] = np.sin(tab[:, 0::2])
            tab[:, 1::2] = np.cos(tab[:, 1::2])
            self.pos_embedding_table = xp.array(tab.astype(np.float32), dtype=backend.FLOAT_TYPE)
        else:
            self.pos_embedding_table = backend.init_zeros_tensor((context_length, C))
            self.pos_embedding_table_grads = self.register_param(self.pos_embedding_table)
        self.embedding_table = embedding_table
        self.parameters.append(self.embedding_table.table)

    def forward(self, input):
        if not isinstance(input, xp.DeviceTensor):
            input = xp.array(np.asarray(input))
        self.input = input
        if input.ndim != 2:
            raise ValueError("token ids must be [batch, time]")
        B, T = input.shape
        if T > self.context_length:
            raise ValueError(f"sequence length {T} exceeds the positional table "
                             f"({self.context_length})")
        self.output = xp.embed(input, self.embedding_table.table, self.pos_embedding_table, T,
                               out_shape=(B, T, self.embedding_table.embed_size))
        return self.output


class GPTEmbedBack(Layer):
    """Tied LM head logits = x @ table^T (reference transformer_adapters.py:167-177). The
    table is already K-contiguous ([V, C]), so the MFMA GEMM reads it in place. Logits rows
    are padded to a multiple of 8 elements so every row starts 16-byte aligned."""

    def __init__(self, embedding_table):
        super(GPTEmbedBack, self).__init__()
        self.embedding_table = embedding_table
        self.is_embed_layer_back = True

    def forward(self, input):
        self.input = input
        table = self.embedding_table.table
        V, C = table.shape
        x2 = input.reshape(-1, C)
        M = x2.shape[0]
        out = xp.empty(input.shape[:-1] + (V,), input.dtype, pitch=_round_up(V, 8))
        xp.gemm(x2, table, M=M, N=V, K=C, lda=x2.pitch, ldb=table.pitch, b_layout=xp.TL_B_NK,
                C=out, ldc=out.pitch)
        self.output = out
        return self.output


class VitMLPHead(Layer):
    """Class-token classifier: x[:, 0, :] @ W + b (reference transformer_adapters.py:76-95).
    Token 0 of each image is read in place with a row stride of L*C."""

    def __init__(self, in_channels, out_channels):
        super(VitMLPHead, self).__init__()
        self.weights = backend.init_random_tensor((in_channels, out_channels),
                                                  divisor=in_channels ** 0.5)
        self.bias = backend.init_zeros_tensor(out_channels)
        self.weight_grads = self.register_param(self.weights)
        self.bias_grads = self.register_param(self.bias)

    def forward(self, input):
        self.input = input
        B, L, C = input.shape
        if not input.contiguous:
            raise ValueError("VitMLPHead needs a contiguous input")
        cls = xp.DeviceTensor((B, C), input.dtype, pitch=L * C, buf=input.buf,
                              offset=input.offset)
        self.output = linear(cls, self.weights, self.bias)
        return self.output


class ScaledEmbedFront(Layer):
    """table[ids] * scale with no positional table (rotary positions are applied inside
    attention). Gemma-style decoders scale by sqrt(d_model). No reference counterpart; the
    gather is GPTEmbedFront's (reference transformer_adapters.py:150)."""

    def __init__(self, embedding_table, scale):
        super(ScaledEmbedFront, self).__init__()
        self.embedding_table = embedding_table
        self.scale = float(np.float32(scale))
        self.parameters.append(self.embedding_table.table)

    def forward(self, input):
        if not isinstance(input, xp.DeviceTensor):
            input = xp.array(np.asarray(input))
        self.input = input
        B, T = input.shape
        self.output = xp.embed(input, self.embedding_table.table, None, T,
                               out_shape=(B, T, self.embedding_table.embed_size), scale=self.scale)
        return self.output
