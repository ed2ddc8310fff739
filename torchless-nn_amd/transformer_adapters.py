"""GPT embedding and prediction layers (reference transformer_adapters.py:108-181) and the
ViT classifier head (reference transformer_adapters.py:76-95) on the MI355X runtime."""
import numpy as np

import backend
import tl_hip as xp
from utils import Layer
from layers import _packed_nk, linear

__all__ = ["VitProjector", "GPTEmbeddingTable", "GPTEmbedFront", "GPTEmbedBack", "VitMLPHead",
           "ScaledEmbedFront"]


def _round_up(n, m):
    return (n + m - 1) // m * m


class VitProjector(Layer):
    """Image -> token sequence (reference transformer_adapters.py:6-55): patches of
    patch_size, flattened in (row, column, channel) order, projected by `projection`
    (no bias), preceded by 1 + num_registers learned tokens, plus positional embeddings.

    bf16 images whose patches have at most 64 features (ViT-S/4: 48) and at most 64
    patches take one launch (tl_vit_project: patch gather, projection on the matrix cores,
    class/register rows and positions in one kernel per image). Other shapes take three,
    with the same result bit for bit: the patch gather (tl_patchify), one batched GEMM that
    writes each image's patch rows after its class/register rows with the positional rows
    added in the epilogue (a residual shared by the whole batch, stride 0), and one gather
    per class/register row that writes that row of every image (row pitch = tokens x dim).
    `fused = False` forces the three-launch form."""

    def __init__(self, input_size: tuple, patch_size: tuple, embedding_dim, num_registers=0):
        super(VitProjector, self).__init__()
        self.batch_size = 0
        self.channels, self.height, self.width = input_size
        self.patch_size = tuple(patch_size)
        self.patches_height = self.height // self.patch_size[0]
        self.patches_width = self.width // self.patch_size[1]
        self.sequence_length = self.patches_height * self.patches_width
        self.token_dim = self.patch_size[0] * self.patch_size[1] * self.channels
        self.embedding_dim = embedding_dim
        self.cls_reg_size = 1 + num_registers
        self.tokens = None
        self.embeddings = None
        E = embedding_dim
        self.projection = backend.init_random_tensor((self.token_dim, E), divisor=self.token_dim ** 0.5)
        self.cls_reg_tokens = backend.init_random_tensor((self.cls_reg_size, E), divisor=E ** 0.5)
        self.positional_embeddings = backend.init_zeros_tensor((self.cls_reg_size + self.sequence_length, E))
        self.projection_grads = self.register_param(self.projection)
        self.cls_reg_token_grads = self.register_param(self.cls_reg_tokens)
        self.positional_embeddings_grads = self.register_param(self.positional_embeddings)
        self._zero_ids = None
        self.fused = True

    def forward(self, input):
        if not isinstance(input, xp.DeviceTensor):
            input = xp.array(np.asarray(input, dtype=np.float32), dtype=self.projection.dtype)
        self.input = input
        if input.ndim != 4 or tuple(input.shape[1:]) != (self.channels, self.height, self.width):
            raise ValueError(f"expected images [B, {self.channels}, {self.height}, {self.width}], "
                             f"got {input.shape}")
        B = self.batch_size = input.shape[0]
        dt = self.projection.dtype
        L, R, E, K = self.sequence_length, self.cls_reg_size, self.embedding_dim, self.token_dim
        out = xp.empty((B, R + L, E), dt)
        if (self.fused and dt is xp.bfloat16 and input.dtype is dt and
                xp.vit_project_ok(input, self.patch_size, E, R)):
            xp.vit_project(input, _packed_nk(self.projection), self.cls_reg_tokens,
                           self.positional_embeddings, self.patch_size, out)
            self.embeddings = out
            self.output = out
            return self.output
        self.tokens = xp.patchify(input, self.patch_size, dtype=dt)  # [B, L, K]
        es = dt.itemsize
        pos = self.positional_embeddings
        # rows R.. of every image: tokens @ projection + positions[R:]
        if dt is xp.bfloat16:
            W, ldb, layout = _packed_nk(self.projection), K, xp.TL_B_NK
        else:
            W, ldb, layout = self.projection, E, xp.TL_B_KN
        body = xp.DeviceTensor((1,), dt, buf=out.buf, offset=out.offset + R * E * es)
        pos_body = xp.DeviceTensor((L, E), dt, buf=pos.buf, offset=pos.offset + R * E * es)
        xp.gemm(self.tokens, W, M=L, N=E, K=K, lda=K, ldb=ldb, b_layout=layout, C=body, ldc=E,
                batch=B, sa=(L * K, 0), sc=((R + L) * E, 0), residual=pos_body, ldr=E,
                sr=(0, 0), family="gemm_batched")
        # rows 0..R-1: the class/register token plus its position, for every image
        if self._zero_ids is None or self._zero_ids.size != B:
            self._zero_ids = xp.zeros((B,), xp.int32)
        for r in range(R):
            tok = xp.DeviceTensor((1, E), dt, buf=self.cls_reg_tokens.buf,
                                  offset=self.cls_reg_tokens.offset + r * E * es)
            prow = xp.DeviceTensor((1, E), dt, buf=pos.buf, offset=pos.offset + r * E * es)
            row = xp.DeviceTensor((1,), dt, buf=out.buf, offset=out.offset + r * E * es)
            xp.embed(self._zero_ids, tok, prow, 1, out=row, ld_out=(R + L) * E)
        self.embeddings = out
        self.output = out
        return self.output


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

    def forward(self, input, pos0=0):
        """`pos0`: the ids sit at positions pos0 .. (a decode step after a cached prefix;
        the reference always starts at 0, transformer_adapters.py:146-153)."""
        if not isinstance(input, xp.DeviceTensor):
            input = xp.array(np.asarray(input))
        self.input = input
        if input.ndim != 2:
            raise ValueError("token ids must be [batch, time]")
        if not input.contiguous:
            input = input.copy()
        B, T = input.shape
        if pos0 < 0 or pos0 + T > self.context_length:
            raise ValueError(f"positions up to {pos0 + T} exceed the positional table "
                             f"({self.context_length})")
        self.output = xp.embed(input, self.embedding_table.table, self.pos_embedding_table, T,
                               pos0=pos0, out_shape=(B, T, self.embedding_table.embed_size))
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
