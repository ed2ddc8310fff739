"""Transformer layers on the MI355X runtime (reference layers.py:195-476).

Same classes, constructor arguments, parameter lists and `forward(x) -> y` contract as the
reference; every forward is a handful of libtl kernel launches on one HIP stream:

  Dense / FFN / projections -> tl_gemm with bias, activation and residual epilogues
  MultiHeadAttention        -> QKV GEMM that scatters head-major Q, K and V^T, then one
                               fused attention kernel (bf16, or fp32 on the fp32 matrix
                               cores) that writes merged heads, or (shapes it does not take,
                               `fused = False`) the batched QK^T GEMM, the causal softmax
                               row kernel and the batched P.V GEMM
  LayerNorm / RMSNorm       -> one row kernel each

The MFMA GEMMs read a weight in a K-contiguous copy ([out, in]) that is packed on the
device the first time the weight is used and again after its buffer has been written (by
`set`, `fill` or any kernel writing into any view of it). bf16 weights always take that copy;
fp32 weights take it for products the fp32 matrix-core kernels run (K % 4 == 0, and either
at least 128 output tiles of 128x128 or K <= 1024 with at least 8 tiles of 64x64), which
doubles their HBM use, and are read in place by the fp32 VALU GEMM otherwise.
"""
import numpy as np

import backend
import tl_hip as xp
from utils import Layer
from activations import act_code_of

__all__ = ["Dense", "Dropout", "MultiHeadAttention", "TransformerFeedForward", "LayerNorm",
           "RMSNorm", "TransformerBlock", "linear", "KVCache", "MultiQueryAttention",
           "GeGLUFeedForward", "GemmaBlock", "DevicePosition"]


def _round_up(n, m):
    return (n + m - 1) // m * m


def _packed_nk(w, prenorm=None):
    """[K, N] weight -> [N, K] (K-contiguous) copy for the MFMA GEMM, cached on the
    weight until its contents change. With `prenorm` (the RMSNorm layer that feeds the
    product) its gain is folded in: B[n, k] = w[k, n] * (gamma_offset + gamma[k])."""
    key = ((w._version,) if prenorm is None else
           (w._version, prenorm.gamma._version, prenorm.gamma_offset))
    if w._aux is not None and w._aux[0] == key:
        return w._aux[1]
    if prenorm is None:
        packed = xp.transpose2d(w)
    else:
        packed = xp.transpose2d_gain(w, prenorm.gamma, prenorm.gamma_offset)
    w._aux = (key, packed)
    return packed


def _warm(*weights):
    """Name the weights of the products that follow the next norm launch to that launch
    (xp.prefetch_hint), so they arrive from the device caches rather than HBM. bf16 weights
    are read by the products as their packed [N, K] copies, which are the ones named; the
    other dtypes are left alone."""
    for w in weights:
        if w.dtype is xp.bfloat16:
            xp.prefetch_hint(_packed_nk(w))


_UNIT_GAIN = {}


def _folds_gain(prenorm, w_dtype):
    """bf16 products fed by an RMSNorm carry its gain in their packed weight."""
    return prenorm is not None and w_dtype is xp.bfloat16 and prenorm.gamma.dtype is xp.bfloat16


def _prenorm(x2d, prenorm, w_dtype):
    """(A operand, norm_eps) of a product that starts with the RMSNorm layer `prenorm`.
    When the weight carries the gain (bf16), a decode step's few rows go in unnormalised and
    the product scales each row by its 1 / rms (no separate launch); more rows are
    normalised first with a unit gain. Otherwise the norm layer runs as it is."""
    if prenorm is None:
        return x2d, None
    if not _folds_gain(prenorm, w_dtype):
        return prenorm.forward(x2d), None
    M, K = x2d.shape
    prenorm.input = x2d
    if M <= 16 and K % 8 == 0 and x2d.pitch % 8 == 0 and x2d.ptr % 16 == 0:
        prenorm.output = None
        return x2d, float(prenorm.eps)
    key = (K, x2d.dtype.name)
    if key not in _UNIT_GAIN:
        _UNIT_GAIN[key] = xp.zeros((K,), x2d.dtype)
    prenorm.output = xp.rmsnorm(x2d, _UNIT_GAIN[key], prenorm.eps, 1.0)
    return prenorm.output, None


def linear(x2d, w, bias=None, act=xp.TL_ACT_NONE, residual=None, out=None, qkv=None,
           family="gemm_mfma", prenorm=None):
    """y = act(x2d @ w + bias) (+ residual), x2d [M, K], w [K, N] (reference `x @ W + b`).
    With `prenorm` (an RMSNorm layer) the product is RMSNorm(x2d) @ w."""
    M, K = x2d.shape
    Kw, N = w.shape
    if Kw != K:
        raise ValueError(f"matmul shape mismatch: {x2d.shape} @ {w.shape}")
    fold = prenorm if _folds_gain(prenorm, w.dtype) else None
    x2d, norm_eps = _prenorm(x2d, prenorm, w.dtype)
    if qkv is None and out is None:
        out = xp.empty((M, N), x2d.dtype)
    # bf16 always; fp32 when the fp32 matrix-core kernels take the product (K % 4 == 0, and
    # either at least 128 output tiles of 128x128 or K <= 1024 with 8 or more 64x64 tiles):
    # both read B as [N, K]
    if w.dtype is xp.bfloat16 or (K % 4 == 0 and (-(-M // 128) * -(-N // 128) >= 128 or
                                                  (K <= 1024 and -(-M // 64) * -(-N // 64) >= 8))):
        B, ldb, layout = _packed_nk(w, fold), K, xp.TL_B_NK
    else:
        B, ldb, layout = w, w.pitch, xp.TL_B_KN
    xp.gemm(x2d, B, M=M, N=N, K=K, lda=x2d.pitch, ldb=ldb, b_layout=layout, C=out,
            ldc=(out.pitch if out is not None else 0), bias=bias, act=act, residual=residual,
            ldr=(residual.pitch if residual is not None else 0), qkv=qkv, family=family,
            norm_eps=norm_eps)
    return out


class Dense(Layer):
    """x @ W + b, W [in, out] (reference layers.py:195-209)."""

    def __init__(self, input_size, output_size):
        super(Dense, self).__init__()
        self.weights = backend.init_random_tensor((input_size, output_size),
                                                  divisor=(0.5 * input_size) ** 0.5)
        self.bias = backend.init_zeros_tensor(output_size)
        self.weight_grads = self.register_param(self.weights)
        self.bias_grads = self.register_param(self.bias)

    def forward(self, input):
        self.input = input
        x2 = input.reshape(-1, input.shape[-1])
        y = linear(x2, self.weights, self.bias)
        self.output = y.reshape(*input.shape[:-1], self.weights.shape[1])
        return self.output


class Dropout(Layer):
    """Identity at inference (reference layers.py:217-233). Sampling a mask is a training
    feature this runtime does not provide, so a non-zero rate outside eval mode raises."""

    def __init__(self, dropout_rate):
        super(Dropout, self).__init__()
        self.dropout_rate = dropout_rate

    def forward(self, input):
        self.input = input
        if self.dropout_rate > 0.0 and self.eval_mode is False:
            raise NotImplementedError(
                "Dropout with rate > 0 in training mode is not supported by the MI355X "
                "runtime; call set_eval(True) (inference) or build with rate 0")
        self.output = self.input
        return self.output


class MultiHeadAttention(Layer):
    """Fused-QKV multi-head attention (reference layers.py:241-307).

    Device layout per call: Q and K as [B, H, T, D], V transposed as [B, H, D, T] (the K
    operand of P.V must be contiguous along T), merged heads as [B, T, C]. The fused path
    never materialises the [B, H, T, T] probabilities, so `softmax` stays None; the unfused
    path keeps them (row pitch rounded up to 8 elements). `fused = False` forces the latter.
    """
    fused = True

    def __init__(self, embedding_dim, context_length, num_heads, decoder=False,
                 attn_dropout_rate=0.0, res_dropout_rate=0.0):
        super(MultiHeadAttention, self).__init__()
        self.embedding_dim = embedding_dim
        self.context_length = context_length
        self.num_heads = num_heads
        self.heads_dim = embedding_dim // num_heads
        self.is_decoder = decoder

        self.query = None
        self.key_t = None
        self.value = None
        self.softmax = None
        self.heads_out = None

        self.attn_dropout = Dropout(attn_dropout_rate)
        self.res_dropout = Dropout(res_dropout_rate)

        C = embedding_dim
        self.qkv_weights = backend.init_random_tensor((C, 3 * C), divisor=(0.5 * C) ** 0.5)
        self.qkv_bias = backend.init_zeros_tensor(3 * C)
        self.out_weights = backend.init_random_tensor((C, C), divisor=(0.5 * C) ** 0.5)
        self.out_bias = backend.init_zeros_tensor(C)

        self.qkv_weight_grads = self.register_param(self.qkv_weights)
        self.qkv_bias_grads = self.register_param(self.qkv_bias)
        self.out_weight_grads = self.register_param(self.out_weights)
        self.out_bias_grads = self.register_param(self.out_bias)

    def forward(self, input, cache=None, layer=0, pos0=0):
        return self._forward(input, None, cache, layer, pos0)

    def _forward(self, input, residual, cache=None, layer=0, pos0=0):
        """Returns heads @ W_o + b_o, plus `residual` when given (fused in the epilogue).
        With a KVCache (not in the reference, whose generation recomputes the window,
        demo.ipynb:1526-1533), a decoder writes this call's keys and values into the cache
        at positions pos0 .. and attends over positions 0 .. pos0 + T - 1."""
        if cache is not None:
            return self._forward_cached(input, residual, cache, layer, pos0)
        self.input = input
        B, T, C = input.shape
        H, D = self.num_heads, self.heads_dim
        if self.is_decoder and T > self.context_length:
            raise ValueError(f"sequence length {T} exceeds the context length "
                             f"{self.context_length} of the causal mask")
        dt = input.dtype
        x2 = input.reshape(B * T, C)
        # the fused kernel takes keys/values with a capacity that is a multiple of 8; the
        # padding positions are never written and never read as values
        fused = self.fused and xp.attention_supported(dt, D, _round_up(T, 8))
        L = _round_up(T, 8) if fused else T
        q = xp.empty((B, H, T, D), dt)
        k = xp.empty((B, H, L, D), dt)
        vt = xp.empty((B, H, D, L), dt)
        linear(x2, self.qkv_weights, self.qkv_bias, qkv=(q, k, vt, T, H, H, D, L, 0))
        self.query, self.key_t, self.value = q, k, vt

        divisor = float(np.float32(D ** 0.5))  # reference layers.py:293 divides by sqrt(D)
        if fused:
            heads = xp.empty((B, T, C), dt)
            if self.attn_dropout.dropout_rate > 0.0 and not self.attn_dropout.eval_mode:
                self.attn_dropout.forward(heads)  # raises: no dropout sampling at inference
            xp.attention(q, k, vt, heads, n_heads_q=H, n_heads_kv=H, divisor=divisor,
                         causal=self.is_decoder, offset=0, seq_k=T)
            self.softmax = None
        else:
            heads = self._unfused(q, k, vt, B, T, C, H, D, dt, divisor)
        self.heads_out = heads

        out = linear(heads.reshape(B * T, C), self.out_weights, self.out_bias,
                     residual=(residual.reshape(B * T, C) if residual is not None else None))
        self.output = out.reshape(B, T, C)
        return self.res_dropout.forward(self.output)

    def _forward_cached(self, input, residual, cache, layer, pos0):
        self.input = input
        B, T, C = input.shape
        H, D = self.num_heads, self.heads_dim
        if not self.is_decoder:
            raise ValueError("a KV cache serves causal (decoder) attention only")
        if pos0 < 0 or pos0 + T > min(cache.capacity, self.context_length):
            raise ValueError(f"positions up to {pos0 + T} exceed the cache ({cache.capacity}) "
                             f"or the context length ({self.context_length})")
        if self.attn_dropout.dropout_rate > 0.0 and not self.attn_dropout.eval_mode:
            self.attn_dropout.forward(input)  # raises: no dropout sampling at inference
        dt, L, Tk = input.dtype, cache.capacity, pos0 + T
        k, vt = cache.k[layer], cache.vt[layer]
        q = xp.empty((B, H, T, D), dt)
        linear(input.reshape(B * T, C), self.qkv_weights, self.qkv_bias,
               qkv=(q, k, vt, T, H, H, D, L, pos0))
        self.query, self.key_t, self.value = q, k, vt
        divisor = float(np.float32(D ** 0.5))
        heads = xp.empty((B, T, C), dt)
        if self.fused and xp.attention_supported(dt, D, L):
            xp.attention(q, k, vt, heads, n_heads_q=H, n_heads_kv=H, divisor=divisor,
                         causal=True, offset=pos0, seq_k=Tk)
            self.softmax = None
        else:
            self.softmax = _attend_cache_unfused(q, k, vt, heads, B, T, Tk, L, H, H, D, dt,
                                                 divisor, pos0)
        self.heads_out = heads
        out = linear(heads.reshape(B * T, C), self.out_weights, self.out_bias,
                     residual=(residual.reshape(B * T, C) if residual is not None else None))
        self.output = out.reshape(B, T, C)
        return self.res_dropout.forward(self.output)

    def _unfused(self, q, k, vt, B, T, C, H, D, dt, divisor):
        ldS = _round_up(T, 8)
        scores = xp.empty((B, H, T, T), dt, pitch=ldS)
        # (Q @ K^T) / sqrt(D): reference layers.py:293 divides after the product
        xp.gemm(q, k, M=T, N=T, K=D, lda=D, ldb=D, b_layout=xp.TL_B_NK, C=scores, ldc=ldS,
                batch=B * H, sa=(T * D, 0), sb=(T * D, 0), sc=(T * ldS, 0),
                divisor=divisor, family="gemm_batched")
        # additive -1e9 causal mask + softmax (reference layers.py:295-300), in place
        probs = xp.softmax(scores, causal=self.is_decoder, period=T, offset=0, out=scores)
        self.softmax = self.attn_dropout.forward(probs)

        heads = xp.empty((B, T, C), dt)
        # P @ V with the head merge folded into the store (reference layers.py:303-304)
        xp.gemm(self.softmax, vt, M=T, N=D, K=T, lda=ldS, ldb=T, b_layout=xp.TL_B_NK, C=heads,
                ldc=C, batch=B * H, batch_inner=H, sa=(H * T * ldS, T * ldS),
                sb=(H * D * T, D * T), sc=(T * C, D), family="gemm_batched")
        return heads

    def set_eval(self, eval_mode):
        self.attn_dropout.set_eval(eval_mode)
        self.res_dropout.set_eval(eval_mode)


class TransformerFeedForward(Layer):
    """act(x W1 + b1) W2 + b2 with a 4x hidden layer (reference layers.py:346-375). GeLU
    and SiLU run in the first GEMM's epilogue."""

    def __init__(self, num_channels, activation, res_dropout_rate=0.0):
        super(TransformerFeedForward, self).__init__()
        self.activation: Layer = activation()
        self.act_code = act_code_of(activation)
        self.dropout = Dropout(res_dropout_rate)
        self.hidden_output = None
        C = num_channels
        self.weights1 = backend.init_random_tensor((C, 4 * C), divisor=(0.5 * C) ** 0.5)
        self.bias1 = backend.init_zeros_tensor(4 * C)
        self.weights2 = backend.init_random_tensor((4 * C, C), divisor=(2 * C) ** 0.5)
        self.bias2 = backend.init_zeros_tensor(C)
        self.weight_grads1 = self.register_param(self.weights1)
        self.bias_grads1 = self.register_param(self.bias1)
        self.weight_grads2 = self.register_param(self.weights2)
        self.bias_grads2 = self.register_param(self.bias2)

    def forward(self, input):
        return self._forward(input, None)

    def _forward(self, input, residual):
        self.input = input
        shape = input.shape
        C = shape[-1]
        x2 = input.reshape(-1, C)
        if self.act_code is not None:
            h = linear(x2, self.weights1, self.bias1, act=self.act_code)
        else:
            h = self.activation.forward(linear(x2, self.weights1, self.bias1))
        self.hidden_output = h
        y = linear(h, self.weights2, self.bias2,
                   residual=(residual.reshape(-1, C) if residual is not None else None))
        self.output = self.dropout.forward(y.reshape(*shape))
        return self.output

    def set_eval(self, eval_mode):
        self.dropout.set_eval(eval_mode)


class LayerNorm(Layer):
    """(x - mean) / sqrt(var + 1e-5) * gamma + beta over the last axis, population
    variance (reference layers.py:395-428)."""

    def __init__(self, num_channels):
        super(LayerNorm, self).__init__()
        self.channels = num_channels
        self.eps = np.float32(1e-5)
        self.gamma = backend.init_zeros_tensor(num_channels).fill(1)
        self.beta = backend.init_zeros_tensor(num_channels)
        self.gamma_grads = self.register_param(self.gamma)
        self.beta_grads = self.register_param(self.beta)

    def forward(self, input):
        self.input = input
        self.output = xp.layernorm(input, self.gamma, self.beta, self.eps)
        return self.output


class RMSNorm(Layer):
    """x / sqrt(mean(x^2) + eps) * (gamma_offset + gamma). Absent from the reference
    (layers.py:394 is a TODO); gamma_offset=1 with gamma=0 init gives Gemma's convention."""

    def __init__(self, num_channels, eps=1e-6, gamma_offset=0.0):
        super(RMSNorm, self).__init__()
        self.channels = num_channels
        self.eps = np.float32(eps)
        self.gamma_offset = float(gamma_offset)
        self.gamma = backend.init_zeros_tensor(num_channels)
        if self.gamma_offset == 0.0:
            self.gamma.fill(1)
        self.gamma_grads = self.register_param(self.gamma)

    def forward(self, input):
        self.input = input
        self.output = xp.rmsnorm(input, self.gamma, self.eps, self.gamma_offset)
        return self.output


class TransformerBlock(Layer):
    """Pre-LN block x + MHA(LN1 x), then + FFN(LN2 .) (reference layers.py:444-467).

    With `fuse_residual` (the default) both residual adds run in the epilogues of the
    out-projection and second FFN GEMMs, so `attn_block.output` and `ffn.output` hold the
    residual stream after each add. With `fuse_residual = False` (on the class or one block)
    the sublayers return their own outputs and the adds are separate launches, as in the
    reference (layers.py:464-466), so `attn_block.output` is heads @ W_o + b_o and
    `ffn.output` is act(. W1 + b1) W2 + b2: per-layer taps read what the reference's do."""
    fuse_residual = True

    def __init__(self, embed_dim, context_length, num_heads, activation, decoder=False,
                 attn_dropout_rate=0.0, res_dropout_rate=0.0):
        super(TransformerBlock, self).__init__()
        self.pre_attn_norm = LayerNorm(embed_dim)
        self.attn_block = MultiHeadAttention(embed_dim, context_length, num_heads,
                                             decoder=decoder,
                                             attn_dropout_rate=attn_dropout_rate,
                                             res_dropout_rate=res_dropout_rate)
        self.pre_ffn_norm = LayerNorm(embed_dim)
        self.ffn = TransformerFeedForward(embed_dim, activation,
                                          res_dropout_rate=res_dropout_rate)
        self.parameters = [*self.pre_attn_norm.parameters, *self.attn_block.parameters,
                           *self.pre_ffn_norm.parameters, *self.ffn.parameters]

    def forward(self, input, cache=None, layer=0, pos0=0):
        """`cache` / `layer` / `pos0`: decode with a KV cache (MultiHeadAttention.forward)."""
        self.input = input
        # each norm launch also pulls the next two products' weights into the device caches
        # (after a forward's 0.8 GB of logits none of them is left there)
        _warm(self.attn_block.qkv_weights, self.attn_block.out_weights)
        if not self.fuse_residual:
            y = input + self.attn_block._forward(self.pre_attn_norm.forward(input), None, cache,
                                                 layer, pos0)
            _warm(self.ffn.weights1, self.ffn.weights2)
            self.output = y + self.ffn._forward(self.pre_ffn_norm.forward(y), None)
            return self.output
        y = self.attn_block._forward(self.pre_attn_norm.forward(input), input, cache, layer, pos0)
        _warm(self.ffn.weights1, self.ffn.weights2)
        self.output = self.ffn._forward(self.pre_ffn_norm.forward(y), residual=y)
        return self.output

    def set_eval(self, eval_mode):
        self.eval_mode = eval_mode
        self.attn_block.set_eval(eval_mode)
        self.ffn.set_eval(eval_mode)


# ---------------------------------------------------------------------------------------
# Gemma-style decoder pieces. The reference has no counterpart: its
# attention is one fused [C, 3C] MHA with absolute positions (layers.py:241-307), its FFN
# is ungated (layers.py:346-375) and generation recomputes the whole window
# (demo.ipynb:1520-1537). Their interfaces follow the Layer protocol above.
# ---------------------------------------------------------------------------------------
_ROPE_TABLES = {}


def _rope_table(T, D, base, pos0):
    """cos/sin table for positions pos0 .. pos0 + T - 1, shared by every layer of a step
    (a handful of recent tables are kept; each is T * D * 4 bytes)."""
    key = (T, D, base, pos0)
    t = _ROPE_TABLES.pop(key, None)
    if t is None:
        t = xp.rope_table(T, D, base, pos0)
        while len(_ROPE_TABLES) >= 8:
            _ROPE_TABLES.pop(next(iter(_ROPE_TABLES)))
    _ROPE_TABLES[key] = t
    return t


class DevicePosition:
    """The position of a decode step kept in device memory (one int64) together with the
    RoPE table of the step's T positions, so a step captured in a graph replays at the
    current position: `refresh()` recomputes the table from the device value and
    `advance(n)` adds n on the device, both stream-ordered."""

    def __init__(self, start, T, head_dim, base=10000.0, table=None):
        self.pos = xp.array(np.array([start], np.int64))
        self.T, self.head_dim, self.base = int(T), int(head_dim), float(base)
        self.table = table if table is not None else xp.empty((2, self.T, self.head_dim // 2),
                                                              xp.float32)

    @classmethod
    def at(cls, pos0, T, head_dim, base):
        """A fixed host position pos0 (its table from the shared host-position tables)."""
        return cls(pos0, T, head_dim, base, table=_rope_table(T, head_dim, base, pos0))

    def refresh(self):
        xp.rope_table_dev(self.table, self.pos, self.base)

    def advance(self, n=1):
        xp.i64_add(self.pos, n)

    def get(self):
        return int(self.pos.get()[0])


class KVCache:
    """Per-layer keys [B, Hkv, L, D] and transposed values [B, Hkv, D, L] in HBM, L a
    multiple of 8; positions at or past the valid length are never read as values."""

    def __init__(self, n_layers, batch, n_kv_heads, capacity, head_dim, dtype):
        self.capacity = _round_up(capacity, 8)
        self.batch, self.n_kv_heads, self.head_dim = batch, n_kv_heads, head_dim
        self.k = [xp.zeros((batch, n_kv_heads, self.capacity, head_dim), dtype) for _ in range(n_layers)]
        self.vt = [xp.zeros((batch, n_kv_heads, head_dim, self.capacity), dtype) for _ in range(n_layers)]
        self.length = 0  # valid positions written so far


class MultiQueryAttention(Layer):
    """Multi-/grouped-query causal attention with rotary positions: num_heads query heads
    share num_kv_heads key/value heads (Shazeer 2019, "Fast Transformer Decoding"; Ainslie
    et al. 2023, GQA), rotate-half RoPE on queries and keys (Su et al. 2021), scores divided
    by sqrt(head_dim), no biases. Weights qkv [C, (Hq + 2 Hkv) D] with columns [Q | K | V]
    and out [Hq D, C]. `forward(x, cache, layer, pos0)` writes this call's keys and values
    into `cache` at positions pos0.. and attends over positions 0 .. pos0 + T - 1."""
    fused = True

    def __init__(self, embedding_dim, context_length, num_heads, num_kv_heads, head_dim,
                 rope_base=10000.0):
        super(MultiQueryAttention, self).__init__()
        if num_heads % num_kv_heads:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        self.embedding_dim, self.context_length = embedding_dim, context_length
        self.num_heads, self.num_kv_heads, self.heads_dim = num_heads, num_kv_heads, head_dim
        self.rope_base = float(rope_base)
        C, N = embedding_dim, (num_heads + 2 * num_kv_heads) * head_dim
        self.qkv_weights = backend.init_random_tensor((C, N), divisor=C ** 0.5)
        self.out_weights = backend.init_random_tensor((num_heads * head_dim, C),
                                                      divisor=(num_heads * head_dim) ** 0.5)
        self.register_param(self.qkv_weights)
        self.register_param(self.out_weights)
        self.softmax = None

    def forward(self, input, cache=None, layer=0, pos0=0):
        return self._forward(input, None, cache, layer, pos0)

    def _forward(self, input, residual, cache=None, layer=0, pos0=0, prenorm=None):
        """`prenorm` (an RMSNorm layer) normalises `input` first (folded into the QKV
        product for a decode step's few rows)."""
        if isinstance(pos0, DevicePosition):
            return self._forward_dev(input, residual, cache, layer, pos0, prenorm)
        B, T, C = input.shape
        Hq, Hkv, D = self.num_heads, self.num_kv_heads, self.heads_dim
        if (cache is not None and self.fused and (Hq // Hkv) * T <= 16 and
                pos0 + T <= min(cache.capacity, self.context_length) and
                xp.attention_decode_dev_supported(input.dtype, D, cache.capacity)):
            # a decode step: the same kernels as a replayed one (position in device memory)
            dpos = DevicePosition.at(pos0, T, D, self.rope_base)
            return self._forward_dev(input, residual, cache, layer, dpos, prenorm)
        self.input = input
        if pos0 + T > self.context_length:
            raise ValueError(f"positions up to {pos0 + T} exceed the context length "
                             f"{self.context_length}")
        dt = input.dtype
        q = xp.empty((B, Hq, T, D), dt)
        if cache is not None:
            if pos0 + T > cache.capacity:
                raise ValueError("KV cache too small")
            k, vt, L = cache.k[layer], cache.vt[layer], cache.capacity
        else:
            L = _round_up(T, 8)
            k, vt = xp.empty((B, Hkv, L, D), dt), xp.empty((B, Hkv, D, L), dt)
        linear(input.reshape(B * T, C), self.qkv_weights, qkv=(q, k, vt, T, Hq, Hkv, D, L, pos0),
               prenorm=prenorm)
        table = _rope_table(T, D, self.rope_base, pos0)
        # queries and this call's cache keys rotated in one launch
        kslice = xp.DeviceTensor((B * Hkv, T, D), dt, buf=k.buf,
                                 offset=k.offset + pos0 * D * dt.itemsize)
        xp.rope2(q, kslice, table, T, n_seq2=B * Hkv, seq_stride2=L * D)
        Tk = pos0 + T
        divisor = float(np.float32(D ** 0.5))
        heads = xp.empty((B, T, Hq * D), dt)
        if self.fused and xp.attention_supported(dt, D, L):
            xp.attention(q, k, vt, heads, n_heads_q=Hq, n_heads_kv=Hkv, divisor=divisor,
                         causal=True, offset=pos0, seq_k=Tk)
        else:
            self._unfused(q, k, vt, heads, B, T, Tk, L, Hq, Hkv, D, dt, divisor, pos0)
        out = linear(heads.reshape(B * T, Hq * D), self.out_weights,
                     residual=(residual.reshape(B * T, C) if residual is not None else None))
        self.output = out.reshape(B, T, C)
        return self.output

    def _forward_dev(self, input, residual, cache, layer, dpos, prenorm=None):
        """Decode at a device position (what a captured step replays): the same kernels and
        arithmetic as the host-position call, with the cache row, the RoPE positions and the
        attended key count read from dpos.pos on the device. The caller keeps the position
        below the cache capacity (rows past it are neither written nor read)."""
        self.input = input
        B, T, C = input.shape
        Hq, Hkv, D = self.num_heads, self.num_kv_heads, self.heads_dim
        if cache is None:
            raise ValueError("decoding at a device position needs a KV cache")
        if dpos.T != T or dpos.head_dim != D or dpos.base != self.rope_base:
            raise ValueError("the device position's RoPE table does not match this call")
        dt = input.dtype
        if not (self.fused and xp.attention_decode_dev_supported(dt, D, cache.capacity)):
            raise ValueError("decoding at a device position needs the fused bf16 attention kernel")
        q = xp.empty((B, Hq, T, D), dt)
        k, vt, L = cache.k[layer], cache.vt[layer], cache.capacity
        linear(input.reshape(B * T, C), self.qkv_weights, qkv=(q, k, vt, T, Hq, Hkv, D, L, dpos.pos),
               prenorm=prenorm)
        heads = xp.empty((B, T, Hq * D), dt)
        div = float(np.float32(D ** 0.5))
        if D >= 64:  # RoPE of the queries and new keys inside the attention kernel
            xp.attention_decode_dev(q, k, vt, heads, dpos.pos, n_heads_q=Hq, n_heads_kv=Hkv,
                                    divisor=div, rope=dpos.table)
        else:
            xp.rope2_dev(q, k, dpos.table, dpos.pos)
            xp.attention_decode_dev(q, k, vt, heads, dpos.pos, n_heads_q=Hq, n_heads_kv=Hkv,
                                    divisor=div)
        out = linear(heads.reshape(B * T, Hq * D), self.out_weights,
                     residual=(residual.reshape(B * T, C) if residual is not None else None))
        self.output = out.reshape(B, T, C)
        return self.output

    def _unfused(self, q, k, vt, heads, B, T, Tk, L, Hq, Hkv, D, dt, divisor, pos0):
        self.softmax = _attend_cache_unfused(q, k, vt, heads, B, T, Tk, L, Hq, Hkv, D, dt,
                                             divisor, pos0)


def _attend_cache_unfused(q, k, vt, heads, B, T, Tk, L, Hq, Hkv, D, dt, divisor, pos0):
    """Causal attention of q [B, Hq, T, D] at positions pos0 .. over the first Tk keys of a
    cache k [B, Hkv, L, D] / vt [B, Hkv, D, L] with materialised probabilities: scores by
    batched products, the causal softmax, P.V into heads [B, T, Hq D]. Returns the
    probabilities [B, Hq, T, Tk] (row pitch a multiple of 8)."""
    g = Hq // Hkv
    ldS = _round_up(Tk, 8)
    scores = xp.empty((B, Hq, T, Tk), dt, pitch=ldS)
    es = dt.itemsize
    for hk in range(Hkv):  # one batched product per kv head: z = (b, query head in group)
        qv = xp.DeviceTensor((1,), dt, buf=q.buf, offset=q.offset + hk * g * T * D * es)
        kv = xp.DeviceTensor((1,), dt, buf=k.buf, offset=k.offset + hk * L * D * es)
        sv = xp.DeviceTensor((1,), dt, buf=scores.buf, offset=scores.offset + hk * g * T * ldS * es)
        xp.gemm(qv, kv, M=T, N=Tk, K=D, lda=D, ldb=D, b_layout=xp.TL_B_NK, C=sv, ldc=ldS,
                batch=B * g, batch_inner=g, sa=(Hq * T * D, T * D), sb=(Hkv * L * D, 0),
                sc=(Hq * T * ldS, T * ldS), divisor=divisor, family="gemm_batched")
    probs = xp.softmax(scores, causal=True, period=T, offset=pos0, out=scores)
    for hk in range(Hkv):
        pv = xp.DeviceTensor((1,), dt, buf=probs.buf, offset=probs.offset + hk * g * T * ldS * es)
        vv = xp.DeviceTensor((1,), dt, buf=vt.buf, offset=vt.offset + hk * D * L * es)
        hv = xp.DeviceTensor((1,), dt, buf=heads.buf, offset=heads.offset + hk * g * D * es)
        xp.gemm(pv, vv, M=T, N=D, K=Tk, lda=ldS, ldb=L, b_layout=xp.TL_B_NK, C=hv,
                ldc=Hq * D, batch=B * g, batch_inner=g, sa=(Hq * T * ldS, T * ldS),
                sb=(Hkv * D * L, 0), sc=(T * Hq * D, D), family="gemm_batched")
    return probs


class GeGLUFeedForward(Layer):
    """act(x W_gate) * (x W_up) then W_down, no biases (Shazeer 2020, "GLU Variants Improve
    Transformer"); act is the tanh-GeLU of reference activations.py:24-28 (GeGLU) or SiLU
    (SwiGLU). The gate and up weights are packed into one [2F, C] operand with interleaved
    rows (gate f, up f), so one GEMM's epilogue forms act(gate) * up."""

    def __init__(self, num_channels, hidden, activation=None):
        super(GeGLUFeedForward, self).__init__()
        from activations import GeLU
        activation = activation or GeLU
        self.act_code = act_code_of(activation)
        if self.act_code not in (xp.TL_ACT_GELU, xp.TL_ACT_SILU):
            raise ValueError("gated FFN supports GeLU or SiLU")
        C, F = num_channels, hidden
        self.hidden = F
        self.gate_weights = backend.init_random_tensor((C, F), divisor=C ** 0.5)
        self.up_weights = backend.init_random_tensor((C, F), divisor=C ** 0.5)
        self.down_weights = backend.init_random_tensor((F, C), divisor=F ** 0.5)
        for w in (self.gate_weights, self.up_weights, self.down_weights):
            self.register_param(w)
        self._pack = None

    def _packed(self, prenorm=None):
        """Gate and up weights interleaved as [2F, C] rows (gate f, up f), with the gain of
        `prenorm` (the RMSNorm feeding the FFN) folded in when given."""
        g, u = self.gate_weights, self.up_weights
        key = ((g._version, u._version) if prenorm is None else
               (g._version, u._version, prenorm.gamma._version, prenorm.gamma_offset))
        if self._pack is None or self._pack[0] != key:
            C, F = g.shape
            packed = xp.empty((2 * F, C), g.dtype)
            for w, at in ((g, 0), (u, C)):
                if prenorm is None:
                    xp.transpose2d(w, out=packed, out_offset=at, ldy=2 * C)
                else:
                    xp.transpose2d_gain(w, prenorm.gamma, prenorm.gamma_offset, out=packed,
                                        out_offset=at, ldy=2 * C)
            self._pack = (key, packed)
        return self._pack[1]

    def forward(self, input):
        return self._forward(input, None)

    def _forward(self, input, residual, prenorm=None):
        self.input = input
        shape = input.shape
        C, F = shape[-1], self.hidden
        wdt = self.gate_weights.dtype
        x2, norm_eps = _prenorm(input.reshape(-1, C), prenorm, wdt)
        M = x2.shape[0]
        h = xp.empty((M, F), input.dtype)
        pack = self._packed(prenorm if _folds_gain(prenorm, wdt) else None)
        xp.gemm(x2, pack, M=M, N=2 * F, K=C, lda=x2.pitch, ldb=C, b_layout=xp.TL_B_NK,
                C=h, ldc=F, act=self.act_code, geglu=True, norm_eps=norm_eps)
        self.hidden_output = h
        y = linear(h, self.down_weights,
                   residual=(residual.reshape(-1, C) if residual is not None else None))
        self.output = y.reshape(*shape)
        return self.output


class GemmaBlock(Layer):
    """Pre-norm decoder block with RMSNorm ((1 + gamma) scale, eps 1e-6), multi-query
    rotary attention and a GeGLU FFN: y = x + Attn(N1 x); z = y + FFN(N2 y). Residual adds
    run in the GEMM epilogues, as in TransformerBlock."""

    def __init__(self, embed_dim, context_length, num_heads, num_kv_heads, head_dim, ffn_hidden,
                 rope_base=10000.0, eps=1e-6):
        super(GemmaBlock, self).__init__()
        self.pre_attn_norm = RMSNorm(embed_dim, eps=eps, gamma_offset=1.0)
        self.attn_block = MultiQueryAttention(embed_dim, context_length, num_heads, num_kv_heads,
                                              head_dim, rope_base)
        self.pre_ffn_norm = RMSNorm(embed_dim, eps=eps, gamma_offset=1.0)
        self.ffn = GeGLUFeedForward(embed_dim, ffn_hidden)
        self.parameters = [*self.pre_attn_norm.parameters, *self.attn_block.parameters,
                           *self.pre_ffn_norm.parameters, *self.ffn.parameters]

    def forward(self, input, cache=None, layer=0, pos0=0):
        self.input = input
        y = self.attn_block._forward(input, input, cache, layer, pos0, prenorm=self.pre_attn_norm)
        self.output = self.ffn._forward(y, y, prenorm=self.pre_ffn_norm)
        return self.output
