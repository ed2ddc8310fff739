"""HIP-graph capture and device-resident positions on the MI355X.

A decode step captured once and replayed must give exactly what the same step gives when
its calls run one by one: the device-position kernels (QKV cache write, RoPE over a cache
slice, decode attention) are checked bit for bit against their host-position forms at
positions across the cache, the graph-driven greedy loop against the eager loop (ids and
every KV-cache byte), and the runtime's capture rules (replays interleaved with eager work,
blocks a live graph writes kept from reuse, host syncs refused during a capture, staged
host-to-device copies taking the host data at call time)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F32 = np.float32


@pytest.fixture(scope="module")
def tl():
    import tl_hip
    tl_hip.ctx()
    import backend
    import gemma
    import layers
    return dict(xp=tl_hip, backend=backend, gemma=gemma, layers=layers)


def _bits(t):
    """Raw device bytes of a tensor (bf16 as uint16), for bit-exact comparison."""
    import tl_hip as xp
    raw = np.empty(t.nrows * t.pitch * t.dtype.itemsize, np.uint8)
    c = xp.ctx()
    xp.check(c.lib.tl_memcpy_d2h(c.handle, raw.ctypes.data, t.ptr, raw.nbytes))
    return raw


def _pos(xp, p):
    return xp.array(np.array([p], np.int64))


@pytest.mark.parametrize("cfg", [(4, 8, 1, 256, 2176, 1), (2, 4, 2, 64, 264, 2),
                                 (3, 12, 12, 32, 72, 1), (1, 8, 1, 128, 1024, 2)])
def test_attention_decode_dev_matches_host_offset(tl, cfg):
    """Bit-exact against tl_attention_fwd at the same position (the grid covers the capacity,
    blocks past the live keys add nothing), with NaN in the cache rows past the live keys."""
    xp = tl["xp"]
    B, Hq, Hkv, D, L, Tq = cfg
    rng = np.random.default_rng(B * 100 + D)
    q = xp.array(rng.standard_normal((B, Hq, Tq, D)).astype(F32), dtype="bf16")
    kh = rng.standard_normal((B, Hkv, L, D)).astype(F32)
    vh = rng.standard_normal((B, Hkv, D, L)).astype(F32)
    for pos in (0, 5, 63, 64, 200, L - Tq):
        if pos + Tq > L:
            continue
        k2, v2 = kh.copy(), vh.copy()
        k2[:, :, pos + Tq:, :] = np.nan
        v2[:, :, :, pos + Tq:] = np.nan
        k = xp.array(k2, dtype="bf16")
        vt = xp.array(v2, dtype="bf16")
        want = xp.empty((B, Tq, Hq * D), xp.bfloat16)
        got = xp.empty((B, Tq, Hq * D), xp.bfloat16)
        div = float(np.float32(D ** 0.5))
        xp.attention(q, k, vt, want, n_heads_q=Hq, n_heads_kv=Hkv, divisor=div, causal=True,
                     offset=pos, seq_k=pos + Tq)
        xp.attention_decode_dev(q, k, vt, got, _pos(xp, pos), n_heads_q=Hq, n_heads_kv=Hkv,
                                divisor=div)
        w, g = want.get(), got.get()
        assert np.all(np.isfinite(w)), (cfg, pos)
        assert np.array_equal(_bits(got), _bits(want)), (cfg, pos)


def _attn64(q, k, v, Hq, Hkv, pos):
    """float64 causal attention of q [B, Hq, Tq, D] at positions pos .. over keys k
    [B, Hkv, >= pos + Tq, D] and values v [B, Hkv, D, >= pos + Tq] -> [B, Tq, Hq * D]."""
    B, _, Tq, D = q.shape
    g = Hq // Hkv
    out = np.zeros((B, Tq, Hq * D))
    for b in range(B):
        for h in range(Hq):
            kk = k[b, h // g].astype(np.float64)
            vv = v[b, h // g].astype(np.float64)
            for t in range(Tq):
                n = pos + t + 1
                sc = kk[:n] @ q[b, h, t].astype(np.float64) / np.sqrt(D)
                e = np.exp(sc - sc.max())
                out[b, t, h * D:(h + 1) * D] = vv[:, :n] @ (e / e.sum())
    return out


@pytest.mark.parametrize("cfg", [(4, 8, 1, 256, 2176, 1), (2, 4, 2, 64, 264, 2),
                                 (1, 8, 1, 128, 1024, 2), (3, 4, 4, 64, 40, 1)])
def test_attention_decode_fused_rope(tl, cfg):
    """Decode attention taking unrotated queries and new cache keys with the RoPE table: the
    new keys are rotated in the cache (within rounding of the oracle's RoPE; no other row
    touched) and the output matches float64 attention over the oracle-rotated operands."""
    from oracle import numpy_ref as ref
    xp = tl["xp"]
    B, Hq, Hkv, D, L, Tq = cfg
    rng = np.random.default_rng(B * 7 + D + Tq)
    qh = ref.round_bf16(rng.standard_normal((B, Hq, Tq, D)).astype(F32))
    kh = ref.round_bf16(rng.standard_normal((B, Hkv, L, D)).astype(F32))
    vh = ref.round_bf16(rng.standard_normal((B, Hkv, D, L)).astype(F32))
    for pos in (0, 63, L - Tq):
        q = xp.array(qh, dtype="bf16")
        k = xp.array(kh, dtype="bf16")
        vt = xp.array(vh, dtype="bf16")
        out = xp.empty((B, Tq, Hq * D), xp.bfloat16)
        table = xp.rope_table(Tq, D, 10000.0, pos)
        xp.attention_decode_dev(q, k, vt, out, _pos(xp, pos), n_heads_q=Hq, n_heads_kv=Hkv,
                                divisor=float(np.float32(D ** 0.5)), rope=table)
        c, s = ref.rope_table(Tq, D, 10000.0, pos)
        knew = ref.round_bf16(ref.rope(kh[:, :, pos:pos + Tq], c, s))
        got_k = k.get()
        assert ref.max_rel(got_k[:, :, pos:pos + Tq], knew) <= 1e-2, pos
        assert np.array_equal(got_k[:, :, :pos], kh[:, :, :pos])
        assert np.array_equal(got_k[:, :, pos + Tq:], kh[:, :, pos + Tq:])
        kr = kh.copy()
        kr[:, :, pos:pos + Tq] = knew
        want = _attn64(ref.round_bf16(ref.rope(qh, c, s)), kr, vh, Hq, Hkv, pos)
        assert ref.max_rel(out.get(), want) <= 2e-2, pos


def test_attention_decode_dev_refuses_prefill_shapes(tl):
    xp = tl["xp"]
    q = xp.zeros((1, 8, 4, 64), xp.bfloat16)  # 8 heads x 4 rows share one kv head: 32 rows
    k = xp.zeros((1, 1, 64, 64), xp.bfloat16)
    vt = xp.zeros((1, 1, 64, 64), xp.bfloat16)
    out = xp.empty((1, 4, 512), xp.bfloat16)
    with pytest.raises(xp.TLError):
        xp.attention_decode_dev(q, k, vt, out, _pos(xp, 0), n_heads_q=8, n_heads_kv=1,
                                divisor=8.0)


@pytest.mark.parametrize("D,T", [(256, 1), (64, 2), (16, 1)])
def test_rope2_dev_matches_rope2_on_cache_slice(tl, D, T):
    """Queries and the cache rows at a device position rotate exactly as rope2 rotates them
    at the host position; rows past the capacity are left alone."""
    xp = tl["xp"]
    B, H, L = 2, 3, 40
    rng = np.random.default_rng(D + T)
    qh = rng.standard_normal((B, 4, T, D)).astype(F32)
    ch = rng.standard_normal((B, H, L, D)).astype(F32)
    for pos in (0, 7, L - T, L - 1):
        q1, c1 = xp.array(qh, dtype="bf16"), xp.array(ch, dtype="bf16")
        q2, c2 = xp.array(qh, dtype="bf16"), xp.array(ch, dtype="bf16")
        p = _pos(xp, pos)
        table = xp.empty((2, T, D // 2), xp.float32)
        xp.rope_table_dev(table, p)
        ref_table = xp.rope_table(T, D, 10000.0, pos)
        assert np.array_equal(table.get(), ref_table.get())
        xp.rope2_dev(q2, c2, table, p)
        n = min(T, L - pos)
        if n == T:
            ks = xp.DeviceTensor((B * H, T, D), xp.bfloat16, buf=c1.buf,
                                 offset=c1.offset + pos * D * 2)
            xp.rope2(q1, ks, ref_table, T, n_seq2=B * H, seq_stride2=L * D)
            assert np.array_equal(_bits(c2), _bits(c1)), pos
            assert np.array_equal(_bits(q2), _bits(q1)), pos
        else:  # the last position: its row rotated, nothing written past the capacity
            want = c1.get()
            got = c2.get()
            assert np.array_equal(got[:, :, :pos], want[:, :, :pos])
            assert not np.array_equal(got[:, :, pos], want[:, :, pos])
            xp.rope(q1, ref_table, out=q1)
            assert np.array_equal(_bits(q2), _bits(q1)), pos


CFGS = {
    "mqa256": dict(vocab=1000, ctx=512, layers=3, d=256, heads=8, kv_heads=1, head_dim=256,
                   ffn=1024, rope_base=10000.0),
    "gqa64": dict(vocab=777, ctx=256, layers=2, d=128, heads=4, kv_heads=2, head_dim=64,
                  ffn=384, rope_base=500.0),
}


def _model(tl, name, seed):
    cfg = CFGS[name]
    model = tl["gemma"].build_gemma(cfg, "bf16")
    tl["gemma"].seed_gemma(model, seed, 0.05)
    return model, cfg


@pytest.mark.parametrize("name,B,T", [("mqa256", 4, 130), ("gqa64", 3, 37)])
def test_device_position_step_matches_host_position_step(tl, name, B, T):
    """Four decode steps at a device position against the same steps at host positions on a
    second cache: logits, next ids and both caches bit-identical after every step."""
    xp, layers = tl["xp"], tl["layers"]
    model, cfg = _model(tl, name, 31)
    ids = np.random.default_rng(32).integers(0, cfg["vocab"], (B, T))
    ca, cb = model.new_cache(B, T + 8), model.new_cache(B, T + 8)
    la = model.forward(ids, ca, 0)
    lb = model.forward(ids, cb, 0)
    tok_a = xp.argmax(model.last_rows(la))
    tok_b = xp.empty((B,), xp.int64)
    xp.argmax(model.last_rows(lb), out=tok_b)
    dpos = layers.DevicePosition(T, 1, cfg["head_dim"], cfg["rope_base"])
    for t in range(4):
        la = model.forward(tok_a.reshape(B, 1), ca, T + t)
        tok_a = xp.argmax(model.last_rows(la))
        lb = model.decode_step(tok_b, cb, dpos)
        dpos.advance(1)
        # logits rows are padded to a multiple of 8 columns: compare the valid columns
        assert np.array_equal(lb.get().view(np.uint32), la.get().view(np.uint32)), t
        assert np.array_equal(tok_b.get(), tok_a.get()), t
        for i in range(cfg["layers"]):
            assert np.array_equal(_bits(cb.k[i]), _bits(ca.k[i])), (t, i)
            assert np.array_equal(_bits(cb.vt[i]), _bits(ca.vt[i])), (t, i)
    assert dpos.get() == T + 4


@pytest.mark.parametrize("name,B,T,n", [("mqa256", 4, 130, 20), ("gqa64", 3, 37, 3),
                                        ("gqa64", 2, 8, 2), ("mqa256", 1, 1, 9)])
def test_graph_greedy_matches_eager_greedy(tl, name, B, T, n):
    """generate_greedy replaying one captured decode step gives the eager loop's ids, and
    leaves every KV-cache byte as the eager loop leaves it."""
    model, cfg = _model(tl, name, 41)
    ids = np.random.default_rng(42 + T).integers(0, cfg["vocab"], (B, T))
    ce, cg = model.new_cache(B, T + n), model.new_cache(B, T + n)
    eager = model.generate_greedy(ids, n, cache=ce, graph=False)
    graph = model.generate_greedy(ids, n, cache=cg, graph=True)
    assert graph.shape == (B, n)
    assert np.array_equal(graph, eager)
    for i in range(cfg["layers"]):
        assert np.array_equal(_bits(cg.k[i]), _bits(ce.k[i])), i
        assert np.array_equal(_bits(cg.vt[i]), _bits(ce.vt[i])), i
    assert cg.length == ce.length == T + n - 1


def test_graph_replays_with_eager_work_between(tl):
    """A captured norm + product + add, replayed five times with eager uploads, kernels and
    frees between the replays: every replay equals the eager result for the current input."""
    xp = tl["xp"]
    rng = np.random.default_rng(51)
    M, C, N = 48, 256, 320
    x = xp.array(rng.standard_normal((M, C)).astype(F32), dtype="bf16")
    g = xp.array(rng.standard_normal(C).astype(F32), dtype="bf16")
    b = xp.array(rng.standard_normal(C).astype(F32), dtype="bf16")
    w = xp.array(rng.standard_normal((C, N)).astype(F32) / 16, dtype="bf16")
    import layers

    def step():
        y = xp.layernorm(x, g, b, 1e-5)
        z = layers.linear(y, w)
        return z + z

    want_first = _bits(step())  # eager: also packs w before the capture
    with xp.capture() as cap:
        out = step()
    for r in range(5):
        xh = rng.standard_normal((M, C)).astype(F32)
        x.set(xh)
        junk = [xp.layernorm(x, g, b, 1e-5) for _ in range(3)]  # eager allocations and frees
        del junk
        cap.launch()
        got = _bits(out)
        want = _bits(step())
        assert np.array_equal(got, want), r
        assert not np.array_equal(got, want_first), r
    cap.destroy()


def test_graph_held_blocks_are_not_reused(tl):
    """A block handed out during a capture and freed by the caller is still written by every
    replay, so the allocator keeps it from new tensors until the graph is destroyed."""
    xp = tl["xp"]
    rng = np.random.default_rng(61)
    x = xp.array(rng.standard_normal((64, 512)).astype(F32), dtype="bf16")
    g = xp.array(np.ones(512, F32), dtype="bf16")
    b = xp.array(np.zeros(512, F32), dtype="bf16")
    xp.layernorm(x, g, b, 1e-5)
    with xp.capture() as cap:
        y = xp.layernorm(x, g, b, 1e-5)
        keep = xp.layernorm(y, g, b, 1e-5)
        y_ptr = y.ptr
        del y
    fresh = [xp.array(np.full((64, 512), 7.0, F32), dtype="bf16") for _ in range(4)]
    assert all(f.ptr != y_ptr for f in fresh)
    cap.launch()
    xp.synchronize()
    for f in fresh:
        assert np.all(f.get() == 7.0)
    want = xp.layernorm(xp.layernorm(x, g, b, 1e-5), g, b, 1e-5)
    assert np.array_equal(_bits(keep), _bits(want))
    cap.destroy()
    assert np.array_equal(_bits(keep), _bits(want))  # the caller's tensor outlives the graph


def test_capture_refuses_host_syncs_and_recovers(tl):
    xp = tl["xp"]
    x = xp.array(np.ones((8, 64), F32), dtype="bf16")
    g = xp.array(np.ones(64, F32), dtype="bf16")
    b = xp.array(np.zeros(64, F32), dtype="bf16")
    with pytest.raises(xp.TLError):
        with xp.capture():
            xp.layernorm(x, g, b, 1e-5)
            xp.synchronize()
    with pytest.raises(xp.TLError):
        with xp.capture():
            x.get()
    with pytest.raises(xp.TLError):
        with xp.capture():
            x.set(np.zeros((8, 64), F32))
    y = xp.layernorm(x, g, b, 1e-5)  # the context works after a refused capture
    assert np.allclose(y.get(), 0.0)
    xp.synchronize()


def test_staged_host_copies_take_the_data_at_call_time(tl):
    """tl_memcpy_h2d returns before the copy runs (pinned staging behind queued work); the
    host buffer is overwritten right after each call, and each device buffer still holds
    what the host held at its call. Also one copy above the staging size (waits)."""
    xp = tl["xp"]
    c = xp.ctx()
    rng = np.random.default_rng(71)
    a = xp.array(rng.standard_normal((2048, 2048)).astype(F32), dtype="bf16")
    import layers
    host = np.empty(1 << 20, np.uint8)
    expect, bufs = [], []
    for i in range(12):
        layers.linear(a, a)  # keeps the stream busy while the copy is queued
        host[:] = rng.integers(0, 256, host.size, dtype=np.uint8)
        expect.append(host.copy())
        d = xp.empty((host.size,), xp.uint8)
        xp.check(c.lib.tl_memcpy_h2d(c.handle, d.ptr, host.ctypes.data, host.size))
        host[:] = 0
        bufs.append(d)
    for want, d in zip(expect, bufs):
        assert np.array_equal(_bits(d)[:want.size], want)
    big = rng.integers(0, 256, 80 << 20, dtype=np.uint8)
    d = xp.empty((big.size // 4,), xp.float32)
    layers.linear(a, a)
    xp.check(c.lib.tl_memcpy_h2d(c.handle, d.ptr, big.ctypes.data, big.size))
    want = big.copy()
    big[:] = 1
    assert np.array_equal(_bits(d), want)


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_captured_forward_matches_predict(tl, dt):
    """Network.capture: the char-level GPT forward (config 1 shape) replayed from one graph
    gives predict()'s probabilities bit for bit for several inputs, host and device ids,
    with eager forwards between the replays."""
    xp = tl["xp"]
    import gpt
    cfg = dict(vocab=65, ctx=128, layers=4, d=128, heads=4, act="gelu")
    net, _ = gpt.build_gpt(cfg, dtype=dt)
    gpt.seed_parameters(net, 3, 0.3 if dt == "fp32" else 0.05)
    rng = np.random.default_rng(4)
    first = rng.integers(0, 65, (4, 128)).astype(np.int32)
    fwd = net.capture(first)
    for r in range(4):
        ids = first if r == 0 else rng.integers(0, 65, (4, 128)).astype(np.int32)
        src = ids if r % 2 == 0 else xp.array(ids)
        got = fwd(src)
        want = net.predict(ids)  # eager, between replays
        assert got is fwd.output
        # probability rows are padded to 72 columns: compare the 65 valid ones
        assert np.array_equal(got.get().view(np.uint32), want.get().view(np.uint32)), r
    with pytest.raises(ValueError):
        fwd(xp.array(first[:2]))
    fwd.destroy()
