"""tl_attention_fwd_noalloc (the allocation-free variant of tl_attention_fwd) through the C
ABI: on the decode path its results equal tl_attention_fwd's bit for bit on two calls in a
row, the second smaller (the static scratch keeps the first call's contents); the prefill
path agrees too; calls from two contexts take the scratch in turn; a call whose partials
exceed the static scratch is refused."""
import ctypes

import numpy as np
import pytest

from oracle import numpy_ref as ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def xp():
    import tl_hip
    tl_hip.ctx()
    return tl_hip


def _operands(xp, rng, B, Hq, Hkv, Tq, Tk, L, D):
    def dev(shape, scale):
        return xp.array(ref.round_bf16(rng.standard_normal(shape).astype(np.float32) * scale),
                        dtype="bf16")
    q = dev((B, Hq, Tq, D), 1.0)
    k = dev((B, Hkv, L, D), 1.0)
    vt = dev((B, Hkv, D, L), 1.0)
    return q, k, vt


def _run(xp, fn, q, k, vt, B, Hq, Hkv, Tq, Tk, L, D, offset):
    out = xp.empty((B, Tq, Hq * D), "bf16")
    out.fill(7.0)
    c = xp.ctx()
    rc = getattr(c.lib, fn)(c.handle, q.ptr, k.ptr, vt.ptr, out.ptr, B, Hq, Hkv, Tq, Tk, D,
                            out.pitch, offset, float(np.float32(D ** 0.5)), 1, L,
                            xp.bfloat16.code)
    assert rc == 0, (fn, rc, xp.last_error())
    return out.get_raw()


# (B, Hq, Hkv, Tq, Tk, L, D): the config-5 decode step first, then a smaller call
CASES = [(4, 8, 1, 1, 2176, 2176, 256), (2, 4, 1, 1, 300, 304, 128)]


def _call(xp, c, fn, q, k, vt, out, B, Hq, Hkv, Tq, Tk, L, D, offset):
    rc = getattr(c.lib, fn)(c.handle, q.ptr, k.ptr, vt.ptr, out.ptr, B, Hq, Hkv, Tq, Tk, D,
                            out.pitch, offset, float(np.float32(D ** 0.5)), 1, L,
                            xp.bfloat16.code)
    assert rc == 0, (fn, rc, xp.last_error())


def test_noalloc_first_call_on_a_fresh_context_allocates_nothing(xp):
    """The no-alloc entry point called first on a fresh context (empty workspace, empty
    allocator) at the config-5 decode size: afterwards the context's workspace is still 0
    bytes and its allocator counters are unchanged, so the partials went to the static
    scratch. tl_attention_fwd on the same context then grows the workspace (the query sees
    it) and writes the same bytes."""
    B, Hq, Hkv, Tq, Tk, L, D = CASES[0]
    print(f"noalloc fresh-context case B={B} Hq={Hq} Tk={Tk} D={D}", flush=True)
    q, k, vt = _operands(xp, np.random.default_rng(11), B, Hq, Hkv, Tq, Tk, L, D)
    got, want = (xp.empty((B, Tq, Hq * D), "bf16").fill(7.0) for _ in range(2))
    xp.synchronize()  # operands were written on the default context's stream
    c2 = xp.Context(xp.ctx().device)
    try:
        assert c2.workspace_bytes() == 0
        stats = c2.mem_stats()
        _call(xp, c2, "tl_attention_fwd_noalloc", q, k, vt, got, B, Hq, Hkv, Tq, Tk, L, D, Tk - Tq)
        c2.sync()
        assert c2.workspace_bytes() == 0
        assert c2.mem_stats() == stats
        _call(xp, c2, "tl_attention_fwd", q, k, vt, want, B, Hq, Hkv, Tq, Tk, L, D, Tk - Tq)
        c2.sync()
        assert c2.workspace_bytes() > 0
    finally:
        c2.destroy()
    assert np.array_equal(got.get_raw(), want.get_raw())


def test_noalloc_calls_from_two_contexts_take_the_scratch_in_turn(xp):
    """Two fresh contexts (two streams) call the no-alloc entry point back to back with no
    host synchronisation in between, each on its own inputs at the config-5 decode size, so
    both calls' partials land at the same static scratch addresses. Each call's stream waits
    for the other context's last call, so every output equals tl_attention_fwd's bit for bit.
    Destroying the context that used the scratch last leaves the other one working."""
    B, Hq, Hkv, Tq, Tk, L, D = CASES[0]
    print(f"noalloc two-context case B={B} Hq={Hq} Tk={Tk} D={D}", flush=True)
    rng = np.random.default_rng(5)
    ops = [_operands(xp, rng, B, Hq, Hkv, Tq, Tk, L, D) for _ in range(2)]
    want = [_run(xp, "tl_attention_fwd", *o, B, Hq, Hkv, Tq, Tk, L, D, Tk - Tq) for o in ops]
    outs = [[xp.empty((B, Tq, Hq * D), "bf16").fill(7.0) for _ in range(3)] for _ in range(2)]
    xp.synchronize()
    ctxs = [xp.Context(xp.ctx().device) for _ in range(2)]
    try:
        for r in range(3):
            for i in range(2):
                _call(xp, ctxs[i], "tl_attention_fwd_noalloc", *ops[i], outs[i][r],
                      B, Hq, Hkv, Tq, Tk, L, D, Tk - Tq)
        for c in ctxs:
            c.sync()
        for i in range(2):
            for r in range(3):
                assert np.array_equal(outs[i][r].get_raw(), want[i]), (i, r)
        ctxs[1].destroy()  # the context that used the scratch last
        again = xp.empty((B, Tq, Hq * D), "bf16").fill(7.0)
        xp.synchronize()
        _call(xp, ctxs[0], "tl_attention_fwd_noalloc", *ops[0], again, B, Hq, Hkv, Tq, Tk, L, D,
              Tk - Tq)
        ctxs[0].sync()
        assert np.array_equal(again.get_raw(), want[0])
    finally:
        for c in ctxs:
            c.destroy()


def test_noalloc_decode_matches_allocating_entry_point_twice(xp):
    rng = np.random.default_rng(2024)
    for B, Hq, Hkv, Tq, Tk, L, D in CASES:
        print(f"noalloc decode case B={B} Hq={Hq} Hkv={Hkv} Tq={Tq} Tk={Tk} L={L} D={D}", flush=True)
        q, k, vt = _operands(xp, rng, B, Hq, Hkv, Tq, Tk, L, D)
        off = Tk - Tq
        want = _run(xp, "tl_attention_fwd", q, k, vt, B, Hq, Hkv, Tq, Tk, L, D, off)
        got = _run(xp, "tl_attention_fwd_noalloc", q, k, vt, B, Hq, Hkv, Tq, Tk, L, D, off)
        assert np.array_equal(got, want)
        # and both agree with the float64 definition
        qf, kf, vf = (xp.bf16_bits_to_f32(t.get_raw()).reshape(t.shape) for t in (q, k, vt))
        s = np.einsum("bhtd,bkd->bhtk", qf.astype(np.float64), kf[:, 0, :Tk].astype(np.float64))
        s /= np.sqrt(D)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        o = np.einsum("bhtk,bdk->bthd", p, vf[:, 0, :, :Tk].astype(np.float64)).reshape(B, Tq, Hq * D)
        assert ref.max_rel(xp.bf16_bits_to_f32(got).reshape(o.shape), o) <= 2e-2
    xp.synchronize()


def test_noalloc_prefill_matches(xp):
    B, Hq, Hkv, Tq, Tk, L, D = 2, 4, 2, 130, 130, 136, 64
    rng = np.random.default_rng(7)
    q, k, vt = _operands(xp, rng, B, Hq, Hkv, Tq, Tk, L, D)
    want = _run(xp, "tl_attention_fwd", q, k, vt, B, Hq, Hkv, Tq, Tk, L, D, 0)
    got = _run(xp, "tl_attention_fwd_noalloc", q, k, vt, B, Hq, Hkv, Tq, Tk, L, D, 0)
    assert np.array_equal(got, want)


def test_noalloc_rejects_partials_beyond_its_scratch(xp):
    # 64 x 1 kv heads x 34 blocks of 64 keys x 16 x (256 + 2) floats > 16 MiB
    B, Hq, Hkv, Tq, Tk, L, D = 64, 8, 1, 1, 2176, 2176, 256
    q = xp.empty((B, Hq, Tq, D), "bf16")
    k = xp.empty((B, Hkv, L, D), "bf16")
    vt = xp.empty((B, Hkv, D, L), "bf16")
    out = xp.empty((B, Tq, Hq * D), "bf16")
    c = xp.ctx()
    rc = c.lib.tl_attention_fwd_noalloc(c.handle, q.ptr, k.ptr, vt.ptr, out.ptr, B, Hq, Hkv, Tq,
                                        Tk, D, out.pitch, Tk - 1, 16.0, 1, L, xp.bfloat16.code)
    assert rc == xp.TL_ERR_INVALID
    assert "allocation-free" in xp.last_error()
    xp.synchronize()
