"""Benchmark: GPT-2-small-shape bf16 prefill forward on one MI355X.

One step = one `Network.predict` of the notebook GPT composition (embedding, 12 decoder
blocks, final LayerNorm, tied LM head, SoftMax) over B=8 x T=1024 token ids that are already
resident in HBM. Prints one JSON line (see the fields below) with:
  value       tokens/s of the whole forward (8192 tokens / step time)
  roofline    the dense bf16 MFMA GEMMs (QKV, out-proj, FFN1, FFN2, LM head): algorithmic
              FLOPs / summed kernel time from HIP events around each launch, vs 2.5 PFLOP/s
  row_kernels standalone LayerNorm / RMSNorm / causal softmax / RoPE
              in GB/s of algorithmic bytes vs 8 TB/s, and vs a plain copy of the same
              bytes timed the same way (the measured ceiling at that size)
  cpu_baseline the NumPy restatement (oracle/) on a bounded sample of the same workload
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "torchless-nn_amd")
sys.path[:0] = [ROOT, PKG]
os.environ.setdefault("XP_RUNTIME", "MI355X")

import numpy as np  # noqa: E402

METRIC = "GPT fwd tokens/sec @1 GPU; norm/softmax/RoPE HBM GB/s; GEMM MFMA % of peak"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
CFG = dict(vocab=50257, ctx=1024, layers=12, d=768, heads=12, act="gelu")
BATCH, SEQ = 8, 1024


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gpt_forward_flops(B, T, cfg):
    C, V, L = cfg["d"], cfg["vocab"], cfg["layers"]
    M = B * T
    dense = L * 2 * M * C * (3 * C + C + 4 * C + 4 * C)
    head = 2 * M * C * V
    attn = L * B * cfg["heads"] * 2 * (2 * T * T * (C // cfg["heads"]))
    return dense, head, attn


def row_kernel_bench(xp, reps=20):
    """BASELINE config 2 standalone row kernels; GB/s of algorithmic bytes per call. Each
    rep uses its own buffers (rotated among >256 MB) so the 256 MB MALL cannot serve them."""
    out = {}
    rng = np.random.default_rng(0)

    def run_ms(fn, nbuf):
        for i in range(2):
            fn(i % nbuf)
        xp.synchronize()
        e0, e1 = xp.Event(), xp.Event()
        e0.record()
        for i in range(reps):
            fn(i % nbuf)
        e1.record()
        return e0.elapsed_ms(e1) / reps

    def copy_gbs(nbytes, nbuf):
        """A plain device copy (tl_cast fp32 -> fp32) moving the same bytes, half read and
        half written, over as many rotating buffers and timed the same way: the measured
        ceiling of a streaming kernel of this size (launch and ramp included)."""
        n = int(nbytes // 8)
        src = [xp.empty((n,), "fp32") for _ in range(nbuf)]
        dst = [xp.empty((n,), "fp32") for _ in range(nbuf)]
        lib, h = xp.lib(), xp.ctx().handle
        ms = run_ms(lambda i: xp.check(lib.tl_cast(h, src[i].ptr, dst[i].ptr, n, 0, 0)), nbuf)
        del src, dst
        return 8.0 * n / (ms * 1e-3) / 1e9

    def timed(name, fn, nbytes, nbuf):
        ms = run_ms(fn, nbuf)
        gbs = nbytes / (ms * 1e-3) / 1e9
        cp = copy_gbs(nbytes, nbuf)
        out[name] = {"gbs": round(gbs, 1), "us": round(ms * 1e3, 2),
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": int(nbytes),
                     "copy_gbs": round(cp, 1), "frac_of_copy": round(gbs / cp, 4)}
        log(f"{name}: {out[name]}")

    for dt, es in (("fp32", 4), ("bf16", 2)):
        R, Cn = 16384, 4096
        host = rng.standard_normal((R, Cn)).astype(np.float32)
        xs = [xp.array(host, dtype=dt) for _ in range(2)]
        ys = [xp.empty((R, Cn), dt) for _ in range(2)]
        g = xp.array(rng.standard_normal(Cn).astype(np.float32), dtype=dt)
        b = xp.array(rng.standard_normal(Cn).astype(np.float32), dtype=dt)
        nb = es * (2.0 * R * Cn + 2 * Cn)
        timed(f"layernorm_{dt}_16384x4096", lambda i: xp.layernorm(xs[i], g, b, np.float32(1e-5), out=ys[i]), nb, 2)
        timed(f"rmsnorm_{dt}_16384x4096", lambda i: xp.rmsnorm(xs[i], g, np.float32(1e-6), out=ys[i]),
              es * (2.0 * R * Cn + Cn), 2)
        del xs, ys
        B, H, T = 8, 12, 1024
        s_host = rng.standard_normal((B, H, T, T)).astype(np.float32)
        ss = [xp.array(s_host, dtype=dt) for _ in range(2)]
        ps = [xp.empty((B, H, T, T), dt) for _ in range(2)]
        del s_host
        kept = B * H * T * (T + 1) / 2
        timed(f"softmax_causal_{dt}_8x12x1024x1024",
              lambda i: xp.softmax(ss[i], causal=True, period=T, out=ps[i]), es * (kept + B * H * T * T), 2)
        del ss, ps
        D = 64
        nrot = 12  # 12 x (25..50 MB in + out) rotated > 256 MB
        r_host = rng.standard_normal((B, H, T, D)).astype(np.float32)
        rx = [xp.array(r_host, dtype=dt) for _ in range(nrot)]
        ry = [xp.empty((B, H, T, D), dt) for _ in range(nrot)]
        tab = xp.rope_table(T, D, 10000.0)
        timed(f"rope_{dt}_8x12x1024x64", lambda i: xp.rope(rx[i], tab, out=ry[i]), es * 2.0 * B * H * T * D, nrot)
        del rx, ry
        # the config-3 vocabulary softmax: [B*T, 50257] logits at a row pitch of 50264
        R, V, P = 8192, 50257, 50264
        vx = []
        for i in range(2):
            full = xp.random_normal((R, P), seed=7, stream=i, std=3.0, dtype=dt)
            vx.append(xp.DeviceTensor((R, V), full.dtype, pitch=P, buf=full.buf, offset=full.offset))
        vy = [xp.empty((R, V), dt, pitch=P) for _ in range(2)]
        timed(f"softmax_vocab_{dt}_8192x50257", lambda i: xp.softmax(vx[i], out=vy[i]), es * 2.0 * R * V, 2)
        del vx, vy
    return out


def gemma_bench(xp, prefill_reps=3, decode_steps=128, graph=True):
    """Gemma-style bf16 decoder (2.5B weights, device-seeded N(0,0.02)):
    prefill B=4 x T=2048 into the KV cache, then `decode_steps` greedy steps at M=4 whose
    ids are fed back on the device. Decode is weight-streaming: every step reads all
    GEMM weights once (the packed [N, K] copies) plus the live KV cache."""
    import gemma
    cfg = gemma.GEMMA_2B
    B, T = 4, 2048
    log("building Gemma-style config-5 model (bf16, device-seeded)")
    model = gemma.build_gemma(cfg, "bf16")
    gemma.seed_gemma(model, 0, 0.02, device=True)
    ids = xp.array(np.random.default_rng(2).integers(0, cfg["vocab"], (B, T)).astype(np.int32))
    cache = model.new_cache(B, T + decode_steps)
    model.forward(ids, cache, 0)  # warm-up; packs every weight once
    xp.synchronize()
    e0, e1 = xp.Event(), xp.Event()
    e0.record()
    for _ in range(prefill_reps):
        logits = model.forward(ids, cache, 0)
    e1.record()
    prefill_ms = e0.elapsed_ms(e1) / prefill_reps
    # the prefill a generation runs: logits of each sequence's last position only
    e0.record()
    for _ in range(prefill_reps):
        model.forward(ids, cache, 0, last_only=True)
    e1.record()
    prefill_last_ms = e0.elapsed_ms(e1) / prefill_reps
    # per-family kernel time of one more full prefill (HIP events around every launch)
    xp.kprof_reset()
    xp.kprof_enable(list(xp.KFAMILY))
    logits = model.forward(ids, cache, 0)
    xp.synchronize()
    pfam = {f: xp.kprof_query(f) for f in xp.KFAMILY}
    xp.kprof_enable([])
    prefill_breakdown = {f: {"ms": round(r["ms"], 3), "launches": r["launches"],
                             "tflops": round(r["flops"] / (r["ms"] * 1e-3) / 1e12, 1) if r["flops"] else None}
                         for f, r in pfam.items() if r["launches"]}
    C, F, V, L = cfg["d"], cfg["ffn"], cfg["vocab"], cfg["layers"]
    Hq, Hkv, D = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    M = B * T
    dense_w = L * (C * (Hq + 2 * Hkv) * D + Hq * D * C + C * 2 * F + F * C)
    attn = L * B * Hq * 2 * 2 * D * (T * (T + 1) / 2)  # causal QK^T and PV
    prefill_flops = 2 * M * (dense_w + C * V) + attn

    def step(nxt, pos):
        lg = model.forward(nxt.reshape(B, 1), cache, pos)
        return xp.argmax(model.last_rows(lg))

    nxt = xp.argmax(model.last_rows(logits))
    for w in range(3):  # warm-up decode steps (positions rewritten by the timed loop)
        step(nxt, T + w)
    xp.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for t in range(decode_steps):
        nxt = step(nxt, T + t)
    e1.record()
    xp.synchronize()
    wall = (time.perf_counter() - t0) / decode_steps * 1e3
    decode_ms = e0.elapsed_ms(e1) / decode_steps
    # the same steps as one captured HIP graph each: the position lives on the device, so
    # one capture replays at every position (same kernels and results as the loop above)
    import layers
    tok = xp.empty((B,), xp.int64)
    xp.argmax(model.last_rows(logits), out=tok)
    dpos = layers.DevicePosition(T, 1, D, cfg["rope_base"])

    def gstep():
        model.decode_step(tok, cache, dpos)
        dpos.advance(1)

    gstep()  # eager at the device position: everything the capture needs exists after it
    graph_ms = gwall = float("nan")
    if graph:
        with xp.capture() as g:
            gstep()
        dpos.pos.set(np.array([T], np.int64))
        xp.synchronize()
        t0 = time.perf_counter()
        e0.record()
        for t in range(decode_steps):
            g.launch()
        e1.record()
        xp.synchronize()
        gwall = (time.perf_counter() - t0) / decode_steps * 1e3
        graph_ms = e0.elapsed_ms(e1) / decode_steps
        g.destroy()
    # per-family kernel time of the decode steps (HIP events around every launch)
    xp.kprof_reset()
    xp.kprof_enable(list(xp.KFAMILY))
    n_prof = 16
    for t in range(n_prof):
        nxt = step(nxt, T + t)
    xp.synchronize()
    fam = {f: xp.kprof_query(f) for f in xp.KFAMILY}
    xp.kprof_enable([])
    decode_breakdown = {f: {"ms_per_step": round(r["ms"] / n_prof, 4),
                            "launches_per_step": r["launches"] // n_prof,
                            "gbs": round(r["bytes"] / (r["ms"] * 1e-3) / 1e9, 1)}
                        for f, r in fam.items() if r["launches"]}
    w_bytes = 2.0 * (dense_w + C * V)
    kv_bytes = 2.0 * L * B * Hkv * D * 2 * (T + decode_steps / 2)
    out = {
        "workload": "Gemma-style decoder (BASELINE config 5): vocab 256000, 18 layers, d 2048, "
                    "8 q heads / 1 kv head of 256, GeGLU FFN 16384; bf16, weights N(0,0.02) "
                    "device-seeded; prefill B=4 T=2048, then greedy decode with KV cache",
        "prefill_ms": round(prefill_ms, 3),
        "prefill_last_only_ms": round(prefill_last_ms, 3),
        "prefill_tokens_per_s": round(M / (prefill_ms * 1e-3), 1),
        "prefill_tflops": round(prefill_flops / (prefill_ms * 1e-3) / 1e12, 1),
        "prefill_flops": prefill_flops,
        "prefill_kernel_breakdown": prefill_breakdown,
        "decode_steps": decode_steps,
        "decode_ms_per_step": round(decode_ms, 4),
        "decode_wall_ms_per_step": round(wall, 4),
        "decode_tokens_per_s": round(B / (decode_ms * 1e-3), 1),
        "decode_bytes_per_step": w_bytes + kv_bytes,
        "decode_hbm_gbs": round((w_bytes + kv_bytes) / (decode_ms * 1e-3) / 1e9, 1),
        "decode_hbm_frac": round((w_bytes + kv_bytes) / (decode_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "decode_kernel_breakdown": decode_breakdown,
    }
    if graph:
        out.update({
            "decode_graph_ms_per_step": round(graph_ms, 4),
            "decode_graph_wall_ms_per_step": round(gwall, 4),
            "decode_graph_tokens_per_s": round(B / (graph_ms * 1e-3), 1),
            "decode_graph_hbm_frac": round((w_bytes + kv_bytes) / (graph_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
    log(f"gemma config 5: {json.dumps(out)}")
    del model, cache, logits
    return out


def vit_bench(xp, steps=10, warmup=3):
    """ViT-S/4 bf16 classifier forward over 512 CIFAR-shaped images
    (65 tokens each) already in HBM; per-step kernel breakdown from HIP events."""
    import vit
    cfg = vit.VIT_S4
    B = 512
    log("building ViT-S/4 config-4 model (bf16)")
    net = vit.build_vit(cfg, "bf16")
    vit.seed_vit(net, 0, 0.02)
    rng = np.random.default_rng(3)
    pix = rng.random((B, 3, 32, 32), dtype=np.float32)
    x = xp.array((pix - np.float32(0.5)) / np.float32(np.sqrt(1.0 / 12.0)), dtype="bf16")
    for _ in range(warmup):
        net.predict(x)
    xp.synchronize()
    e0, e1 = xp.Event(), xp.Event()
    e0.record()
    for _ in range(steps):
        net.predict(x)
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    xp.kprof_reset()
    xp.kprof_enable(list(xp.KFAMILY))
    for _ in range(steps):
        net.predict(x)
    xp.synchronize()
    fam = {f: xp.kprof_query(f) for f in xp.KFAMILY}
    xp.kprof_enable([])
    d, L, T = cfg["d"], cfg["layers"], 65
    M = B * T
    dense = L * 2 * M * d * 12 * d + 2 * B * 64 * 48 * d + 2 * B * d * cfg["classes"]
    attn = L * B * cfg["heads"] * 2 * 2 * T * T * (d // cfg["heads"])
    out = {
        "workload": "ViT-S/4 classifier forward (BASELINE config 4): 512 images 3x32x32, patch 4 "
                    "(64 tokens + CLS), 8 encoder layers, d 384, 6 heads, MLP 1536 GeLU, 10 "
                    "classes; bf16, weights N(0,0.02) seeded, pixels uniform normalised",
        "ms_per_step": round(ms, 4),
        "images_per_s": round(B / (ms * 1e-3), 1),
        "tokens_per_s": round(M / (ms * 1e-3), 1),
        "tflops": round((dense + attn) / (ms * 1e-3) / 1e12, 1),
        "flops": dense + attn,
        "kernel_breakdown": {f: {"ms_per_step": round(r["ms"] / steps, 4),
                                 "launches_per_step": r["launches"] // steps}
                             for f, r in fam.items() if r["launches"]},
    }
    log(f"vit config 4: {json.dumps(out)}")
    del net, x
    return out


VENDOR_SHAPES = {"qkv": (768, 2304), "out_proj": (768, 768), "ffn1": (768, 3072),
                 "ffn2": (3072, 768), "lm_head": (768, 50257)}  # (K, N) at M = 8192


def vendor_gemm_child(reps=20):
    """Child process of vendor_gemm_compare: times PyTorch's F.linear (bias, bf16; hipBLASLt
    on ROCm) at the config-3 shapes and prints {name: microseconds} as JSON. It runs in its
    own process because PyTorch carries its own HIP runtime, which does not see the GPU in a
    process where libtl.so has already loaded the system one."""
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "torch sees no GPU"}))
        return
    M, out = BATCH * SEQ, {}
    for name, (K, N) in VENDOR_SHAPES.items():
        a = torch.randn(M, K, device="cuda", dtype=torch.bfloat16)
        w = torch.randn(N, K, device="cuda", dtype=torch.bfloat16) * 0.02
        b = torch.randn(N, device="cuda", dtype=torch.bfloat16) * 0.02
        for _ in range(3):
            torch.nn.functional.linear(a, w, b)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(reps):
            torch.nn.functional.linear(a, w, b)
        t1.record()
        torch.cuda.synchronize()
        out[name] = t0.elapsed_time(t1) / reps * 1e3
        del a, w, b
    print(json.dumps(out), flush=True)


def vendor_gemm_compare(xp, reps=20):
    """The config-3 dense products (M = 8192, bias epilogue, bf16) through this library's
    tl_gemm and through the vendor library behind PyTorch's F.linear (hipBLASLt on ROCm),
    each timed with events over `reps` back-to-back calls on hot operands: a reference point
    for what the matrix cores reach at these shapes, not part of the product."""
    import subprocess
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-child"],
                           capture_output=True, text=True, timeout=300)
        vend = json.loads(r.stdout.strip().splitlines()[-1])
    except Exception as e:  # noqa: BLE001  (a measurement leg only)
        log(f"vendor GEMM comparison skipped: {type(e).__name__}: {e}")
        return None
    if "error" in vend:
        log(f"vendor GEMM comparison skipped: {vend['error']}")
        return None
    M, out = BATCH * SEQ, {}
    for name, (K, N) in VENDOR_SHAPES.items():
        a = xp.random_normal((M, K), 1, 0, std=1.0, dtype="bf16")
        bt = xp.random_normal((N, K), 2, 0, std=0.02, dtype="bf16")
        bias = xp.random_normal((N,), 3, 0, std=0.02, dtype="bf16")
        ldc = (N + 7) // 8 * 8
        c = xp.empty((M, N), "bf16", pitch=ldc)
        fn = lambda: xp.gemm(a, bt, M=M, N=N, K=K, lda=K, ldb=K, b_layout=xp.TL_B_NK, C=c,
                             ldc=ldc, bias=bias)
        fn()
        e0, e1 = xp.Event(), xp.Event()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        ours = e0.elapsed_ms(e1) / reps * 1e3
        del a, bt, bias, c
        fl = 2.0 * M * N * K
        out[name] = {"tl_us": round(ours, 1), "vendor_us": round(vend[name], 1),
                     "tl_tflops": round(fl / (ours * 1e-6) / 1e12, 1),
                     "vendor_tflops": round(fl / (vend[name] * 1e-6) / 1e12, 1)}
    log(f"vendor GEMM comparison: {json.dumps(out)}")
    return out


def gpt2_fp32_bench(xp, steps=3, warmup=1):
    """The headline model in fp32, the reference's default FLOAT_TYPE (what a drop-in user
    runs without XP_FLOAT=bf16): products on the fp32 matrix cores and attention fused in
    fp32 (16x16x4 fp32 MFMA, online softmax)."""
    import gpt
    net, _ = gpt.build_gpt(CFG, dtype="fp32")
    gpt.seed_parameters(net, 0)
    ids = xp.array(np.random.default_rng(1).integers(0, CFG["vocab"], (BATCH, SEQ)).astype(np.int32))
    for _ in range(warmup):
        net.predict(ids)
    xp.synchronize()
    e0, e1 = xp.Event(), xp.Event()
    e0.record()
    for _ in range(steps):
        net.predict(ids)
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    xp.kprof_reset()
    xp.kprof_enable(list(xp.KFAMILY))
    net.predict(ids)
    xp.synchronize()
    fam = {f: xp.kprof_query(f) for f in xp.KFAMILY}
    xp.kprof_enable([])
    out = {"workload": "GPT-2-small-shape prefill (config 3 shape) in fp32: B 8, T 1024",
           "ms_per_step": round(ms, 3), "tokens_per_s": round(BATCH * SEQ / (ms * 1e-3), 1),
           "kernel_breakdown": {f: {"ms_per_step": round(r["ms"], 3), "launches_per_step": r["launches"],
                                    "tflops": round(r["flops"] / (r["ms"] * 1e-3) / 1e12, 1) if r["flops"] else None}
                                for f, r in fam.items() if r["launches"]}}
    log(f"gpt2 fp32: {json.dumps(out)}")
    del net
    return out


CHAR_CFG = dict(vocab=65, ctx=128, layers=4, d=128, heads=4, act="gelu")


def char_gpt_bench(xp, steps=50, warmup=5):
    """BASELINE config 1, the reference's own CPU-runnable case: the char-level GPT forward in
    fp32 (vocab 65, ctx 128, 4 layers, d 128, 4 heads, GeLU, batch 4 x 128 ids) on the device.
    Too small for a roofline (0.95 GFLOP, ~50 launches): reported as latency."""
    import gpt
    net, _ = gpt.build_gpt(CHAR_CFG, dtype="fp32")
    gpt.seed_parameters(net, 0)
    ids = xp.array(np.random.default_rng(0).integers(0, 65, (4, 128)).astype(np.int32))
    for _ in range(warmup):
        net.predict(ids)
    xp.synchronize()
    e0, e1 = xp.Event(), xp.Event()
    e0.record()
    for _ in range(steps):
        net.predict(ids)
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    t0 = time.perf_counter()
    for _ in range(steps):
        net.predict(ids)
    host_ms = (time.perf_counter() - t0) / steps * 1e3  # issue time (the queue runs ahead)
    xp.synchronize()
    # the same forward captured once as a HIP graph and replayed (one host call per forward)
    fwd = net.capture(ids)
    fwd(ids)
    xp.synchronize()
    e0.record()
    t0 = time.perf_counter()
    for _ in range(steps):
        fwd(ids)
    graph_host_ms = (time.perf_counter() - t0) / steps * 1e3
    e1.record()
    graph_ms = e0.elapsed_ms(e1) / steps
    fwd.destroy()
    xp.kprof_reset()
    xp.kprof_enable(list(xp.KFAMILY))
    for _ in range(steps):
        net.predict(ids)
    xp.synchronize()
    fam = {f: xp.kprof_query(f) for f in xp.KFAMILY}
    xp.kprof_enable([])
    out = {"workload": "char-level GPT forward (BASELINE config 1): vocab 65, ctx 128, 4 layers, "
                       "d 128, 4 heads, GeLU, fp32, batch 4 x 128 token ids, weights seeded",
           "ms_per_step": round(ms, 4), "tokens_per_s": round(512 / (ms * 1e-3), 1),
           "host_issue_ms_per_step": round(host_ms, 4),
           "graph_ms_per_step": round(graph_ms, 4),
           "graph_tokens_per_s": round(512 / (graph_ms * 1e-3), 1),
           "graph_host_ms_per_step": round(graph_host_ms, 4),
           "kernel_breakdown": {f: {"ms_per_step": round(r["ms"] / steps, 4),
                                    "launches_per_step": r["launches"] // steps}
                                for f, r in fam.items() if r["launches"]}}
    log(f"char gpt config 1: {out}")
    return out


def cpu_baseline_char_gpt(runs=3):
    """Config 1 on the host: the oracle's NumPy forward (op for op the reference's
    XP_RUNTIME=CPU path), median of `runs` after one warm-up."""
    from oracle import numpy_ref as ref
    params = ref.gpt_params(CHAR_CFG, 0)
    ids = np.random.default_rng(0).integers(0, 65, (4, 128))
    ref.gpt_forward(ids, params, CHAR_CFG)
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        ref.gpt_forward(ids, params, CHAR_CFG)
        ts.append(time.perf_counter() - t0)
    ms = float(np.median(ts)) * 1e3
    return {"ms_per_step": round(ms, 3), "tokens_per_s": round(512 / (ms * 1e-3), 1),
            "kind": "port", "sample": f"the whole config-1 forward, median of {runs} runs"}


def _blas_info():
    """(threads, "vendor version") of the BLAS NumPy calls, from threadpoolctl."""
    try:
        from threadpoolctl import threadpool_info
        blas = [i for i in threadpool_info() if i.get("user_api") == "blas"]
        if blas:
            b = blas[0]
            return int(b.get("num_threads", 1)), f"{b.get('internal_api', '?')} {b.get('version', '?')}"
    except Exception:
        pass
    return 1, "unknown"


def cpu_baseline(sample_seqs=2, sample_T=SEQ, runs=3):
    """The oracle's NumPy forward (op for op the reference's CPU runtime) on a bounded sample
    of the workload: `sample_seqs` sequences of T tokens of the same model; one warm-up run,
    then the median of `runs`."""
    from oracle import numpy_ref as ref
    threads, blas = _blas_info()
    params = ref.gpt_params(CFG, 0)
    ids = np.random.default_rng(1).integers(0, CFG["vocab"], (sample_seqs, sample_T))
    ref.gpt_forward(ids, params, CFG)
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        ref.gpt_forward(ids, params, CFG)
        ts.append(time.perf_counter() - t0)
    dt = float(np.median(ts))
    return {"value": round(sample_seqs * sample_T / dt, 1), "unit": "tokens/s",
            "cores": threads, "kind": "port",
            "sample": (f"{sample_seqs} x {sample_T} tokens of the same GPT-2-small-shape forward, "
                       f"fp32 NumPy (oracle/numpy_ref.py); one warm-up, then the median of {runs} "
                       f"runs ({', '.join(f'{t:.2f}' for t in ts)} s); sgemm multi-threaded on "
                       f"{threads} threads of {blas} (OPENBLAS_NUM_THREADS="
                       f"{os.environ.get('OPENBLAS_NUM_THREADS', 'unset')}), NumPy ufuncs "
                       f"single-threaded; os.cpu_count()={os.cpu_count()}, "
                       f"affinity={len(os.sched_getaffinity(0))}")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-row-kernels", action="store_true")
    ap.add_argument("--only-row-kernels", action="store_true",
                    help="only time the standalone row kernels (a tuning run, no model)")
    ap.add_argument("--no-gemma", action="store_true", help="skip the config-5 decoder section")
    ap.add_argument("--no-vit", action="store_true", help="skip the config-4 ViT section")
    ap.add_argument("--no-gpt2-fp32", action="store_true", help="skip the fp32 GPT-2 section")
    ap.add_argument("--no-char", action="store_true", help="skip the config-1 section")
    ap.add_argument("--no-graph", action="store_true",
                    help="skip the config-5 decode replayed from a HIP graph (profiling runs)")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip the hipBLASLt (PyTorch F.linear) GEMM comparison")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a plain fp32 copy kernel of 256 MiB three times (the "
                         "reference dispatch for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--vendor-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.vendor_child:
        vendor_gemm_child()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    import tl_hip as xp
    import gpt
    xp.ctx()
    if args.calibrate_copy:
        n = 64 << 20  # 64 Mi fp32 = 256 MiB read + 256 MiB written per dispatch
        src, dst = xp.empty((n,), "fp32").fill(1.0), xp.empty((n,), "fp32")
        for _ in range(3):
            xp.check(xp.lib().tl_cast(xp.ctx().handle, src.ptr, dst.ptr, n, 0, 0))
        xp.synchronize()
        del src, dst
        log("copy calibration: 3 x cast_vec_kernel<float,float> over 256 MiB")
    if args.only_row_kernels:
        print(json.dumps({"row_kernels": row_kernel_bench(xp)}), flush=True)
        return
    log("building GPT-2-small-shape model (bf16) and seeding weights")
    net, _ = gpt.build_gpt(CFG, dtype="bf16")
    gpt.seed_parameters(net, 0)
    ids = xp.array(np.random.default_rng(1).integers(0, CFG["vocab"], (BATCH, SEQ)).astype(np.int32))
    xp.synchronize()

    for i in range(args.warmup):
        net.predict(ids)
    xp.synchronize()
    log(f"warmup done ({args.warmup} steps)")

    e0, e1 = xp.Event(), xp.Event()
    xp.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        out = net.predict(ids)
    e1.record()
    xp.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1) / args.steps
    tokens_s = BATCH * SEQ / (ms * 1e-3)
    log(f"timed {args.steps} steps: {ms:.3f} ms/step (event), wall {wall / args.steps * 1e3:.3f} ms/step")
    del out

    # per-launch kernel profile: the same K steps again with HIP events around every launch
    xp.kprof_reset()
    xp.kprof_enable(list(xp.KFAMILY))
    for _ in range(args.steps):
        net.predict(ids)
    xp.synchronize()
    fam = {f: xp.kprof_query(f) for f in xp.KFAMILY}
    xp.kprof_enable([])
    breakdown = {}
    for f, r in fam.items():
        if r["launches"]:
            breakdown[f] = {"ms_per_step": round(r["ms"] / args.steps, 4),
                            "launches_per_step": r["launches"] // args.steps,
                            "tflops": round(r["flops"] / (r["ms"] * 1e-3) / 1e12, 1) if r["flops"] else None,
                            "gbs": round(r["bytes"] / (r["ms"] * 1e-3) / 1e9, 1)}
    log(f"breakdown: {json.dumps(breakdown)}")
    g = fam["gemm_mfma"]
    achieved = g["flops"] / (g["ms"] * 1e-3) / 1e12 if g["ms"] else 0.0
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_traffic_gpt2_small_bf16_prefill.json")
    if os.path.exists(tpath):  # rocprofv3 FETCH_SIZE / WRITE_SIZE, calibrated (see the file)
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
    roofline = {"bound": "mfma", "kernel": "gemm_mfma_kernel (QKV, out-proj, FFN1, FFN2, LM head)",
                "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "avg_launch_us": round(g["ms"] / max(1, g["launches"]) * 1e3, 2),
                "flops_per_launch": round(g["flops"] / max(1, g["launches"])),
                "traffic": traffic, "traffic_unit": "bytes per launch (HBM, measured)"}

    rows = {} if args.no_row_kernels else row_kernel_bench(xp)
    gem = None if args.no_gemma else gemma_bench(xp, graph=not args.no_graph)
    vit_line = None if args.no_vit else vit_bench(xp)
    char = None if args.no_char else char_gpt_bench(xp)
    f32 = None if args.no_gpt2_fp32 else gpt2_fp32_bench(xp)
    vendor = None if args.no_vendor else vendor_gemm_compare(xp)
    cpu = None if args.no_cpu_baseline else cpu_baseline()
    if char is not None and not args.no_cpu_baseline:
        char["cpu_baseline"] = cpu_baseline_char_gpt()
        log(f"char gpt config 1 cpu baseline: {char['cpu_baseline']}")
    if cpu:
        log(f"cpu baseline: {cpu}")

    dense, head, attn = gpt_forward_flops(BATCH, SEQ, CFG)
    line = {
        "metric": METRIC, "value": round(tokens_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: weights N(0,0.02) seeded, token ids uniform in [0,50257) seeded",
        "config": {"workload": "GPT-2-small-shape decoder prefill (BASELINE config 3)",
                   "global_batch": BATCH, "seq_len": SEQ, "vocab": CFG["vocab"],
                   "layers": CFG["layers"], "d_model": CFG["d"], "heads": CFG["heads"],
                   "ffn": 4 * CFG["d"], "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "gemm_flops_per_step": {"dense": dense, "lm_head": head, "attention_full": attn},
        "kernel_breakdown": breakdown,
        "row_kernels": rows,
        "gemma_decoder": gem,
        "vit_classifier": vit_line,
        "char_gpt": char,
        "gpt2_fp32": f32,
        "vendor_gemm": vendor,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
