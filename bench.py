"""Benchmark of the uLLM attention path on one MI355X.

Headline workload: Qwen2.5-1.5B-shaped decode
attention -- batch 1, 12 query heads, 2 KV heads, head_dim 128, f16 KV cache
of 4096 positions, 28 layers back to back.  One step = the attention of all
28 layers for one decoded token, inputs resident in HBM.  The KV sets rotate
over >= 512 MiB so the 256 MiB Infinity Cache cannot serve them.

Also reported on the same line: causal prefill (configs[2], Qwen3-4B-shaped,
S=2048 bf16) in TFLOP/s, the cfg1 (f32, configs[0]) and cfg4 (Gemma-3 head_dim
256: a 6-layer sliding-window/global decode group and its S=1024 prefill)
rows, long-context decode (configs[4], 32K bf16), the roofline of the
dominant kernel, the CPU oracle on a bounded sample, and the GPU outputs of
the SplitMix64 inputs against the oracle's.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only PART] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode-attn µs/layer + HBM GB/s at 4K ctx; prefill-attn TFLOP/s (1 GPU)"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", choices=["all", "decode", "prefill", "long", "append", "proj",
                                       "matmul", "paged", "cfg1", "cfg4", "f32prefill", "f32decode",
                                       "copy",
                                       "floor"],
                    default="all")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    return ap.parse_args()


def decode_workload(torch, A, H, Hk, D, L, n_layer, dt, min_bytes, windows=None, first=None):
    """Rotating sets of per-layer (q, K, V) plus one captured graph per set.
    windows[l]: the sliding window of layer l (0: global).  first: (q, K, V)
    CPU tensors for layer 0 of set 0 (the SplitMix64 layer the CPU baseline
    runs too); every other layer is torch-random."""
    dev = torch.device("cuda")
    windows = windows or [0] * n_layer
    esz = torch.finfo(dt).bits // 8
    visible = [min(L, w) if w > 0 else L for w in windows]
    layer_bytes = [2 * n * Hk * D * esz for n in visible]
    alloc = 2 * L * Hk * D * esz * n_layer
    n_sets = max(1, math.ceil(min_bytes / alloc))
    g = torch.Generator(device=dev).manual_seed(1234)
    sets = []
    for _ in range(n_sets):
        k = torch.randn(n_layer, L, Hk * D, generator=g, device=dev).to(dt)
        v = torch.randn(n_layer, L, Hk * D, generator=g, device=dev).to(dt)
        q = torch.randn(n_layer, 1, H, D, generator=g, device=dev)
        sets.append((q, k, v))
    if first is not None:
        sets[0][0][0].copy_(first[0].view(1, H, D))
        sets[0][1][0].copy_(first[1])
        sets[0][2][0].copy_(first[2])
    lens = torch.tensor([L], dtype=torch.int32, device=dev)
    nws = max(A.decode_workspace_bytes(1, H, Hk, D, L, w) for w in set(windows))
    ws = torch.zeros(max(nws, 256), dtype=torch.uint8, device=dev)
    out = torch.empty(n_layer, 1, H, D, device=dev)
    scale = 1.0 / math.sqrt(D)

    def step_eager(si, events=None):
        q, k, v = sets[si]
        for li in range(n_layer):
            if events is not None:
                events[li][0].record()
            A.attn_decode(q[li], k[li], v[li], lens, L, Hk, window=windows[li], scale=scale,
                          out=out[li], workspace=ws)
            if events is not None:
                events[li][1].record()

    # Warm the kernels, then capture one graph per set (no memsets inside).
    for si in range(n_sets):
        step_eager(si)
    torch.cuda.synchronize()
    graphs = []
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        for si in range(n_sets):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=cap):
                step_eager(si)
            graphs.append(gr)
    torch.cuda.current_stream().wait_stream(cap)
    torch.cuda.synchronize()
    return dict(sets=sets, graphs=graphs, step_eager=step_eager, layer_bytes=layer_bytes,
                n_sets=n_sets, out=out, n_layer=n_layer)


def first_layer_out(torch, wl):
    """Output of layer 0 of set 0 after an eager pass (the synth layer)."""
    wl["step_eager"](0)
    torch.cuda.synchronize()
    return wl["out"][0].reshape(-1).cpu().numpy()


def time_graph_steps(torch, wl, steps, warmup):
    graphs, n = wl["graphs"], wl["n_sets"]
    for i in range(warmup):
        graphs[i % n].replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    t0.record()
    for i in range(steps):
        graphs[i % n].replay()
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    return t0.elapsed_time(t1) / steps, wall


def bench_decode(torch, A, args, H, Hk, D, L, n_layer, dt, label, windows=None, first=None):
    wl = decode_workload(torch, A, H, Hk, D, L, n_layer, dt, 2 * MALL_BYTES, windows, first)
    ms_step, wall = time_graph_steps(torch, wl, args.steps, args.warmup)
    # One decode-attention op per layer = the split-KV kernel plus its merge
    # kernel, back to back in the graph; events bracket the whole timed region
    # on the stream the graphs run on.
    us_layer = ms_step * 1000.0 / n_layer
    lb = sum(wl["layer_bytes"]) / n_layer  # mean algorithmic bytes per layer
    res = dict(label=label, ms_per_step=ms_step, us_per_layer=us_layer,
               gbps_step=lb / (us_layer * 1e3), layer_bytes=lb, n_sets=wl["n_sets"],
               wall_s=wall, step_bytes=sum(wl["layer_bytes"]))
    if first is not None:
        res["first_out"] = first_layer_out(torch, wl)
    del wl
    torch.cuda.empty_cache()
    return res


def bench_prefill(torch, A, args, S, H, Hk, D, dt, window=0, first=None):
    """Causal prefill of S rows, timed as a graph of back-to-back launches.
    first: (q, K, V) CPU tensors to run instead of torch-random inputs (the
    SplitMix64 inputs the CPU baseline runs too); their output is returned."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(99)
    if first is not None:
        q, k, v = (t.to(dev) for t in first)
    else:
        q = torch.randn(S, H * D, generator=g, device=dev).to(dt)
        k = torch.randn(S, Hk * D, generator=g, device=dev).to(dt)
        v = torch.randn(S, Hk * D, generator=g, device=dev).to(dt)
    out = torch.empty(S, H * D, device=dev)
    run = lambda: A.attn_prefill(q, k, v, H, Hk, D, window=window, out=out)  # noqa: E731
    for _ in range(max(3, args.warmup)):
        run()
    torch.cuda.synchronize()
    # A graph of back-to-back launches: the events bracket GPU work only, not
    # per-launch event and dispatch gaps.
    reps = 20
    gr = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(gr, stream=st):
            for _ in range(reps):
                run()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    gr.replay()
    torch.cuda.synchronize()
    n = max(3, min(args.steps // 20, 20))
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(n):
        gr.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / (n * reps)
    n = n * reps
    # (query, key) pairs the mask keeps: row i sees min(i + 1, window) keys
    pairs = S * (S + 1) / 2
    if 0 < window < S:
        pairs -= (S - window) * (S - window + 1) / 2
    flop = 4.0 * D * H * pairs
    res = dict(ms=ms, tflops=flop / (ms * 1e-3) / 1e12, flop=flop, launches=n)
    if first is not None:
        run()
        torch.cuda.synchronize()
        res["out"] = out.cpu().numpy()
    return res


def bench_prefill_paged(torch, A, args, S, H, Hk, D, dt, page):
    """cfg3 prefill with K/V in pages of `page` positions shuffled over a
    pool (chunked-prefill layout), timed like bench_prefill."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(99)
    q = torch.randn(S, H * D, generator=g, device=dev).to(dt)
    n_pages = (S + page - 1) // page
    kp = torch.randn(n_pages, page, Hk * D, generator=g, device=dev).to(dt)
    vp = torch.randn(n_pages, page, Hk * D, generator=g, device=dev).to(dt)
    table = torch.randperm(n_pages, generator=g, device=dev).to(torch.int32)
    out = torch.empty(S, H * D, device=dev)
    run = lambda: A.attn_prefill_paged(q, kp, vp, table, H, Hk, D, out=out)  # noqa: E731
    for _ in range(3):
        run()
    torch.cuda.synchronize()
    reps = 20
    gr = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(gr, stream=st):
            for _ in range(reps):
                run()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    gr.replay()
    torch.cuda.synchronize()
    n = max(3, min(args.steps // 20, 20))
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(n):
        gr.replay()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / (n * reps)
    flop = 4.0 * D * H * S * (S + 1) / 2
    return dict(ms=ms, tflops=flop / (ms * 1e-3) / 1e12, page=page)


def bench_append(torch, A, args, S, H, Hk, D, dt):
    """cfg3's fused append: S rows of f32 q/k/v -> Q/K RMSNorm -> NeoX RoPE
    (theta 1e6) -> q (bf16) and the K/V cache rows (bf16).  HBM-bound: the
    algorithmic bytes are the f32 rows read, the (cos, sin) rows read and the
    bf16 rows written; timed as a graph of launches (no host overhead)."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn(S, H * D, generator=g, device=dev)
    k = torch.randn(S, Hk * D, generator=g, device=dev)
    v = torch.randn(S, Hk * D, generator=g, device=dev)
    qn = 1.0 + 0.1 * torch.randn(D, generator=g, device=dev)
    kn = 1.0 + 0.1 * torch.randn(D, generator=g, device=dev)
    kc = torch.empty(S, Hk * D, dtype=dt, device=dev)
    vc = torch.empty_like(kc)
    qo = torch.empty(S, H * D, dtype=dt, device=dev)
    cs = A.rope_table(S, D, 1e6)
    run = lambda: A.qkv_append(q, k, v, kc, vc, cs, start_pos=0, n_head=H, n_kv_head=Hk,  # noqa: E731
                               head_dim=D, q_norm=qn, k_norm=kn, q_out=qo)
    for _ in range(3):
        run()
    torch.cuda.synchronize()
    reps = 20
    gr = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(gr, stream=st):
            for _ in range(reps):
                run()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    gr.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = max(3, min(args.steps // 20, 20))
    t0.record()
    for _ in range(n):
        gr.replay()
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / (n * reps)
    esz = torch.finfo(dt).bits // 8
    nbytes = S * (H + 2 * Hk) * D * 4 + S * D * 4 + 2 * D * 4 + S * (H + 2 * Hk) * D * esz
    return dict(us=us, bytes=nbytes, gbps=nbytes / (us * 1e3))


def bench_proj(torch, A, args, hidden, H, Hk, D, wdt):
    """Decode-side Q/K/V projection + fused append for one token (Qwen3-4B
    shape): HBM-bound on the weights.  Algorithmic bytes = the three weight
    matrices + x + the outputs; timed as a graph of launches, the weights
    rotated over enough copies to exceed the MALL."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(11)
    wbytes = (H + 2 * Hk) * D * hidden * torch.finfo(wdt).bits // 8
    n_sets = max(1, math.ceil(2 * MALL_BYTES / wbytes))
    sets = []
    for _ in range(n_sets):
        sets.append(tuple((0.02 * torch.randn(n * D, hidden, generator=g, device=dev)).to(wdt)
                          for n in (H, Hk, Hk)))
    x = torch.randn(1, hidden, generator=g, device=dev)
    qn = 1.0 + 0.1 * torch.randn(D, generator=g, device=dev)
    kn = 1.0 + 0.1 * torch.randn(D, generator=g, device=dev)
    n_ctx = 4096
    kc = torch.zeros(n_ctx, Hk * D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    qo = torch.empty(1, H * D, device=dev)
    cs = A.rope_table(n_ctx, D, 1e6)
    run = lambda si: A.qkv_proj_append(x, *sets[si], kc, vc, cs, start_pos=n_ctx - 1, n_head=H,  # noqa: E731
                                       n_kv_head=Hk, head_dim=D, q_norm=qn, k_norm=kn, q_out=qo)
    for si in range(n_sets):
        run(si)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(gr, stream=st):
            for si in range(n_sets):
                run(si)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    gr.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = max(3, min(args.steps // 20, 20))
    t0.record()
    for _ in range(n):
        gr.replay()
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / (n * n_sets)
    nbytes = wbytes + hidden * 4 + H * D * 4 + 2 * Hk * D * 2
    return dict(us=us, bytes=nbytes, gbps=nbytes / (us * 1e3), n_sets=n_sets)


def bench_matmul(torch, A, args, S, hidden, outs):
    """Prefill-side Q/K/V projections (forward.rs:799-801): one batched matmul
    per weight over S token rows, f32 activations x bf16 weights.  Algorithmic
    work = 2 S hidden sum(outs) FLOP; the matrix cores execute twice that
    (activation hi + lo halves).  Timed as a graph of launches."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(13)
    x = torch.randn(S, hidden, generator=g, device=dev)
    ws = [(0.02 * torch.randn(o, hidden, generator=g, device=dev)).to(torch.bfloat16) for o in outs]
    ys = [torch.empty(S, o, device=dev) for o in outs]
    run = lambda: [A.matmul(w, x, y) for w, y in zip(ws, ys)]  # noqa: E731
    run()
    torch.cuda.synchronize()
    reps = 4
    gr = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(gr, stream=st):
            for _ in range(reps):
                run()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    gr.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = max(3, min(args.steps // 20, 20))
    t0.record()
    for _ in range(n):
        gr.replay()
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / (n * reps)
    flop = 2 * S * hidden * sum(outs)
    return dict(us=us, flop=flop, tflops=flop / (us * 1e6))


def bench_paged(torch, A, args, H, Hk, D, B, lo, hi, n_layer, page, dt):
    """cfg5 batch 8: independent sequences with ragged lengths in [lo, hi]
    (SplitMix64), 48 layers per step, over a paged cache (page positions per
    page, pages of a layer shuffled over its pool) and, for comparison, over
    the contiguous layout ullm_hip_attn_decode takes.  Layer l reads pool
    l % 4: consecutive layers never share data, and 4 pools exceed the MALL.
    Algorithmic bytes per layer = sum(len) x 2 x Hk x D x 2."""
    import numpy as np

    from ullm_amd import synth
    dev = torch.device("cuda")
    lens = synth.ragged_lengths(5, B, lo, hi)
    L_ = max(lens)
    kvs = Hk * D
    need = [(n + page - 1) // page for n in lens]
    n_pages = sum(need)
    stride = (L_ + page - 1) // page
    n_pool = 4
    g = torch.Generator(device=dev).manual_seed(21)
    rng = np.random.default_rng(21)
    pools, tables = [], []
    for _ in range(n_pool):
        kp = torch.randn(n_pages, page, kvs, generator=g, device=dev).to(dt)
        vp = torch.randn(n_pages, page, kvs, generator=g, device=dev).to(dt)
        perm = rng.permutation(n_pages)
        t = np.full((B, stride), -1, np.int32)
        i = 0
        for b in range(B):
            t[b, :need[b]] = perm[i:i + need[b]]
            i += need[b]
        pools.append((kp, vp))
        tables.append(torch.from_numpy(t).to(dev))
    q = torch.randn(n_layer, B, H, D, generator=g, device=dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty(n_layer, B, H, D, device=dev)
    nws = int(A.L.lib().ullm_hip_paged_decode_workspace_bytes(B, H, Hk, D, L_, 0))
    ws = torch.zeros(max(nws, 256), dtype=torch.uint8, device=dev)

    def paged_step():
        for li in range(n_layer):
            kp, vp = pools[li % n_pool]
            A.attn_decode_paged(q[li], kp, vp, tables[li % n_pool], sl, L_, Hk, out=out[li],
                                workspace=ws)

    cont = []
    for _ in range(n_pool):
        kc = torch.randn(B, L_, kvs, generator=g, device=dev).to(dt)
        vc = torch.randn(B, L_, kvs, generator=g, device=dev).to(dt)
        cont.append((kc, vc))
    wsc = A.new_decode_workspace(B, H, Hk, D, L_)

    def cont_step():
        for li in range(n_layer):
            kc, vc = cont[li % n_pool]
            A.attn_decode(q[li], kc, vc, sl, L_, Hk, out=out[li], seq_stride=L_ * kvs,
                          workspace=wsc)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            with torch.cuda.graph(gr, stream=st):
                fn()
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        for _ in range(2):
            gr.replay()
        torch.cuda.synchronize()
        n = max(3, min(args.steps // 30, 10))
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(n):
            gr.replay()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) * 1e3 / (n * n_layer)

    us_p = timed(paged_step)
    us_c = timed(cont_step)
    lb = sum(lens) * 2 * Hk * D * torch.finfo(dt).bits // 8
    return dict(lens=lens, page=page, us_paged=us_p, us_contig=us_c, layer_bytes=lb,
                gbps_paged=lb / (us_p * 1e3), gbps_contig=lb / (us_c * 1e3))


def bench_copy(torch):
    """Plain copy of known size: the calibration kernel for FETCH/WRITE_SIZE."""
    n = 256 << 20
    a = torch.ones(n // 4, device="cuda")
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    return dict(bytes_each_way=n)


def bench_floor(torch, A):
    """Read floors beside the decode op: ullm_hip_stream_read over a distinct
    buffer per graph node (rotated past the MALL), at the cfg2 layer size
    (4 MiB) and the cfg5 layer size (64 MiB), plus a 16-byte read (the cost
    of a graph node itself).  Same launch path as the decode op."""
    import ctypes as C

    lib = A.L.lib()
    dev = torch.device("cuda")
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    res = {}
    for name, nbytes, nodes, grid in (("node", 16, 56, 1), ("read_4MiB", 4 << 20, 140, 1024),
                                      ("read_64MiB", 64 << 20, 48, 2048)):
        pool = torch.ones(max(nbytes * nodes // 4, 4), dtype=torch.float32, device=dev)
        base = pool.data_ptr()
        step = nbytes if name != "node" else 0
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            with torch.cuda.graph(g, stream=cap):
                st = C.c_void_p(cap.cuda_stream)
                for i in range(nodes):
                    A.L.check(lib.ullm_hip_stream_read(C.c_void_p(base + i * step), nbytes, grid,
                                                       C.c_void_p(sink.data_ptr()), st))
        torch.cuda.current_stream().wait_stream(cap)
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        reps = 20
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(reps):
            g.replay()
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1000.0 / (reps * nodes)
        res[name + "_us"] = round(us, 3)
        if name != "node":
            res[name + "_gbps"] = round(nbytes / (us * 1e3), 1)
            res[name + "_frac"] = round(nbytes / (us * 1e3) / HBM_PEAK_GBS, 4)
        del g, pool
    return res


def synth_decode_layer(torch, H, Hk, D, L, dt, seed):
    """One decode layer from SplitMix64 (ullm_amd.synth): q [H*D] f32, K/V
    [L, Hk*D] rounded to the cache dtype.  The GPU bench runs it as its first
    layer and the CPU baseline runs the very same values."""
    from ullm_amd import synth

    return (synth.randn(seed, 1, (H * D,)), synth.randn(seed, 2, (L, Hk * D), dt),
            synth.randn(seed, 3, (L, Hk * D), dt))


def cpu_baseline_decode(layer, H, Hk, D, L, budget_s=12.0, window=0):
    """The oracle (single thread, the reference's serial schedule) on the
    synth layer, repeated for about budget_s seconds."""
    import numpy as np

    from oracle import oracle as ora

    q = layer[0].numpy().astype(np.float32)
    kc = layer[1].float().numpy()
    vc = layer[2].float().numpy()
    scale = 1.0 / math.sqrt(D)
    done, t0 = 0, time.perf_counter()
    ref = None
    while time.perf_counter() - t0 < budget_s:
        ref = ora.attn_decode(q, kc, vc, L - 1, H, Hk, D, scale, window=window)
        done += 1
    el = time.perf_counter() - t0
    return dict(value=el / done * 1e6, layers=done, seconds=el, ref=ref)


def cpu_baseline_prefill(first, S, H, Hk, D):
    """The oracle's full causal prefill over the synth inputs (every row of
    every head), single thread."""
    from oracle import oracle as ora

    q, k, v = (t.float().numpy() for t in first)
    t0 = time.perf_counter()
    ref = ora.attn_prefill(q, k, v, S, 0, H, Hk, D, 1.0 / math.sqrt(D))
    el = time.perf_counter() - t0
    flop = 4.0 * D * H * S * (S + 1) / 2
    return dict(ms=el * 1e3, gflops=flop / el / 1e9, ref=ref)


def parity(out, ref):
    """max-abs and rel-L2 of the GPU output against the oracle's."""
    import numpy as np

    o = np.asarray(out, dtype=np.float64).reshape(-1)
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    return dict(max_abs=float(np.max(np.abs(o - r))),
                rel_l2=float(np.linalg.norm(o - r) / max(np.linalg.norm(r), 1e-30)))


def load_traffic():
    p = os.path.join(ROOT, "profiles", "decode_cfg2_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build targets ONE GPU; --gpus {args.gpus} is not supported "
              "(sharding over several GPUs is not built; it runs on one GPU)", file=sys.stderr)
        sys.exit(2)
    import torch

    from ullm_amd import attention as A

    A.L.lib()  # fail loudly if the HIP library is missing
    if args.only == "copy":
        print(json.dumps(bench_copy(torch)))
        return
    if args.only == "floor":
        print(json.dumps(bench_floor(torch, A)))
        return
    want = lambda k: args.only in ("all", k)  # noqa: E731
    res = {}
    # Layer 0 of the cfg2 run and the cfg3 prefill inputs come from SplitMix64
    # (ullm_amd.synth), so the CPU baseline runs exactly what the GPU ran.
    syn2 = synth_decode_layer(torch, 12, 2, 128, 4096, torch.float16, seed=2)
    syn3 = None
    if want("decode"):
        res["cfg2"] = bench_decode(torch, A, args, 12, 2, 128, 4096, 28, torch.float16, "cfg2",
                                   first=syn2)
    if want("prefill"):
        from ullm_amd import synth

        syn3 = tuple(synth.randn(3, t, (2048, n * 128), torch.bfloat16)
                     for t, n in ((1, 32), (2, 8), (3, 8)))
        res["cfg3"] = bench_prefill(torch, A, args, 2048, 32, 8, 128, torch.bfloat16, first=syn3)
        res["cfg3_paged"] = bench_prefill_paged(torch, A, args, 2048, 32, 8, 128, torch.bfloat16,
                                                256)
    if want("f32prefill"):
        # The reference's own cache dtype (f32) through the MFMA prefill.
        res["f32_prefill"] = bench_prefill(torch, A, args, 2048, 32, 8, 128, torch.float32)
        res["f32_prefill_d256"] = bench_prefill(torch, A, args, 1024, 8, 4, 256, torch.float32)
    if want("cfg1"):
        res["cfg1"] = bench_decode(torch, A, args, 32, 8, 64, 512, 28, torch.float32, "cfg1")
    if want("f32decode"):
        # cfg5's shape over the reference's own f32 cache (128 MiB per layer).
        res["f32_long"] = bench_decode(torch, A, argparse.Namespace(steps=max(5, args.steps // 10),
                                                                    warmup=3),
                                       32, 4, 128, 32768, 12, torch.float32, "f32_long")
    if want("cfg4"):
        # One step = a 6-layer group: 5 sliding-window layers (1024 keys) and
        # the global layer, at context 8192 (forward.rs:450-454 / lib.rs:1183-1186).
        res["cfg4"] = bench_decode(torch, A, argparse.Namespace(steps=max(10, args.steps // 4),
                                                                warmup=3),
                                   8, 4, 256, 8192, 6, torch.float16, "cfg4",
                                   windows=[1024] * 5 + [0])
        res["cfg4_prefill"] = bench_prefill(torch, A, args, 1024, 8, 4, 256, torch.float16,
                                            window=1024)
        # A long prompt: the global layer and a sliding-window layer at S=8192.
        res["cfg4_prefill_8k"] = bench_prefill(torch, A, args, 8192, 8, 4, 256, torch.float16)
        res["cfg4_prefill_8k_w"] = bench_prefill(torch, A, args, 8192, 8, 4, 256, torch.float16,
                                                 window=1024)
    if want("append"):
        res["append"] = bench_append(torch, A, args, 2048, 32, 8, 128, torch.bfloat16)
    if want("proj"):
        res["proj"] = bench_proj(torch, A, args, 2560, 32, 8, 128, torch.bfloat16)
    if want("matmul"):
        res["matmul"] = bench_matmul(torch, A, args, 2048, 2560, (4096, 1024, 1024))
    if want("paged"):
        res["paged"] = bench_paged(torch, A, args, 32, 4, 128, 8, 4096, 32768, 48, 256,
                                   torch.bfloat16)
    if want("long"):
        res["cfg5"] = bench_decode(torch, A, argparse.Namespace(steps=max(5, args.steps // 10),
                                                                warmup=3),
                                   32, 4, 128, 32768, 48, torch.bfloat16, "cfg5")
    if args.only == "all":
        res["floor"] = bench_floor(torch, A)
    if args.only != "all":
        for r in res.values():
            r.pop("first_out", None)
            r.pop("out", None)
        print(json.dumps(res))
        return

    d, p, lc, ap, pj = res["cfg2"], res["cfg3"], res["cfg5"], res["append"], res["proj"]
    mm, pg = res["matmul"], res["paged"]
    c1, c4, c4p = res["cfg1"], res["cfg4"], res["cfg4_prefill"]
    traffic = load_traffic()
    line = {
        "metric": METRIC,
        "value": round(d["us_per_layer"], 4),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_step"], 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "cfg2 Qwen2.5-1.5B-shaped decode attention: batch 1, 12 q heads, "
                        "2 kv heads, head_dim 128, f16 KV cache 4096, 28 layers per step "
                        "(HIP graph per step, KV sets rotated over "
                        f"{d['n_sets']} x 28 layers to defeat the MALL; layer 0 of set 0 is "
                        "SplitMix64 data, the rest torch-random)",
            "batch": 1, "n_head": 12, "n_kv_head": 2, "head_dim": 128, "ctx": 4096,
            "layers": 28, "kv_dtype": "f16",
        },
        "decode_gbps": round(d["gbps_step"], 1),
        "prefill": {"workload": "cfg3 Qwen3-4B-shaped causal prefill, S=2048, 32/8 heads, "
                                "head_dim 128, bf16 (SplitMix64 inputs)", "ms": round(p["ms"], 4),
                    "tflops": round(p["tflops"], 2),
                    "flop_causal": p["flop"],
                    "paged": {"page": res["cfg3_paged"]["page"],
                              "ms": round(res["cfg3_paged"]["ms"], 4),
                              "tflops": round(res["cfg3_paged"]["tflops"], 2)}},
        "cfg1_decode": {"workload": "cfg1 Llama-3.2-1B-shaped decode: 32/8 heads, head_dim 64, "
                                    "f32 KV 512, 28 layers per graph (rotated past the MALL)",
                        "kernel": "decode_block_kernel<F32,64,1,32> (bf16 hi + lo MFMA) + "
                                  "decode_merge_kernel",
                        "us_per_layer": round(c1["us_per_layer"], 3),
                        "algorithmic_bytes": int(c1["layer_bytes"]),
                        "gbps": round(c1["gbps_step"], 1),
                        "frac_hbm": round(c1["gbps_step"] / HBM_PEAK_GBS, 4)},
        "cfg4_decode": {"workload": "cfg4 Gemma-3-4B-shaped decode group: 8/4 heads, head_dim "
                                    "256, f16 KV, context 8192; 6 layers per step = 5 sliding-"
                                    "window layers (1024 keys) + 1 global layer, rotated past "
                                    "the MALL",
                        "kernel": "window layers decode_block_kernel<F16,256,1,16>, global layer "
                                  "decode_mfma_kernel<F16,256,false,4>; each + decode_merge_kernel",
                        "us_per_group": round(c4["ms_per_step"] * 1e3, 3),
                        "us_per_layer": round(c4["us_per_layer"], 3),
                        "algorithmic_bytes_per_group": int(c4["step_bytes"]),
                        "gbps": round(c4["gbps_step"], 1),
                        "frac_hbm": round(c4["gbps_step"] / HBM_PEAK_GBS, 4)},
        "cfg4_prefill": {"workload": "cfg4 causal prefill, S=1024, 8/4 heads, head_dim 256, "
                                     "f16, window 1024 (= causal at this length)",
                         "kernel": "prefill16_kernel<F16,2,2> (two key streams, value columns split over two workgroups)",
                         "ms": round(c4p["ms"], 4), "tflops": round(c4p["tflops"], 2),
                         "flop_causal": c4p["flop"],
                         "frac_mfma": round(c4p["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4)},
        "cfg4_prefill_8k": {"workload": "cfg4 shapes at an 8192-token prompt: 8/4 heads, "
                                        "head_dim 256, f16; global layer (causal) and a "
                                        "sliding-window layer (window 1024)",
                            "kernel": "prefill16_kernel<F16,1,1> (one key stream)",
                            "global": {"ms": round(res["cfg4_prefill_8k"]["ms"], 4),
                                       "tflops": round(res["cfg4_prefill_8k"]["tflops"], 2),
                                       "frac_mfma": round(res["cfg4_prefill_8k"]["tflops"]
                                                          / MFMA_BF16_PEAK_TFLOPS, 4)},
                            "window_1024": {"ms": round(res["cfg4_prefill_8k_w"]["ms"], 4),
                                            "tflops": round(res["cfg4_prefill_8k_w"]["tflops"], 2),
                                            "frac_mfma": round(res["cfg4_prefill_8k_w"]["tflops"]
                                                               / MFMA_BF16_PEAK_TFLOPS, 4)}},
        "f32_prefill": {"workload": "cfg3 shape (S=2048, 32/8 heads, head_dim 128) over an f32 "
                                    "cache, the reference's own cache dtype: Q.K on bf16 hi + lo "
                                    "halves of Q and K, P.V in f16",
                        "kernel": "prefill16_kernel<F32,KS,1,128> (f32 tiles by LDS DMA, "
                                  "split in LDS into bf16 hi/lo K and f16 V)",
                        "ms": round(res["f32_prefill"]["ms"], 4),
                        "tflops": round(res["f32_prefill"]["tflops"], 2),
                        "frac_mfma": round(res["f32_prefill"]["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4),
                        "note": "the matrix cores execute 2x the algorithmic FLOP (three bf16 "
                                "products for Q.K)",
                        "head_dim_256": {
                            "workload": "cfg4 shape (S=1024, 8/4 heads, head_dim 256, causal) "
                                        "over an f32 cache",
                            "kernel": "prefill16_kernel<F32,1,2,256> (one key stream, value "
                                      "columns split over two workgroups)",
                            "ms": round(res["f32_prefill_d256"]["ms"], 4),
                            "tflops": round(res["f32_prefill_d256"]["tflops"], 2),
                            "frac_mfma": round(res["f32_prefill_d256"]["tflops"]
                                               / MFMA_BF16_PEAK_TFLOPS, 4)}},
        "f32_long_decode": {"workload": "cfg5's shape (32/4 heads, head_dim 128, batch 1, 32768 "
                                        "keys) over an f32 cache, the reference's own cache "
                                        "dtype; 12 layers per graph",
                            "kernel": "decode_dma_kernel<F32,128,2> (f32 tiles by LDS DMA, bf16 "
                                      "hi + lo MFMAs) + decode_merge_kernel",
                            "us_per_layer": round(res["f32_long"]["us_per_layer"], 3),
                            "algorithmic_bytes": int(res["f32_long"]["layer_bytes"]),
                            "gbps": round(res["f32_long"]["gbps_step"], 1),
                            "frac_hbm": round(res["f32_long"]["gbps_step"] / HBM_PEAK_GBS, 4)},
        "long_decode": {"workload": "cfg5 Qwen3-30B-A3B-shaped decode, 32/4 heads, head_dim "
                                    "128, bf16 KV 32768, 48 layers",
                        "us_per_layer": round(lc["us_per_layer"], 3),
                        "gbps": round(lc["gbps_step"], 1),
                        "frac_hbm": round(lc["gbps_step"] / HBM_PEAK_GBS, 4),
                        "read_floor_us": res["floor"]["read_64MiB_us"],
                        "read_floor_frac": res["floor"]["read_64MiB_frac"]},
        "append": {"workload": "cfg3 fused append: 2048 rows, 32/8 heads, head_dim 128, f32 "
                               "q/k/v in, Q/K RMSNorm + NeoX RoPE, bf16 q and KV rows out",
                   "kernel": "qkv_append_kernel<128,BF16,BF16>",
                   "us": round(ap["us"], 3), "algorithmic_bytes": ap["bytes"],
                   "gbps": round(ap["gbps"], 1),
                   "frac_hbm": round(ap["gbps"] / HBM_PEAK_GBS, 4)},
        "qkv_proj": {"workload": "Qwen3-4B-shaped decode Q/K/V projection + fused append: "
                                 "hidden 2560, 32/8 heads, head_dim 128, bf16 weights, Q/K "
                                 "RMSNorm + NeoX RoPE, bf16 cache",
                     "kernel": "qkv_proj_kernel<128,BF16,F32,BF16>",
                     "us": round(pj["us"], 3), "algorithmic_bytes": pj["bytes"],
                     "gbps": round(pj["gbps"], 1),
                     "frac_hbm": round(pj["gbps"] / HBM_PEAK_GBS, 4)},
        "prefill_proj": {"workload": "Qwen3-4B-shaped prefill Q/K/V projections: 2048 token "
                                     "rows, hidden 2560 -> 4096 + 1024 + 1024, f32 activations, "
                                     "bf16 weights, f32 out (three launches)",
                         "kernel": "matmul_bf16_kernel",
                         "us": round(mm["us"], 2), "flop": mm["flop"],
                         "tflops": round(mm["tflops"], 1),
                         "frac_mfma": round(mm["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4),
                         "note": "activations run as bf16 hi + lo: the matrix cores "
                                 "execute 2x the algorithmic FLOP"},
        "paged_decode": {"workload": "cfg5 batch 8, ragged lengths in [4096, 32768] "
                                     f"(SplitMix64: {pg['lens']}), 32/4 heads, head_dim 128, "
                                     "bf16, 48 layers; paged cache with "
                                     f"{pg['page']}-position pages shuffled over the pool, and "
                                     "the contiguous layout for comparison",
                         "us_per_layer": round(pg["us_paged"], 3),
                         "gbps": round(pg["gbps_paged"], 1),
                         "frac_hbm": round(pg["gbps_paged"] / HBM_PEAK_GBS, 4),
                         "contiguous_us_per_layer": round(pg["us_contig"], 3),
                         "contiguous_gbps": round(pg["gbps_contig"], 1),
                         "algorithmic_bytes": pg["layer_bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(d["gbps_step"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(d["gbps_step"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("bytes_per_launch") if traffic else None,
                     "traffic_measured_at": traffic.get("commit") if traffic else None,
                     "kernel": "decode_block_kernel<F16,128,1,32> + decode_merge_kernel<128,4,2,256> "
                               "(one decode-attention op per layer)",
                     "algorithmic_bytes": int(d["layer_bytes"]),
                     "us_per_launch": round(d["us_per_layer"], 3),
                     "read_floor": {
                         "note": "ullm_hip_stream_read of the same 4 MiB as one graph node: the "
                                 "best a single read-only launch of this size reaches here",
                         "us": res["floor"]["read_4MiB_us"],
                         "frac": res["floor"]["read_4MiB_frac"],
                         "graph_node_us": res["floor"]["node_us"]}},
        "roofline_prefill": {"bound": "mfma", "achieved": round(p["tflops"], 2),
                             "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(p["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4),
                             "kernel": "prefill4_kernel<BF16,128>"},
    }
    if not args.no_cpu:
        # The oracle on rank 0's host, one thread (the reference's attention
        # loop is serial, lib.rs:917-938), on the SplitMix64 layer the GPU ran
        # as layer 0: about 12 s of repeated layers, then the full cfg3 prefill.
        cd = cpu_baseline_decode(syn2, 12, 2, 128, 4096)
        cp = cpu_baseline_prefill(syn3, 2048, 32, 8, 128)
        line["cpu_baseline"] = {
            "value": round(cd["value"], 1), "unit": "us/layer", "cores": 1, "kind": "port",
            "sample": f"{cd['layers']} repetitions of the cfg2 SplitMix64 layer (the GPU run's "
                      f"layer 0) in {cd['seconds']:.1f} s on 1 thread, oracle/ref_attention.c "
                      f"-O2; then the full cfg3 prefill (all 2048 rows x 32 heads, the GPU run's "
                      f"SplitMix64 inputs) in {cp['ms']:.0f} ms = {cp['gflops']:.2f} GFLOP/s",
            "prefill_ms": round(cp["ms"], 1),
            "prefill_gflops": round(cp["gflops"], 3),
            "host_cpu": _cpu_model(),
            "host_cpu_id": _cpu_id(),
            "nproc": os.cpu_count(),
        }
        # The same inputs through the GPU path: its output against the oracle's.
        line["parity"] = {"cfg2_layer0": parity(d["first_out"], cd["ref"]),
                          "cfg3_prefill": parity(p["out"], cp["ref"]),
                          "tolerance": {"max_abs": 2e-3, "rel_l2": 1e-3}}
    print(json.dumps(line))


def _cpu_id():
    """lscpu's vendor / family / model / stepping (the model name alone can be
    generic on a virtualised host)."""
    import subprocess

    keys = ("Vendor ID", "CPU family", "Model", "Stepping", "Thread(s) per core",
            "Core(s) per socket", "Socket(s)")
    out = {}
    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10)
        for ln in r.stdout.splitlines():
            k, _, v = ln.partition(":")
            if k.strip() in keys:
                out[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return out


def _cpu_model():
    """The host CPU's model name, as lscpu reports it (/proc/cpuinfo otherwise)."""
    import subprocess

    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10)
        for ln in r.stdout.splitlines():
            if ln.strip().startswith("Model name:"):
                return ln.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()
