"""Decode benchmark: Llama-3-8B-shaped bf16 greedy decode at context 8192.

One step = one full decode token (embed, 32 x [attention block, SwiGLU
block], final norm + LM head, device argmax feeding the next DecodeStep),
replayed as a HIP graph with no host round trip.  The KV cache is prefilled
with N(0, 1) values so every timed token attends over ~8k positions; weights
are random N(0, 0.02) bf16 generated on the device (synthetic data).

Prints one JSON line (rank 0, N=1 only): decode tokens/s, the dominant
kernel's HBM roofline from HIP-event timings taken in this run, a per-kernel
table, and the CPU oracle timed on the host on a bounded sample of the same
workload (with a greedy-token parity check against the GPU).
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tokens/sec @ Llama-3-8B shape ctx 8192; kernel HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0

LLAMA3_8B = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, hidden=14336, vocab=128256,
                 max_seq=8192, theta=500000.0, eps=1e-5)


class Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def token_bytes(c, ctx):
    """Algorithmic HBM bytes of one decode token at context `ctx` (bf16
    weights and KV, fp32 activations; scratch excluded)."""
    head = c.dim // c.n_heads
    q, kv = head * c.n_heads, head * c.n_kv_heads
    per_layer_w = (q + 2 * kv) * c.dim + c.dim * q + 3 * c.hidden * c.dim
    weights = 2 * (c.n_layers * per_layer_w + c.vocab * c.dim)
    kv_read = c.n_layers * 2 * ctx * kv * 2
    return weights + kv_read


def kernel_bytes(c, ctx, split=128):
    """Algorithmic bytes per launch of each per-layer kernel (GEMV: d*n*2 +
    4n + 4d [+ 4d residual]; attention: 2*ctx*kv_dim*2 + q and out)."""
    head = c.dim // c.n_heads
    q, kv = head * c.n_heads, head * c.n_kv_heads
    return {
        "gate_up_swiglu": 2 * c.hidden * c.dim * 2 + 4 * c.dim * 2 + 4 * c.hidden,
        "qkv_rope_store": (q + 2 * kv) * c.dim * 2 + 4 * c.dim * 2 + 4 * q + 2 * 2 * kv,
        "w2_residual": c.dim * c.hidden * 2 + 4 * c.hidden + 4 * c.dim * 2,
        "wo_residual": c.dim * q * 2 + 4 * q + 4 * c.dim * 2,
        "attention_partial": 2 * ctx * kv * 2 + 8 * q,
        # the merge reads each live split's (acc, m, l) once and writes out
        "attention_combine": c.n_heads * -(-ctx // split) * (head + 2) * 4 + 4 * q,
        "lm_head": c.vocab * c.dim * 2 + 4 * c.dim * 2 + 4 * c.vocab,
    }


def time_kernels(rt, model, c, weights, ctx, reps, split=0, use_graph=True):
    """Average duration of each fused kernel: HIP events on the model's
    stream around batches of L back-to-back launches (one per layer, so
    nothing is served from cache), replayed as one captured graph unless
    use_graph is False."""
    import ammon_amd
    from ammon_amd import Timer
    from ammon_amd._abi import BF16, F32, call, check, lib

    L, head = c.n_layers, c.dim // c.n_heads
    q, kv = head * c.n_heads, head * c.n_kv_heads
    stream = model.stream
    x = rt.alloc(c.dim * 4)
    rt.fill_normal(x, F32, c.dim, 5, 900)
    qb, hb, xb = rt.alloc(q * 4), rt.alloc(c.hidden * 4), rt.alloc(q * 4)
    xr = rt.alloc(c.dim * 4)
    rt.fill_normal(xr, F32, c.dim, 5, 901)
    logits = rt.alloc(c.vocab * 4)
    step = rt.step(1, ctx - 1)
    table = rt.upload(ammon_amd.rope_table_host(c.theta, head, c.max_seq))
    if not split:
        split = int(ammon_amd._abi.lib.ammon_attention_default_split_for(
            rt.handle, c.n_heads, c.n_kv_heads, head, c.kv_dtype, c.max_seq))
    part_bytes = ammon_amd.attention_scratch_bytes(c.n_heads, head, c.max_seq, split)
    part = rt.alloc(part_bytes)
    rt.synchronize()

    def w(name, l, per):
        return ctypes.c_void_p(int(weights[name]) + l * per * 2)

    def kv_ptr(l):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        call("ammon_llama_kv_layer", model.handle, l, ctypes.byref(k), ctypes.byref(v))
        return k, v

    rms = lambda name, l: ctypes.c_void_p(int(weights[name]) + l * c.dim * 4)
    # per kernel: the entry point and its arguments for each of the L layers
    launches = {
        "qkv_rope_store": ("ammon_qkv_rope_store", lambda l: (
            rt.handle, stream, x, rms("rms_att", l), F32, c.eps, w("wq", l, q * c.dim),
            w("wk", l, kv * c.dim), w("wv", l, kv * c.dim), BF16, c.dim, c.n_heads,
            c.n_kv_heads, head, qb, *kv_ptr(l), BF16, c.max_seq, step, table)),
        "attention_partial": ("ammon_attention_partial", lambda l: (
            rt.handle, stream, qb, c.n_heads, *kv_ptr(l), BF16, c.n_kv_heads, head, c.max_seq,
            step, split, part)),
        "attention_combine": ("ammon_attention_combine", lambda l: (
            rt.handle, stream, part, c.n_heads, head, c.max_seq, step, split, xb)),
        "wo_residual": ("ammon_gemv", lambda l: (
            rt.handle, stream, w("wo", l, c.dim * q), BF16, c.dim, q, xb, xr, xr)),
        "gate_up_swiglu": ("ammon_gate_up_swiglu", lambda l: (
            rt.handle, stream, x, rms("rms_ffn", l), F32, c.eps, w("w1", l, c.hidden * c.dim),
            w("w3", l, c.hidden * c.dim), BF16, c.dim, c.hidden, hb)),
        "w2_residual": ("ammon_gemv", lambda l: (
            rt.handle, stream, w("w2", l, c.dim * c.hidden), BF16, c.dim, c.hidden, hb, xr,
            xr)),
        "lm_head": ("ammon_gemv_rmsnorm", lambda l: (
            rt.handle, stream, x, weights["rms_final"], F32, c.eps, weights["wcls"], BF16,
            c.vocab, c.dim, logits)),
    }
    out = {}
    nbytes = kernel_bytes(c, ctx, split)
    timer = Timer(rt)
    for name, (entry, args_of) in launches.items():
        fn = getattr(lib, entry)
        per_layer = [args_of(l) for l in range(L)]

        def run_layers():
            for a in per_layer:
                check(fn(*a))

        graph = None
        if use_graph:
            # the L launches as one graph: no host launch overhead between them
            call("ammon_capture_begin", rt.handle, stream)
            run_layers()
            graph = ctypes.c_void_p()
            call("ammon_capture_end", rt.handle, stream, ctypes.byref(graph))
            body = lambda: call("ammon_graph_launch", rt.handle, graph, stream)
        else:
            body = run_layers
        body()  # warm the launch path
        samples = []
        for _ in range(reps):
            # one event pair around L back-to-back launches on the model's
            # stream (one per layer, distinct weights): average per launch
            timer.start(stream)
            body()
            timer.stop(stream)
            samples.append(timer.elapsed_ms() / L)
        if graph is not None:
            call("ammon_graph_destroy", rt.handle, graph)
        ms = float(np.median(samples))
        out[name] = {"avg_us": round(ms * 1e3, 3), "bytes": nbytes[name],
                     "gbs": round(nbytes[name] / (ms * 1e-3) / 1e9, 1),
                     "frac": round(nbytes[name] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "launches": reps * L}
    timer.close()
    return out


def cpu_baseline(rt, model, c, weights, start_pos, token0, gpu_tokens, budget_s):
    """The oracle (C, OpenMP over output rows) decoding the same positions
    from the same weights and KV prefix on the host cores."""
    import oracle
    from ammon_amd._abi import BF16, call

    t0 = time.time()
    host = {}
    for name, buf in weights.items():
        dt = np.float32 if name.startswith("rms") else np.uint16
        host[name] = buf.download(buf.nbytes // np.dtype(dt).itemsize, dt)
    shapes = oracle.weight_shapes(oracle.LlamaConfig(
        **{k: LLAMA3_8B[k] for k in ("dim", "n_layers", "n_heads", "n_kv_heads", "hidden",
                                     "vocab", "max_seq")}))
    host = {k: v.reshape(shapes[k]) for k, v in host.items()}
    ocfg = oracle.LlamaConfig(dim=c.dim, n_layers=c.n_layers, n_heads=c.n_heads,
                              n_kv_heads=c.n_kv_heads, hidden=c.hidden, vocab=c.vocab,
                              max_seq=c.max_seq, theta=c.theta, eps=c.eps, w_dtype=BF16,
                              kv_dtype=BF16)
    om = oracle.Model(ocfg, host)
    head = c.dim // c.n_heads
    kv_n = c.n_kv_heads * c.max_seq * head
    for l in range(c.n_layers):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        call("ammon_llama_kv_layer", model.handle, l, ctypes.byref(k), ctypes.byref(v))
        for src, get in ((k, oracle._lib.orc_model_key_cache),
                         (v, oracle._lib.orc_model_value_cache)):
            hm = np.empty(kv_n, np.uint16)
            call("ammon_memcpy", rt.handle, hm.ctypes.data, src, hm.nbytes, 2, None)
            rt.synchronize()
            pm = oracle_layout(hm, c.n_kv_heads, c.max_seq, head)
            ctypes.memmove(get(om._handle, l), pm.ctypes.data, pm.nbytes)
    setup_s = time.time() - t0
    log(f"cpu baseline: weights + cache on host in {setup_s:.1f}s; decoding")
    tokens, times = [], []
    tok = token0
    pos = start_pos
    while pos < c.max_seq:
        t1 = time.perf_counter()
        logits = om.step(tok, pos)
        times.append(time.perf_counter() - t1)
        tok = oracle.sample_argmax(logits)
        tokens.append(tok)
        pos += 1
        if sum(times) > budget_s:
            break
    om.close()
    n = len(times)
    agree = [int(a) == int(b) for a, b in zip(tokens, gpu_tokens[:n])]
    return {
        "value": round(n / sum(times), 4), "unit": "tokens/s", "cores": oracle.num_threads(),
        "kind": "port",
        "sample": (f"{n} greedy decode tokens of the same model at positions {start_pos}.."
                   f"{start_pos + n - 1} (ctx ~8192), oracle C restatement, -O3, OpenMP over "
                   f"output rows"),
        "seconds": round(sum(times), 2),
        "token_parity": bool(all(agree)), "tokens_compared": n,
        **cpu_info(),
    }


MFMA_BF16_PEAK_TFLOPS = 2500.0

# The kernel with the largest share of the token: the gate/up GEMV + SwiGLU
# (32 launches per token, 235 MB each at the Llama-3-8B shape).
DOMINANT = "gate_up_swiglu"
DOMINANT_NAME = "ammon_gemv_bf16_v_swiglu (gate/up GEMV + SwiGLU, RMSNorm prologue)"


def prefill_measure(rt, model, c, prompt_lengths=(16, 512), reps=3):
    """Prompt prefill (one pass per layer: GEMMs on matrix cores, token-
    batched attention) of T-token prompts from position 0: whole-model
    time, and the gate/up GEMM + SwiGLU alone (events on the model's stream
    around one launch per layer's weights, so no launch finds its 235 MB of
    weights in the 256 MB MALL).  Short prompts are HBM-bound on W (bytes: W once +
    x + hb); long ones are matrix-core bound, the bf16 W against x split
    into three bf16 parts (three MFMAs per product: issued TFLOP/s = 3 x
    algorithmic)."""
    from ammon_amd import Timer
    from ammon_amd._abi import BF16, F32, call

    out = {}
    timer = Timer(rt)
    stream = model.stream
    w1 = ctypes.c_void_p(int(model.weights["w1"]))
    w3 = ctypes.c_void_p(int(model.weights["w3"]))
    for T in prompt_lengths:
        prompt = (np.arange(T) * 7919 % c.vocab).astype(np.int32)
        model.prefill(prompt)  # warm: scratch allocation, first launches
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            model.prefill(prompt)  # synchronises
            ts.append(time.perf_counter() - t0)
        ms = min(ts) * 1e3
        x = rt.alloc(T * c.dim * 4)
        rt.fill_normal(x, F32, T * c.dim, 1, 7)
        hb = rt.alloc(T * c.hidden * 4)
        per = c.hidden * c.dim * 2  # bytes of one layer's w1 (and w3)
        layer_args = [(rt.handle, stream, x, T, ctypes.c_void_p(w1.value + l * per),
                       ctypes.c_void_p(w3.value + l * per), BF16, c.dim, c.hidden, hb)
                      for l in range(c.n_layers)]
        call("ammon_prefill_gate_up_swiglu", *layer_args[-1])
        timer.start(stream)
        for args in layer_args:
            call("ammon_prefill_gate_up_swiglu", *args)
        timer.stop(stream)
        us = timer.elapsed_ms() * 1e3 / len(layer_args)
        x.free()
        hb.free()
        nbytes = 2 * c.hidden * c.dim * 2 + T * c.dim * 4 + T * c.hidden * 4
        flops = 2.0 * T * 2 * c.hidden * c.dim
        gemm = {"kernel": "ammon_gemm_bf16_swiglu (gate/up GEMM + SwiGLU)", "avg_us": round(us, 2),
                "bytes": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                "mfma_frac": round(3 * flops / (us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}
        out[str(T)] = {"tokens": T, "ms": round(ms, 3), "tokens_per_s": round(T / ms * 1e3, 1),
                       "gate_up_gemm": gemm}
        log(f"prefill T={T}: {ms:.2f} ms ({T / ms * 1e3:.0f} tok/s); gate/up GEMM {us:.1f} us, "
            f"{gemm['gbs']:.0f} GB/s, {gemm['tflops']:.1f} TFLOP/s")
    timer.close()
    return out


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "hbm_traffic_llama3_8b_ctx8192.json")


def measured_traffic(kernel, algorithmic_bytes):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE and WRITE_SIZE passes over this benchmark, each
    scaled by the counter's reading for the copy probe).  Empty when the
    summary is missing or was taken on a different shape."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)["kernels"][kernel]
    except (OSError, KeyError, ValueError):
        return {}
    if rec.get("algorithmic_bytes") != algorithmic_bytes:
        return {}
    return {"traffic_bytes": rec["traffic_bytes"],
            "source": "profiles/" + os.path.basename(TRAFFIC_FILE)}


COPY_PROBE_N = 1 << 26  # fp32 elements per operand (256 MiB)


def copy_probe(rt, reps=4):
    """out = a + b over COPY_PROBE_N floats: reads 2 * 256 MiB and writes
    256 MiB per launch.  Under rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE
    calibrate the counters' units against a known byte count."""
    from ammon_amd._abi import F32, call
    bufs = [rt.alloc(COPY_PROBE_N * 4) for _ in range(3)]
    for i, b in enumerate(bufs[:2]):
        rt.fill_normal(b, F32, COPY_PROBE_N, 11, i)
    for _ in range(reps):
        call("ammon_add", rt.handle, None, bufs[0], bufs[1], bufs[2], COPY_PROBE_N)
    rt.synchronize()
    log(f"copy probe: {reps} x ammon_add over {COPY_PROBE_N} floats "
        f"(read {8 * COPY_PROBE_N} B, write {4 * COPY_PROBE_N} B per launch)")
    for b in bufs:
        b.free()


def cpu_info():
    """Host the CPU legs run on: model name, cores this process may use,
    OMP_NUM_THREADS."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "affinity_cores": len(os.sched_getaffinity(0)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def graph_ms(rt, stream, launch_all, reps=5):
    """Median ms of one replay of a graph that captures launch_all() on
    `stream` (events around each replay, after one warm replay)."""
    from ammon_amd import Timer
    from ammon_amd._abi import call

    call("ammon_capture_begin", rt.handle, stream)
    launch_all()
    graph = ctypes.c_void_p()
    call("ammon_capture_end", rt.handle, stream, ctypes.byref(graph))
    timer = Timer(rt)
    try:
        call("ammon_graph_launch", rt.handle, graph, stream)
        samples = []
        for _ in range(reps):
            timer.start(stream)
            call("ammon_graph_launch", rt.handle, graph, stream)
            timer.stop(stream)
            samples.append(timer.elapsed_ms())
    finally:
        timer.close()
        call("ammon_graph_destroy", rt.handle, graph)
    return float(np.median(samples))


def cpu_seconds(fn, budget_s, at_least=1):
    """Seconds per call of fn() on the host: repeated until budget_s (and at
    least `at_least` calls)."""
    n, t0 = 0, time.perf_counter()
    while n < at_least or time.perf_counter() - t0 < budget_s:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n


def rate(nbytes, us):
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"avg_us": round(us, 3), "bytes": int(nbytes), "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def read_chain_us(rt, stream, sources, nbytes, max_launches=32):
    """Per-launch µs of a captured graph of back-to-back ammon_stream_read
    launches of `nbytes` each over distinct slices of the `sources` buffers
    (so no launch finds its bytes in a cache), median of 5 replays."""
    from ammon_amd._abi import call
    nbytes = -(-int(nbytes) // 16) * 16
    slices = [int(b) + i * nbytes for b in sources for i in range(b.nbytes // nbytes)]
    slices = slices[:max_launches]

    def launch_all():
        for ptr in slices:
            call("ammon_stream_read", rt.handle, stream, ctypes.c_void_p(ptr), nbytes)
    return graph_ms(rt, stream, launch_all) * 1e3 / len(slices)


# launches per token of each timed kernel in the decode graph; embed and the
# argmax's second pass (kilobytes each) are the two others
LAUNCHES = {"qkv_rope_store": 32, "attention_partial": 32, "attention_combine": 32,
            "wo_residual": 32, "gate_up_swiglu": 32, "w2_residual": 32, "lm_head": 1}


def launch_floor(rt, model, kernels, ms_per_step):
    """The read floor of the decode's launch list.  For each launch, the
    chained time of a pure read of its algorithmic bytes (ammon_stream_read:
    two workgroups per CU, contiguous shares, nothing written), against the
    kernel's own average; 32 x the per-layer launches + the LM head + two
    kilobyte launches (embed, the argmax's second pass, each floored by a
    16 KiB read) give the token time of a launch list whose every kernel
    streamed like a plain read.  Sources: the w1, w2 and w3 stacks (3.76 GB
    each).  Also the plain read of a whole stack (the device's streaming
    ceiling)."""
    srcs = [model.weights[n] for n in ("w1", "w2", "w3")]
    stream = model.stream
    by = {}
    floor_ms = 2 * read_chain_us(rt, stream, srcs, 16384) * 1e-3
    for name, n in LAUNCHES.items():
        k = kernels[name]
        f = read_chain_us(rt, stream, srcs, k["bytes"])
        by[name] = {"bytes": k["bytes"], "floor_us": round(f, 3), "kernel_us": k["avg_us"],
                    "excess_us": round(k["avg_us"] - f, 3), "launches_per_token": n}
        floor_ms += n * f * 1e-3
        log(f"read floor {name:18s} {k['bytes'] / 1e6:9.1f} MB: {f:8.2f} us "
            f"(kernel {k['avg_us']:.2f} us, +{k['avg_us'] - f:.2f})")
    log(f"launch-list read floor {floor_ms:.4f} ms/token = {1e3 / floor_ms:.1f} tok/s; "
        f"measured {ms_per_step:.4f} ms ({floor_ms / ms_per_step:.3f} of the floor's rate)")
    floor = {"kernel": "ammon_stream_read (pure read, 2 workgroups per CU, contiguous shares)",
             "by_launch": by, "ms_per_token": round(floor_ms, 4),
             "tokens_per_s": round(1e3 / floor_ms, 1),
             "measured_ms_per_token": round(ms_per_step, 4),
             "measured_over_floor_rate": round(floor_ms / ms_per_step, 4)}
    sizes = {}
    for nbytes in (1073741824, srcs[0].nbytes):
        us = read_chain_us(rt, stream, srcs, nbytes)
        sizes[str(nbytes)] = rate(nbytes, us)
        log(f"stream read {nbytes / 2**20:7.0f} MiB: {us:8.2f} us ({sizes[str(nbytes)]['gbs']:.0f} GB/s)")
    ceiling = dict(sizes[str(srcs[0].nbytes)])
    ceiling["kernel"] = "ammon_stream_read (pure read, 2 workgroups per CU, contiguous shares)"
    ceiling["by_size"] = sizes
    return floor, ceiling


C3_CTX = (1024, 4096, 8192)


def c3_attention(rt, stream, cpu_budget):
    """Single-layer decode attention, 32 q / 8 kv heads of 128, bf16 KV, at
    position ctx - 1 of a cache of ctx positions: split partials + merge
    (ammon_attention_decode).  Caches rotate through a 1.07 GB pool (one
    per launch, a graph of all of them), so no launch reads from cache what
    an earlier one brought in.  CPU leg: the oracle's split-8 pair on the
    first cache of the pool; parity: the GPU output against it."""
    import oracle
    from ammon_amd import attention_scratch_bytes, kv_unpermute
    from ammon_amd._abi import BF16, F32, call, lib

    q_heads, kv_heads, head = 32, 8, 128
    pool_elems = 32 * 2 * kv_heads * 8192 * head  # 32 layers' K and V at 8192
    pool = rt.alloc(pool_elems * 2)
    rt.fill_normal(pool, BF16, pool_elems, 7, 300)
    qh = oracle.normal(q_heads * head, 301).reshape(q_heads, head)
    q = rt.upload(qh)
    out = rt.alloc(q_heads * head * 4)
    rt.synchronize()
    lines = {}
    for ctx in C3_CTX:
        split = int(lib.ammon_attention_default_split_for(rt.handle, q_heads, kv_heads, head, BF16,
                                                          ctx))
        part_bytes = attention_scratch_bytes(q_heads, head, ctx, split)
        part = rt.alloc(part_bytes)
        per = kv_heads * ctx * head  # elements of one K (or V) cache
        pairs = pool_elems // (2 * per)
        step = rt.step(0, ctx - 1)
        ptr = lambda i: ctypes.c_void_p(int(pool) + i * per * 2)

        def launch_all():
            for i in range(pairs):
                call("ammon_attention_decode", rt.handle, stream, q, q_heads, ptr(2 * i),
                     ptr(2 * i + 1), BF16, kv_heads, head, ctx, step, split, part, part_bytes,
                     out)

        us = graph_ms(rt, stream, launch_all) * 1e3 / pairs
        nbytes = 2 * ctx * kv_heads * head * 2 + 8 * q_heads * head
        line = rate(nbytes, us)
        line.update({"split": split, "launches_timed": pairs})
        # parity and CPU leg on the pool's first cache
        call("ammon_attention_decode", rt.handle, stream, q, q_heads, ptr(0), ptr(1), BF16,
             kv_heads, head, ctx, step, split, part, part_bytes, out)
        rt.synchronize(stream)
        got = out.download((q_heads, head))
        kv = []
        for i in (0, 1):
            hm = np.empty((kv_heads, ctx, head), np.uint16)
            call("ammon_memcpy", rt.handle, hm.ctypes.data, ptr(i), hm.nbytes, 2, None)
            rt.synchronize()
            kv.append(kv_unpermute(hm, kv_heads, ctx, head))
        want = oracle.attention(qh, kv[0], kv[1], BF16, ctx - 1)
        line["rel_err_vs_oracle"] = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
        s = cpu_seconds(lambda: oracle.attention(qh, kv[0], kv[1], BF16, ctx - 1), cpu_budget)
        line["cpu_us"] = round(s * 1e6, 1)
        lines[str(ctx)] = line
        part.free()
        log(f"C3 ctx {ctx}: {us:.2f} us ({line['gbs']:.0f} GB/s, frac {line['frac']:.3f}); "
            f"cpu {s * 1e6:.0f} us; rel err {line['rel_err_vs_oracle']:.1e}")
    pool.free()
    return {"workload": "single-layer decode attention, 32 q / 8 kv heads of 128, bf16 KV, "
                        "position ctx - 1; partials + merge per launch", "ctx": lines}


def c2_kernels(rt, stream, tok_emb, cpu_budget):
    """The isolated kernels: embedding gather of 4096 ids from the 128256 x
    4096 table (bf16 and fp32; 32 id sets per timed graph), RMSNorm over 64
    and 1 rows of 4096 (eps 1e-5; inputs rotated through a 1 GiB pool), RoPE
    (theta 500000) of Q [32 x 128] and K [8 x 128] with the cache store at 64
    random positions, SwiGLU over 14336.  The last two move kilobytes: their
    times are launch latency, not bandwidth."""
    import oracle
    from ammon_amd import rope_table_host
    from ammon_amd._abi import BF16, F32, call

    out = {}
    vocab, dim, rows = 128256, 4096, 4096
    rng = np.random.default_rng(1002)
    id_sets = [rt.upload(rng.integers(0, vocab, rows).astype(np.uint32)) for _ in range(32)]
    x = rt.alloc(rows * dim * 4)
    tab32 = rt.alloc(vocab * dim * 4)
    rt.fill_normal(tab32, F32, vocab * dim, 9, 1)
    rt.synchronize()
    host_bf16 = tok_emb.download(vocab * dim, np.uint16).reshape(vocab, dim)
    host_ids = id_sets[0].download(rows, np.uint32)
    for name, table, dt, es in (("embed_bf16", tok_emb, BF16, 2), ("embed_f32", tab32, F32, 4)):
        def launch_all(table=table, dt=dt):
            for ids in id_sets:
                call("ammon_embed_rows", rt.handle, stream, table, dt, vocab, dim, ids, rows, x)
        us = graph_ms(rt, stream, launch_all) * 1e3 / len(id_sets)
        out[name] = rate(rows * dim * (es + 4) + 4 * rows, us)
        if dt == BF16:
            call("ammon_embed_rows", rt.handle, stream, table, dt, vocab, dim, id_sets[0], rows, x)
            rt.synchronize(stream)
            got = x.download((rows, dim))
            want = oracle.embed(host_bf16, BF16, host_ids)
            out[name]["bit_exact_vs_oracle"] = bool(np.array_equal(got, want))
            s = cpu_seconds(lambda: oracle.embed(host_bf16, BF16, host_ids), cpu_budget)
            out[name]["cpu_us"] = round(s * 1e6, 1)
    tab32.free()
    del host_bf16
    # RMSNorm, in place over slices of a 1 GiB pool
    pool_floats = 1 << 28
    pool = rt.alloc(pool_floats * 4)
    rt.fill_normal(pool, F32, pool_floats, 9, 2)
    w = rt.alloc(dim * 4)
    rt.fill_normal(w, F32, dim, 9, 3, 1.0, 0.2)
    rt.synchronize()
    for nrows in (64, 1):
        # at most 1024 launches per graph, spread over the whole pool
        n = min(pool_floats // (nrows * dim), 1024)
        stride = pool_floats // n * 4
        sl = lambda i, stride=stride: ctypes.c_void_p(int(pool) + i * stride)

        def launch_all(n=n, nrows=nrows, sl=sl):
            for i in range(n):
                call("ammon_rmsnorm", rt.handle, stream, sl(i), w, F32, sl(i), nrows, dim, 1e-5)
        us = graph_ms(rt, stream, launch_all, reps=3) * 1e3 / n
        out[f"rmsnorm_{nrows}x{dim}"] = rate(nrows * dim * 8 + dim * 4, us)
    xh = oracle.normal(64 * dim, 9).reshape(64, dim)
    wh = oracle.normal(dim, 10, mean=1.0, std=0.2)
    out[f"rmsnorm_64x{dim}"]["cpu_us"] = round(
        cpu_seconds(lambda: oracle.rmsnorm(xh, wh), cpu_budget) * 1e6, 1)
    pool.free()
    # RoPE + K store, SwiGLU: launch-latency bound
    q_heads, kv_heads, head, seq = 32, 8, 128, 8192
    table = rt.upload(rope_table_host(500000.0, head, seq))
    qb = rt.alloc(q_heads * head * 4)
    kp = rt.alloc(kv_heads * head * 4)
    kc = rt.alloc(kv_heads * seq * head * 2)
    rt.fill_normal(qb, F32, q_heads * head, 9, 4)
    rt.fill_normal(kp, F32, kv_heads * head, 9, 5)
    steps = [rt.step(0, int(p)) for p in rng.integers(0, seq, 64)]

    def rope_all():
        for st in steps:
            call("ammon_rope_store", rt.handle, stream, qb, q_heads, kp, kv_heads, head, kc, BF16,
                 seq, st, table)
    us = graph_ms(rt, stream, rope_all) * 1e3 / len(steps)
    out["rope_store"] = rate(4 * q_heads * head * 2 + 4 * kv_heads * head + 2 * kv_heads * head,
                             us)
    hb = rt.alloc(14336 * 4)
    hb2 = rt.alloc(14336 * 4)
    rt.fill_normal(hb, F32, 14336, 9, 6)
    rt.fill_normal(hb2, F32, 14336, 9, 7)

    def swiglu_all():
        for _ in range(64):
            call("ammon_swiglu", rt.handle, stream, hb, hb2, 14336)
    us = graph_ms(rt, stream, swiglu_all) * 1e3 / 64
    out["swiglu_14336"] = rate(3 * 4 * 14336, us)
    g = oracle.normal(14336, 11)
    u = oracle.normal(14336, 12)
    out["swiglu_14336"]["cpu_us"] = round(cpu_seconds(lambda: oracle.swiglu(g, u), cpu_budget) * 1e6,
                                          1)
    for k, v in out.items():
        log(f"C2 {k}: {v['avg_us']:.2f} us ({v['gbs']:.0f} GB/s)"
            + (f"; cpu {v['cpu_us']:.0f} us" if "cpu_us" in v else ""))
    return {"workload": "isolated kernels: embed 4096 ids of 128256 x 4096, RMSNorm 64 and 1 "
                        "rows x 4096, RoPE + K store (32/8 heads of 128), SwiGLU 14336",
            "kernels": out}


C1 = dict(dim=288, n_layers=6, n_heads=6, n_kv_heads=6, hidden=768, vocab=32000, max_seq=256,
          theta=10000.0, eps=1e-5)


def c1_decode(rt, cpu_budget):
    """The tiny fp32 decoder (dim 288, 6 layers, 6 heads of 48, SwiGLU 768,
    vocab 32000), seeded 8-token prompt, max_new_tokens 256: 255 greedy steps
    by the reference's loop on the device (tokens/s with the reference's
    formula) and by the oracle on the host from the same weights."""
    import oracle
    from ammon_amd import LlamaModel
    from ammon_amd._abi import F32

    c = Cfg(**C1, w_dtype=F32, kv_dtype=F32)
    m = LlamaModel.synthetic(rt, c, seed=1000, std=0.02)
    prompt = np.random.default_rng(1001).integers(1, c.vocab, 8).astype(np.int32)
    m.generate_tokens_device(prompt, 256)  # warm: graph capture
    toks, _, tps = m.generate_tokens_device(prompt, 256)
    toks_h, _, tps_h = m.generate_tokens(prompt, 256)
    host = {}
    shapes = oracle.weight_shapes(oracle.LlamaConfig(**{k: C1[k] for k in (
        "dim", "n_layers", "n_heads", "n_kv_heads", "hidden", "vocab", "max_seq")}))
    for name, buf in m.weights.items():
        host[name] = buf.download(shapes[name], np.float32)
    m.close()
    om = oracle.Model(oracle.LlamaConfig(**C1), host)
    t0 = time.perf_counter()
    want, _ = om.generate_tokens(prompt, 256)
    cpu_s = time.perf_counter() - t0
    om.close()
    line = {"tokens_per_s_device_loop": round(tps, 1), "tokens_per_s_host_loop": round(tps_h, 1),
            "steps": 255, "token_parity": bool(np.array_equal(toks, want) and
                                                np.array_equal(toks_h, want)),
            "cpu": {"tokens_per_s": round(255 / cpu_s, 1), "seconds": round(cpu_s, 2),
                    "cores": oracle.num_threads(), "kind": "port",
                    "sample": "the full 255-step greedy run"}}
    log(f"C1: {tps:.0f} tok/s device loop, {tps_h:.0f} host loop; cpu {255 / cpu_s:.1f} tok/s; "
        f"parity {line['token_parity']}")
    return line


C4_FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "golden",
                          "c4_greedy.npz")


def c4_generate(rt, cpu_budget):
    """The Llama-3-8B-shaped greedy decode as configured: 32 layers, bf16
    weights N(0, 0.02) (weight seed 1003), a seeded 16-token prompt and
    max_new_tokens 528 -- 527 steps, 512 generated -- with tokens/s by the
    reference's formula (src/generate.rs:73-84: steps after the first over
    the time from the end of the first) for the device loop and the host
    loop.  With the reference's fp32 cache the tokens are checked against
    the oracle's run stored in tests/golden/c4_greedy.npz: all 527 equal, or
    equal up to a step where the runs part at a near tie (the oracle's top-2
    margin within twice the logits' 1e-4 normwise tolerance); with a bf16
    cache (the headline's storage) the same loops are timed.  CPU leg:
    the oracle on the same weights from the same prompt for a bounded number
    of steps, with token parity against the GPU's."""
    import oracle
    from ammon_amd import LlamaModel
    from ammon_amd._abi import BF16, F32

    f = np.load(C4_FIXTURE)
    c4 = json.loads(str(f["config"]))
    prompt = np.asarray(f["prompt"], np.int32)
    max_new = int(f["max_new_tokens"])
    want = np.asarray(f["tokens"], np.int32)
    margins, scales = f["margins"].astype(np.float64), f["scales"].astype(np.float64)

    def parity(got):
        """True if equal, or equal up to a parting at a near tie."""
        bad = np.nonzero(np.asarray(got) != want)[0]
        if bad.size == 0:
            return True
        i = int(bad[0])
        return i >= len(prompt) - 1 and margins[i] <= 2e-4 * scales[i]
    line = {"workload": "Llama-3-8B-shaped greedy decode, 16-token seeded prompt, "
                        f"max_new_tokens {max_new} ({max_new - 1} steps, "
                        f"{max_new - len(prompt)} generated); bf16 weights",
            "steps": max_new - 1}
    weights = None
    for kv_name, kv in (("kv_f32", F32), ("kv_bf16", BF16)):
        c = Cfg(**c4, w_dtype=BF16, kv_dtype=kv)
        if weights is None:
            m = LlamaModel.synthetic(rt, c, seed=int(f["weight_seed"]), std=0.02)
            weights = m.weights
        else:
            m = LlamaModel(rt, c, weights)
        m.generate_tokens_device(prompt, 16)  # warm: graph capture
        toks, _, tps = m.generate_tokens_device(prompt, max_new)
        toks_h, _, tps_h = m.generate_tokens(prompt, max_new)
        r = {"tokens_per_s_device_loop": round(tps, 1), "tokens_per_s_host_loop": round(tps_h, 1),
             "loops_agree": bool(np.array_equal(toks, toks_h))}
        if kv == F32:
            r["tokens_equal_oracle_fixture"] = bool(np.array_equal(toks, want) and
                                                   np.array_equal(toks_h, want))
            r["tokens_match_oracle_up_to_near_tie"] = bool(parity(toks) and parity(toks_h))
            gpu_toks = toks
        line[kv_name] = r
        m.close()
        log(f"C4 {kv_name}: {tps:.1f} tok/s device loop, {tps_h:.1f} host loop" +
            (f"; tokens equal the oracle's fixture: {r['tokens_equal_oracle_fixture']}"
             if kv == F32 else ""))
    if cpu_budget > 0:
        c = Cfg(**c4, w_dtype=BF16, kv_dtype=F32)
        shapes = oracle.weight_shapes(oracle.LlamaConfig(**{k: c4[k] for k in (
            "dim", "n_layers", "n_heads", "n_kv_heads", "hidden", "vocab", "max_seq")}))
        host = {}
        for name, buf in weights.items():
            host[name] = buf.download(shapes[name],
                                      np.float32 if name.startswith("rms") else np.uint16)
        om = oracle.Model(oracle.LlamaConfig(**c4, w_dtype=BF16, kv_dtype=F32), host)
        tok, toks, times = int(prompt[0]), [], []
        for pos in range(max_new - 1):
            t0 = time.perf_counter()
            logits = om.step(tok, pos)
            times.append(time.perf_counter() - t0)
            tok = int(prompt[pos + 1]) if pos < len(prompt) - 1 else int(oracle.sample_argmax(logits))
            toks.append(tok)
            if sum(times) > cpu_budget:
                break
        om.close()
        n = len(times)
        line["cpu"] = {"tokens_per_s": round(n / sum(times), 2), "steps": n,
                       "cores": oracle.num_threads(), "kind": "port",
                       "sample": f"the first {n} of the {max_new - 1} steps, fp32 cache",
                       "token_parity": bool(np.array_equal(toks, gpu_toks[:n]))}
        log(f"C4 cpu: {line['cpu']['tokens_per_s']} tok/s over {n} steps; parity "
            f"{line['cpu']['token_parity']}")
    for buf in weights.values():
        buf.free()
    return line


C5 = dict(dim=8192, n_layers=1, n_heads=64, n_kv_heads=8, hidden=28672, vocab=128256,
          max_seq=32768, theta=500000.0, eps=1e-5)


def c5_layer(rt, cpu_budget, steps=16):
    """One Llama-3-70B-shaped layer + final norm + LM head, bf16 weights and
    KV, the cache prefilled N(0, 1): greedy decode steps at positions
    32752..32767 as one graph per step; ms per step against the HBM roofline
    of its bytes.  CPU leg: the oracle on the same weights and cache, a few
    steps from 32752, with token parity."""
    import oracle
    from ammon_amd import LlamaModel, Timer, kv_unpermute
    from ammon_amd._abi import BF16, F32, call

    c = Cfg(**C5, w_dtype=BF16, kv_dtype=BF16)
    head = c.dim // c.n_heads
    m = LlamaModel.synthetic(rt, c, seed=70, std=0.02)
    for i, name in enumerate(("rms_att", "rms_ffn", "rms_final")):
        rt.fill_normal(m.weights[name], F32, c.dim, 71, i, 1.0, 0.2)
    kv_n = c.n_kv_heads * c.max_seq * head
    k, v = ctypes.c_void_p(), ctypes.c_void_p()
    call("ammon_llama_kv_layer", m.handle, 0, ctypes.byref(k), ctypes.byref(v))
    rt.fill_normal(k, BF16, kv_n, 72, 0)
    rt.fill_normal(v, BF16, kv_n, 72, 1)
    rt.synchronize()
    start = c.max_seq - steps
    m.decode(128000, start - 8, 8)  # warm: graph capture
    timer = Timer(rt)
    timer.start(m.stream)
    m.decode(128000, start, steps)
    timer.stop(m.stream)
    ms = timer.elapsed_ms() / steps
    timer.close()
    gpu_tokens = m.read_tokens(start, steps)
    nbytes = token_bytes(c, c.max_seq - steps // 2)
    line = {"ms_per_step": round(ms, 4), "step_bytes": nbytes,
            "roofline_ms": round(nbytes / (HBM_PEAK_GBS * 1e9) * 1e3, 4),
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if cpu_budget > 0:
        shapes = oracle.weight_shapes(oracle.LlamaConfig(**{kk: C5[kk] for kk in (
            "dim", "n_layers", "n_heads", "n_kv_heads", "hidden", "vocab", "max_seq")}))
        host = {}
        for name, buf in m.weights.items():
            dt = np.float32 if name.startswith("rms") else np.uint16
            host[name] = buf.download(shapes[name], dt)
        om = oracle.Model(oracle.LlamaConfig(**C5, w_dtype=BF16, kv_dtype=BF16), host)
        for src, get in ((k, oracle._lib.orc_model_key_cache), (v, oracle._lib.orc_model_value_cache)):
            hm = np.empty((c.n_kv_heads, c.max_seq, head), np.uint16)
            call("ammon_memcpy", rt.handle, hm.ctypes.data, src, hm.nbytes, 2, None)
            rt.synchronize()
            pm = kv_unpermute(hm, c.n_kv_heads, c.max_seq, head)
            ctypes.memmove(get(om._handle, 0), pm.ctypes.data, pm.nbytes)
        # the GPU decode from `start` began with token 128000
        tok, toks, times = 128000, [], []
        for pos in range(start, c.max_seq):
            t0 = time.perf_counter()
            logits = om.step(tok, pos)
            times.append(time.perf_counter() - t0)
            tok = int(oracle.sample_argmax(logits))
            toks.append(tok)
            if sum(times) > cpu_budget:
                break
        om.close()
        line["cpu"] = {"ms_per_step": round(1e3 * sum(times) / len(times), 1),
                       "steps": len(times), "cores": oracle.num_threads(), "kind": "port",
                       "token_parity": bool(np.array_equal(toks, gpu_tokens[: len(toks)]))}
    m.close()
    log(f"C5: {ms:.3f} ms/step (roofline {line['roofline_ms']:.3f} ms, frac {line['frac']:.3f})"
        + (f"; cpu {line['cpu']['ms_per_step']:.0f} ms/step, parity {line['cpu']['token_parity']}"
           if "cpu" in line else ""))
    return line


def oracle_layout(head_major, kv_heads, seq, head):
    from ammon_amd import kv_unpermute
    return kv_unpermute(head_major.reshape(kv_heads, seq, head), kv_heads, seq, head)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--kernel-reps", type=int, default=3)
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of CPU decode for the baseline (0 skips it)")
    ap.add_argument("--no-graph", action="store_true", help="replay launches without a graph")
    ap.add_argument("--split", type=int, default=0,
                    help="attention split length (0: the library's choice)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prompt-prefill lines")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other workloads' lines (C1-C5) and the stream ceiling")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain streaming kernel of known size (ammon_add over "
                         "256 MiB operands), the calibration for HBM byte counters")
    ap.add_argument("--config", choices=("c1", "c2", "c3", "c4", "c5"),
                    help="run only that workload's line (no headline) and print it as JSON: "
                         "for profiling one workload on its own")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the decode "
              f"path here is single-device.", file=sys.stderr)
        sys.exit(2)

    import ammon_amd
    from ammon_amd import Runtime, Timer
    from ammon_amd._abi import BF16, call

    if args.config:
        rt = Runtime(0)
        cb = 0.0 if args.no_cpu else args.cpu_budget
        if args.copy_probe:
            copy_probe(rt)
        small = 0.5 if cb > 0 else 0.0

        def c2_alone():
            from ammon_amd._abi import BF16
            vocab, dim = LLAMA3_8B["vocab"], LLAMA3_8B["dim"]
            table = rt.alloc(vocab * dim * 2)
            rt.fill_normal(table, BF16, vocab * dim, 2024, 0, 0.0, 0.02)
            try:
                return c2_kernels(rt, None, table, small)
            finally:
                table.free()

        fn = {"c1": lambda: c1_decode(rt, cb), "c2": c2_alone,
              "c3": lambda: c3_attention(rt, None, small),
              "c4": lambda: c4_generate(rt, min(cb, 10.0)),
              "c5": lambda: c5_layer(rt, min(cb, 10.0))}
        print(json.dumps({"config": args.config, args.config: fn[args.config]()}), flush=True)
        return

    c = Cfg(**LLAMA3_8B, w_dtype=BF16, kv_dtype=BF16)
    total = args.steps + args.warmup
    if total >= c.max_seq:
        sys.exit("steps + warmup must be below the context length")
    start_pos = c.max_seq - total
    rt = Runtime(0)
    log(f"device {rt.info.arch.decode()} cus={rt.info.compute_units}; generating weights")
    t0 = time.time()
    model = ammon_amd.LlamaModel.synthetic(rt, c, seed=2024, std=0.02,
                                           use_graph=not args.no_graph, split_len=args.split)
    head = c.dim // c.n_heads
    kv_n = c.n_kv_heads * c.max_seq * head
    for l in range(c.n_layers):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        call("ammon_llama_kv_layer", model.handle, l, ctypes.byref(k), ctypes.byref(v))
        rt.fill_normal(k, BF16, kv_n, 7, 2 * l)
        rt.fill_normal(v, BF16, kv_n, 7, 2 * l + 1)
    rt.synchronize()
    # the decode graph: the step's launch list with the LM head carrying the
    # argmax's first pass, plus the argmax's second pass
    launches = model.launches + 1
    log(f"weights + KV prefill in {time.time() - t0:.1f}s; launches/token={launches}")

    if args.copy_probe:
        copy_probe(rt)

    token0 = 128000
    stream = model.stream
    # Warmup continues the same greedy chain the timed steps extend; the
    # first decode captures the token graph.
    model.decode(token0, start_pos, args.warmup)
    warm = model.read_tokens(start_pos, args.warmup)
    next_token = int(warm[-1]) if args.warmup else token0
    timer = Timer(rt)
    t_wall = time.perf_counter()
    timer.start(stream)
    model.decode(next_token, start_pos + args.warmup, args.steps)
    timer.stop(stream)
    ms = timer.elapsed_ms()
    wall = time.perf_counter() - t_wall
    timer.close()
    gpu_tokens = model.read_tokens(start_pos, total)
    ms_per_step = ms / args.steps
    tps = 1000.0 / ms_per_step
    ctx_mid = start_pos + args.warmup + args.steps // 2
    tok_bytes = token_bytes(c, ctx_mid)
    log(f"{args.steps} tokens in {ms:.2f} ms (wall {wall * 1e3:.1f} ms): {tps:.1f} tok/s, "
        f"{tok_bytes / (ms_per_step * 1e-3) / 1e9:.0f} GB/s per token stream")

    kernels = time_kernels(rt, model, c, model.weights, ctx_mid, args.kernel_reps, args.split,
                           use_graph=not args.no_graph)
    for k, v in kernels.items():
        log(f"  {k:18s} {v['avg_us']:9.2f} us  {v['gbs']:7.1f} GB/s  frac {v['frac']:.3f}")
    dom = kernels[DOMINANT]
    traffic = measured_traffic(DOMINANT, dom["bytes"])

    cpu = None
    if args.cpu_budget > 0 and not args.no_cpu:
        cpu = cpu_baseline(rt, model, c, model.weights, start_pos, token0, gpu_tokens,
                           args.cpu_budget)
        log(f"cpu baseline: {cpu}")

    # after the CPU baseline: prefill rewrites the first cache positions
    prefill = None if args.no_prefill else prefill_measure(rt, model, c)

    # the other workloads, each with its CPU leg (not part of `value`)
    extras = {}
    if not args.no_configs:
        cb = 0.0 if args.no_cpu else args.cpu_budget
        small = 0.5 if cb > 0 else 0.0
        for name, fn in (("launch_floor", lambda: launch_floor(rt, model, kernels, ms_per_step)),
                         ("c3", lambda: c3_attention(rt, stream, small)),
                         ("c2", lambda: c2_kernels(rt, stream, model.weights["tok_emb"], small)),
                         ("c1", lambda: c1_decode(rt, cb)),
                         ("c4", lambda: c4_generate(rt, min(cb, 10.0))),
                         ("c5", lambda: c5_layer(rt, min(cb, 10.0)))):
            try:
                extras[name] = fn()
            except Exception as e:  # recorded in the JSON line; the headline stands
                extras[name] = {"error": f"{type(e).__name__}: {e}"}
                log(f"{name} failed: {extras[name]['error']}")

    # (floor, ceiling), or an error record in the floor's place
    lf = extras.pop("launch_floor", None)
    floor, ceiling = lf if isinstance(lf, tuple) else (lf, None)
    result = {
        "metric": METRIC,
        "value": round(tps, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": ("Llama-3-8B-shaped greedy decode at context 8192: 32 layers, dim 4096, "
                         "32 q / 8 kv heads of 128, SwiGLU 14336, vocab 128256, RoPE theta "
                         "500000; bf16 weights and KV cache, fp32 activations and "
                         "accumulation; random N(0, 0.02) weights, KV prefilled N(0, 1)"),
            "batch": 1,
            "positions": [start_pos + args.warmup, c.max_seq - 1],
            "graph_replay": not args.no_graph,
            "launches_per_token": launches,
            "token_bytes": tok_bytes,
            "token_hbm_gbs": round(tok_bytes / (ms_per_step * 1e-3) / 1e9, 1),
            "token_roofline_frac": round(tok_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                         4),
        },
        "roofline": {
            "kernel": DOMINANT_NAME,
            "bound": "hbm",
            "achieved": dom["gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dom["frac"],
            "traffic": traffic.get("traffic_bytes"),
            "traffic_source": traffic.get("source"),
            "bytes_per_launch": dom["bytes"],
            "avg_launch_us": dom["avg_us"],
        },
        "kernels": kernels,
        "prefill": prefill,
        "cpu_baseline": cpu,
        "launch_floor": floor,
        "stream_read_ceiling": ceiling,
        "configs": {k: extras[k] for k in ("c1", "c2", "c3", "c4", "c5") if k in extras},
    }
    model.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
