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


def kernel_bytes(c, ctx):
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
    logits = rt.alloc(c.vocab * 4)
    step = rt.step(1, ctx - 1)
    table = rt.upload(ammon_amd.rope_table_host(c.theta, head, c.max_seq))
    if not split:
        split = int(ammon_amd._abi.lib.ammon_attention_default_split(rt.handle, c.n_kv_heads, c.max_seq))
    part = rt.alloc(ammon_amd.attention_scratch_bytes(c.n_heads, head, c.max_seq, split))
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
    nbytes = kernel_bytes(c, ctx)
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
    }


MFMA_BF16_PEAK_TFLOPS = 2500.0


def prefill_measure(rt, model, c, prompt_lengths=(16, 512), reps=3):
    """Prompt prefill (one pass per layer: GEMMs on matrix cores, token-
    batched attention) of T-token prompts from position 0: whole-model
    time, and the gate/up GEMM + SwiGLU alone (events around 10 launches on
    the model's stream).  Short prompts are HBM-bound on W (bytes: W once +
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
        args = (rt.handle, stream, x, T, w1, w3, BF16, c.dim, c.hidden, hb)
        call("ammon_prefill_gate_up_swiglu", *args)
        timer.start(stream)
        for _ in range(10):
            call("ammon_prefill_gate_up_swiglu", *args)
        timer.stop(stream)
        us = timer.elapsed_ms() * 1e3 / 10
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
    ap.add_argument("--persistent", action="store_true",
                    help="one persistent cooperative kernel per token")
    ap.add_argument("--split", type=int, default=0,
                    help="attention split length (0: the library's choice)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prompt-prefill lines")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain streaming kernel of known size (ammon_add over "
                         "256 MiB operands), the calibration for HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the decode "
              f"path here is single-device.", file=sys.stderr)
        sys.exit(2)

    import ammon_amd
    from ammon_amd import Runtime, Timer
    from ammon_amd._abi import BF16, call

    c = Cfg(**LLAMA3_8B, w_dtype=BF16, kv_dtype=BF16)
    total = args.steps + args.warmup
    if total >= c.max_seq:
        sys.exit("steps + warmup must be below the context length")
    start_pos = c.max_seq - total
    rt = Runtime(0)
    log(f"device {rt.info.arch.decode()} cus={rt.info.compute_units}; generating weights")
    t0 = time.time()
    model = ammon_amd.LlamaModel.synthetic(rt, c, seed=2024, std=0.02,
                                           use_graph=not args.no_graph, split_len=args.split,
                                           persistent=args.persistent)
    head = c.dim // c.n_heads
    kv_n = c.n_kv_heads * c.max_seq * head
    for l in range(c.n_layers):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        call("ammon_llama_kv_layer", model.handle, l, ctypes.byref(k), ctypes.byref(v))
        rt.fill_normal(k, BF16, kv_n, 7, 2 * l)
        rt.fill_normal(v, BF16, kv_n, 7, 2 * l + 1)
    rt.synchronize()
    # the decode graph: the step's launch list with the LM head carrying the
    # argmax's first pass, plus the argmax's second pass (one launch when
    # persistent)
    launches = 1 if args.persistent else model.launches + 1
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
    dom = kernels["gate_up_swiglu"]
    traffic = measured_traffic("gate_up_swiglu", dom["bytes"])

    cpu = None
    if args.cpu_budget > 0 and not args.no_cpu:
        cpu = cpu_baseline(rt, model, c, model.weights, start_pos, token0, gpu_tokens,
                           args.cpu_budget)
        log(f"cpu baseline: {cpu}")

    # after the CPU baseline: prefill rewrites the first cache positions
    prefill = None if args.no_prefill else prefill_measure(rt, model, c)

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
            "kernel": "ammon_gemv_bf16_v_swiglu (gate/up GEMV + SwiGLU, RMSNorm prologue)",
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
    }
    model.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
