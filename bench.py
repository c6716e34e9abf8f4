"""Benchmark of the quantized compute path on one MI355X.

Headline workload (BASELINE metric "quant matvec HBM GB/s (% of peak) at
14336x4096 b=1; decode-attn tok/s @32k ctx"): one step = one batch-1 Q4_K
matvec of the Llama-3-8B FFN up projection (W 14336x4096, config 3), with the
weights resident in HBM.  Steps rotate over enough weight copies that the
working set exceeds twice the 256 MB last-level cache, so every step streams
W from HBM.  value = algorithmic bytes per step * steps / elapsed.

The JSON line also carries, measured the same way in shorter runs, the other
configurations (Q4_0 at the target shape and 4096^2, Q8_0 B=1/4/8, Q6_K, the
prefill GEMM, INT8 KV quantization and paged INT8 decode attention), the
roofline record of the headline kernel and the CPU oracle baseline.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ssd-llm_amd"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
LLC_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    # ~9 ms of untimed replays: the first millisecond after a pause runs up to 5% slow
    ap.add_argument("--warmup", type=int, default=1000)
    ap.add_argument("--no-extras", action="store_true", help="only the headline workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--profile-pass", action="store_true",
                    help="short run for hardware-counter passes: a Q8_0 dequant of known size (the "
                         "counter calibration), then a few launches of every configuration's kernels; "
                         "prints no JSON")
    ap.add_argument("--ceiling", action="store_true",
                    help="plain streaming-read bandwidth versus size and the cost of an empty launch "
                         "(libssdq_probe.so), timed like the matvecs; prints one JSON line")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="fp16 matrix-core rate of a register-operand MFMA loop (random or zero operands, "
                         "0-4 VALU instructions per MFMA; libssdq_probe.so) and torch's fp16 GEMM at the "
                         "config-4 shapes; prints one JSON line")
    ap.add_argument("--hipblaslt", action="store_true",
                    help="torch's fp16 GEMM (hipBLASLt) of the config-4 layer shapes on already "
                         "dequantized weights, for comparison with the Q4_K prefill GEMM; prints one JSON line")
    ap.add_argument("--layer", action="store_true",
                    help="only the decoder-layer case (one Llama-3-8B layer from resident weights, "
                         "ssdq_decode_layer_dev), for a kernel trace of its steps; prints one JSON line")
    ap.add_argument("--eager", action="store_true",
                    help="launch every matvec step from Python instead of replaying captured HIP graphs")
    return ap.parse_args()


def copies_for(nbytes):
    return max(2, min(64, (2 * LLC_BYTES) // max(1, nbytes) + 1))


class Timer:
    """Events on the stream the kernels are launched on (torch's current stream).

    Short kernels (the matvecs take ~10 us) are replayed from HIP graphs of up
    to GRAPH_CHUNK captured launches, so the host's per-launch cost (ctypes
    marshalling, ~15 us) does not set the step time.  A timed block is exactly
    `steps` launches (whole replays of the chunk graph, then one replay of a
    graph of the remainder), bracketed by device synchronizations.  Each block
    is enqueued twice in a row, its start event between the two: the first,
    untimed copy keeps the device busy (and at its working clock) while the
    host enqueues the timed one, so the events time the device executing
    exactly the block's launches, not the host submitting them or the device
    leaving idle.

    Warm-up runs at least `warmup` launches and at least MIN_WARM_S seconds,
    in whole replays, then further untimed blocks until two consecutive blocks
    agree within SETTLE_TOL (at most SETTLE_MAX_S seconds: the first
    milliseconds after a pause run up to 5% slow).  Then at least MIN_BLOCKS
    and up to MAX_BLOCKS blocks are timed (STAB_S seconds); the reported time
    is their median, and the first of them is kept beside it."""

    GRAPH_CHUNK = 50
    MIN_WARM_S = 0.05
    SETTLE_TOL = 0.01
    SETTLE_MAX_S = 1.0
    STAB_S = 0.02
    MIN_BLOCKS = 5
    MAX_BLOCKS = 11

    def __init__(self, torch, graph=True):
        self.torch = torch
        self.graph = graph
        self.e0 = torch.cuda.Event(enable_timing=True)
        self.e1 = torch.cuda.Event(enable_timing=True)

    def _block(self, body):
        torch = self.torch
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        body()  # untimed lead copy
        self.e0.record()
        body()
        self.e1.record()
        torch.cuda.synchronize()
        return self.e0.elapsed_time(self.e1) * 1e-3, time.perf_counter() - t0

    def run(self, fn, steps, warmup, graph=None, stability=True):
        """Times `steps` launches of fn(i).  Returns a dict: t (the median event
        seconds of the timed blocks), t_median (the same), t_first (the first
        timed block), wall (its host seconds), steps, chunk (launches per graph
        replay, 0 when eager), warm_launches, settle_blocks (untimed blocks
        until two agreed) and blocks (timed blocks)."""
        torch = self.torch
        use_graph = self.graph if graph is None else graph
        if not use_graph:
            def body():
                for i in range(steps):
                    fn(i)
            warm, t0 = 0, time.perf_counter()
            while warm < warmup or time.perf_counter() - t0 < self.MIN_WARM_S:
                fn(warm)
                warm += 1
            chunk, graphs = 0, None
        else:
            chunk = min(self.GRAPH_CHUNK, steps)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):  # the library sizes its workspace for this stream
                for i in range(2):
                    fn(i)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for i in range(chunk):
                    fn(i)
            rem = steps % chunk
            g_rem = None
            if rem:
                g_rem = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g_rem, stream=side):
                    for i in range(rem):
                        fn(i)
            graphs = (g, g_rem)
            full = steps // chunk

            def body():
                for _ in range(full):
                    g.replay()
                if g_rem is not None:
                    g_rem.replay()
            warm, t0 = 0, time.perf_counter()
            while warm < warmup or time.perf_counter() - t0 < self.MIN_WARM_S:
                g.replay()
                warm += chunk
                if warm % (20 * chunk) == 0:
                    torch.cuda.synchronize()
            torch.cuda.synchronize()
        settle = 0
        if stability:
            prev, t1 = self._block(body)[0], time.perf_counter()
            settle = 1
            while time.perf_counter() - t1 < self.SETTLE_MAX_S:
                cur = self._block(body)[0]
                settle += 1
                if abs(cur - prev) <= self.SETTLE_TOL * min(cur, prev):
                    break
                prev = cur
        t_first, wall = self._block(body)
        times = [t_first]
        if stability:
            t1 = time.perf_counter()
            while len(times) < self.MAX_BLOCKS and (time.perf_counter() - t1 < self.STAB_S
                                                    or len(times) < self.MIN_BLOCKS):
                times.append(self._block(body)[0])
        del graphs
        med = sorted(times)[len(times) // 2]
        return {"t": med, "t_median": med, "t_first": t_first, "wall": wall, "steps": steps, "chunk": chunk,
                "warm_launches": warm, "settle_blocks": settle, "blocks": len(times)}


def matvec_case(torch, ssdq, synth, dtype, out_dim, in_dim, batch, seed_cfg):
    rb = ssdq.row_bytes(dtype, in_dim)
    wbytes = out_dim * rb
    n = copies_for(wbytes)
    base = torch.from_numpy(synth.quant_weights(dtype, out_dim, in_dim, synth.seed(seed_cfg, 0))).cuda()
    ws = [base] + [base.clone() for _ in range(n - 1)]
    x = torch.randn(batch * in_dim, device="cuda")
    y = torch.empty(batch * out_dim, device="cuda")
    algo_bytes = wbytes + 4 * batch * (in_dim + out_dim)

    def step(i):
        ssdq.matvec(dtype, ws[i % n], x, y, out_dim, in_dim, batch)

    return step, algo_bytes, 2.0 * batch * out_dim * (in_dim // ssdq.block_size(dtype)) * ssdq.block_size(dtype)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 (the sharding across GPUs "
                                   "is designed, not run: the boxes here have one GPU each)"}))
        sys.exit(2)
    import numpy as np
    import torch

    import ssdq
    from ssdq import synth

    torch.cuda.set_device(0)
    if args.profile_pass:
        profile_pass(torch, ssdq, synth)
        return
    if args.ceiling:
        print(json.dumps(read_ceiling(torch)))
        return
    if args.hipblaslt:
        print(json.dumps(hipblaslt_layer(torch)))
        return
    if args.mfma_ceiling:
        print(json.dumps(mfma_ceiling(torch)))
        return
    timer = Timer(torch, graph=not args.eager)
    if args.layer:
        print(json.dumps({"decode_layer_llama3_8b_q4k_ctx4096": decode_layer_case(torch, ssdq, synth, timer)}))
        return

    # ---------------------------------------------------------- headline
    step, algo_bytes, _ = matvec_case(torch, ssdq, synth, ssdq.Q4_K, 14336, 4096, 1, 3)
    tm = timer.run(step, args.steps, args.warmup)
    steps, wall = tm["steps"], tm["wall"]
    sec_per_step = tm["t"] / steps
    value = algo_bytes / sec_per_step / 1e9

    result = {
        "metric": "quant matvec HBM GB/s (% of peak) at 14336x4096 b=1; decode-attn tok/s @32k ctx",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec_per_step * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded GGUF Q4_K blocks per config 3, x ~ N(0,1)); weights HBM-resident, "
                "rotated over copies larger than 2x the last-level cache",
        "config": {"workload": "Q4_K matvec 14336x4096 batch 1 (Llama-3-8B FFN up, config 3)",
                   "out_dim": 14336, "in_dim": 4096, "batch": 1,
                   "weight_copies": copies_for(14336 * ssdq.row_bytes(ssdq.Q4_K, 4096)),
                   "weights": "GGUF Q4_K", "activations": "f32", "accumulate": "f32",
                   "launch": "eager" if args.eager else
                   f"hip graph replays of {tm['chunk']} launches (remainder in a second graph)",
                   "warmup_launches_run": tm["warm_launches"],
                   "timing": {"value_from": "median of the timed blocks of exactly `steps` launches",
                              "settle_blocks": tm["settle_blocks"], "timed_blocks": tm["blocks"],
                              "first_block_GB/s": round(algo_bytes * steps / tm["t_first"] / 1e9, 1),
                              "median_GB/s": round(algo_bytes * steps / tm["t_median"] / 1e9, 1)}},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles("q4k_matvec_14336x4096"),
            "kernel": "mv_b1r<Q4_K>", "algo_bytes_per_launch": algo_bytes,
        },
        "host_wall_s": round(wall, 4),
    }

    if not args.no_extras:
        result["extras"] = extras(torch, ssdq, synth, timer, np)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(np, synth, ssdq, sec_per_step)
    print(json.dumps(result))


CAL_ELEMS = 1 << 26  # Q8_0 dequant calibration: 71,303,168 B read, 268,435,456 B written


def profile_pass(torch, ssdq, synth):
    """Launch sequence profiled with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE, SQ_*).

    Dispatches, in order (each section on its own weight copies, so every
    launch streams from HBM):
      3 x dequant_kernel (Q8_0, CAL_ELEMS elements): a plain streaming kernel
          whose bytes are known exactly, used to scale the counters to bytes;
      20 x the headline Q4_K 14336x4096 batch-1 matvec (config 3);
      20 x Q4_0 4096x4096 and 20 x Q4_0 14336x4096 (config 1, north-star shape);
      20 x Q8_0 11008x4096 at B = 1, 4 and 8 (config 2);
      20 x Q6_K 4096x14336 (config 3; K slices + slice_reduce_kernel);
      3 x the config-4 prefill GEMM layer (q/k/v and gate/up fused, o, down);
      3 x INT8 quantize of 8 x 32768 x {K, V} rows of 1024 (config 5a);
      5 x paged INT8 decode attention, 8 x 32k context (config 5b)."""
    nb = CAL_ELEMS // 32
    raw = torch.randint(0, 256, (nb * 34,), dtype=torch.uint8, device="cuda")
    raw.view(nb, 34)[:, 0:2] = torch.tensor([0x00, 0x3C], dtype=torch.uint8, device="cuda")  # d = 1.0
    out = torch.empty(CAL_ELEMS, device="cuda")
    torch.cuda.synchronize()
    for _ in range(3):
        ssdq.dequant(ssdq.Q8_0, raw, CAL_ELEMS, out)
    torch.cuda.synchronize()
    del raw, out
    print(f"profile pass: calibration read {nb * 34} B write {CAL_ELEMS * 4} B", flush=True)
    for name, dt, od, idim, b, cfg in [("q4k_matvec_14336x4096", ssdq.Q4_K, 14336, 4096, 1, 3),
                                       ("q4_0_matvec_4096x4096", ssdq.Q4_0, 4096, 4096, 1, 1),
                                       ("q4_0_matvec_14336x4096", ssdq.Q4_0, 14336, 4096, 1, 1),
                                       ("q8_0_matvec_11008x4096_b1", ssdq.Q8_0, 11008, 4096, 1, 2),
                                       ("q8_0_matvec_11008x4096_b4", ssdq.Q8_0, 11008, 4096, 4, 2),
                                       ("q8_0_matvec_11008x4096_b8", ssdq.Q8_0, 11008, 4096, 8, 2),
                                       ("q6_k_matvec_4096x14336", ssdq.Q6_K, 4096, 14336, 1, 3)]:
        step, algo_bytes, _ = matvec_case(torch, ssdq, synth, dt, od, idim, b, cfg)
        step(0)
        torch.cuda.synchronize()
        for i in range(20):
            step(i)
        torch.cuda.synchronize()
        print(f"profile pass: {name} x20, algorithmic bytes {algo_bytes}", flush=True)
        del step
        torch.cuda.empty_cache()
    layer_fused, flops = gemm_layer(torch, ssdq, synth)
    layer_fused(0)
    torch.cuda.synchronize()
    for i in range(3):
        layer_fused(i)
    torch.cuda.synchronize()
    print(f"profile pass: prefill GEMM layer x3, {flops:.0f} FLOP per layer", flush=True)
    del layer_fused
    torch.cuda.empty_cache()
    n_rows, dim = 8 * 32768 * 2, 1024
    xk = torch.randn(n_rows * dim, device="cuda")
    codes = torch.empty(n_rows * dim, dtype=torch.int8, device="cuda")
    scales = torch.empty(n_rows, device="cuda")
    for _ in range(3):
        ssdq.kv_quantize_rows(xk, codes, scales, n_rows, dim)
    torch.cuda.synchronize()
    print(f"profile pass: kv quantize x3, algorithmic bytes {n_rows * dim * 5 + n_rows * 4}", flush=True)
    del xk
    attn = attention_case(torch, ssdq, synth, codes, scales)
    for i in range(5):
        attn(i)
    torch.cuda.synchronize()
    print("profile pass: paged attention x5, algorithmic bytes 539295744", flush=True)


def gemm_layer(torch, ssdq, synth):
    """The config-4 layer as the bench runs it: q/k/v and gate/up each one GEMM
    over shared X (multi entry point), o and down alone.  Returns (fn, FLOP)."""
    layer = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
             ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
    M = 512
    W, Y = {}, {}
    flops = 0
    for i, (nm, N, K) in enumerate(layer):
        W[nm] = torch.from_numpy(synth.quant_weights(ssdq.Q4_K, N, K, synth.seed(4, i))).cuda()
        Y[nm] = torch.empty(M * N, device="cuda")
        flops += 2.0 * M * N * K
    X = {4096: torch.randn(M, 4096, device="cuda").to(torch.bfloat16).view(torch.int16),
         14336: torch.randn(M, 14336, device="cuda").to(torch.bfloat16).view(torch.int16)}
    dims = {nm: (N, K) for nm, N, K in layer}
    groups = [("q", "k", "v"), ("o",), ("gate", "up"), ("down",)]

    def layer_fused(i):
        for g in groups:
            K = dims[g[0]][1]
            ssdq.gemm_q4k_bf16_multi([W[n] for n in g], X[K], [Y[n] for n in g], M, [dims[n][0] for n in g], K)

    def layer_separate(i):
        for nm, N, K in layer:
            ssdq.gemm_q4k_bf16(W[nm], X[K], Y[nm], M, N, K)

    layer_fused.separate = layer_separate
    return layer_fused, flops


def decode_layer_case(torch, ssdq, synth, timer, ctx=4096):
    """One Llama-3-8B decoder layer for one token from resident weights
    (ssdq_decode_layer_dev): Q4_K projections, Q6_K down, `ctx` earlier tokens
    in the layer's paged INT8 pool (block 16).  Layers are rotated over copies
    larger than twice the last-level cache.  Algorithmic bytes: the layer's
    weight bytes, the K/V codes and scales of ctx + 1 tokens, and the block
    table; the activations (tens of KB) are left out."""
    import numpy as np
    n_embd, n_head, n_kv, hd, n_ff, bs = 4096, 32, 8, 128, 14336, 16
    kv_dim = n_kv * hd
    types = {"attn_q": ssdq.Q4_K, "attn_k": ssdq.Q4_K, "attn_v": ssdq.Q4_K, "attn_output": ssdq.Q4_K,
             "ffn_gate": ssdq.Q4_K, "ffn_up": ssdq.Q4_K, "ffn_down": ssdq.Q6_K}
    t = synth.decoder_layer(n_embd, n_head, n_kv, hd, n_ff, types, synth.seed(7, 0))
    g = synth.rng(synth.seed(7, 20))
    norms = [(0.5 + g.random(n_embd)).astype(np.float32) for _ in range(2)]
    wbytes = sum(v[2].nbytes for v in t.values()) + 2 * 4 * n_embd
    max_blocks = (ctx + 1 + bs - 1) // bs
    kvbytes = (ctx + 1) * (2 * kv_dim + 8) + 4 * max_blocks
    n = copies_for(wbytes)
    store = ssdq.WeightStore()
    for layer in range(n):
        for name, (dt, dims, raw) in t.items():
            store.put(f"blk.{layer}.{name}.weight", dt, dims, raw)
        store.put(f"blk.{layer}.attn_norm.weight", ssdq.F32, (n_embd,), norms[0])
        store.put(f"blk.{layer}.ffn_norm.weight", ssdq.F32, (n_embd,), norms[1])
    # per layer: a pool of max_blocks physical blocks behind a shuffled table,
    # the earlier tokens' codes random, scales ~ U[0.01, 0.03]
    pools = []
    for layer in range(n):
        rows = max_blocks * bs
        pools.append((torch.randint(-127, 128, (rows * kv_dim,), dtype=torch.int8, device="cuda"),
                      torch.rand(rows, device="cuda") * 0.02 + 0.01,
                      torch.randint(-127, 128, (rows * kv_dim,), dtype=torch.int8, device="cuda"),
                      torch.rand(rows, device="cuda") * 0.02 + 0.01,
                      torch.from_numpy(g.permutation(max_blocks).astype(np.int32)).cuda()))
    tables = [p[4].cpu().numpy() for p in pools]
    slots = [torch.tensor([int(tb[ctx // bs]) * bs + ctx % bs], dtype=torch.int32, device="cuda") for tb in tables]
    ctx_len = torch.tensor([ctx + 1], dtype=torch.int32, device="cuda")
    cfg = ssdq.layer_config(n_embd, n_head, n_kv, hd, n_ff, 500000.0, 1e-5)
    sbytes, _ = ssdq.decode_layer_scratch(cfg)
    scratch = torch.zeros(sbytes, dtype=torch.uint8, device="cuda")
    hidden = torch.randn(n_embd, device="cuda")

    def step(i):
        layer = i % n
        kc, ks, vc, vs, bt = pools[layer]
        ssdq.decode_layer(store, layer, cfg, hidden, ctx, kc, ks, vc, vs, bs, bt, max_blocks, slots[layer],
                          ctx_len, max_blocks * bs, scratch=scratch)

    tr = timer.run(step, 100, 200)
    per = tr["t_median"] / tr["steps"]
    nbytes = wbytes + kvbytes
    ok = bool(torch.isfinite(hidden).all())
    del pools, scratch
    store.close()
    torch.cuda.empty_cache()
    return {"us": round(per * 1e6, 2), "GB/s": round(nbytes / per / 1e9, 1),
            "pct_hbm_peak": round(100 * nbytes / per / 1e9 / HBM_PEAK_GBS, 2), "bytes": nbytes,
            "layers_rotated": n, "context": ctx, "hidden_finite": ok,
            "note": "ssdq_decode_layer_dev: 9 steps in 7 kernel launches (the two RMSNorms folded into the QKV and "
                    "SwiGLU launches, the token's INT8 append into the attention launch, the residual add into "
                    "the down projection's slice reduction), one HIP graph replay per 50 layers"}


def attention_case(torch, ssdq, synth, codes, scales):
    """Config 5b on an INT8 pool (codes [2 * 8 * 32768, 1024]: K rows, then V rows)."""
    n_seq, n_head, n_kv, hd, bs, ctx = 8, 32, 8, 128, 16, 32768
    mb = ctx // bs
    kc = codes[: n_seq * mb * bs * n_kv * hd]
    vc = codes[n_seq * mb * bs * n_kv * hd:]
    ks = scales[: n_seq * mb * bs]
    vs = scales[n_seq * mb * bs:]
    tables = torch.from_numpy(synth.block_tables(n_seq, mb, synth.seed(5, 3))).cuda()
    cl = torch.full((n_seq,), ctx, dtype=torch.int32, device="cuda")
    q = torch.randn(n_seq * n_head * hd, device="cuda")
    o = torch.empty_like(q)
    return lambda i: ssdq.paged_attention_int8(q, kc, ks, vc, vs, tables, cl, o, n_seq, n_head, n_kv, hd, bs, mb,
                                               ctx)


def _probe_lib():
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "ssd-llm_amd", "libssdq_probe.so"))
    lib.ssdq_probe_read.restype = ctypes.c_int
    lib.ssdq_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]
    lib.ssdq_probe_read_nt.restype = ctypes.c_int
    lib.ssdq_probe_read_nt.argtypes = lib.ssdq_probe_read.argtypes
    lib.ssdq_probe_empty.restype = ctypes.c_int
    lib.ssdq_probe_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.ssdq_probe_mfma.restype = ctypes.c_int
    lib.ssdq_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_void_p]
    return lib


def read_ceiling(torch):
    """Plain streaming reads (16-byte loads, 4 in flight per thread, one
    contiguous slice per workgroup) of buffers from 4 MB to 512 MB, each rotated
    over copies larger than twice the last-level cache and timed like the
    matvecs (graph replays); the best of several launch shapes per size.  Also
    the time per launch of an empty kernel (256 x 256 and 256 x 768 threads)."""
    lib = _probe_lib()
    timer = Timer(torch)
    sink = torch.zeros(65536, dtype=torch.int32, device="cuda")
    stream = lambda: torch.cuda.current_stream().cuda_stream
    out = {"read": [], "read_nontemporal": [], "empty_kernel_us": {}}
    for mb in (4, 8, 16, 33.1, 48, 64, 128, 256, 512):
        nbytes = int(mb * 1e6) // 16 * 16 if mb == 33.1 else int(mb * (1 << 20))
        if mb == 33.1:
            nbytes = 33103872  # the headline matvec's algorithmic bytes
        n = copies_for(nbytes)
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1) for _ in range(n)]
        for key, fn in (("read", lib.ssdq_probe_read), ("read_nontemporal", lib.ssdq_probe_read_nt)):
            best = None
            for grid, block in ((256, 768), (512, 512), (1024, 256), (2048, 256), (2048, 512), (4096, 256)):
                def step(i, grid=grid, block=block, fn=fn):
                    rc = fn(bufs[i % n].data_ptr(), nbytes, sink.data_ptr(), grid, block, stream())
                    if rc != 0:
                        raise RuntimeError(f"{key} probe: hip error {rc}")
                tr = timer.run(step, 200, 200)
                us = tr["t_median"] / tr["steps"] * 1e6
                if best is None or us < best[0]:
                    best = (us, grid, block)
            out[key].append({"bytes": nbytes, "us": round(best[0], 3), "GB/s": round(nbytes / best[0] / 1e3, 1),
                             "pct_hbm_peak": round(100 * nbytes / best[0] / 1e3 / HBM_PEAK_GBS, 2),
                             "grid": best[1], "block": best[2]})
        del bufs
        torch.cuda.empty_cache()
    for grid, block in ((256, 256), (256, 768)):
        tr = timer.run(lambda i: lib.ssdq_probe_empty(grid, block, stream()), 200, 200)
        out["empty_kernel_us"][f"{grid}x{block}"] = round(tr["t_median"] / tr["steps"] * 1e6, 3)
    return out


def mfma_ceiling(torch):
    """The fp16 matrix-core rate on this part: an MFMA loop with register
    operands (eight independent v_mfma_f32_16x16x32_f16 chains per wave, 512
    workgroups) on random or all-zero fp16 operands, with 0, 2 or 4 independent
    VALU instructions after each MFMA; and torch.matmul in fp16 (hipBLASLt) at
    the config-4 shapes and at 8192^3, on random and on zero inputs.  HIP
    events around eager launches, best of 5."""
    lib = _probe_lib()
    stream = lambda: torch.cuda.current_stream().cuda_stream
    src = {"random": (torch.rand(4096 * 8, device="cuda") * 2 - 1).to(torch.float16),
           "zero": torch.zeros(4096 * 8, dtype=torch.float16, device="cuda")}
    out = {"mfma_loop": [], "torch_matmul_fp16": []}
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def best_ms(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        best = None
        for _ in range(reps):
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1)
            best = ms if best is None else min(best, ms)
        return best

    grid, iters = 512, 4000
    for block in (256, 512):
        sink = torch.empty(grid * block, device="cuda")
        for nv in (0, 1, 2):
            for kind in ("random", "zero"):
                def launch(kind=kind, nv=nv, block=block, sink=sink):
                    rc = lib.ssdq_probe_mfma(src[kind].data_ptr(), sink.data_ptr(), iters, nv, grid, block, stream())
                    if rc != 0:
                        raise RuntimeError(f"ssdq_probe_mfma: hip error {rc}")
                ms = best_ms(launch)
                flop = 16384.0 * 8 * iters * grid * (block // 64)
                tf = flop / ms / 1e9
                out["mfma_loop"].append({"operands": kind, "valu_per_mfma": 2 * nv, "block": block,
                                         "waves_per_simd": block // 128, "ms": round(ms, 4),
                                         "TFLOP/s": round(tf, 1), "pct_bf16_peak": round(100 * tf / BF16_PEAK_TFLOPS, 2)})
    for M, N, K in ((512, 28672, 4096), (512, 6144, 4096), (512, 4096, 4096), (512, 4096, 14336), (8192, 8192, 8192)):
        for kind in ("random", "zero"):
            a = torch.randn(M, K, device="cuda", dtype=torch.float16)
            b = torch.randn(K, N, device="cuda", dtype=torch.float16)
            if kind == "zero":
                a.zero_()
                b.zero_()
            ms = best_ms(lambda: torch.matmul(a, b), 5)
            tf = 2.0 * M * N * K / ms / 1e9
            out["torch_matmul_fp16"].append({"M": M, "N": N, "K": K, "inputs": kind, "us": round(ms * 1e3, 1),
                                             "TFLOP/s": round(tf, 1),
                                             "pct_bf16_peak": round(100 * tf / BF16_PEAK_TFLOPS, 2)})
            del a, b
    return out


def hipblaslt_layer(torch):
    """torch.matmul in fp16 (hipBLASLt) over the config-4 layer: X [512, K] fp16
    times already-dequantized fp16 weights [K, N] for the seven matrices (4x the
    Q4_K weight bytes), timed as a whole layer with HIP events."""
    M = 512
    layer = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
             ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
    W = {nm: torch.randn(K, N, device="cuda", dtype=torch.float16) * 0.02 for nm, N, K in layer}
    X = {K: torch.randn(M, K, device="cuda", dtype=torch.float16) for K in (4096, 14336)}
    Y = {}
    flops = sum(2.0 * M * N * K for _, N, K in layer)

    def run(i):
        for nm, N, K in layer:
            Y[nm] = torch.matmul(X[K], W[nm])
    timer = Timer(torch)
    tr = timer.run(run, 20, 10, graph=False)
    t = tr["t_median"] / tr["steps"]
    per = {}
    for nm, N, K in layer:
        tr1 = timer.run(lambda i, nm=nm, K=K: torch.matmul(X[K], W[nm]), 20, 10, graph=False)
        per[nm] = round(tr1["t_median"] / tr1["steps"] * 1e6, 2)
    return {"what": "torch.matmul fp16 (hipBLASLt), config-4 layer shapes, M = 512, dequantized fp16 weights",
            "ms_per_layer": round(t * 1e3, 4), "TFLOP/s": round(flops / t / 1e12, 1),
            "pct_bf16_peak": round(100 * flops / t / 1e12 / BF16_PEAK_TFLOPS, 2), "us_per_matrix": per}


def traffic_from_profiles(key):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    calibrated on a copy kernel), recorded in profiles/hbm_traffic.txt."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.txt")
    try:
        for line in open(path):
            parts = line.split()
            if len(parts) >= 2 and parts[0] == key:
                return float(parts[1])
    except OSError:
        pass
    return None


def extras(torch, ssdq, synth, timer, np):
    out = {}
    cases = [
        ("q4_0_matvec_14336x4096_b1", ssdq.Q4_0, 14336, 4096, 1, 1),
        ("q4_0_matvec_4096x4096_b1", ssdq.Q4_0, 4096, 4096, 1, 1),
        ("q8_0_matvec_11008x4096_b1", ssdq.Q8_0, 11008, 4096, 1, 2),
        ("q8_0_matvec_11008x4096_b4", ssdq.Q8_0, 11008, 4096, 4, 2),
        ("q8_0_matvec_11008x4096_b8", ssdq.Q8_0, 11008, 4096, 8, 2),
        ("q6_k_matvec_4096x14336_b1", ssdq.Q6_K, 4096, 14336, 1, 3),
        ("q4_k_matvec_4096x14336_b1", ssdq.Q4_K, 4096, 14336, 1, 3),  # FFN down: K-sliced rows
        ("q5_k_matvec_4096x14336_b1", ssdq.Q5_K, 4096, 14336, 1, 3),
        ("q4_k_matvec_28672x8192_b1", ssdq.Q4_K, 28672, 8192, 1, 3),  # a 70B-sized FFN up projection
    ]
    # the reference's other matvec_quantized types at the north-star shape
    for k, dt in enumerate(ssdq.MATVEC_EXTRA_TYPES):
        cases.append((f"{ssdq.TYPE_NAMES[dt].lower()}_matvec_14336x4096_b1", dt, 14336, 4096, 1, 6 + k))
    for name, dt, od, idim, b, cfg in cases:
        step, nbytes, _ = matvec_case(torch, ssdq, synth, dt, od, idim, b, cfg)
        tr = timer.run(step, 200, 500)
        t, n = tr["t_median"], tr["steps"]
        gbs = nbytes / (t / n) / 1e9
        out[name] = {"GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                     "us": round(t / n * 1e6, 3)}
        torch.cuda.empty_cache()

    # decode-layer ops on quantized weights (Llama-3-8B shapes, batch 1): the
    # fused launch against the same projections as separate matvec launches
    def layer_case(name, dts_rows, fused, n_embd=4096):
        base = []
        nbytes = 4 * n_embd
        for i, (dt, rows) in enumerate(dts_rows):
            w = torch.from_numpy(synth.quant_weights(dt, rows, n_embd, synth.seed(5, 8 + i))).cuda()
            base.append((dt, w, rows, torch.empty(rows, device="cuda")))
            nbytes += w.numel() + 4 * rows
        n = copies_for(nbytes)  # weights rotated over copies larger than 2x the last-level cache
        sets = [base] + [[(dt, w.clone(), r, y) for dt, w, r, y in base] for _ in range(n - 1)]
        x = torch.randn(n_embd, device="cuda")
        tr = timer.run(lambda i: fused(sets[i % n], x), 200, 500)
        tf, nf = tr["t_median"], tr["steps"]
        tr = timer.run(lambda i: [ssdq.matvec(dt, w, x, y, r, n_embd) for dt, w, r, y in sets[i % n]], 200, 500)
        ts, ns = tr["t_median"], tr["steps"]
        del sets, base
        out[name] = {"us": round(tf / nf * 1e6, 3), "GB/s": round(nbytes / (tf / nf) / 1e9, 1),
                     "pct_hbm_peak": round(100 * nbytes / (tf / nf) / 1e9 / HBM_PEAK_GBS, 2),
                     "separate_matvecs_us": round(ts / ns * 1e6, 3)}
        torch.cuda.empty_cache()

    def qkv(m, x):
        (dq, wq, rq, q), (_, wk, rk, k), (_, wv, rv, v) = m
        ssdq.qkv_rope((dq,) * 3, (wq, wk, wv), x, q, k, v, rq, rk, 4096, 128, 4000, 500000.0)

    def swi(m, x):
        (dt, wg, r, h), (_, wu, _, _) = m
        ssdq.swiglu(dt, wg, wu, x, h, r, 4096)

    gnorm = torch.rand(4096, device="cuda") + 0.5

    def head(m, x):
        (dt, w, r, y), = m
        ssdq.rmsnorm_matvec(dt, w, x, gnorm, 1e-5, y, r, 4096)

    layer_case("decode_qkv_rope_q4k_4096", [(ssdq.Q4_K, 4096), (ssdq.Q4_K, 1024), (ssdq.Q4_K, 1024)], qkv)
    layer_case("decode_swiglu_q4k_14336x4096", [(ssdq.Q4_K, 14336), (ssdq.Q4_K, 14336)], swi)
    layer_case("decode_output_head_rmsnorm_q6k_128256x4096", [(ssdq.Q6_K, 128256)], head)
    out["decode_layer_llama3_8b_q4k_ctx4096"] = decode_layer_case(torch, ssdq, synth, timer)

    # INT8 KV swap slots: 1024 blocks of 16 tokens x 1024 (one layer of a 16k-token
    # context) gathered into the reference's slot format and scattered back
    bs_, kv_, nb_, npool_ = 16, 1024, 1024, 4096
    kc_ = torch.randint(-127, 128, (npool_ * bs_ * kv_,), dtype=torch.int8, device="cuda")
    vc_ = torch.randint(-127, 128, (npool_ * bs_ * kv_,), dtype=torch.int8, device="cuda")
    ks_, vs_ = torch.rand(npool_ * bs_, device="cuda"), torch.rand(npool_ * bs_, device="cuda")
    ids_ = torch.randperm(npool_, device="cuda")[:nb_].to(torch.int32)
    nf_ = torch.full((nb_,), bs_, dtype=torch.int32, device="cuda")
    sb_ = ssdq.kv_slot_bytes(bs_, kv_)
    for where, slots_ in (("device", torch.empty(nb_ * sb_, dtype=torch.uint8, device="cuda")),
                          ("pinned_host", torch.empty(nb_ * sb_, dtype=torch.uint8).pin_memory())):
        tr = timer.run(lambda i: ssdq.kv_swap_out(kc_, ks_, vc_, vs_, ids_, nf_, nb_, bs_, kv_, npool_,
                                                   slots_), 50, 5)
        t, n = tr["t_median"], tr["steps"]
        tr = timer.run(lambda i: ssdq.kv_swap_in(slots_, ids_, nb_, bs_, kv_, npool_, kc_, ks_, vc_, vs_,
                                                  None), 50, 5)
        ti, ni = tr["t_median"], tr["steps"]
        out[f"kv_swap_out_int8_1024x16x1024_to_{where}"] = {
            "GB/s": round(nb_ * sb_ / (t / n) / 1e9, 1), "us": round(t / n * 1e6, 2),
            "swap_in_GB/s": round(nb_ * sb_ / (ti / ni) / 1e9, 1), "swap_in_us": round(ti / ni * 1e6, 2),
            "bytes": nb_ * sb_}
    del kc_, vc_, ks_, vs_
    torch.cuda.empty_cache()

    # the synchronous host-pointer twin (MetalCompute::matvec_quantized contract):
    # W and x cross PCIe on every call, so this is the PCIe-inclusive rate
    w_host = synth.quant_weights(ssdq.Q4_K, 14336, 4096, synth.seed(3, 0))
    x_host = synth.normal_f32(4096, 1)
    with ssdq.Context() as ctx:
        ctx.matvec_quantized(w_host, x_host, 14336, 4096, ssdq.Q4_K)
        reps, t0 = 0, time.perf_counter()
        while reps < 20:
            ctx.matvec_quantized(w_host, x_host, 14336, 4096, ssdq.Q4_K)
            reps += 1
        el = (time.perf_counter() - t0) / reps
    hb = w_host.size + 4 * (4096 + 14336)
    out["host_twin_q4k_matvec_14336x4096_pcie_inclusive"] = {
        "GB/s": round(hb / el / 1e9, 2), "us": round(el * 1e6, 1),
        "note": "ssdq_matvec_quantized: host W and x copied in, y copied out, per call"}

    # config 4: one Llama-3-8B layer of Q4_K prefill GEMMs at M = 512.  q/k/v
    # and gate/up read the same X and run as one GEMM each (multi entry point);
    # the seven separate GEMMs are timed as well.
    layer_fused, flops = gemm_layer(torch, ssdq, synth)
    t = timer.run(layer_fused, 5, 1, graph=False)["t_median"]
    t_sep = timer.run(layer_fused.separate, 5, 1, graph=False)["t_median"]
    tfl = flops / (t / 5) / 1e12
    out["prefill_gemm_q4k_layer_m512"] = {"TFLOP/s": round(tfl, 2),
                                          "pct_bf16_peak": round(100 * tfl / BF16_PEAK_TFLOPS, 2),
                                          "ms_per_layer": round(t / 5 * 1e3, 3),
                                          "ms_per_layer_seven_separate_gemms": round(t_sep / 5 * 1e3, 3),
                                          "note": "q/k/v and gate/up each one GEMM over shared X"}
    del layer_fused
    torch.cuda.empty_cache()

    # config 5a: INT8 quantize of 8 x 32768 tokens x {K, V} x 1024
    n_rows, dim = 8 * 32768 * 2, 1024
    xk = torch.randn(n_rows * dim, device="cuda")
    codes = torch.empty(n_rows * dim, dtype=torch.int8, device="cuda")
    scales = torch.empty(n_rows, device="cuda")
    t = timer.run(lambda i: ssdq.kv_quantize_rows(xk, codes, scales, n_rows, dim), 20, 3, graph=False)["t_median"]
    qbytes = n_rows * dim * 5 + n_rows * 4
    out["kv_int8_quantize_8x32768x2x1024"] = {"GB/s": round(qbytes / (t / 20) / 1e9, 1),
                                              "pct_hbm_peak": round(100 * qbytes / (t / 20) / 1e9 / HBM_PEAK_GBS, 2),
                                              "us": round(t / 20 * 1e6, 1)}
    del xk
    # config 5b: paged INT8 GQA decode attention, reusing the quantized pool
    n_seq = 8
    t = timer.run(attention_case(torch, ssdq, synth, codes, scales), 50, 5, graph=False)["t_median"]
    abytes = 536870912 + 2097152 + 131072 + 131072 + 65536
    step_s = t / 50
    out["paged_int8_decode_attention_32k"] = {
        "tok/s": round(n_seq / step_s, 1), "GB/s": round(abytes / step_s / 1e9, 1),
        "pct_hbm_peak": round(100 * abytes / step_s / 1e9 / HBM_PEAK_GBS, 2),
        "us_per_step": round(step_s * 1e6, 2)}
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, min_s):
    """Seconds per call of fn() over calls adding up to at least min_s (after one warm-up call)."""
    fn()
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= min_s:
            return el / reps, reps


def cpu_baseline(np, synth, ssdq, gpu_sec_per_step):
    """The CPU oracle (the C restatement of the reference's functions) on this
    host's cores, for every configuration: single thread like the reference
    (every matvec_*_cpu and the INT8 quantizer are single-threaded), and all
    cores (up to 16) with output rows, token rows or (sequence, head) pairs
    sharded over threads as tensor_parallel.rs:45-96 shards rows.  Each figure is
    the mean over calls adding up to ~1.5 s (single thread) or ~0.5 s (all
    cores) on a bounded sample of the configuration's work, scaled to its unit."""
    from concurrent.futures import ThreadPoolExecutor
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ssdq_oracle as o
    nt = min(16, os.cpu_count() or 1)
    pool = ThreadPoolExecutor(nt)
    S1, SN = 1.5, 0.5
    cfgs = {}

    def mv_entry(name, dt, od, idim, batch, cfg, sample):
        w = synth.quant_weights(dt, od, idim, synth.seed(cfg, 0))
        x = synth.normal_f32((batch, idim), synth.seed(cfg, 1))
        nbytes = w.size + 4 * batch * (idim + od)

        def step(threads):
            for b in range(batch):  # batch_scheduler.rs:242-276: one matvec per row
                o.matvec(dt, w, x[b], od, idim, threads=threads)
        t1, r1 = _timed(lambda: step(1), S1)
        tn, rn = _timed(lambda: step(nt), SN)
        cfgs[name] = {"unit": "GB/s", "1_thread": round(nbytes / t1 / 1e9, 3),
                      f"{nt}_threads": round(nbytes / tn / 1e9, 3), "ms_per_step_1_thread": round(t1 * 1e3, 2),
                      "sample": f"{r1} + {rn} {sample}"}
        return t1, r1, nbytes

    t_head, r_head, head_bytes = mv_entry("3_q4_k_matvec_14336x4096_b1", ssdq.Q4_K, 14336, 4096, 1, 3,
                                          "whole Q4_K matvecs 14336x4096")
    mv_entry("3_q6_k_matvec_4096x14336_b1", ssdq.Q6_K, 4096, 14336, 1, 3, "whole Q6_K matvecs 4096x14336")
    mv_entry("1_q4_0_matvec_4096x4096_b1", ssdq.Q4_0, 4096, 4096, 1, 1, "whole Q4_0 matvecs 4096x4096")
    for b in (1, 4, 8):
        mv_entry(f"2_q8_0_matvec_11008x4096_b{b}", ssdq.Q8_0, 11008, 4096, b, 2,
                 f"steps of {b} Q8_0 matvecs 11008x4096")

    # config 4: per-token matvecs of the seven Q4_K matrices over widened bf16
    # rows (transformer.rs:166-196); the sample is T tokens through the layer
    layer = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096),
             (4096, 14336)]
    ws = [synth.quant_weights(ssdq.Q4_K, n, k, synth.seed(4, i)) for i, (n, k) in enumerate(layer)]
    T1, TN = 1, 4 * nt
    xs = {k: synth.f32_to_bf16_bits(synth.normal_f32((TN, k), synth.seed(4, 8 + (k > 4096)))) for k in (4096, 14336)}

    def gemm_tokens(T, threads):
        for w, (n, k) in zip(ws, layer):
            o.gemm_q4k_bf16(w, xs[k][:T], T, n, k, threads=threads)
    flop_tok = 2.0 * sum(n * k for n, k in layer)
    t1, r1 = _timed(lambda: gemm_tokens(T1, 1), S1)
    tn, rn = _timed(lambda: gemm_tokens(TN, nt), SN)
    cfgs["4_prefill_q4k_layer_m512"] = {
        "unit": "TFLOP/s", "1_thread": round(T1 * flop_tok / t1 / 1e12, 5),
        f"{nt}_threads": round(TN * flop_tok / tn / 1e12, 5),
        "ms_per_512_token_layer_1_thread": round(t1 / T1 * 512 * 1e3, 1),
        "sample": f"{r1} x {T1} token(s) (1 thread) and {rn} x {TN} tokens ({nt} threads) through the seven "
                  f"matrices; scaled to 512 tokens by token count"}
    del ws, xs

    # config 5a: INT8 row quantize (block_swap.rs:36-60), rows of 1024
    dim, rows1 = 1024, 8192
    kv = synth.normal_f32((rows1 * nt, dim), synth.seed(5, 0))
    qb_row = 5 * dim + 4
    t1, r1 = _timed(lambda: o.quantize_rows(kv[:rows1], rows1, dim), S1)

    def quant_all():
        list(pool.map(lambda i: o.quantize_rows(kv[i * rows1:(i + 1) * rows1], rows1, dim), range(nt)))
    tn, rn = _timed(quant_all, SN)
    cfgs["5a_kv_int8_quantize_rows_1024"] = {
        "unit": "GB/s", "1_thread": round(rows1 * qb_row / t1 / 1e9, 3),
        f"{nt}_threads": round(nt * rows1 * qb_row / tn / 1e9, 3),
        "sample": f"{r1} x {rows1} rows (1 thread), {rn} x {nt * rows1} rows ({nt} threads) of the 524,288-row "
                  f"config; GB/s by 5 B per element + 4 B per row"}
    del kv

    # config 5b: paged INT8 GQA decode attention at 32k context, one step of
    # one sequence (32 heads) on one thread; all cores take the 8 sequences
    n_head, n_kv, hd, bs, ctx = 32, 8, 128, 16, 32768
    mb = ctx // bs
    g = np.random.default_rng(5)
    kc = g.integers(-127, 128, (mb * bs * n_kv * hd,), dtype=np.int8)
    vc = g.integers(-127, 128, (mb * bs * n_kv * hd,), dtype=np.int8)
    ks = g.uniform(0.005, 0.03, mb * bs).astype(np.float32)
    vs = g.uniform(0.005, 0.03, mb * bs).astype(np.float32)
    tab = synth.block_tables(1, mb, synth.seed(5, 3))
    q = synth.normal_f32((n_head * hd,), synth.seed(5, 4))
    cl = np.array([ctx], np.int32)

    def attn_seq():
        o.paged_attention_int8(q, kc, ks, vc, vs, tab, cl, 1, n_head, n_kv, hd, bs, mb)
    t1, r1 = _timed(attn_seq, S1)

    def attn_all():
        list(pool.map(lambda i: attn_seq(), range(8)))
    tn, rn = _timed(attn_all, SN)
    step_bytes_seq = 536870912 // 8 + 2097152 // 8
    cfgs["5b_paged_int8_decode_attention_32k"] = {
        "unit": "tok/s", "1_thread": round(1.0 / t1, 3), f"{nt}_threads": round(8 / tn, 3),
        "1_thread_GB/s": round(step_bytes_seq / t1 / 1e9, 3),
        "sample": f"{r1} single-sequence steps (32 heads, 32768 tokens) on 1 thread: tok/s = 8 / (8 x the "
                  f"sequence time); {rn} steps of all 8 sequences on {nt} threads"}
    pool.shutdown()

    return {"value": round(head_bytes / t_head / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{r_head} single-thread Q4_K matvecs 14336x4096 ({t_head * 1e3:.1f} ms each) on "
                      f"{os.cpu_count()} visible host cores ({_cpu_model()})",
            "gpu_over_cpu": round(t_head / gpu_sec_per_step, 1),
            "cpu_model": _cpu_model(), "host_cores_visible": os.cpu_count(), "threads_all_cores": nt,
            "configs": cfgs}


if __name__ == "__main__":
    main()
