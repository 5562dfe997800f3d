#!/usr/bin/env python3
"""Benchmark of the batch-1 quantized decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload: a Llama-2-7B-shaped decoder (dim 4096, 32
layers, 32 heads x 128, SwiGLU hidden 11008, vocab 32000) with random-init
N(0, 0.02) weights quantized to INT4, group 64 (scale = amax/7), activations
Q8 per group of 64, fp32 KV cache.  128 random prompt ids are forced, then
W warmup and K timed greedy steps run through the engine's captured
hipGraph with the argmax on the device (the decode loop of runq.c:681-718).
A "step" is one decode position; value = K / timed seconds (tok/s).

Also reported on the same JSON line:
  roofline      the decode's dominant kernel, the w1|w3 GEMV of the step
                (22016 x 4096, RMSNorm + Q8 prologue, SwiGLU epilogue),
                launched by the engine with the decode's own arguments over
                the 32 layers' weights (1.6 GB, so the 256 MB MALL cannot
                serve them) and timed live with HIP events on the engine's
                stream: algorithmic bytes per launch / mean duration, against
                the 8 TB/s HBM3E peak;
  decode_gemv   the same for all five GEMV kinds of the step, and the
                aggregate GEMV fraction of peak over one step;
  runq_tok_s    the reference's own tok/s formula, (positions - 1) /
                elapsed (runq.c:710-716), over the whole generation
                (prefill + warmup + timed steps);
  gemv_c2_int8, gemv_c3_int4
                BASELINE configs 2 and 3: the four Llama-2-7B GEMV shapes,
                pre-quantized activations, rotating >= 1 GiB weight sets;
  cpu_baseline  the reference's CPU runner (v1-int8-vnni/runq.c, AVX-512
                VNNI, OpenMP), compiled from its own source, decoding the
                7B shape at its native INT8 group 32 on this host's cores;
  cpu_reference the host CPU (model, AVX-512 VNNI), matmul_q8 GB/s on the
                config-2 shapes (group 32: the reference's own code; group
                64: the C port, as runq fixes QBLOCK = 32) and the config-1
                model's end-to-end tok/s through the compiled reference.

--decode-only runs the decode alone (no microbenchmarks, no CPU legs): the
form the committed rocprofv3 kernel statistics are taken from.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "llama2-min-inference_amd")
sys.path.insert(0, PKG)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "batch-1 decode tok/s, Llama-2-7B-shape INT4; GEMV achieved HBM GB/s (% peak)"


def gemv_bytes(rows, cols, bits, group):
    """Algorithmic bytes of one GEMV: weights + weight scales + activations
    + activation scales + fp32 output."""
    return rows * cols * bits // 8 + rows * (cols // group) * 4 + cols + (cols // group) * 4 + rows * 4


def step_bytes(cfg, group, pos):
    """Algorithmic bytes of one decode step at position pos (INT4 weights)."""
    d, h, L, V = cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.vocab_size
    kv = d * cfg.n_kv_heads // cfg.n_heads
    per_layer = (gemv_bytes(d + 2 * kv, d, 4, group) + gemv_bytes(d, d, 4, group)
                 + gemv_bytes(2 * h, d, 4, group) + gemv_bytes(d, h, 4, group))
    kv_read = L * 2 * (pos + 1) * kv * 4
    kv_write = L * 2 * kv * 4
    return L * per_layer + gemv_bytes(V, d, 4, group) + kv_read + kv_write + d * 4


def time_gemv(torch, abi, rows, cols, bits, group, min_bytes=1 << 30, reps=20):
    """Mean duration (ms) of the GEMV over rotating weight sets, HIP events
    on the stream the kernel is launched on."""
    wbytes = rows * cols * bits // 8
    nb = cols // group
    nset = max(2, -(-min_bytes // (wbytes + rows * nb * 4)))
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    ws = [torch.randint(0, 256, (wbytes,), dtype=torch.uint8, device="cuda", generator=g) for _ in range(nset)]
    ss = [torch.rand(rows * nb, dtype=torch.float32, device="cuda", generator=g) * 1e-3 for _ in range(nset)]
    xq = torch.randint(-127, 128, (cols,), dtype=torch.int8, device="cuda", generator=g)
    xs = torch.rand(nb, dtype=torch.float32, device="cuda", generator=g)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream()
    name = "l2q_gemv_q4" if bits == 4 else "l2q_gemv_q8"
    fn = getattr(abi.lib(), name)

    def launch(i):
        rc = fn(out.data_ptr(), xq.data_ptr(), xs.data_ptr(), ws[i % nset].data_ptr(), ss[i % nset].data_ptr(),
                rows, cols, group, None, st.cuda_stream)
        if rc:
            abi.check(rc)

    for i in range(nset):
        launch(i)
    torch.cuda.synchronize()
    n = nset * reps
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(n):
        launch(i)
    e1.record(st)
    e1.synchronize()
    ms = e0.elapsed_time(e1) / n
    del ws, ss
    torch.cuda.empty_cache()
    return ms, n


def time_attention(torch, abi, host, ctx, mode, reps=50, n_heads=32, hs=128, max_t=4096):
    """Mean duration (ms) of one layer's decode attention at context ctx
    (32 heads x 128, cache of 4096 positions): mode
    "exact" (fp32 cache, the reference's order), "split" (fp32 cache,
    split-context, the config's 1e-5 tolerance) or "int8" (int8 cache); and
    its algorithmic bytes (K and V read, q read, output written).  Mode
    "split1" is the engine's tolerance-mode form (L2Q_ATTN_SPLIT_CONTEXT:
    one kernel, the engine's K layout); "int8split" the int8 cache split over
    the context (the int8-KV engine's form)."""
    kv8 = mode in ("int8", "int8split")
    g = torch.Generator(device="cuda")
    g.manual_seed(ctx)
    q = torch.randn(n_heads * hs, device="cuda", generator=g)
    out = torch.empty_like(q)
    st = torch.cuda.current_stream()
    if kv8:
        k = torch.randint(-127, 128, (n_heads * max_t * hs,), dtype=torch.int8, device="cuda", generator=g)
        v = torch.randint(-127, 128, (n_heads * max_t * hs,), dtype=torch.int8, device="cuda", generator=g)
        ks = torch.rand(n_heads * max_t, device="cuda", generator=g) * 0.02
        vs = torch.rand(n_heads * max_t, device="cuda", generator=g) * 0.02
        args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), ks.data_ptr(), vs.data_ptr(), out.data_ptr())
        fn = "l2q_attention_kv8_ex" if mode == "int8split" else "l2q_attention_kv8"
        nbytes = 2 * ctx * n_heads * (hs + 4)
    else:
        k = torch.randn(n_heads * max_t * hs, device="cuda", generator=g)
        v = torch.randn(n_heads * max_t * hs, device="cuda", generator=g)
        args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr())
        fn = "l2q_attention_split" if mode == "split" else "l2q_attention_ex"
        nbytes = 2 * ctx * n_heads * hs * 4
    nbytes += 2 * n_heads * hs * 4
    # exact, split1: the engine's K layout (and, exact, its choice of kernels)
    extra = {"exact": (abi.L2Q_ATTN_K_INTERLEAVED,),
             "split1": (abi.L2Q_ATTN_K_INTERLEAVED | abi.L2Q_ATTN_SPLIT_CONTEXT,),
             "int8split": (abi.L2Q_ATTN_SPLIT_CONTEXT,)}.get(mode, ())

    def launch():
        abi.call(fn, *args, ctx - 1, n_heads, n_heads, hs, max_t, *extra, torch.cuda.current_stream().cuda_stream)

    for _ in range(3):
        launch()
    torch.cuda.synchronize()
    # the launches are replayed from a captured graph: a short attention
    # takes less time than one launch through ctypes
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            launch()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    graph.replay()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps, nbytes


def time_gemm(torch, abi, rows, cols, T, bits=4, group=64, reps=20):
    """Mean duration (ms) of the batched prefill GEMM (l2q_gemm_q) of T
    tokens, HIP events on its stream; one weight set (the MALL may hold it)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(rows + T)
    nb = cols // group
    w = torch.randint(0, 256, (rows * cols * bits // 8,), dtype=torch.uint8, device="cuda", generator=g)
    ws = torch.rand(rows * nb, device="cuda", generator=g) * 1e-3
    xq = torch.randint(-127, 128, (T * cols,), dtype=torch.int8, device="cuda", generator=g)
    xs = torch.rand(T * nb, device="cuda", generator=g)
    out = torch.empty(T * rows, device="cuda")
    st = torch.cuda.current_stream()

    def launch():
        abi.call("l2q_gemm_q", bits, out.data_ptr(), xq.data_ptr(), xs.data_ptr(), w.data_ptr(), ws.data_ptr(),
                 rows, cols, group, T, st.cuda_stream)

    launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        launch()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


C2_SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008), (32000, 4096)]


def cpu_info():
    """Model name and the AVX-512 VNNI flag of this host (Linux)."""
    model, flags = None, set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if model is None and line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                elif not flags and line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return {"model": model, "avx512_vnni": "avx512_vnni" in flags, "avx512f": "avx512f" in flags,
            "nproc": os.cpu_count(), "omp_threads": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))}


def cpu_matmul(reps=3, rotate_bytes=1 << 30):
    """matmul_q8 (runq.c:142-159) on the config-2 shapes in GB/s of the
    config-2 algorithmic bytes: group 32 through the reference's own function
    (compiled runq.c), group 64 through the C port (oracle.c orc_matmul_q8),
    since runq fixes its group at QBLOCK = 32.  Each timed pass calls the
    function once on each of n distinct weight copies, n * (weight + scale
    bytes) >= rotate_bytes (1 GiB, well above the host's last-level cache),
    so every call streams its weights from DRAM; the figure is the median over
    `reps` passes of the mean call time."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle_py as O
    rng = np.random.default_rng(5)
    # one arena of weight bytes, filled by tiling 64 MiB of random bytes
    arena = np.empty(rotate_bytes + (140 << 20), dtype=np.uint8)
    tile = rng.integers(0, 256, 64 << 20, dtype=np.uint8)
    for o in range(0, arena.size, tile.size):
        n = min(tile.size, arena.size - o)
        arena[o:o + n] = tile[:n]
    del tile
    out = {}
    for rows, cols in C2_SHAPES:
        x = rng.standard_normal(cols).astype(np.float32)
        res = {}
        for group, kind in ((32, "reference"), (64, "port")):
            if kind == "reference" and not O.ref_available():
                continue
            wb = rows * cols
            nsc = rows * (cols // group)
            ncopy = -(-rotate_bytes // (wb + 4 * nsc))
            wcopies = [arena[(k * wb) % (arena.size - wb):][:wb] for k in range(ncopy)]
            scopies = [(rng.random(nsc, dtype=np.float32) * np.float32(1e-3)) for _ in range(ncopy)]
            xq, xs, xt = O.quantize_act(x, group)
            if kind == "reference":
                def fn(k):
                    return O.ref_matmul_q8(xq, xs, xt, wcopies[k], scopies[k], rows, cols)
            else:
                def fn(k):
                    return O.matmul(8, xq, xs, xt, wcopies[k], scopies[k], rows, cols, group, want_dots=False)
            for k in range(ncopy):   # untimed pass: page-in
                fn(k)
            ts = []
            for _ in range(reps):
                t = time.perf_counter()
                for k in range(ncopy):
                    fn(k)
                ts.append((time.perf_counter() - t) / ncopy)
            t = float(np.median(ts))
            b = gemv_bytes(rows, cols, 8, group)
            res[f"G{group}"] = {"kind": kind, "ms": round(t * 1e3, 3), "GB/s": round(b / t / 1e9, 1),
                                "weight_copies": ncopy}
            del wcopies, scopies
        out[f"{rows}x{cols}"] = res
    del arena
    return out


def cpu_c1():
    """BASELINE config 1 on the compiled reference runq.c: the stories15M-shaped
    INT8 group-32 model, 16 prompt ids then 240 greedy steps, tok/s by the
    reference's formula ((pos - 1) / elapsed from the end of step 1)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle_py as O
    from llama2q import host
    if not O.ref_available():
        return None
    ck = host.synth_checkpoint(host.config_15m(), 8, 32, seed=1234)
    prompt = [int(v) for v in host.uniform_ints(16, 1234, 100, 3, 32000)]
    ref = O.RefRunq(image=ck.data)
    token = prompt[0]
    t0 = 0.0
    for pos in range(256):
        lg = ref.forward(token, pos)
        token = prompt[pos + 1] if pos < len(prompt) - 1 else O.ref_argmax(lg)
        if pos == 0:
            t0 = time.perf_counter()
    el = time.perf_counter() - t0
    ref.close()
    return {"tok_s": round(255 / el, 1), "positions": 256, "kind": "reference"}


def cpu_baseline(seconds_budget=20.0):
    """The reference runq.c (AVX-512 VNNI + OpenMP) on this host: 7B-shaped
    INT8 group-32 decode (its own format; the reference has no CPU INT4
    path).  Timed as the reference does: from the end of the first step."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle_py as O
    from llama2q import host
    if not O.ref_available():
        return None
    cfg = host.config_7b(seq_len=4096)
    t0 = time.time()
    ck = host.synth_checkpoint(cfg, 8, 32, seed=11)
    t_synth = time.time() - t0
    ref = O.RefRunq(image=ck.data)
    prompt = [int(v) for v in host.uniform_ints(64, 11, 100, 3, cfg.vocab_size)]
    ref.forward(prompt[0], 0)                 # first step: not timed (runq.c:710)
    t0 = time.time()
    n = 0
    while True:
        n += 1
        ref.forward(prompt[n], n)
        el = time.time() - t0
        if el > seconds_budget or n + 1 >= len(prompt):
            break
    ref.close()
    del ck
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(n / el, 3), "unit": "tok/s", "cores": cores, "kind": "reference",
            "sample": f"runq.c forward, Llama-2-7B shape INT8 group 32 (7.96 GB, random-init), "
                      f"{n} decode steps at positions 1..{n} after one untimed step; OpenMP threads={cores}; "
                      f"checkpoint synthesis {t_synth:.1f}s not timed"}


LONG_PROMPT = 3000   # prompt positions before the long-context decode figures


def decode_rate(torch, Engine, ck, prompt, warmup, steps, **options):
    """Greedy decode of an engine built with `options`: the prompt prefilled
    (once untimed, which allocates the prefill buffers, then once timed: the
    same positions rewrite the same cache rows), `warmup` untimed steps,
    then `steps` timed steps through the captured graph with the device
    argmax (host loop)."""
    e = Engine(ck, max_steps=len(prompt) + warmup + steps, **options)
    e.prefill(prompt[:-1], 0, logits=False)
    torch.cuda.synchronize()
    tp = time.perf_counter()
    e.prefill(prompt[:-1], 0, logits=False)
    torch.cuda.synchronize()
    prefill_ms = (time.perf_counter() - tp) * 1e3
    tok, p = prompt[-1], len(prompt) - 1
    for _ in range(warmup):
        tok = e.forward_argmax(tok, p)
        p += 1
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(steps):
        tok = e.forward_argmax(tok, p)
        p += 1
    torch.cuda.synchronize()
    el = time.perf_counter() - t
    e.close()
    return {"tok_s": round(steps / el, 2), "ms_per_step": round(el * 1e3 / steps, 4), "steps": steps,
            "positions": [p - steps, p - 1], "prefill_ms": round(prefill_ms, 3), "prefill_positions": len(prompt) - 1}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--kv8-steps", type=int, default=64,
                    help="greedy steps timed again with the int8 KV cache engine (0: skip)")
    ap.add_argument("--prefill-reps", type=int, default=3,
                    help="timed repeats of the batched prefill of the forced prompt (mean reported)")
    ap.add_argument("--decode-only", action="store_true",
                    help="the decode and its own GEMV kernels alone: no microbenchmarks of other "
                         "kernel forms, no int8-KV decode, no CPU legs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a 256 MiB device copy (x4): a kernel of known traffic for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the decode path is single-device; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)

    import torch
    from llama2q import abi, host
    from llama2q.model import Engine
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    cfg = host.config_7b(seq_len=4096)
    group = 64
    t0 = time.time()
    ck = host.synth_checkpoint(cfg, 4, group, seed=2024, q4_divisor=7.0)
    t_synth = time.time() - t0
    max_steps = args.prompt + args.warmup + args.steps
    prompt = [int(v) for v in host.uniform_ints(args.prompt, 2024, 100, 3, cfg.vocab_size)]

    # secondary figures: the same greedy decode with the int8 KV cache and
    # with the tolerance-mode attention, at the bench window and after a
    # long prompt (a context of ~3000 positions)
    kv8 = decode_modes = None
    if args.kv8_steps > 0 and not args.decode_only:
        n2 = args.kv8_steps
        kv8 = decode_rate(torch, Engine, ck, prompt, args.warmup, n2, kv8=True)
        long_prompt = [int(v) for v in host.uniform_ints(LONG_PROMPT, 2025, 100, 3, cfg.vocab_size)]
        decode_modes = {
            "note": "tok/s of greedy decode through the captured graph (device argmax), per engine option; "
                    "attn_split = L2Q_ENGINE_ATTN_SPLIT (split-context attention, equal to the exact order up "
                    "to rounding), kv8 = L2Q_ENGINE_KV_INT8; prefill_ms: the batched prefill of the "
                    "prompt's prefill_positions (host-timed, warm)",
            "attn_split": decode_rate(torch, Engine, ck, prompt, args.warmup, n2, attn_split=True),
            "long_context": {name: decode_rate(torch, Engine, ck, long_prompt, args.warmup, n2, **kw)
                             for name, kw in (("exact", {}), ("attn_split", {"attn_split": True}),
                                              ("kv8", {"kv8": True}))},
        }

    eng = Engine(ck, max_steps=max_steps)
    del ck

    # the forced prompt positions in one batched prefill: once untimed (the
    # first call allocates the prefill buffers), then the mean of
    # --prefill-reps timed repeats (each rewrites the same KV rows); then
    # warmup greedy steps
    eng.prefill(prompt[:-1], 0, logits=False)
    torch.cuda.synchronize()
    reps = max(1, args.prefill_reps)
    tp = time.perf_counter()
    for _ in range(reps):
        eng.prefill(prompt[:-1], 0, logits=False)
    torch.cuda.synchronize()
    prefill_s = (time.perf_counter() - tp) / reps
    token = prompt[-1]
    pos = args.prompt - 1
    for _ in range(args.warmup):
        token = eng.forward_argmax(token, pos)
        pos += 1
    torch.cuda.synchronize()
    pos_start = pos
    t0 = time.perf_counter()
    for _ in range(args.steps):
        token = eng.forward_argmax(token, pos)
        pos += 1
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gen_end = time.perf_counter()
    # the reference's tok/s formula over the whole generation: positions run
    # minus one over the time from the first forward (the prefill) on
    n_pos = pos
    runq_tok_s = (n_pos - 1) / (gen_end - tp)
    # the same positions replayed back to back without per-token host sync
    dev_ms = eng.time_steps([prompt[i % len(prompt)] for i in range(args.steps)], pos_start)

    # the step's GEMV kernels, launched by the engine with the decode's own
    # arguments, rotating over the layers' weights (HIP events)
    d, h, L = cfg.dim, cfg.hidden_dim, cfg.n_layers
    kv = d * cfg.n_kv_heads // cfg.n_heads
    kinds = [("qkv", abi.L2Q_GEMV_QKV, d + 2 * kv, d, L), ("wo", abi.L2Q_GEMV_WO, d, d, L),
             ("w13", abi.L2Q_GEMV_W13, 2 * h, d, L), ("w2", abi.L2Q_GEMV_W2, d, h, L),
             ("wcls", abi.L2Q_GEMV_CLASSIFIER, cfg.vocab_size, d, 1)]
    # each kernel launched alone n times in a row by the engine with the
    # decode's arguments, rotating over the 32 layers' weights (>= 1 GiB for
    # the layer kinds); HIP events around the run
    decode_gemv = {}
    tot_b = tot_us = 0.0
    for name, kind, r, c, per_step in kinds:
        n = 4 * L if per_step > 1 else 32
        us = eng.time_gemv(kind, n) * 1e3 / n
        b = gemv_bytes(r, c, 4, group)
        decode_gemv[name] = {"rows": r, "cols": c, "us": round(us, 3), "bytes": b,
                             "GB/s": round(b / us / 1e3, 1), "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                             "per_step": per_step, "launches": n}
        tot_b += per_step * b
        tot_us += per_step * us
    decode_gemv["aggregate"] = {"bytes_per_step": int(tot_b), "us_per_step": round(tot_us, 1),
                                "GB/s": round(tot_b / tot_us / 1e3, 1),
                                "frac": round(tot_b / tot_us / 1e3 / HBM_PEAK_GBS, 4)}
    eng.close()

    ms_per_step = elapsed * 1e3 / args.steps
    tok_s = args.steps / elapsed
    avg_bytes = np.mean([step_bytes(cfg, group, p) for p in range(pos_start, pos_start + args.steps)])

    # BASELINE configs 2 and 3: the four 7B shapes, pre-quantized activations
    gemv_c2 = gemv_c3 = attention = gemm_t = None
    if not args.decode_only:
        gemv_c2, gemv_c3 = {}, {}
        for bits, dst in ((8, gemv_c2), (4, gemv_c3)):
            for r, c in C2_SHAPES:
                ms, n = time_gemv(torch, abi, r, c, bits, group)
                b = gemv_bytes(r, c, bits, group)
                dst[f"{r}x{c}"] = {"us": round(ms * 1e3, 3), "bytes": b, "GB/s": round(b / ms / 1e6, 1),
                                   "frac": round(b / ms / 1e6 / HBM_PEAK_GBS, 4), "launches": n}

        # one layer's attention at the BASELINE config-4 contexts: fp32 cache in
        # the exact order and split over the context, int8 cache
        attention = {}
        for ctx in (256, 1024, 2048, 4096):
            for name in ("exact", "split", "split1", "int8", "int8split"):
                ms, nbytes = time_attention(torch, abi, host, ctx, name)
                attention[f"{name}_ctx{ctx}"] = {"us": round(ms * 1e3, 2), "bytes": nbytes,
                                                 "GB/s": round(nbytes / ms / 1e6, 1)}

        # the batched prefill GEMM at T = 128 tokens (INT4 g64, 7B shapes);
        # each launch includes the activation preparation kernel
        gemm_t = {}
        for name, _, r, c, _ in kinds:
            ms = time_gemm(torch, abi, r, c, 128)
            gemm_t[name] = {"us": round(ms * 1e3, 2), "int8_TOPS": round(2 * r * c * 128 / ms / 1e9, 2),
                            "weight_GB/s": round(gemv_bytes(r, c, 4, group) / ms / 1e6, 1)}

    traffic = None
    tpath = os.path.join(REPO, "profiles", "gemv_q4_g64_w13_decode_traffic.txt")
    if os.path.exists(tpath):
        with open(tpath) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch="):
                    traffic = int(line.split("=", 1)[1])

    cpu = cpu_ref = None
    if not args.decode_only and not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_seconds)
        cpu_ref = {"host": cpu_info(), "matmul_q8": cpu_matmul(), "c1_decode": cpu_c1()}

    dom = decode_gemv["w13"] if decode_gemv else None
    roofline = None
    if dom:
        roofline = {"bound": "hbm", "achieved": dom["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": dom["frac"], "traffic": traffic,
                    "kernel": "k_gemv<4,64,2,2,2,2,11>: the decode's w1|w3 GEMV, 22016 x 4096, RMSNorm + Q8 "
                              "prologue, SwiGLU epilogue, launched by the engine with the step's arguments "
                              "over the 32 layers' weights (1.6 GB), back to back",
                    "bytes_per_launch": dom["bytes"], "mean_us": dom["us"]}

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xint8",
        "data": "synthetic (random-init N(0,0.02) weights, seeded random prompt ids)",
        "config": {"workload": "Llama-2-7B-shape INT4 g64 batch-1 greedy decode (BASELINE config 5)",
                   "dim": cfg.dim, "layers": cfg.n_layers, "heads": cfg.n_heads, "hidden": cfg.hidden_dim,
                   "vocab": cfg.vocab_size, "group": group, "prompt_tokens": args.prompt,
                   "positions": [pos_start, pos_start + args.steps - 1], "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "runq_tok_s": round(runq_tok_s, 2),
        "decode_gemv": decode_gemv,
        "step_bytes_avg": int(avg_bytes),
        "step_effective_GBs": round(avg_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "device_replay_ms_per_step": round(dev_ms / args.steps, 4),
        "gemv_c2_int8": gemv_c2,
        "gemv_c3_int4": gemv_c3,
        "attention_c4": attention,
        "prefill_gemm_t128": gemm_t,
        "prefill": {"tokens": args.prompt - 1, "ms": round(prefill_s * 1e3, 3),
                    "tok_s": round((args.prompt - 1) / prefill_s, 1),
                    "reps": max(1, args.prefill_reps),
                    "note": "batched prefill of the forced prompt positions (int8 MFMA GEMMs, host-timed mean "
                            "of warm repeats, includes the per-chunk token upload)"},
        "kv8_decode": kv8,
        "decode_modes": decode_modes,
        "cpu_reference": cpu_ref,
        "synth_seconds": round(t_synth, 1),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
