"""Benchmark of the K-quant decode hot path on one MI355X.

One step = one pass of the hot path over one batch of synthetic input at BASELINE config 2: the
activation vector x (f32[3072], N(0,1)) is quantized to per-32 int8 blocks (quantize_q8x4) and
multiplied by the 128256 x 3072 Q6_K output head (matvec_q6k_q8) into f32 logits. Every weight
matrix of every leg is drawn from N(0, 0.02) and quantized to its ggml type on the GPU (ggml's
reference quantizers, kernelcore_amd/synth.py), then repacked; two copies of the head alternate so
the 256 MB Infinity Cache cannot hold them.

value = algorithmic bytes per step (ggml weight bytes + x + y, 323,730,432 B) / GPU time per step
over the K timed steps (HIP events on the stream, the median of --reps repetitions), with every
input resident in HBM. roofline: the same bytes over the matvec kernel's own average duration (the
same launches without the quantizer, between two events) against the 8 TB/s HBM peak. Before each
leg the GPU runs about 0.3 s of work so that its clocks have ramped up. Also reported: config 1
(Q4_K 3072 x 3072) rotated over 200 weight copies (>1 GB), the Q4_K matvec at config 2's shape,
config 3 (the prefill matmuls), configs 4 and 5 (prefill and greedy decode of the Llama-3.2-3B and
Qwen3-8B shapes), each a median of --reps repetitions, and beside each leg the same work on the
host cores: the oracle's vectorised kernels (oracle/kc_oracle_simd.c: AVX-512 VNNI or AVX2
integer dots, chosen by CPUID; OpenMP over every host thread), bounded samples stated in each leg.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--reps R] [--no-cpu] [--calibrate]
"""
import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import kernelcore_amd as kc  # noqa: E402
from kernelcore_amd import synth  # noqa: E402

PEAK_HBM_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # dense fp16 MFMA
PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA (the bound the config-3 workload names: 8-bit products)
METRIC = "Q4_K matvec HBM GB/s (% of peak); decode tok/s, 3B-shape Q4_K_M, 1 GPU"


class Timer:
    """Timed kc events on one stream."""

    def __init__(self, stream):
        self.stream = stream

    def event(self):
        e = C.c_void_p()
        kc.call("kcEventCreateTimed", C.byref(e))
        return e

    def record(self, e):
        kc.call("kcEventRecord", e, self.stream)

    @staticmethod
    def ms(a, b):
        v = C.c_float()
        kc.call("kcEventElapsedTime", C.byref(v), a, b)
        return v.value


def med(xs):
    return float(statistics.median(xs))


def new_stream():
    s = C.c_void_p()
    kc.call("kcStreamCreate", C.byref(s))
    return s


def warm_clocks(stream, seconds=0.3):
    """About `seconds` of streaming work on the stream, so that the timed work that follows runs at
    the GPU's sustained clocks rather than during their ramp."""
    n = 16 << 20
    a, b, o = kc.Buffer(n * 4), kc.Buffer(n * 4), kc.Buffer(n * 4)
    args = kc.VectorAddArgs(a.ptr, b.ptr, o.ptr, n)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            kc.launch("vector_add", args, stream)
        kc.call("kcStreamSynchronize", stream)
    for x in (a, b, o):
        x.free()


def time_launches(stream, fn, steps, reps):
    """Per repetition: the GPU time of `steps` calls of fn (events around them on the stream)."""
    t = Timer(stream)
    e0, e1 = t.event(), t.event()
    out = []
    for _ in range(reps):
        kc.call("kcStreamSynchronize", stream)
        t.record(e0)
        for i in range(steps):
            fn(i)
        t.record(e1)
        kc.call("kcStreamSynchronize", stream)
        out.append(Timer.ms(e0, e1))
    for e in (e0, e1):
        kc.call("kcEventDestroy", e)
    return out


def matvec_run(qtype, rows, k, copies, steps, warmup, seed, reps, graph=False):
    """quantize + matvec per step over `copies` weight streams; median timings of `reps` repetitions."""
    nb = k // 32
    f32, blocks = kc.Buffer(rows * k * 4), kc.Buffer(rows * (k // 256) * (210 if qtype == "q6k" else 144))
    streams = [synth.quantized_stream(qtype, rows, k, seed + i, f32=f32, blocks=blocks) for i in range(copies)]
    f32.free()
    blocks.free()
    x = (np.random.default_rng(seed + 99).standard_normal(k)).astype(np.float32)
    bx, bq, bd, by = kc.Buffer.of(x), kc.Buffer(nb * 32), kc.Buffer(nb * 8), kc.Buffer(rows * 4)
    s = new_stream()
    qa = kc.QuantizeArgs(bx.ptr, bq.ptr, bd.ptr, nb)
    mas = [kc.MatvecQ4Q8Args(w.ptr, bq.ptr, bd.ptr, by.ptr, None, rows, k) for w in streams]
    name = f"matvec_{qtype}_q8"

    def step(i):
        kc.launch("quantize_q8x4", qa, s)
        kc.launch(name, mas[i % copies], s)

    warm_clocks(s)
    for i in range(max(warmup, copies)):
        step(i)
    region = time_launches(s, step, steps, reps)  # the timed steps: quantize + matvec
    kernel = time_launches(s, lambda i: kc.launch(name, mas[i % copies], s), steps, reps)  # the matvec alone
    # the dispatch floor: the same number of back-to-back launches of a kernel that does nothing
    # measurable (a 256-element vector_add), for the share of a small kernel's time that is launch
    a, b, o = kc.Buffer(1024), kc.Buffer(1024), kc.Buffer(1024)
    va = kc.VectorAddArgs(a.ptr, b.ptr, o.ptr, 256)
    floor = time_launches(s, lambda i: kc.launch("vector_add", va, s), steps, reps)
    out = {"region_ms": med(region), "kernel_ms": med(kernel) / steps, "floor_ms": med(floor) / steps,
           "region_reps_ms": [round(v, 4) for v in region]}
    if graph:
        # The matvecs over the whole rotation captured once as a HIP graph and replayed (the
        # launches then cost the graph's dispatch instead of one host call each); the same for
        # the vector_add, the floor under the graph.
        def replay_ms(launch_one):
            g = C.c_void_p()
            kc.call("kcStreamBeginCapture", s)
            for i in range(copies):
                launch_one(i)
            kc.call("kcStreamEndCapture", s, C.byref(g))
            nrep = max(1, steps // copies)
            t = time_launches(s, lambda _: kc.call("kcGraphLaunch", g, s), nrep, reps)
            kc.call("kcGraphDestroy", g)
            return med(t) / (nrep * copies)

        out["graph_kernel_ms"] = replay_ms(lambda i: kc.launch(name, mas[i], s))
        out["graph_floor_ms"] = replay_ms(lambda i: kc.launch("vector_add", va, s))
    y = by.download(np.float32)
    kc.call("kcStreamDestroy", s)
    for buf in streams + [bx, bq, bd, by, a, b, o]:
        buf.free()
    out["finite"] = bool(np.all(np.isfinite(y)))
    return out


def prefill_matmul_run(steps, seed, reps):
    """the FFN of one layer over a 512-token prompt on the MFMA matmul --
    gate and up (8192 x 3072) and down (3072 x 8192), Q4_K, per-256 int8 activations. One step
    = the three matmuls; 2 * rows * k * 512 operations each."""
    n = 512
    shapes = [(8192, 3072), (8192, 3072), (3072, 8192)]
    ws = [synth.quantized_stream("q4k", r, k, seed + i) for i, (r, k) in enumerate(shapes)]
    rng = np.random.default_rng(seed + 50)
    xs = [kc.Buffer.of(rng.standard_normal(k * n).astype(np.float32)) for k in (3072, 8192)]
    qs = [kc.Buffer(n * k // 256 * 85 * 4) for k in (3072, 8192)]
    ys = [kc.Buffer(r * n * 4) for r, _ in shapes]
    s = new_stream()
    for x, q, k in zip(xs, qs, (3072, 8192)):
        kc.launch("quantize_cols_k", kc.QuantizeColsArgs(x.ptr, q.ptr, None, k, n), s)
    args = [kc.MatmulKQ8Args(wt.ptr, qs[0 if k == 3072 else 1].ptr, y.ptr, None, r, k, n, 8)
            for wt, y, (r, k) in zip(ws, ys, shapes)]

    def step(_):
        for a in args:
            kc.launch("matmul_q4k_q8kx8", a, s)

    warm_clocks(s)
    for i in range(3):
        step(i)
    ms = med(time_launches(s, step, steps, reps)) / steps
    kc.call("kcStreamDestroy", s)
    finite = all(np.all(np.isfinite(y.download(np.float32))) for y in ys)
    for b in ws + xs + qs + ys:
        b.free()
    ops = sum(2 * r * k * n for r, k in shapes)
    tops = ops / (ms * 1e-3) / 1e12
    return {"workload": "BASELINE config 3: gate + up (8192x3072) + down (3072x8192) Q4_K matmuls, 512 tokens, "
                        "weights N(0, 0.02) quantized as ggml does",
            "ms_per_step": round(ms, 4), "ops_per_step": ops, "achieved_tops": round(tops, 1),
            "peak_tops": PEAK_F16_TFLOPS, "mfma_util": round(tops / PEAK_F16_TFLOPS, 4),
            "peak_int8_tops": PEAK_INT8_TOPS, "mfma_util_int8": round(tops / PEAK_INT8_TOPS, 4), "reps": reps,
            "mfma": "v_mfma_f32_32x32x16_f16 on exact small-integer operands", "finite": bool(finite)}


# Llama-3.2-3B architecture, Q4_K_M layout (Q6_K for attn_v / ffn_down / output)
LLAMA32_3B = dict(n_layer=28, n_embd=3072, n_head=24, n_head_kv=8, head_dim=128, n_ff=8192, n_vocab=128256,
                  norm_eps=1e-5, rope_theta=500000.0, rope_neox=0, qk_norm=0, max_ctx=1024, max_batch=512)
CFG4_NAME = "BASELINE config 4: 28-layer Llama-3.2-3B shape"
# Qwen3-8B architecture (per-head q/k RMSNorm, NEOX RoPE), 1024-token prefill
# then 256 decode steps (context up to 1280)
QWEN3_8B = dict(n_layer=36, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=12288, n_vocab=151936,
                norm_eps=1e-6, rope_theta=1000000.0, rope_neox=1, qk_norm=1, max_ctx=1536, max_batch=1024)
CFG5_NAME = "BASELINE config 5: 36-layer Qwen3-8B shape (per-head q/k RMSNorm, NEOX RoPE)"


def decode_bytes(w, cfg, ctx):
    """HBM bytes one decode token reads: every weight tensor but the embedding (one row of it),
    the f16 K and V caches over ctx positions, and the logits written."""
    emb_row = cfg["n_embd"] // 256 * 144
    wb = sum(a.nbytes for (tid, _), a in w.items() if tid != 0) + emb_row
    kv = 2 * cfg["n_layer"] * ctx * cfg["n_head_kv"] * cfg["head_dim"] * 2
    return wb + kv + cfg["n_vocab"] * 4


def ggml_backend_decode_run(cfg, n_ctx, n_decode, seed, reps, modes=(1, 0), profile=0):
    """The drop-in path: single-token decode steps of cfg through the ggml backend core
    (kcGgmlGraphCompute) on the graph llama.cpp builds for them (kernelcore_amd/ggml_graph.py: the
    reference op sequence, the backend's fusions, no driver-level fusion), at context n_ctx
    onwards. The KV view spans n_ctx + n_decode rows rounded up to 256 (llama.cpp pads n_kv so),
    so every step has the same nodes and the backend launches its kept graph again; per step the
    host updates the position, cache row and mask inputs (three small copies) and calls
    graph_compute, which returns once the step has run. Weights N(0, 0.02) quantized on the device
    (the types of kcModelTensorInfo), norms N(1, 0.05), caches zero (the step time does not depend
    on their values). Also timed: the same steps with graphs off (launches one by one). profile 1 / 2:
    the backends made with GGML_KERNELCORE_PROFILE's setting, their host times per call and (2: every
    launch timed alone, no graph) the device time per launch name added to the result."""
    from kernelcore_amd import ggml_graph as gg

    s = gg.LayerShape.of_model(cfg, (n_ctx + n_decode + 255) // 256 * 256)
    n_kv = s.kv_size
    bufs, seeds = [], iter(range(seed, seed + 10000))

    def alloc(nbytes, type_, ne):
        if type_ in ("q4k", "q6k"):
            b = synth.quantized_stream(type_, ne[1], ne[0], next(seeds))
        else:
            b = kc.Buffer(nbytes)
            if type_ == "f32" and ne[1] == 1 and ne[0] in (s.n_embd, s.hd):  # norm weights
                kc.launch("fill_normal_f32", kc.FillNormalArgs(b.ptr, ne[0], next(seeds), 1.0, 0.05))
            else:
                kc.call("kcMemset", b.ptr, 0, nbytes)
        bufs.append(b)
        return b.ptr

    t0 = time.perf_counter()
    g = gg.Graph(alloc)
    io, _, _, logits = gg.decoder(g, s, cfg["n_layer"], 1, n_kv)
    kc.synchronize()
    setup_s = time.perf_counter() - t0
    x = np.random.default_rng(seed).standard_normal(s.n_embd).astype(np.float32)
    kc.call("kcMemcpy", io["x"].data, x.ctypes.data, x.nbytes, kc.HOST_TO_DEVICE)
    mask = np.full(n_kv, -np.inf, np.float16)
    nodes = kc.GgmlNodes(g.nodes)  # the node array built once, as llama.cpp hands over its cgraph's

    def step(p):
        pos = np.array([p], np.int32)
        kc.call("kcMemcpy", io["pos"].data, pos.ctypes.data, 4, kc.HOST_TO_DEVICE)
        idx = pos.astype(np.int64)
        kc.call("kcMemcpy", io["kv_idx"].data, idx.ctypes.data, 8, kc.HOST_TO_DEVICE)
        mask[:p + 1] = 0.0
        kc.call("kcMemcpy", io["mask"].data, mask.ctypes.data, mask.nbytes, kc.HOST_TO_DEVICE)
        be.compute(nodes)

    out = {"workload": f"{cfg['n_layer']}-layer decode steps at context {n_ctx}..{n_ctx + n_decode} through "
                       f"kcGgmlGraphCompute on llama.cpp's graph ({len(g.nodes)} nodes per step, KV view of {n_kv} rows)",
           "setup_s": round(setup_s, 1)}
    for graphs in modes:
        be = kc.GgmlBackend(graphs=graphs, profile=profile)
        mask[:] = -np.inf
        for p in range(n_ctx - 4, n_ctx):  # warm-up (records the kept graph)
            step(p)
        times = []
        for _ in range(reps):
            mask[:] = -np.inf
            w0 = time.perf_counter()
            for p in range(n_ctx, n_ctx + n_decode):
                step(p)
            times.append(time.perf_counter() - w0)
        st = be.stats()
        prof = be.profile() if profile >= 2 else None
        be.close()
        ms = med(times) / n_decode * 1e3
        key = "kept_graph" if graphs else "eager"
        out[key] = {"tok_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4),
                    "launches_per_token": round(st["launches"] / st["computes"], 1),
                    "graphs_recorded": st["graphs_recorded"], "graphs_reused": st["graphs_reused"]}
        if profile >= 1:  # the library's host clock per graph_compute call (warm-up calls included)
            out[key]["profile"] = {f"{k}_per_call": round(st[k] / st["computes"], 4)
                                   for k in ("compute_ms", "record_ms", "run_ms")}
            out[key]["profile"]["calls"] = st["computes"]
        if prof:  # device ms per launch name, summed over the calls
            out[key]["profile"]["launches"] = {k: [n, round(v, 4)] for k, (n, v) in sorted(prof.items())}
    lg = np.empty(s.n_vocab, np.float32)
    kc.call("kcMemcpy", lg.ctypes.data, logits.data, lg.nbytes, kc.DEVICE_TO_HOST)
    out["finite"] = bool(np.all(np.isfinite(lg)))
    for b in bufs:
        b.free()
    return out


def ggml_backend_prefill_run(cfg, n_prompt, seed, reps, graphs=1):
    """The drop-in path for a prompt: one n_prompt-token step of cfg (positions 0 .., the causal
    mask, the KV view of n_prompt rows rounded up to 256) through kcGgmlGraphCompute on the graph
    llama.cpp builds (the last layer keeps only the last row after its attention; the head gives
    that row's logits), with the backend claiming attention over the whole prompt (attn_tokens =
    n_prompt: one flash_attn_f16 kernel). The same step is computed reps times (the kept graph after
    the first); weights as the decode leg's."""
    from kernelcore_amd import ggml_graph as gg

    n_kv = (n_prompt + 255) // 256 * 256
    s = gg.LayerShape.of_model(cfg, n_kv)
    bufs, seeds = [], iter(range(seed, seed + 10000))

    def alloc(nbytes, type_, ne):
        if type_ in ("q4k", "q6k"):
            b = synth.quantized_stream(type_, ne[1], ne[0], next(seeds))
        else:
            b = kc.Buffer(nbytes)
            if type_ == "f32" and ne[1] == 1 and ne[0] in (s.n_embd, s.hd):  # norm weights
                kc.launch("fill_normal_f32", kc.FillNormalArgs(b.ptr, ne[0], next(seeds), 1.0, 0.05))
            else:
                kc.call("kcMemset", b.ptr, 0, nbytes)
        bufs.append(b)
        return b.ptr

    g = gg.Graph(alloc)
    io, _, _, logits = gg.decoder(g, s, cfg["n_layer"], n_prompt, n_kv)
    x = np.random.default_rng(seed).standard_normal(n_prompt * s.n_embd).astype(np.float32)
    pos = np.arange(n_prompt, dtype=np.int32)
    mrow = io["mask"].ne[0]
    mask = np.where(np.arange(mrow)[None, :] <= pos[:, None], 0.0, -np.inf).astype(np.float16)
    for name, a in (("x", x), ("pos", pos), ("kv_idx", pos.astype(np.int64)), ("mask", mask)):
        kc.call("kcMemcpy", io[name].data, a.ctypes.data, a.nbytes, kc.HOST_TO_DEVICE)
    kc.synchronize()
    nodes = kc.GgmlNodes(g.nodes)
    be = kc.GgmlBackend(graphs=graphs, attn_tokens=n_prompt)
    be.compute(nodes)  # records the kept graph
    times = []
    for _ in range(reps):
        w0 = time.perf_counter()
        be.compute(nodes)
        times.append(time.perf_counter() - w0)
    st = be.stats()
    be.close()
    lg = np.empty(s.n_vocab, np.float32)
    kc.call("kcMemcpy", lg.ctypes.data, logits.data, lg.nbytes, kc.DEVICE_TO_HOST)
    for b in bufs:
        b.free()
    ms = med(times) * 1e3
    return {"workload": f"{cfg['n_layer']}-layer {n_prompt}-token prompt through kcGgmlGraphCompute on llama.cpp's "
                        f"graph ({len(g.nodes)} nodes, KV view of {n_kv} rows)",
            "prefill_tok_s": round(n_prompt / ms * 1e3, 1), "prefill_ms": round(ms, 3),
            "launches": round(st["launches"] / st["computes"], 1), "reps": reps,
            "finite": bool(np.all(np.isfinite(lg)))}


def model_run(cfg, n_prompt, n_decode, seed, reps, eager=False, name=CFG4_NAME):
    """A random n_prompt-token prompt (one batched forward), then n_decode greedy decode steps
    (graph-replayed, argmax on the device). A warm-up prompt + 4 steps first (builds the decode
    graph); then `reps` repetitions of: reset the cache, the timed prompt, the timed decode.
    Returns the leg's figures (medians) and the weights (for the CPU leg)."""
    t0 = time.perf_counter()
    w = synth.model_weights(cfg, seed)
    m = kc.Model(**cfg)
    for (tid, layer), a in w.items():
        m.set_tensor(tid, layer, a)
    kc.synchronize()
    setup_s = time.perf_counter() - t0
    prompt = np.random.default_rng(seed + 7).integers(0, cfg["n_vocab"], n_prompt).astype(np.int32)
    warm_clocks(m.stream())
    m.forward(prompt)
    if not eager:
        m.generate(4)
    t = Timer(m.stream())
    e = [t.event() for _ in range(3)]
    pre, dec, pre_ev, dec_ev = [], [], [], []
    for _ in range(reps):
        m.reset()
        kc.synchronize()
        w0 = time.perf_counter()
        t.record(e[0])
        logits = m.forward(prompt)
        t.record(e[1])
        w1 = time.perf_counter()
        if eager:  # one kcModelForward per token, argmax on the host (kernel tracing without graphs)
            toks = [int(np.argmax(logits))]
            for _ in range(n_decode):
                toks.append(int(np.argmax(m.forward([toks[-1]]))))
        else:
            toks = m.generate(n_decode + 1)  # the first token comes from the prompt's logits
        t.record(e[2])
        kc.call("kcStreamSynchronize", m.stream())
        w2 = time.perf_counter()
        pre.append(w1 - w0)
        dec.append(w2 - w1)
        pre_ev.append(Timer.ms(e[0], e[1]))
        dec_ev.append(Timer.ms(e[1], e[2]))
        assert m.position() == n_prompt + n_decode
    for x in e:
        kc.call("kcEventDestroy", x)
    m.close()
    bpt = decode_bytes(w, cfg, n_prompt + n_decode // 2)
    dec_s = med(dec)
    gbs = bpt * n_decode / dec_s / 1e9
    out = {"workload": f"{name}, Q4_K_M weights N(0, 0.02) quantized as ggml does, "
                       f"{n_prompt}-token prompt then {n_decode} greedy decode steps, f16 KV cache",
           "prefill_tok_s": round(n_prompt / med(pre), 1), "decode_tok_s": round(n_decode / dec_s, 1),
           "prefill_ms": round(med(pre) * 1e3, 3), "ms_per_decode_token": round(dec_s / n_decode * 1e3, 4),
           "reps": reps, "decode_tok_s_reps": [round(n_decode / d, 1) for d in dec],
           "gpu_event_ms": {"prefill": round(med(pre_ev), 3), "decode": round(med(dec_ev), 3)},
           "decode_bytes_per_token": bpt, "decode_hbm_gbs": round(gbs, 1), "decode_frac": round(gbs / PEAK_HBM_GBS, 4),
           "setup_s": round(setup_s, 2), "finite": bool(np.all(np.isfinite(logits))),
           "first_tokens": [int(x) for x in toks[:4]], "decode": "eager" if eager else "graph"}
    return out, w


# ---- the CPU legs: the oracle's vectorised kernels on the host cores ----------------------------------------


def cpu_info():
    import oracle

    O = oracle.lib()
    level = int(O.kco_simd_level())
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except (OSError, StopIteration):
        model = "unknown"
    return {"threads": int(O.kco_max_threads()), "vnni": level == 2,
            "variant": ["scalar", "simd-avx2", "simd-avx512vnni"][level], "cpu": model}


def cpu_entry(value, unit, info, sample):
    return {"value": round(value, 3), "unit": unit, "cores": info["threads"], "kind": "port",
            "variant": info["variant"], "vnni": info["vnni"], "sample": f"{sample}; {info['cpu']}"}


def sample_median(fn, seconds, reps=5, max_n=200):
    """Median over `reps` samples of the seconds per call of fn, each sample as many calls as fit in
    seconds / reps (at least one)."""
    fn()  # warm
    per = []
    for _ in range(reps):
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds / reps or n >= max_n:
                break
        per.append(el / n)
    return med(per), per


def cpu_matvec(qtype, rows, k, seed, seconds, nbytes):
    """The oracle's matvec (per-32 activations, integer dots) over the same matrix: GB/s."""
    import oracle

    O = oracle.lib()
    info = cpu_info()
    w = synth.quantized_matrix(qtype, rows, k, seed)
    x = np.random.default_rng(seed + 99).standard_normal(k).astype(np.float32)
    xq, xd = oracle.quantize_q8x4(O, x)
    y = np.zeros(rows, np.float32)
    fn = getattr(O, f"kco_matvec_{qtype}_q8_simd")
    per, _ = sample_median(lambda: fn(w, xq, xd, y, rows, k, info["threads"]), seconds)
    return cpu_entry(nbytes / per / 1e9, "GB/s", info,
                     f"median of 5 samples of full {rows}x{k} {qtype.upper()} matvecs, {per * 1e3:.2f} ms each")


def cpu_matmul_cfg3(seed, seconds):
    """Config 3 on the host: the oracle's per-256 matmuls (integer sums per super-block), TOP/s."""
    import oracle

    O = oracle.lib()
    info = cpu_info()
    n = 512
    shapes = [(8192, 3072), (8192, 3072), (3072, 8192)]
    ws = [synth.quantized_matrix("q4k", r, k, seed + i) for i, (r, k) in enumerate(shapes)]
    rng = np.random.default_rng(seed + 50)
    qs = {}
    for k in (3072, 8192):
        q = np.zeros(n * (k // 256 * 85), np.int32)
        O.kco_quantize_cols_k(rng.standard_normal(k * n).astype(np.float32), q, k, n)
        qs[k] = q
    ys = [np.zeros(r * n, np.float32) for r, _ in shapes]

    def step():
        for wt, y, (r, k) in zip(ws, ys, shapes):
            O.kco_matmul_q4k_q8k_simd(wt, qs[k], y, r, k, n, info["threads"])

    per, _ = sample_median(step, seconds, max_n=50)
    ops = sum(2 * r * k * n for r, k in shapes)
    return cpu_entry(ops / per / 1e12, "TOP/s", info,
                     f"median of 5 samples of the full config-3 step (three matmuls, 512 columns), "
                     f"{per * 1e3:.0f} ms each")


def cpu_model(cfg, w, n_prompt, n_decode):
    """The oracle model on the host: the prompt in one forward (prefill tok/s), then greedy decode
    steps at the GPU's context (decode tok/s, the median step)."""
    from oracle.model import OracleModel

    info = cpu_info()
    o = OracleModel(cfg, w, threads=info["threads"])
    prompt = np.random.default_rng(12345).integers(0, cfg["n_vocab"], n_prompt).astype(np.int32)
    t0 = time.perf_counter()
    lo = o.forward(prompt)
    pre = time.perf_counter() - t0
    steps = []
    for _ in range(n_decode):
        tok = int(np.argmax(lo))
        t1 = time.perf_counter()
        lo = o.forward([tok])
        steps.append(time.perf_counter() - t1)
    d = med(steps)
    return {"prefill_tok_s": round(n_prompt / pre, 2), "decode_tok_s": round(1.0 / d, 3), "unit": "tok/s",
            "cores": info["threads"], "kind": "port", "variant": info["variant"], "vnni": info["vnni"],
            "sample": f"one {n_prompt}-token prompt ({pre:.1f} s), then {n_decode} greedy decode steps at context "
                      f"{n_prompt}..{n_prompt + n_decode - 1} (median {d * 1e3:.0f} ms); oracle/model.py with the "
                      f"vectorised matvecs / matmuls and flash attention; {info['cpu']}"}


def bytes_cfg2(rows=128256, k=3072):
    return rows * (k // 256) * 210 + k * 4 + rows * 4


def bytes_cfg1(rows=3072, k=3072):
    return rows * (k // 256) * 144 + k * 4 + rows * 4


def calibrate(n=64 << 20):
    """A vector_add of known size (reads 2n floats, writes n) for scaling PMC byte counters."""
    a, b, o = kc.Buffer(n * 4), kc.Buffer(n * 4), kc.Buffer(n * 4)
    for _ in range(3):
        kc.launch("vector_add", kc.VectorAddArgs(a.ptr, b.ptr, o.ptr, n))
    for x in (a, b, o):
        x.free()
    return {"vector_add_n": n, "read_bytes": 8 * n, "write_bytes": 4 * n}


def traffic_from_profile():
    """HBM bytes per launch of the dominant kernel from the committed PMC summary, if present."""
    p = os.path.join(HERE, "profiles", "traffic_matvec_q6k_cfg2.json")
    try:
        return json.load(open(p)).get("traffic_bytes")
    except (OSError, ValueError):
        return None


def note(msg):
    print(msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--reps", type=int, default=5, help="timed repetitions per leg (their median is reported)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU legs")
    ap.add_argument("--calibrate", action="store_true", help="also run a known-size vector_add (PMC scaling)")
    ap.add_argument("--skip-cfg1", action="store_true", help="only the config-2 workload (short profiling runs)")
    ap.add_argument("--skip-model", action="store_true", help="skip the config-3 matmul and the model legs")
    ap.add_argument("--decode-steps", type=int, default=128)
    ap.add_argument("--decode-steps5", type=int, default=256, help="decode steps of the config-5 leg")
    ap.add_argument("--skip-cfg5", action="store_true", help="skip the config-5 (Qwen3-8B shape) model leg")
    ap.add_argument("--eager-decode", action="store_true",
                    help="decode with one kcModelForward per token instead of the replayed graph")
    ap.add_argument("--no-graph", action="store_true",
                    help="time config 1 and the ggml-backend legs by eager launches only (no graph capture: for "
                         "kernel traces)")
    ap.add_argument("--only-model", action="store_true",
                    help="run only the config-3 matmul and the model legs (profiling); prints their JSON")
    ap.add_argument("--only-cfg3", action="store_true",
                    help="run only the config-3 matmul leg (counter profiles); prints its JSON")
    ap.add_argument("--skip-ggml", action="store_true", help="skip the ggml-backend decode leg")
    ap.add_argument("--only-ggml", action="store_true", help="run only the ggml-backend decode leg; prints its JSON")
    ap.add_argument("--ggml-profile", type=int, default=0,
                    help="with --only-ggml: the backend decode legs with GGML_KERNELCORE_PROFILE's setting (1, 2)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    reps = max(1, args.reps)
    cpu = not args.no_cpu and not args.only_model

    kc.init()
    props = kc.device_properties()
    note(f"# device: {props.name.decode()} ({props.worker_count} CUs)")
    mm = mdl = mdl5 = ggml_leg = ggml_pre = ggml_leg5 = ggml_pre5 = None
    modes, gr = ((0,), 0) if args.no_graph else ((1, 0), 1)

    def ggml_cfg5():
        # config 5 (Qwen3-8B shape: the per-head q / k norms, NEOX RoPE) through the backend: decode at
        # context 1024 onwards (a quarter of the model leg's steps), then the 1024-token prompt
        d = ggml_backend_decode_run(QWEN3_8B, 1024, max(args.decode_steps5 // 4, 8), seed=9900, reps=reps, modes=modes,
                                    profile=args.ggml_profile if args.only_ggml else 0)
        note(f"# ggml backend cfg5 decode done: {d[('kept_graph' if gr else 'eager')]['tok_s']} tok/s")
        p = ggml_backend_prefill_run(QWEN3_8B, 1024, seed=9950, reps=reps, graphs=gr)
        note(f"# ggml backend cfg5 prefill done: {p['prefill_tok_s']} tok/s")
        return d, p

    if args.only_ggml:
        res = {"ggml_backend_decode_cfg4": ggml_backend_decode_run(LLAMA32_3B, 512, args.decode_steps, seed=9700,
                                                                   reps=reps, modes=modes, profile=args.ggml_profile),
               "ggml_backend_prefill_cfg4": ggml_backend_prefill_run(LLAMA32_3B, 512, seed=9800, reps=reps, graphs=gr)}
        if not args.skip_cfg5:
            res["ggml_backend_decode_cfg5"], res["ggml_backend_prefill_cfg5"] = ggml_cfg5()
        print(json.dumps(res), flush=True)
        return
    if args.only_cfg3:
        print(json.dumps({"prefill_matmul_cfg3": prefill_matmul_run(max(args.steps // 5, 5), seed=7000, reps=reps)}),
              flush=True)
        return
    if args.only_model or not args.skip_model:
        mm = prefill_matmul_run(max(args.steps // 5, 5), seed=7000, reps=reps)
        note(f"# cfg3 done: {mm['achieved_tops']} TOP/s")
        mdl, w4 = model_run(LLAMA32_3B, 512, args.decode_steps, seed=9000, reps=reps, eager=args.eager_decode)
        note(f"# cfg4 done: prefill {mdl['prefill_tok_s']} tok/s, decode {mdl['decode_tok_s']} tok/s")
        if cpu:
            mdl["cpu_baseline"] = cpu_model(LLAMA32_3B, w4, 512, 8)
            note(f"# cfg4 cpu done: {mdl['cpu_baseline']['decode_tok_s']} tok/s")
        del w4
        if not args.skip_cfg5:
            mdl5, w5 = model_run(QWEN3_8B, 1024, args.decode_steps5, seed=9500, reps=reps, eager=args.eager_decode,
                                 name=CFG5_NAME)
            note(f"# cfg5 done: prefill {mdl5['prefill_tok_s']} tok/s, decode {mdl5['decode_tok_s']} tok/s")
            if cpu:
                mdl5["cpu_baseline"] = cpu_model(QWEN3_8B, w5, 1024, 4)
            del w5
        if cpu:
            mm["cpu_baseline"] = cpu_matmul_cfg3(7000, 10.0)
        if not args.skip_ggml:
            ggml_leg = ggml_backend_decode_run(LLAMA32_3B, 512, args.decode_steps, seed=9700, reps=reps)
            note(f"# ggml backend decode done: {ggml_leg['kept_graph']['tok_s']} tok/s (kept graph)")
            ggml_pre = ggml_backend_prefill_run(LLAMA32_3B, 512, seed=9800, reps=reps, graphs=gr)
            note(f"# ggml backend prefill done: {ggml_pre['prefill_tok_s']} tok/s")
            if not args.skip_cfg5:
                ggml_leg5, ggml_pre5 = ggml_cfg5()
    if args.only_model:
        res = {"prefill_matmul_cfg3": mm, "model_cfg4": mdl}
        if ggml_leg:
            res["ggml_backend_decode_cfg4"] = ggml_leg
            res["ggml_backend_prefill_cfg4"] = ggml_pre
        if ggml_leg5:
            res["ggml_backend_decode_cfg5"] = ggml_leg5
            res["ggml_backend_prefill_cfg5"] = ggml_pre5
        if mdl5:
            res["model_cfg5"] = mdl5
        print(json.dumps(res), flush=True)
        return
    rows2, k2 = 128256, 3072
    r2 = matvec_run("q6k", rows2, k2, copies=2, steps=args.steps, warmup=args.warmup, seed=1000, reps=reps)
    note(f"# cfg2 done: kernel {r2['kernel_ms'] * 1e3:.1f} us")
    rows1 = k1 = 3072
    copies1 = 200  # 200 x 5.3 MB > 1 GB: the Infinity Cache cannot hold the rotation
    r1 = r1l = None
    if not args.skip_cfg1:
        r1 = matvec_run("q4k", rows1, k1, copies=copies1, steps=max(args.steps, copies1), warmup=args.warmup,
                        seed=5000, reps=reps, graph=not args.no_graph)
        note(f"# cfg1 done: kernel {r1['kernel_ms'] * 1e3:.2f} us")
        # The Q4_K kernel at a streaming size: config 2's shape (128256 x 3072) as Q4_K, 2 rotating
        # copies (369 MB > the 256 MB Infinity Cache).
        r1l = matvec_run("q4k", rows2, k2, copies=2, steps=args.steps, warmup=args.warmup, seed=6000, reps=reps)
        note(f"# q4k large done: kernel {r1l['kernel_ms'] * 1e3:.1f} us")
    cal = calibrate() if args.calibrate else None

    b2 = bytes_cfg2(rows2, k2)
    ms_step = r2["region_ms"] / args.steps
    value = b2 / (ms_step * 1e-3) / 1e9
    achieved = b2 / (r2["kernel_ms"] * 1e-3) / 1e9
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 x q6_k (int32 dot, f32 scale)", "data": "synthetic",
        "config": {"workload": "BASELINE config 2: quantize_q8x4 + matvec_q6k_q8, 128256x3072 Q6_K output head "
                               "(N(0, 0.02) quantized as ggml does), batch 1, 2 rotating weight copies",
                   "rows": rows2, "k": k2, "bytes_per_step": b2, "reps": reps,
                   "region_reps_ms": r2["region_reps_ms"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic_from_profile(),
                     "traffic_source": "not measured in this run: the committed rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE "
                                       "figure of the same kernel and launch (profiles/traffic_matvec_q6k_cfg2.json)",
                     "kernel": "matvec_q6k_q8", "kernel_us": round(r2["kernel_ms"] * 1e3, 2)},
    }
    if r1:
        b1 = bytes_cfg1(rows1, k1)
        if "graph_kernel_ms" not in r1:
            r1["graph_kernel_ms"] = r1["graph_floor_ms"] = float("nan")
        a1 = b1 / (r1["graph_kernel_ms"] * 1e-3) / 1e9
        out["q4k_matvec_cfg1"] = {
            "achieved_gbs": round(a1, 1), "frac": round(a1 / PEAK_HBM_GBS, 4),
            "kernel_us": round(r1["graph_kernel_ms"] * 1e3, 3), "graph_floor_us": round(r1["graph_floor_ms"] * 1e3, 3),
            "eager_kernel_us": round(r1["kernel_ms"] * 1e3, 3), "eager_floor_us": round(r1["floor_ms"] * 1e3, 3),
            "eager_achieved_gbs": round(b1 / (r1["kernel_ms"] * 1e-3) / 1e9, 1), "bytes": b1,
            "rotation": f"{copies1} weight copies",
            "note": "kernel_us: the matvecs over the rotation replayed as one HIP graph (the launch cost "
                    "amortised over the graph), per matvec; "
                    "eager_kernel_us: the same launches one host call each; *_floor_us: the same launch counts of a "
                    "256-element vector_add (what a launch costs however small)"}
        if cpu:
            out["q4k_matvec_cfg1"]["cpu_baseline"] = cpu_matvec("q4k", rows1, k1, 5000, 5.0, bytes_cfg1(rows1, k1))
    if r1l:
        bl = bytes_cfg1(rows2, k2)
        al = bl / (r1l["kernel_ms"] * 1e-3) / 1e9
        out["q4k_matvec_large"] = {"workload": f"matvec_q4k_q8, {rows2}x{k2} Q4_K (config 2's shape), batch 1, "
                                               "2 rotating weight copies", "achieved_gbs": round(al, 1),
                                   "frac": round(al / PEAK_HBM_GBS, 4), "kernel_us": round(r1l["kernel_ms"] * 1e3, 2),
                                   "bytes": bl}
    if mm:
        out["prefill_matmul_cfg3"] = mm
    if mdl:
        out["model_cfg4"] = mdl
    if mdl5:
        out["model_cfg5"] = mdl5
    if ggml_leg:
        out["ggml_backend_decode_cfg4"] = ggml_leg
        out["ggml_backend_prefill_cfg4"] = ggml_pre
    if ggml_leg5:
        out["ggml_backend_decode_cfg5"] = ggml_leg5
        out["ggml_backend_prefill_cfg5"] = ggml_pre5
    if cal:
        out["calibration"] = cal
    if cpu:
        out["cpu_baseline"] = cpu_matvec("q6k", rows2, k2, 1000, 10.0, b2)
    if not (r2["finite"] and (r1 is None or r1["finite"]) and (r1l is None or r1l["finite"])
            and (mm is None or mm["finite"]) and (mdl is None or mdl["finite"]) and (mdl5 is None or mdl5["finite"])):
        out["warning"] = "non-finite outputs"
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
