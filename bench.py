"""Benchmark of the K-quant decode hot path on one MI355X.

One step = one pass of the hot path over one batch of synthetic input at BASELINE config 2: the
activation vector x (f32[3072], N(0,1)) is quantized to per-32 int8 blocks (quantize_q8x4) and
multiplied by the 128256 x 3072 Q6_K output head (matvec_q6k_q8) into f32 logits. Weights are
seeded random ggml blocks with bounded fp16 scales (the reference tests' generator), repacked on
the GPU; two copies alternate so the 256 MB Infinity Cache cannot hold them.

value = algorithmic bytes per step (ggml weight bytes + x + y, 323,730,432 B) / wall time per step,
with every input resident in HBM. roofline: the same bytes over the matvec kernel's own average
duration (HIP events around each launch on its stream) against the 8 TB/s HBM peak. Also reported:
config 1 (Q4_K 3072 x 3072) rotated over >1 GB of weight copies, the Q4_K matvec at config 2's
shape, config 3 (the prefill matmuls), configs 4 and 5 (prefill and decode of the Llama-3.2-3B and
Qwen3-8B shapes), and the same-run CPU baselines (oracle/kc_oracle.c on the host cores, bounded
samples of config-2 matvecs and of decode steps).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--calibrate]
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import kernelcore_amd as kc  # noqa: E402

PEAK_HBM_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # dense fp16 MFMA
METRIC = "Q4_K matvec HBM GB/s (% of peak); decode tok/s, 3B-shape Q4_K_M, 1 GPU"


def random_blocks(qtype, rows, k, seed):
    """Random ggml blocks, fp16 scales in [2^-9, 2^-6) (tests/test_llm_kernels.cpp:205-219)."""
    rng = np.random.default_rng(seed)
    bb = kc.BLOCK_BYTES[qtype]
    n = rows * (k // 256)
    b = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    half = lambda: (0x1800 + rng.integers(0, 0x0C00, size=n)).astype(np.uint16).view(np.uint8).reshape(n, 2)
    if qtype == "q4k":
        b[:, 0:2], b[:, 2:4] = half(), half()
    else:
        b[:, 208:210] = half()
    return b.reshape(-1)


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


def matvec_run(qtype, rows, k, copies, steps, warmup, seed):
    """quantize + matvec per step over `copies` weight streams; returns timings."""
    nb = k // 32
    streams = [kc.upload_weights(qtype, random_blocks(qtype, rows, k, seed + i), rows, k) for i in range(copies)]
    x = (np.random.default_rng(seed + 99).standard_normal(k)).astype(np.float32)
    bx, bq, bd, by = kc.Buffer.of(x), kc.Buffer(nb * 32), kc.Buffer(nb * 8), kc.Buffer(rows * 4)
    s = C.c_void_p()
    kc.call("kcStreamCreate", C.byref(s))
    qa = kc.QuantizeArgs(bx.ptr, bq.ptr, bd.ptr, nb)
    mas = [kc.MatvecQ4Q8Args(w.ptr, bq.ptr, bd.ptr, by.ptr, None, rows, k) for w in streams]
    name = f"matvec_{qtype}_q8"
    for i in range(warmup):
        kc.launch("quantize_q8x4", qa, s)
        kc.launch(name, mas[i % copies], s)
    kc.call("kcStreamSynchronize", s)
    t = Timer(s)
    t0, t1, k0, k1 = t.event(), t.event(), t.event(), t.event()
    kc.synchronize()
    # the timed steps: quantize + matvec, back to back on one stream
    wall0 = time.perf_counter()
    t.record(t0)
    for i in range(steps):
        kc.launch("quantize_q8x4", qa, s)
        kc.launch(name, mas[i % copies], s)
    t.record(t1)
    kc.call("kcStreamSynchronize", s)
    kc.synchronize()
    wall = time.perf_counter() - wall0
    # the matvec kernel alone: the same launches without the quantizer, averaged between two events
    t.record(k0)
    for i in range(steps):
        kc.launch(name, mas[i % copies], s)
    t.record(k1)
    kc.call("kcStreamSynchronize", s)
    region_ms = Timer.ms(t0, t1)
    kernel_ms = Timer.ms(k0, k1) / steps
    y = by.download(np.float32)
    for e in (t0, t1, k0, k1):
        kc.call("kcEventDestroy", e)
    kc.call("kcStreamDestroy", s)
    for b in streams + [bx, bq, bd, by]:
        b.free()
    return {"kernel_ms": kernel_ms, "region_ms": region_ms, "wall_s": wall, "finite": bool(np.all(np.isfinite(y)))}


def calibrate(n=64 << 20):
    """A vector_add of known size (reads 2n floats, writes n) for scaling PMC byte counters."""
    a, b, o = kc.Buffer(n * 4), kc.Buffer(n * 4), kc.Buffer(n * 4)
    for _ in range(3):
        kc.launch("vector_add", kc.VectorAddArgs(a.ptr, b.ptr, o.ptr, n))
    for x in (a, b, o):
        x.free()
    return {"vector_add_n": n, "read_bytes": 8 * n, "write_bytes": 4 * n}


def cpu_baseline(rows, k, seconds=10.0):
    """The oracle's config-2 matvec on the host cores (OpenMP), a bounded sample of full passes."""
    import oracle

    O = oracle.lib()
    threads = int(O.kco_max_threads())
    w = random_blocks("q6k", rows, k, 4001)
    x = np.random.default_rng(4002).standard_normal(k).astype(np.float32)
    xq, xd = oracle.quantize_q8x4(O, x)
    y = np.zeros(rows, np.float32)
    O.kco_matvec_q6k_q8_mt(w, xq, xd, y, rows, k, threads)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        O.kco_matvec_q6k_q8_mt(w, xq, xd, y, rows, k, threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 200:
            break
    per = el / n
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except (OSError, StopIteration):
        model = "unknown"
    return {"value": round(bytes_cfg2(rows, k) / per / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} full config-2 Q6_K matvecs ({rows}x{k}, per-32 int8 activations) in {el:.1f} s, "
                      f"{per * 1e3:.1f} ms each, OpenMP over {threads} threads of {model}"}


# Llama-3.2-3B architecture, Q4_K_M layout (Q6_K for attn_v / ffn_down / output)
LLAMA32_3B = dict(n_layer=28, n_embd=3072, n_head=24, n_head_kv=8, head_dim=128, n_ff=8192, n_vocab=128256,
                  norm_eps=1e-5, rope_theta=500000.0, rope_neox=0, qk_norm=0, max_ctx=1024, max_batch=512)
CFG5_NAME = "BASELINE config 5: 36-layer Qwen3-8B shape (per-head q/k RMSNorm, NEOX RoPE)"
# Qwen3-8B architecture (per-head q/k RMSNorm, NEOX RoPE), 1024-token prefill
# then 256 decode steps (context up to 1280)
QWEN3_8B = dict(n_layer=36, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=12288, n_vocab=151936,
                norm_eps=1e-6, rope_theta=1000000.0, rope_neox=1, qk_norm=1, max_ctx=1536, max_batch=1024)


def model_weights(m, cfg, seed):
    """{(tensor id, layer): bytes} for every tensor of model m: random ggml blocks (random_blocks)
    or norm weights in [0.8, 1.2); shapes from kcModelTensorInfo."""
    rng = np.random.default_rng(seed)
    out = {}
    ids = [(t, -1) for t in (0, 1, 2)]
    per_layer = [3, 4, 5, 6, 7, 8, 9, 10, 11] + ([12, 13] if cfg["qk_norm"] else [])
    ids += [(t, l) for l in range(cfg["n_layer"]) for t in per_layer]
    for tid, layer in ids:
        qt, rows, k, _ = m.tensor_info(tid, layer)
        if qt == 0:
            out[(tid, layer)] = rng.uniform(0.8, 1.2, k).astype(np.float32)
        else:
            out[(tid, layer)] = random_blocks("q6k" if qt == 14 else "q4k", rows, k, seed + 1000 * tid + layer + 1)
    return out


def decode_bytes(w, cfg, ctx):
    """HBM bytes one decode token reads: every weight tensor but the embedding (one row of it),
    the f16 K and V caches over ctx positions, and the logits written."""
    emb_row = cfg["n_embd"] // 256 * 144
    wb = sum(a.nbytes for (tid, _), a in w.items() if tid != 0) + emb_row
    kv = 2 * cfg["n_layer"] * ctx * cfg["n_head_kv"] * cfg["head_dim"] * 2
    return wb + kv + cfg["n_vocab"] * 4


def model_run(cfg, n_prompt, n_decode, seed, cpu_seconds, eager=False,
              name="BASELINE config 4: 28-layer Llama-3.2-3B shape"):
    """a random n_prompt-token prompt (one batched forward), then n_decode greedy
    decode steps (graph-replayed, argmax on the device). A warm-up prompt + 4 steps first (builds
    the decode graph), then the cache is reset and the timed prompt and decode run."""
    m = kc.Model(**cfg)
    t0 = time.perf_counter()
    w = model_weights(m, cfg, seed)
    for (tid, layer), a in w.items():
        m.set_tensor(tid, layer, a)
    kc.synchronize()
    setup_s = time.perf_counter() - t0
    prompt = np.random.default_rng(seed + 7).integers(0, cfg["n_vocab"], n_prompt).astype(np.int32)
    m.forward(prompt)
    if not eager:
        m.generate(4)
    m.reset()
    kc.synchronize()
    t = Timer(m.stream())
    e = [t.event() for _ in range(3)]
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
    prefill_ms, decode_ms = Timer.ms(e[0], e[1]), Timer.ms(e[1], e[2])
    for x in e:
        kc.call("kcEventDestroy", x)
    assert m.position() == n_prompt + n_decode
    m.close()
    bpt = decode_bytes(w, cfg, n_prompt + n_decode // 2)
    dec_s = w2 - w1
    gbs = bpt * n_decode / dec_s / 1e9
    out = {"workload": f"{name}, Q4_K_M random weights, "
                       f"{n_prompt}-token prompt then {n_decode} greedy decode steps, f16 KV cache",
           "prefill_tok_s": round(n_prompt / (w1 - w0), 1), "decode_tok_s": round(n_decode / dec_s, 1),
           "prefill_ms": round((w1 - w0) * 1e3, 3), "ms_per_decode_token": round(dec_s / n_decode * 1e3, 4),
           "gpu_event_ms": {"prefill": round(prefill_ms, 3), "decode": round(decode_ms, 3)},
           "decode_bytes_per_token": bpt, "decode_hbm_gbs": round(gbs, 1), "decode_frac": round(gbs / PEAK_HBM_GBS, 4),
           "setup_s": round(setup_s, 2), "finite": bool(np.all(np.isfinite(logits))),
           "first_tokens": [int(x) for x in toks[:4]], "decode": "eager" if eager else "graph"}
    if cpu_seconds > 0:
        out["cpu_baseline"] = cpu_decode_baseline(cfg, w, cpu_seconds)
    return out


def cpu_decode_baseline(cfg, w, seconds):
    """The oracle model's decode (oracle/model.py: the same step on the host, OpenMP matvecs) from
    an empty cache, a bounded number of tokens."""
    import oracle
    from oracle.model import OracleModel

    threads = int(oracle.lib().kco_max_threads())
    o = OracleModel(cfg, w, threads=threads)
    o.forward([1])  # warm
    n, t0 = 0, time.perf_counter()
    tok = 1
    while True:
        tok = int(np.argmax(o.forward([tok])))
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 64:
            break
    return {"value": round(n / el, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} greedy decode tokens at context 2..{n + 1} (the GPU decodes at {cfg['max_batch']}+), "
                      f"{el / n * 1e3:.0f} ms each; the matvecs OpenMP over {threads} threads"}


def prefill_matmul_run(steps, seed):
    """the FFN of one layer over a 512-token prompt on the MFMA matmul --
    gate and up (8192 x 3072) and down (3072 x 8192), Q4_K, per-256 int8 activations. One step
    = the three matmuls; 2 * rows * k * 512 operations each."""
    n = 512
    shapes = [(8192, 3072), (8192, 3072), (3072, 8192)]
    ws = [kc.upload_weights("q4k", random_blocks("q4k", r, k, seed + i), r, k) for i, (r, k) in enumerate(shapes)]
    rng = np.random.default_rng(seed + 50)
    xs = [kc.Buffer.of(rng.standard_normal(k * n).astype(np.float32)) for k in (3072, 8192)]
    qs = [kc.Buffer(n * k // 256 * 85 * 4) for k in (3072, 8192)]
    ys = [kc.Buffer(r * n * 4) for r, _ in shapes]
    s = C.c_void_p()
    kc.call("kcStreamCreate", C.byref(s))
    for x, q, k in zip(xs, qs, (3072, 8192)):
        kc.launch("quantize_cols_k", kc.QuantizeColsArgs(x.ptr, q.ptr, None, k, n), s)
    args = [kc.MatmulKQ8Args(wt.ptr, qs[0 if k == 3072 else 1].ptr, y.ptr, None, r, k, n, 8)
            for wt, y, (r, k) in zip(ws, ys, shapes)]
    for _ in range(2):
        for a in args:
            kc.launch("matmul_q4k_q8kx8", a, s)
    t = Timer(s)
    e0, e1 = t.event(), t.event()
    kc.call("kcStreamSynchronize", s)
    t.record(e0)
    for _ in range(steps):
        for a in args:
            kc.launch("matmul_q4k_q8kx8", a, s)
    t.record(e1)
    kc.call("kcStreamSynchronize", s)
    ms = Timer.ms(e0, e1) / steps
    for x in (e0, e1):
        kc.call("kcEventDestroy", x)
    kc.call("kcStreamDestroy", s)
    finite = all(np.all(np.isfinite(y.download(np.float32))) for y in ys)
    for b in ws + xs + qs + ys:
        b.free()
    ops = sum(2 * r * k * n for r, k in shapes)
    tops = ops / (ms * 1e-3) / 1e12
    return {"workload": "BASELINE config 3: gate + up (8192x3072) + down (3072x8192) Q4_K matmuls, 512 tokens",
            "ms_per_step": round(ms, 4), "ops_per_step": ops, "achieved_tops": round(tops, 1),
            "peak_tops": PEAK_F16_TFLOPS, "mfma_util": round(tops / PEAK_F16_TFLOPS, 4),
            "mfma": "v_mfma_f32_32x32x16_f16 on exact small-integer operands", "finite": bool(finite)}


def bytes_cfg2(rows=128256, k=3072):
    return rows * (k // 256) * 210 + k * 4 + rows * 4


def bytes_cfg1(rows=3072, k=3072):
    return rows * (k // 256) * 144 + k * 4 + rows * 4


def traffic_from_profile():
    """HBM bytes per launch of the dominant kernel from the committed PMC summary, if present."""
    p = os.path.join(HERE, "profiles", "traffic_matvec_q6k_cfg2.json")
    try:
        return json.load(open(p)).get("traffic_bytes")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--calibrate", action="store_true", help="also run a known-size vector_add (PMC scaling)")
    ap.add_argument("--skip-cfg1", action="store_true", help="only the config-2 workload (short profiling runs)")
    ap.add_argument("--skip-model", action="store_true", help="skip the config-3 matmul and config-4 model legs")
    ap.add_argument("--decode-steps", type=int, default=128)
    ap.add_argument("--decode-steps5", type=int, default=256, help="decode steps of the config-5 leg")
    ap.add_argument("--skip-cfg5", action="store_true", help="skip the config-5 (Qwen3-8B shape) model leg")
    ap.add_argument("--eager-decode", action="store_true",
                    help="decode with one kcModelForward per token instead of the replayed graph")
    ap.add_argument("--only-model", action="store_true",
                    help="run only the config-3 matmul and config-4 model legs (profiling); prints their JSON")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    kc.init()
    props = kc.device_properties()
    print(f"# device: {props.name.decode()} ({props.worker_count} CUs)", file=sys.stderr, flush=True)
    if args.only_model:
        mm = prefill_matmul_run(max(args.steps // 5, 5), seed=7000)
        mdl = model_run(LLAMA32_3B, 512, args.decode_steps, seed=9000, cpu_seconds=0, eager=args.eager_decode)
        res = {"prefill_matmul_cfg3": mm, "model_cfg4": mdl}
        if not args.skip_cfg5:
            res["model_cfg5"] = model_run(QWEN3_8B, 1024, args.decode_steps5, seed=9500, cpu_seconds=0,
                                          eager=args.eager_decode, name=CFG5_NAME)
        print(json.dumps(res), flush=True)
        return
    rows2, k2 = 128256, 3072
    r2 = matvec_run("q6k", rows2, k2, copies=2, steps=args.steps, warmup=args.warmup, seed=1000)
    print(f"# cfg2 done: kernel {r2['kernel_ms'] * 1e3:.1f} us", file=sys.stderr, flush=True)
    rows1 = k1 = 3072
    copies1 = 200  # 200 x 5.3 MB > 1 GB: the Infinity Cache cannot hold the rotation
    r1 = None
    if not args.skip_cfg1:
        r1 = matvec_run("q4k", rows1, k1, copies=copies1, steps=max(args.steps, copies1), warmup=args.warmup,
                        seed=5000)
        print(f"# cfg1 done: kernel {r1['kernel_ms'] * 1e3:.2f} us", file=sys.stderr, flush=True)
    # The Q4_K kernel at a streaming size: config 2's shape (128256 x 3072) as Q4_K, 2 rotating
    # copies (369 MB > the 256 MB Infinity Cache).
    r1l = None
    if not args.skip_cfg1:
        r1l = matvec_run("q4k", rows2, k2, copies=2, steps=args.steps, warmup=args.warmup, seed=6000)
        print(f"# q4k large done: kernel {r1l['kernel_ms'] * 1e3:.1f} us", file=sys.stderr, flush=True)
    cal = calibrate() if args.calibrate else None
    mm = mdl = mdl5 = None
    if not args.skip_model:
        mm = prefill_matmul_run(max(args.steps // 5, 5), seed=7000)
        print(f"# cfg3 done: {mm['achieved_tops']} TOP/s", file=sys.stderr, flush=True)
        mdl = model_run(LLAMA32_3B, 512, args.decode_steps, seed=9000, cpu_seconds=0 if args.no_cpu else 10.0,
                        eager=args.eager_decode)
        print(f"# cfg4 done: prefill {mdl['prefill_tok_s']} tok/s, decode {mdl['decode_tok_s']} tok/s",
              file=sys.stderr, flush=True)
        if not args.skip_cfg5:
            mdl5 = model_run(QWEN3_8B, 1024, args.decode_steps5, seed=9500,
                             cpu_seconds=0 if args.no_cpu else 10.0, eager=args.eager_decode, name=CFG5_NAME)
            print(f"# cfg5 done: prefill {mdl5['prefill_tok_s']} tok/s, decode {mdl5['decode_tok_s']} tok/s",
                  file=sys.stderr, flush=True)

    b2 = bytes_cfg2(rows2, k2)
    ms_step = r2["region_ms"] / args.steps
    value = b2 / (ms_step * 1e-3) / 1e9
    achieved = b2 / (r2["kernel_ms"] * 1e-3) / 1e9
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 x q6_k (int32 dot, f32 scale)", "data": "synthetic",
        "config": {"workload": "BASELINE config 2: quantize_q8x4 + matvec_q6k_q8, 128256x3072 Q6_K output head, "
                               "batch 1, 2 rotating weight copies", "rows": rows2, "k": k2, "bytes_per_step": b2},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic_from_profile(),
                     "kernel": "matvec_q6k_q8", "kernel_us": round(r2["kernel_ms"] * 1e3, 2)},
    }
    if r1:
        a1 = bytes_cfg1(rows1, k1) / (r1["kernel_ms"] * 1e-3) / 1e9
        out["q4k_matvec_cfg1"] = {"achieved_gbs": round(a1, 1), "frac": round(a1 / PEAK_HBM_GBS, 4),
                                  "kernel_us": round(r1["kernel_ms"] * 1e3, 3), "bytes": bytes_cfg1(rows1, k1),
                                  "rotation": f"{copies1} weight copies"}
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
    if cal:
        out["calibration"] = cal
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(rows2, k2)
    if not (r2["finite"] and (r1 is None or r1["finite"]) and (r1l is None or r1l["finite"]) and (mm is None or mm["finite"])
            and (mdl is None or mdl["finite"]) and (mdl5 is None or mdl5["finite"])):
        out["warning"] = "non-finite outputs"
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
