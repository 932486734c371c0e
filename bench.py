"""Benchmark of the K-quant decode hot path on one MI355X.

One step = one pass of the hot path over one batch of synthetic input at BASELINE config 2: the
activation vector x (f32[3072], N(0,1)) is quantized to per-32 int8 blocks (quantize_q8x4) and
multiplied by the 128256 x 3072 Q6_K output head (matvec_q6k_q8) into f32 logits. Weights are
seeded random ggml blocks with bounded fp16 scales (the reference tests' generator), repacked on
the GPU; two copies alternate so the 256 MB Infinity Cache cannot hold them.

value = algorithmic bytes per step (ggml weight bytes + x + y, 323,730,432 B) / wall time per step,
with every input resident in HBM. roofline: the same bytes over the matvec kernel's own average
duration (HIP events around each launch on its stream) against the 8 TB/s HBM peak. Also reported:
config 1 (Q4_K 3072 x 3072) rotated over >1 GB of weight copies, and the same-run CPU baseline
(oracle/kc_oracle.c on the host cores, a bounded sample of config-2 matvecs).

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
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    kc.init()
    props = kc.device_properties()
    print(f"# device: {props.name.decode()} ({props.worker_count} CUs)", file=sys.stderr, flush=True)
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
    cal = calibrate() if args.calibrate else None

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
    if cal:
        out["calibration"] = cal
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(rows2, k2)
    if not (r2["finite"] and (r1 is None or r1["finite"])):
        out["warning"] = "non-finite outputs"
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
