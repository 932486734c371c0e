"""BASELINE configs 4 and 5 at full size through the ggml backend core, node by node.

The decoder graph llama.cpp builds (kernelcore_amd/ggml_graph.py: the op order of
docs/cuda_cpu_poc_plan.md:1156-1158 and llm/llm_model.cpp:287-360) for every layer of the
Llama-3.2-3B shape (28 layers) and the Qwen3-8B shape (36 layers), with their vocabularies and
N(0, 0.02) weights quantized as ggml does (kernelcore_amd/synth.py), runs through
kcGgmlGraphCompute with kernel option ggml_extra_fusions = 1: the reference's launches
(ggml-kernelcore.cpp:706-792: its fused norms and SwiGLU, one launch per other node), so that every
node the reference writes is written. Each step's nodes sit in memory of their own, and after the step
every node of every layer is checked against the oracle applied to the GPU's own inputs to that node
-- so each op is held to its own bar and nothing compounds, however deep the model (the layer
test's bars, tests/test_gpu_ggml_backend.py):
  - [ADD +] RMS_NORM + MUL: the sum and the normed rows bit-exact; Qwen3's per-head q / k norms
    bit-exact;
  - MUL_MAT: one column (decode, and the last layer's FFN and the head of a prompt) bit-exact against
    the oracle's per-32 matvec; a batch (the MFMA matmuls) within 1e-3 of the oracle's per-256 matmul;
  - ROPE within the f32 angle's ulps (rope_check; 2e-5 of the largest value, the layer tests' bar,
    holds only at small positions); SET_ROWS: both fp16 caches bit-exact, rows written and
    rows untouched; FLASH_ATTN_EXT within its sum order's ulps (attn_check); SWIGLU within 2e-6 relative (exp2 ulps);
    the residual ADDs bit-exact; the head's logits bit-exact.
Config 4: a 512-token prompt, then 128 decode steps to context 640 (the cache's size). Config 5: a
1024-token prompt, a 200-token chunk that continues it (causal attention over cache and chunk), then
56 decode steps to context 1280. The decode steps share one graph over the whole KV view (the mask
hides the rows not yet written), as llama.cpp pads n_kv: the backend records it once and launches
the kept graph for every later step. Eight decode steps are checked, spread from the first to the
last. Every token of every node is checked."""
import ctypes as C
import os
import sys
import time

import numpy as np
import pytest

import kernelcore_amd as kc
import oracle
from kernelcore_amd import ggml_graph as gg
from kernelcore_amd import synth
from tests import kq
from tests.test_gpu_configs import CFG4, CFG5

pytestmark = pytest.mark.gpu
O = oracle.lib()
THREADS = max(1, min(16, os.cpu_count() or 1))
LAYER_IDS = dict(attn_norm=3, wq=4, wk=5, wv=6, wo=7, ffn_norm=8, wg=9, wu=10, wd=11, q_norm=12, k_norm=13)


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


# ---- the oracle on given inputs ----------------------------------------------------------------

def norm_oracle(x, w, n, eps, batch, a=None, b=None):
    """The fused [ADD +] RMS_NORM + MUL of `rows` rows (their f32 sum and normed output): per-256
    (sumsq_part / add_sumsq_f + norm_mul_q8k) for a batch node, per-32 (norm_mul_q8) for one row."""
    rows = (x if a is None else a).size // n
    nb, nsb = n // 32, n // 256
    sq = np.zeros(rows * nb * 11, np.int32)
    if a is not None:
        x = np.zeros(n * rows, np.float32)
        O.kco_add_sumsq_f(np.ascontiguousarray(a, np.float32).reshape(-1), np.ascontiguousarray(b, np.float32).reshape(-1),
                          x, sq, n, rows)
    else:
        x = np.ascontiguousarray(x, np.float32).reshape(-1).copy()
        O.kco_sumsq_part(x, sq, n, rows)
    y = np.zeros(n * rows, np.float32)
    if batch:
        O.kco_norm_mul_q8k(x, w, y, np.zeros(rows * nsb * 85, np.int32), sq, n, rows, np.float32(eps))
    else:
        O.kco_norm_mul_q8(x, w, y, sq, n, rows, np.float32(eps))
    return x.reshape(rows, n), y.reshape(rows, n)


def mm_oracle(qtype, blocks, x, rows, k, batch):
    """A MUL_MAT's columns x ([n, k]): the per-256 activations and matmul of a batch node, else the
    per-32 activations and matvec of a one-column node (the vectorised forms, bit-identical to the
    scalar restatement)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, k)
    n = x.shape[0]
    y = np.zeros(n * rows, np.float32)
    if batch:
        q = np.zeros(n * (k // 256 * 85), np.int32)
        O.kco_quantize_cols_k(x.reshape(-1), q, k, n)
        getattr(O, f"kco_matmul_{qtype}_q8k_simd")(blocks, q, y, rows, k, n, THREADS)
    else:
        assert n == 1
        xq, xd = oracle.quantize_q8x4(O, x[0])
        getattr(O, f"kco_matvec_{qtype}_q8_simd")(blocks, xq, xd, y, rows, k, THREADS)
    return y.reshape(n, rows)


def rope_check(x, got, want, pos, hd, nh, base, neox, what):
    """ROPE against the oracle within what f32 leaves open: both take the angle pos * 2^(-i/pairs *
    log2 base) the same way, up to an ulp of exp2 and of the product (the GPU's and the C library's
    exp2f), so the angles agree to 4 ulps (2^-21 relative: 3e-5 rad at angle 241, position 299),
    and sin / cos with the rotation's roundings add 8 ulps of one; the bound per element is the pair's
    norm times (angle * 2^-21 + 2^-20). A wrong sign, pair, position or frequency is off by the
    pair's norm itself."""
    pairs = hd // 2
    x = np.asarray(x, np.float64).reshape(-1, nh, hd)
    x0, x1 = (x[..., :pairs], x[..., pairs:]) if neox else (x[..., 0::2], x[..., 1::2])
    theta = np.asarray(pos, np.float64)[:, None, None] * base ** (-np.arange(pairs) / pairs)
    tp = (theta * 2.0 ** -21 + 2.0 ** -20) * np.hypot(x0, x1)
    tol = np.concatenate([tp, tp], axis=-1) if neox else np.repeat(tp, 2, axis=-1)
    err = np.abs(np.asarray(got, np.float64).reshape(tol.shape) - np.asarray(want, np.float64).reshape(tol.shape))
    worst = float((err / (tol + 1e-30)).max())
    assert worst <= 1.0, (what, worst, float(err.max()))


def attn_check(q, kcache, vcache, mask, d, scale, got, what):
    """FLASH_ATTN_EXT against the oracle's within what f32 sum order leaves open. Each output is
    sum_j p_j v_j / sum_j p_j over T keys; the oracle sums keys in order, the GPU in blocks and
    split chunks. Summation noise grows as sqrt(T) ulps of sum_j p_j |v_j| / sum_j p_j (the oracle
    on |V| gives it), and the scores' own ulps (dot product order, exp2) move each p_j by about
    2^-20. So the bound per element is that magnitude times (8 sqrt(T) 2^-24 + 2^-19): 1.9e-5 of it
    at 1224 keys. (A fixed 2e-6 of the largest output, the layer tests' bar, held to 1024 keys;
    outputs are averages with cancellation, so the magnitude can be far above the output.) A key
    missed or taken in excess, a wrong scale, head or row is off by 1e-3 of the magnitude or more."""
    q = np.ascontiguousarray(q, np.float32).reshape(-1)
    m = np.ascontiguousarray(mask).reshape(-1).view(np.uint16)
    want = np.zeros(q.size, np.float32)
    mag = np.zeros(q.size, np.float32)
    O.kco_flash_attn_f16_mt(q, kcache, vcache, m, want, C.byref(d), np.float32(scale), THREADS)
    O.kco_flash_attn_f16_mt(q, kcache, np.ascontiguousarray(vcache & 0x7FFF), m, mag, C.byref(d), np.float32(scale),
                            THREADS)
    tol = (8.0 * np.sqrt(d.T) * 2.0 ** -24 + 2.0 ** -19) * mag.astype(np.float64)
    err = np.abs(np.asarray(got, np.float64).reshape(-1) - want)
    worst = float((err / (tol + 1e-30)).max())
    assert worst <= 1.0, (what, worst, float(err.max()), kq.rel_diff(got.reshape(-1), want))
    return worst


def same_bits(got, want, what):
    g, w = kq.bits(got).reshape(-1), kq.bits(want).reshape(-1)
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} differ, first at {bad[0]}"


# ---- the model in the backend's buffers -----------------------------------------------------------

class Decoder:
    """cfg's weights in the backend's buffers (kcWeightSetTensor), its fp16 KV caches, the host copies
    of the ggml blocks (for the oracle); graph(N, n_kv) builds llama.cpp's step graph over them with
    every node in device memory of its own."""

    def __init__(self, cfg, seed):
        self.cfg = cfg
        self.s = gg.LayerShape.of_model(cfg, cfg["max_ctx"])
        self.w = synth.model_weights(cfg, seed)
        self.bufs = []
        wg = gg.Graph(self._alloc)
        self.W = {"layers": [gg.layer_weights(wg, self.s) for _ in range(cfg["n_layer"])],
                  "output_norm": wg.leaf("f32", [self.s.n_embd], buffer="weights"),
                  "output": wg.leaf("q6k", [self.s.n_embd, self.s.n_vocab], buffer="weights")}
        self.keep = wg
        for l, lw in enumerate(self.W["layers"]):
            for name, tid in LAYER_IDS.items():
                if name in lw:
                    self._set(lw[name], self.w[(tid, l)])
            for c in ("k_cache", "v_cache"):
                kc.call("kcMemset", lw[c].data, 0, self.s.kv_dim * self.s.kv_size * 2)
        self._set(self.W["output_norm"], self.w[(1, -1)])
        self._set(self.W["output"], self.w[(2, -1)])
        self.blocks = [{n: self.w[(LAYER_IDS[n], l)] for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
                       for l in range(cfg["n_layer"])]
        self.emb = self.w[(0, -1)].reshape(cfg["n_vocab"], -1)

    def _alloc(self, nbytes, type_, ne, into=None):
        if type_ in ("q4k", "q6k"):
            nbytes = kc.weight_alloc_size(type_, ne[1], ne[0])
        b = kc.Buffer(nbytes)
        (self.bufs if into is None else into).append(b)
        return b.ptr

    def _set(self, t, data):
        qt = {v: k for k, v in kc.GGML_TYPE.items()}[t.type]
        if qt in ("q4k", "q6k"):
            kc.weight_set(qt, t.ne[1], t.ne[0], t.data, data)
        else:
            put(t, data)

    def embed(self, tokens):
        """GET_ROWS of the embedding (the CPU backend's part in llama.cpp): dequantized rows."""
        E = self.cfg["n_embd"]
        return np.concatenate([oracle.dequant(O, "q4k", self.emb[t], 1, E) for t in tokens]).astype(np.float32)

    def graph(self, N, n_kv):
        step = []
        g = gg.Graph(lambda nbytes, type_, ne: self._alloc(nbytes, type_, ne, step))
        io, _, layers, logits = gg.decoder(g, self.s, self.cfg["n_layer"], N, n_kv, weights=self.W)
        return Step(self, g, io, layers, logits, N, n_kv, step)

    def caches(self):
        n = self.s.kv_size * self.s.kv_dim
        return [(get(lw["k_cache"], np.uint16, n), get(lw["v_cache"], np.uint16, n)) for lw in self.W["layers"]]

    def free(self):
        for b in self.bufs:
            b.free()


def put(t, a):
    a = np.ascontiguousarray(a)
    kc.call("kcMemcpy", t.data, a.ctypes.data, a.nbytes, kc.HOST_TO_DEVICE)


def get(t, dtype, count=None):
    n = count if count is not None else int(np.prod([t.ne[d] for d in range(4)]))
    out = np.empty(n, dtype)
    kc.call("kcMemcpy", out.ctypes.data, t.data, out.nbytes, kc.DEVICE_TO_HOST)
    return out


class Step:
    """One step's graph: N tokens at positions p0.., attending over the first n_kv cache rows."""

    def __init__(self, D, g, io, layers, logits, N, n_kv, bufs):
        self.D, self.g, self.io, self.layers, self.logits = D, g, io, layers, logits
        self.N, self.n_kv, self.bufs = N, n_kv, bufs
        self.nodes = kc.GgmlNodes(g.nodes)
        self.out_cur = logits.src[1].contents  # the output norm's MUL (the head's input)

    def set_inputs(self, tokens, p0):
        N = self.N
        assert len(tokens) == N and p0 + N <= self.n_kv
        self.tokens, self.p0 = np.asarray(tokens), p0
        self.x = self.D.embed(tokens)
        self.pos = np.arange(p0, p0 + N, dtype=np.int32)
        m = np.full((N, self.io["mask"].ne[0]), -np.inf, np.float16)
        for i in range(N):
            m[i, :p0 + i + 1] = 0.0
        self.mask = m
        put(self.io["x"], self.x)
        put(self.io["pos"], self.pos)
        put(self.io["kv_idx"], self.pos.astype(np.int64))
        put(self.io["mask"], m)

    def free(self):
        for b in self.bufs:
            b.free()


# ---- the node checks ------------------------------------------------------------------------------

def check_step(S, before):
    """Every node of every layer of the step just computed, against the oracle on the GPU's inputs to
    that node; before: each layer's (k, v) cache contents ahead of the step. Returns the logits."""
    D, s, N = S.D, S.D.s, S.N
    E, hd, eps = s.n_embd, s.hd, s.eps
    batch = N > 1
    tol = 1e-3 if N >= 64 else 0
    rows = np.arange(N)
    n_layer = len(S.layers)
    f32 = lambda t: get(t, np.float32)
    ff = np.ones(hd // 2, np.float32)

    worst = {"matmul": 0.0, "attention": 0.0}

    def mm_check(qt, blocks, x, got, what, b=batch, t=tol):
        want = mm_oracle(qt, blocks, x, got.shape[1], x.shape[1], b)
        if t == 0:
            same_bits(got, want, what)
        else:
            r = kq.rel_diff(got, want)
            assert r < t, (what, r)
            worst["matmul"] = max(worst["matmul"], r)

    x_in, res = S.x.reshape(N, E), None  # res: the ADD fused into this layer's attention norm
    for l, t in enumerate(S.layers):
        B, last = D.blocks[l], l == n_layer - 1
        where = f"layer {l}"
        # attention norm ([ADD +] RMS_NORM + MUL): the sum (the previous layer's out) and cur bit-exact
        if res is None:
            _, y = norm_oracle(x_in[rows], D.w[(3, l)], E, eps, batch)
        else:
            xs, y = norm_oracle(None, D.w[(3, l)], E, eps, batch, a=res[0][rows], b=res[1][rows])
            same_bits(x_in[rows], xs, f"{where} residual out (fused ADD)")
        cur = f32(t["cur"]).reshape(N, E)
        same_bits(cur[rows], y, f"{where} attn norm")
        # q / k / v
        q = f32(t["q"]).reshape(N, s.q_dim)
        k = f32(t["k"]).reshape(N, s.kv_dim)
        v = f32(t["v"]).reshape(N, s.kv_dim)
        for got, w in ((q, "wq"), (k, "wk"), (v, "wv")):
            mm_check(s.types[w], B[w], cur[rows], got[rows], f"{where} {w}")
        qs, ks = q, k
        if s.qk_norm:  # Qwen3's per-head norms (RMS_NORM + MUL: one rms_norm launch with the weight)
            qs, ks = f32(t["qn"]).reshape(N, s.q_dim), f32(t["kn"]).reshape(N, s.kv_dim)
            for src, got, wid, nh, what in ((q, qs, 12, s.n_head, "q norm"), (k, ks, 13, s.n_head_kv, "k norm")):
                want = np.zeros(len(rows) * nh * hd, np.float32)
                O.kco_rms_norm(np.ascontiguousarray(src[rows]).reshape(-1), D.w[(wid, l)], want, hd, len(rows) * nh,
                               np.float32(eps))
                same_bits(got[rows], want, f"{where} {what}")
        # RoPE of the GPU's q and k
        qr = f32(t["qr"]).reshape(N, s.q_dim)
        kr = f32(t["kr"]).reshape(N, s.kv_dim)
        for src, got, nh, what in ((qs, qr, s.n_head, "rope q"), (ks, kr, s.n_head_kv, "rope k")):
            want = np.zeros(len(rows) * nh * hd, np.float32)
            O.kco_rope_ggml(np.ascontiguousarray(src[rows]).reshape(-1), want, S.pos[rows], ff, hd, nh, len(rows),
                            np.log2(s.base), int(s.neox))
            rope_check(src[rows], got[rows], want, S.pos[rows], hd, nh, s.base, s.neox, f"{where} {what}")
        # SET_ROWS: the new rows are fp16 of the GPU's roped k and its v, every other row untouched
        kcache = get(t["k_cache"], np.uint16, s.kv_size * s.kv_dim)
        vcache = get(t["v_cache"], np.uint16, s.kv_size * s.kv_dim)
        for src, got, old, what in ((kr, kcache, before[l][0], "k cache"), (v, vcache, before[l][1], "v cache")):
            want = old.copy()
            pairs = s.kv_dim // 2
            O.kco_set_rows_f16(np.ascontiguousarray(src).reshape(-1), S.pos.astype(np.int64), want, pairs, N, s.kv_dim,
                               pairs, s.kv_size)
            bad = np.flatnonzero(got != want)
            assert bad.size == 0, f"{where} {what}: {bad.size} values differ, first at row {bad[0] // s.kv_dim}"
        # FLASH_ATTN_EXT over the GPU's caches and roped q, the step's mask
        n_pad = S.mask.shape[1]
        d = oracle.FaDims(H=s.n_head, T=S.n_kv, D=hd, group=s.n_head // s.n_head_kv, tp=(S.n_kv + 7) // 8 * 8,
                          k_row=s.kv_dim // 2, k_head=hd // 2, v_row=s.kv_dim // 2, v_head=hd // 2, N=len(rows),
                          q_tok=hd * s.n_head, q_head=hd, m_row=n_pad // 2, has_mask=1, H_kv=s.n_head_kv)
        attn = f32(t["attn"]).reshape(N, s.q_dim)
        r = attn_check(qr[rows], kcache, vcache, S.mask[rows], d, 1.0 / hd ** 0.5, attn[rows], f"{where} attention")
        worst["attention"] = max(worst["attention"], r)
        # o
        o = f32(t["o"]).reshape(N, E)
        mm_check(s.types["wo"], B["wo"], attn[rows], o[rows], f"{where} wo")
        # FFN: ADD + RMS_NORM + MUL fused (the last layer of a batch: the last token's row only)
        if last and batch:
            frows, fbatch, ftol = np.array([0]), False, 0
            xs, y = norm_oracle(None, D.w[(8, l)], E, eps, False, a=o[N - 1], b=x_in[N - 1])
            ffn_inp = f32(t["ffn_inp"]).reshape(1, E)
            same_bits(ffn_inp, xs, f"{where} ffn_inp (last row)")
        else:
            frows, fbatch, ftol = rows, batch, tol
            xs, y = norm_oracle(None, D.w[(8, l)], E, eps, batch, a=o[rows], b=x_in[rows])
            ffn_inp = f32(t["ffn_inp"]).reshape(N, E)
            same_bits(ffn_inp[rows], xs, f"{where} ffn_inp")
        cur2 = f32(t["cur2"]).reshape(-1, E)
        same_bits(cur2[frows], y, f"{where} ffn norm")
        gate = f32(t["gate"]).reshape(-1, s.n_ff)
        up = f32(t["up"]).reshape(-1, s.n_ff)
        mm_check(s.types["wg"], B["wg"], cur2[frows], gate[frows], f"{where} wg", fbatch, ftol)
        mm_check(s.types["wu"], B["wu"], cur2[frows], up[frows], f"{where} wu", fbatch, ftol)
        act = f32(t["act"]).reshape(-1, s.n_ff)
        want = np.zeros(len(frows) * s.n_ff, np.float32)
        O.kco_silu_mul(np.ascontiguousarray(gate[frows]).reshape(-1), np.ascontiguousarray(up[frows]).reshape(-1), want,
                       want.size)
        assert np.allclose(act[frows].reshape(-1), want, rtol=2e-6, atol=1e-30), (where, "swiglu")
        down = f32(t["down"]).reshape(-1, E)
        mm_check(s.types["wd"], B["wd"], act[frows], down[frows], f"{where} wd", fbatch, ftol)
        # the residual ADD is fused into the next norm (checked there: sum and output)
        x_in, res = f32(t["out"]).reshape(-1, E), (down, ffn_inp)
        same_bits(x_in, down + ffn_inp, f"{where} out")
    # the output norm (fused with the last residual ADD) and the head, one row: bit-exact
    xs, y = norm_oracle(None, D.w[(1, -1)], E, eps, False, a=res[0][-1], b=res[1][-1])
    same_bits(x_in[-1], xs, "last layer out (fused ADD)")
    same_bits(get(S.out_cur, np.float32), y, "output norm")
    logits = get(S.logits, np.float32)
    same_bits(logits, mm_oracle("q6k", D.w[(2, -1)], y, s.n_vocab, E, False), "head")
    return logits, worst


def run_config(name, cfg, seed, chunks, decode_to, check_at):
    """chunks: the batch steps (token counts); then single tokens from the end of the last chunk to
    context decode_to, checked at the decode steps in check_at (negative: from the end)."""
    t0 = time.time()
    D = Decoder(cfg, seed)
    note(f"{name}: weights ready in {time.time() - t0:.1f} s")
    kc.set_option("ggml_extra_fusions", 1)
    be = kc.GgmlBackend(graphs=1, attn_tokens=max(chunks))
    try:
        rng = np.random.default_rng(seed + 1)
        p = 0
        for n in chunks:
            S = D.graph(n, p + n)
            names, _ = kc.ggml_graph_plan(S.g.nodes, attn_tokens=max(chunks))
            assert not any(x.startswith("decode_") or x == "matmul_group" for x in names), names
            S.set_inputs(rng.integers(0, cfg["n_vocab"], n).astype(np.int32), p)
            before = D.caches()
            t1 = time.time()
            be.compute(S.nodes)
            t2 = time.time()
            logits, worst = check_step(S, before)
            note(f"{name}: {n} tokens to context {p + n}: {len(S.g.nodes)} nodes checked; worst MFMA product "
                 f"{worst['matmul']:.1e} of 1e-3, worst attention {worst['attention']:.2f} of its bound "
                 f"(gpu {t2 - t1:.2f} s, check {time.time() - t2:.1f} s)")
            S.free()
            p += n
        n_steps = decode_to - p
        check = {i % n_steps for i in check_at}
        S = D.graph(1, decode_to)  # one graph over the whole KV view for every decode step
        for i in range(n_steps):
            tok = int(np.argmax(logits))
            S.set_inputs([tok], p)
            before = D.caches() if i in check else None
            be.compute(S.nodes)
            if i in check:
                t2 = time.time()
                logits, worst = check_step(S, before)
                note(f"{name}: decode step {i} at context {p + 1}: {len(S.g.nodes)} nodes checked; worst attention "
                     f"{worst['attention']:.2f} of its bound ({time.time() - t2:.1f} s)")
            else:
                logits = get(S.logits, np.float32)
            assert np.all(np.isfinite(logits))
            p += 1
        st = be.stats()
        assert st["graphs_reused"] == n_steps - 1, st  # the kept graph launched for every later step
        S.free()
        note(f"{name}: {len(chunks)} batch steps and {n_steps} decode steps to context {p}, "
             f"{time.time() - t0:.1f} s")
    finally:
        be.close()
        kc.set_option("ggml_extra_fusions", 0)
        D.free()


def test_config4_every_node_through_the_backend():
    run_config("config 4 (ggml)", CFG4, 204, chunks=[512], decode_to=640, check_at=[0, 1, 21, 42, 64, 85, 106, -1])


def test_config5_every_node_through_the_backend():
    run_config("config 5 (ggml)", CFG5, 205, chunks=[1024, 200], decode_to=1280, check_at=[0, 1, 10, 19, 28, 37, 46, -1])
