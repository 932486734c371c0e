"""The ggml backend core (include/kernelcore/ggml_backend.h) on the GPU: graph_compute
(integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp:706-792) over the layer graph
llama.cpp builds (kernelcore_amd/ggml_graph.py), every node's output checked against the oracle on the
GPU's own inputs to that node, so that each op is held to its own bar and nothing compounds:
  - [ADD +] RMS_NORM + MUL (fused): bit-exact against the oracle's fused restatement;
  - MUL_MAT q/k/v, o, gate/up, down: the oracle's quantizer and product on the node's f32 input --
    bit-exact (matvec per column, column-tiled matmul), 1e-3 on the MFMA matmul (64 columns);
  - ROPE: 2e-5 of the largest value (the layer tests' bar); SET_ROWS: the whole fp16 cache
    bit-exact (rows written, rows untouched); FLASH_ATTN_EXT: 2e-6 relative;
  - SWIGLU: 2e-6 relative (exp2 ulps); the residual ADDs: bit-exact.
Then the graph paths: a backend recording graphs and one launching eagerly give bit-identical
layers, and the kept graph, launched again for new input values with eager work and
synchronizations between, matches the eager backend on every call (and is not recorded again)."""
import ctypes as C
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
import oracle
from kernelcore_amd import ggml_graph as gg
from oracle.model import OracleModel
from tests import kq

pytestmark = pytest.mark.gpu
O = oracle.lib()


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


class Layer:
    """A layer graph over device memory with seeded contents: weights (N(0, 0.02) quantized to K-quant
    blocks, uploaded through kcWeightSetTensor), norm weights, the token inputs, and a cache holding p0
    earlier rows."""

    def __init__(self, shape, N, p0, seed, share=False, outputs=()):
        """share: the computed nodes placed as ggml's allocator places them (gg.share_memory: freed
        memory reused, in-place ops), after marking the tensors named in `outputs` graph outputs."""
        self.s, self.N, self.p0, self.n_kv = shape, N, p0, p0 + N
        self.bufs = {}
        self.g = gg.Graph(self._alloc)
        self.t = gg.llama_layer(self.g, shape, N, self.n_kv)
        for name in outputs:
            self.t[name].output = 1
        if share:
            gg.share_memory(self.g, lambda n: self._alloc(n, "f32", [n // 4]))
        s, t = shape, self.t
        self.blocks = {}
        for i, name in enumerate(("wq", "wk", "wv", "wo", "wg", "wu", "wd")):
            w = t[name]
            qt, k, rows = s.types[name], w.ne[0], w.ne[1]
            # N(0, 0.02) quantized as ggml does: activations and attention scores of a real model's size
            # (random block bytes make scores of ~1e5, where the softmax is too sharp to compare)
            self.blocks[name] = oracle.quantize_weights(O, qt, kq.randn(rows * k, seed + i, 0.02), rows, k)
            kc.weight_set(qt, rows, k, w.data, self.blocks[name])
        self.attn_norm = kq.uniform(s.n_embd, seed + 10, 0.5, 1.5)
        self.ffn_norm = kq.uniform(s.n_embd, seed + 11, 0.5, 1.5)
        self.put("attn_norm", self.attn_norm)
        self.put("ffn_norm", self.ffn_norm)
        if s.qk_norm:  # Qwen3's per-head q / k norm weights
            self.put("q_norm", kq.uniform(s.hd, seed + 15, 0.5, 1.5))
            self.put("k_norm", kq.uniform(s.hd, seed + 16, 0.5, 1.5))
        pos = np.arange(p0, p0 + N, dtype=np.int32)
        self.pos = pos
        self.put("pos", pos)
        self.put("kv_idx", pos.astype(np.int64))
        n_pad = t["mask"].ne[0]
        m = np.full((N, n_pad), -np.inf, np.float16)
        for i in range(N):
            m[i, :p0 + i + 1] = 0.0
        self.mask = m.reshape(-1).view(np.uint16)
        self.put("mask", self.mask)
        if t["ff"] is not None:
            self.ff = kq.uniform(s.hd // 2, seed + 12, 1.0, 4.0)
            self.put("ff", self.ff)
        else:
            self.ff = np.ones(s.hd // 2, np.float32)
        rng = np.random.default_rng(seed + 13)
        for c in ("k_cache", "v_cache"):
            cache = np.zeros((s.kv_size, s.kv_dim), np.float16)
            cache[:p0] = rng.standard_normal((p0, s.kv_dim)).astype(np.float16)
            self.put(c, cache.reshape(-1).view(np.uint16))
        self.set_x(seed + 14)

    def _alloc(self, nbytes, type_, ne):
        if type_ in ("q4k", "q6k"):
            nbytes = kc.weight_alloc_size(type_, ne[1], ne[0])
        b = kc.Buffer(nbytes)
        self.bufs[b.ptr] = b
        return b.ptr

    def put(self, name, arr):
        a = np.ascontiguousarray(arr)
        kc.call("kcMemcpy", self.t[name].data, a.ctypes.data, a.nbytes, kc.HOST_TO_DEVICE)

    def get(self, name, dtype, count=None):
        t = self.t[name]
        n = count if count is not None else int(np.prod([t.ne[d] for d in range(4)]))
        out = np.empty(n, dtype)
        kc.call("kcMemcpy", out.ctypes.data, t.data, out.nbytes, kc.DEVICE_TO_HOST)
        return out

    def set_x(self, seed):
        self.x = kq.randn(self.s.n_embd * self.N, seed, 1.0)
        self.put("x", self.x)

    def free(self):
        for b in self.bufs.values():
            b.free()


def fused_norm_oracle(x, w, n, rows, eps, a=None, b=None):
    """The oracle's add_sumsq_f / sumsq_part + norm_mul_q8[k] (its f32 output)."""
    nb, nsb = n // 32, n // 256
    sq = np.zeros(rows * nb * 11, np.int32)
    if a is not None:
        x = np.zeros(n * rows, np.float32)
        O.kco_add_sumsq_f(a, b, x, sq, n, rows)
    else:
        x = x.copy()
        O.kco_sumsq_part(x, sq, n, rows)
    y = np.zeros(n * rows, np.float32)
    if rows > 1:
        O.kco_norm_mul_q8k(x, w, y, np.zeros(rows * nsb * 85, np.int32), sq, n, rows, eps)
    else:
        O.kco_norm_mul_q8(x, w, y, sq, n, rows, eps)
    return x, y


def mul_mat_oracle(qtype, blocks, xcols, rows, k):
    """The launches the backend makes for a MUL_MAT with default switches: one column -> quantize_q8x4
    + matvec; a batch -> per-256 slots (quantize_cols_k) + the per-256 matmul."""
    ncols = xcols.shape[0]
    if ncols == 1:
        xq, xd = oracle.quantize_q8x4(O, xcols[0])
        y = np.zeros(rows, np.float32)
        getattr(O, f"kco_matvec_{qtype}_q8")(blocks, xq, xd, y, rows, k)
        return y.reshape(1, rows)
    q = np.zeros(ncols * (k // 256 * 85), np.int32)
    O.kco_quantize_cols_k(np.ascontiguousarray(xcols).reshape(-1), q, k, ncols)
    y = np.zeros(rows * ncols, np.float32)
    getattr(O, f"kco_matmul_{qtype}_q8k")(blocks, q, y, rows, k, ncols)
    return y.reshape(ncols, rows)


def check_mm(L, name, wname, xname, tol, xcols=None):
    s = L.s
    w = L.t[wname]
    rows, k = w.ne[1], w.ne[0]
    if xcols is None:
        xcols = L.get(xname, np.float32).reshape(L.N, k)
    got = L.get(name, np.float32).reshape(L.N, rows)
    want = mul_mat_oracle(s.types[wname], L.blocks[wname], xcols, rows, k)
    if tol == 0:
        assert np.array_equal(kq.bits(got), kq.bits(want)), name
    else:
        assert kq.rel_diff(got, want) < tol, name


def check_layer(L, names=()):
    """names: the plan's launches. The fused decode launches leave some intermediates unwritten
    (decode_norm_*: the normed rows; decode_matvec_add: the o / down products; decode_*swiglu: gate,
    up and their SWIGLU); they are then taken from the oracle's chain on the GPU's written tensors."""
    s, N = L.s, L.N
    mm_tol = 1e-3 if N >= 64 else 0
    norm_fused = "decode_norm_matvec" in names
    ffn_norm_fused = "decode_norm_swiglu" in names
    swiglu_fused = ffn_norm_fused or "decode_swiglu" in names
    add_fused = "decode_matvec_add" in names
    # attention norm (fused): y bit-exact
    _, y = fused_norm_oracle(L.x, L.attn_norm, s.n_embd, N, s.eps)
    if not norm_fused:
        assert np.array_equal(kq.bits(L.get("cur", np.float32)), kq.bits(y)), "attn norm"
    for name, w in (("q", "wq"), ("k", "wk"), ("v", "wv")):
        check_mm(L, name, w, "cur", mm_tol, xcols=y.reshape(N, s.n_embd) if norm_fused else None)
    # rope of q and k from the GPU's q and k
    for src, dst, nh in (("q", "qr", s.n_head), ("k", "kr", s.n_head_kv)):
        x = L.get(src, np.float32)
        want = np.zeros_like(x)
        O.kco_rope_ggml(x, want, L.pos, L.ff, s.hd, nh, N, np.log2(s.base), int(s.neox))
        got = L.get(dst, np.float32)
        assert np.abs(got - want).max() <= 2e-5 * max(1.0, np.abs(want).max()), dst
    # the caches: the new rows are fp16 of the GPU's k (roped) and v, every other row untouched
    for src, cache, before in (("kr", "k_cache", L.k_before), ("v", "v_cache", L.v_before)):
        want = before.copy()
        pairs = s.kv_dim // 2
        O.kco_set_rows_f16(L.get(src, np.float32), L.pos.astype(np.int64), want, pairs, N, s.kv_dim, pairs,
                           s.kv_size)
        assert np.array_equal(L.get(cache, np.uint16), want), cache
    # attention over the GPU's caches and roped q
    d = oracle.FaDims(H=s.n_head, T=L.n_kv, D=s.hd, group=s.n_head // s.n_head_kv, tp=(L.n_kv + 7) // 8 * 8,
                      k_row=s.kv_dim // 2, k_head=s.hd // 2, v_row=s.kv_dim // 2, v_head=s.hd // 2, N=N,
                      q_tok=s.hd * s.n_head, q_head=s.hd, m_row=L.t["mask"].ne[0] // 2, has_mask=1, H_kv=s.n_head_kv)
    want = np.zeros(N * s.n_head * s.hd, np.float32)
    O.kco_flash_attn_f16(L.get("qr", np.float32), L.get("k_cache", np.uint16), L.get("v_cache", np.uint16), L.mask,
                         want, C.byref(d), np.float32(1.0 / s.hd ** 0.5))
    assert kq.rel_diff(L.get("attn", np.float32), want) < 2e-6, "attention"
    attn = L.get("attn", np.float32).reshape(N, s.n_head * s.hd)
    # a batch of 64+ columns: o's second K half is added inside the FFN norm (o holds the first half)
    o_folded = N >= 64 and "matmul_group" in names
    if add_fused or o_folded:
        o = mul_mat_oracle(s.types["wo"], L.blocks["wo"], attn, s.n_embd, s.n_head * s.hd).reshape(-1)
    else:
        check_mm(L, "o", "wo", "attn", mm_tol)
        o = L.get("o", np.float32)
    if o_folded:  # x = x_in + (o1 + o2) against the oracle's o; the norm of the GPU's x bit-exact
        xg = L.get("ffn_inp", np.float32)
        assert kq.rel_diff(xg, L.x + o) < mm_tol, "ffn_inp"
        x, y = fused_norm_oracle(xg, L.ffn_norm, s.n_embd, N, s.eps)
    else:
        # residual ADD fused with the FFN norm: x = o + x_in, y = norm(x) * w, both bit-exact
        x, y = fused_norm_oracle(None, L.ffn_norm, s.n_embd, N, s.eps, a=o, b=L.x)
        assert np.array_equal(kq.bits(L.get("ffn_inp", np.float32)), kq.bits(x)), "ffn_inp"
    if not ffn_norm_fused:
        assert np.array_equal(kq.bits(L.get("cur2", np.float32)), kq.bits(y)), "ffn norm"
    cur2 = y.reshape(N, s.n_embd)
    if swiglu_fused:
        # gate, up and the GLU's f32 results are not written: the down projection (or the layer output)
        # against the oracle's chain (a value within an ulp of a rounding tie may quantize one step
        # apart: exp2 ulps of the two silu)
        g = mul_mat_oracle(s.types["wg"], L.blocks["wg"], cur2, s.n_ff, s.n_embd)
        u = mul_mat_oracle(s.types["wu"], L.blocks["wu"], cur2, s.n_ff, s.n_embd)
        act = np.zeros(g.size, np.float32)
        O.kco_silu_mul(g.reshape(-1), u.reshape(-1), act, g.size)
        down = mul_mat_oracle(s.types["wd"], L.blocks["wd"], act.reshape(N, s.n_ff), s.n_embd, s.n_ff).reshape(-1)
        if not add_fused:
            assert kq.rel_diff(L.get("down", np.float32), down) < 1e-4, "down (fused swiglu)"
            down = L.get("down", np.float32)
        want = down + L.get("ffn_inp", np.float32)
        assert kq.rel_diff(L.get("out", np.float32), want) < 1e-4, "out"
        if not add_fused:
            assert np.array_equal(kq.bits(L.get("out", np.float32)), kq.bits(want)), "out"
    else:
        check_mm(L, "gate", "wg", "cur2", mm_tol)
        check_mm(L, "up", "wu", "cur2", mm_tol)
        g, u = L.get("gate", np.float32), L.get("up", np.float32)
        want = np.zeros_like(g)
        O.kco_silu_mul(g, u, want, g.size)
        assert np.allclose(L.get("act", np.float32), want, rtol=2e-6, atol=1e-30), "swiglu"
        check_mm(L, "down", "wd", "act", mm_tol)
        want = L.get("down", np.float32) + L.get("ffn_inp", np.float32)
        assert np.array_equal(kq.bits(L.get("out", np.float32)), kq.bits(want)), "out"


CASES = [
    ("decode", gg.LayerShape(), 1, 40, {}),
    ("decode, NEOX rope with frequency factors, head_dim 128", gg.LayerShape(n_embd=1024, neox=True, freq_factors=True),
     1, 300, {}),
    ("batch of 8", gg.LayerShape(), 8, 100, {}),
    ("batch of 64 (MFMA matmuls)", gg.LayerShape(), 64, 64, dict(attn_tokens=64)),
]


@pytest.mark.parametrize("graphs", [1, 0])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_layer_graph_matches_the_oracle_node_by_node(case, graphs):
    name, shape, N, p0, cfg = case
    note(f"ggml layer: {name}, N={N}, p0={p0}, graphs={graphs}")
    # the roped q and k as graph outputs: one token's fused attention writes them only when something
    # outside it reads them, and this test checks every node
    L = Layer(shape, N, p0, seed=300 + N, outputs=("qr", "kr"))
    L.k_before, L.v_before = L.get("k_cache", np.uint16), L.get("v_cache", np.uint16)
    be = kc.GgmlBackend(graphs=graphs, **cfg)
    names, _ = kc.ggml_graph_plan(L.g.nodes, graphs=graphs, **cfg)
    be.compute(L.g.nodes)
    st = be.stats()
    assert st["computes"] == 1 and st["graphs_recorded"] == graphs
    assert st["launches"] == len([n for n in names if n not in "[]"])
    check_layer(L, names)
    be.close()
    L.free()


@pytest.mark.parametrize("live", [False, True], ids=["dead-intermediates", "live-intermediates"])
@pytest.mark.parametrize("shape", [gg.LayerShape(), gg.LayerShape(n_embd=1024, neox=True, freq_factors=True),
                                   gg.LayerShape(n_embd=1024, n_head=8, n_head_kv=2, head_dim=128, neox=True,
                                                 qk_norm=True)],
                         ids=["llama", "neox-ff", "qwen3-qk-norm"])
def test_fused_decode_matvecs_equal_one_launch_per_node(shape, live):
    """One input column: the norms inside the q / k / v and gate / up / SWIGLU launches, the o and
    down products with their residual ADDs, ROPE with the cache rows, the attention output
    quantized in its merge -- every output both write (q, k, v, the caches, the attention, the two
    residual sums) equals the reference's one launch per node bit for bit. The roped q and k (and
    Qwen3's normed q and k) are written by the fused attention only when something outside it reads
    them: live, they are graph outputs and compared as well."""
    qk = ("qr", "kr") + (("qn", "kn") if shape.qk_norm else ())
    L = Layer(shape, 1, 90, seed=808, outputs=qk if live else ())
    names, _ = kc.ggml_graph_plan(L.g.nodes)
    attn = "norm_rope_flash_decode_q8" if shape.qk_norm else "rope_flash_decode_q8"
    assert names == ["decode_norm_matvec", attn, "decode_matvec_add",
                     "decode_norm_swiglu", "decode_matvec_add"]
    kept = ("q", "k", "v", "attn", "ffn_inp", "out") + (qk if live else ())  # what both write
    got = {}
    for opt in (1, 0):
        kc.set_option("ggml_extra_fusions", opt)
        try:
            be = kc.GgmlBackend(graphs=1)
            be.compute(L.g.nodes)
            kc.synchronize()
            got[opt] = {n: L.get(n, np.float32) for n in kept}
            got[opt]["k_cache"], got[opt]["v_cache"] = L.get("k_cache", np.uint16), L.get("v_cache", np.uint16)
            be.close()
        finally:
            kc.set_option("ggml_extra_fusions", 0)
    for n in got[0]:
        a, b = got[0][n], got[1][n]
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b), n
    L.free()


@pytest.mark.parametrize("attn_path", [2, 3], ids=["one-head", "gqa"])
@pytest.mark.parametrize("shape", [gg.LayerShape(), gg.LayerShape(n_embd=1024, neox=True)], ids=["D64", "D128"])
def test_batch_attention_with_an_irregular_mask(shape, attn_path):
    """The matrix-core FLASH_ATTN_EXT of a batch with ggml's mask as given, not causal: random holes,
    keys 64-127 masked for every query (two whole key blocks skipped), a query with a single key,
    keys past the prompt open to the first queries; against the oracle on the GPU's own inputs. Both
    kernels: one query head per workgroup (attn_path 2) and the query heads of a KV head in one
    workgroup (3), each the default for some grid size."""
    kc.set_option("attn_path", attn_path)
    try:
        _irregular_mask_case(shape)
    finally:
        kc.set_option("attn_path", 0)


def _irregular_mask_case(shape):
    N, p0 = 40, 150
    L = Layer(shape, N, p0, seed=919)
    rng = np.random.default_rng(5)
    n_pad = L.t["mask"].ne[0]
    m = np.where(rng.random((N, n_pad)) < 0.3, -np.inf, 0.0).astype(np.float16)
    m[:, L.n_kv:] = -np.inf
    m[:, 64:128] = -np.inf
    m[3, :] = -np.inf
    m[3, 5] = 0.0
    m[:4, p0 + N - 1] = 0.0  # the last key, ahead of these queries' positions
    m[7, 130:140] = np.float16(-2.5)  # finite penalties, not only 0 / -inf
    _masked_case(L, N, m)


def _masked_case(L, N, m):
    """L's layer with mask m through the backend (the masked matrix-core attention), against the
    oracle on the GPU's own inputs."""
    names, _ = kc.ggml_graph_plan(L.g.nodes, attn_tokens=N)
    assert "attn_masked" in names
    L.mask = m.reshape(-1).view(np.uint16)
    L.put("mask", L.mask)
    n_pad = L.t["mask"].ne[0]
    # cache rows past the view (the last key block may reach past n_kv) hold Inf: keys past T must
    # not reach the products (p = 0 times Inf is NaN)
    for c in ("k_cache", "v_cache"):
        cache = L.get(c, np.uint16).reshape(L.s.kv_size, L.s.kv_dim)
        cache[L.n_kv:] = 0x7C00
        L.put(c, cache.reshape(-1))
    be = kc.GgmlBackend(graphs=1, attn_tokens=N)
    be.compute(L.g.nodes)
    kc.synchronize()
    s = L.s
    d = oracle.FaDims(H=s.n_head, T=L.n_kv, D=s.hd, group=s.n_head // s.n_head_kv, tp=(L.n_kv + 7) // 8 * 8,
                      k_row=s.kv_dim // 2, k_head=s.hd // 2, v_row=s.kv_dim // 2, v_head=s.hd // 2, N=N,
                      q_tok=s.hd * s.n_head, q_head=s.hd, m_row=n_pad // 2, has_mask=1, H_kv=s.n_head_kv)
    want = np.zeros(N * s.n_head * s.hd, np.float32)
    O.kco_flash_attn_f16(L.get("qr", np.float32), L.get("k_cache", np.uint16), L.get("v_cache", np.uint16), L.mask,
                         want, C.byref(d), np.float32(1.0 / s.hd ** 0.5))
    assert kq.rel_diff(L.get("attn", np.float32), want) < 2e-6
    be.close()
    L.free()


@pytest.mark.parametrize("attn_path", [2, 3], ids=["one-head", "gqa"])
@pytest.mark.parametrize("p0", [64, 62], ids=["rows16B", "rows4B"])
def test_batch_attention_with_a_window_mask(p0, attn_path):
    """A sliding-window mask (each query sees its last 70 positions) over 192 queries: the later
    query tiles see none of the first key blocks, which the kernels then do not load; one query of a
    later tile also sees key 3 (its tile keeps every block from 0 on), and one row holds a finite
    penalty. Mask rows of 256 halves (16-byte loads in the kernels' scan of the mask) and of 254
    (4-byte loads); both kernels; against the oracle on the GPU's own inputs."""
    shape = gg.LayerShape(n_embd=1024, neox=True, kv_size=256)
    N = 192
    kc.set_option("attn_path", attn_path)
    try:
        L = Layer(shape, N, p0, seed=931)
        n_pad = L.t["mask"].ne[0]
        assert n_pad == p0 + N and (n_pad % 8 == 0) == (p0 == 64)
        key = np.arange(n_pad)[None, :]
        pos = p0 + np.arange(N)[:, None]
        m = np.where((key <= pos) & (key > pos - 70), 0.0, -np.inf).astype(np.float16)
        m[150, 3] = 0.0
        m[120, pos[120, 0] - 10] = np.float16(-1.5)
        _masked_case(L, N, m)
    finally:
        kc.set_option("attn_path", 0)


def test_batch_attention_past_the_score_limit():
    """A prompt whose score matrix passes 2^24 values (32 heads x 1024 tokens x 1024 keys, as BASELINE
    config 5's prompt): claimed because it runs on the masked matrix-core kernel, which keeps no score
    matrix; against the oracle on the GPU's own inputs (causal mask with a block of holes)."""
    shape = gg.LayerShape(n_embd=2048, n_head=32, n_head_kv=8, head_dim=64, n_ff=1024, kv_size=1024)
    N, p0 = 1024, 0
    note("ggml attention past the score limit: 32 heads, 1024 tokens")
    L = Layer(shape, N, p0, seed=929)
    names, _ = kc.ggml_graph_plan(L.g.nodes, attn_tokens=N)
    assert "attn_masked" in names
    n_pad = L.t["mask"].ne[0]
    m = L.mask.view(np.float16).reshape(N, n_pad).copy()
    m[600:700, 100:164] = -np.inf
    L.mask = m.reshape(-1).view(np.uint16)
    L.put("mask", L.mask)
    be = kc.GgmlBackend(graphs=0, attn_tokens=N)
    be.compute(L.g.nodes)
    kc.synchronize()
    s = L.s
    d = oracle.FaDims(H=s.n_head, T=L.n_kv, D=s.hd, group=s.n_head // s.n_head_kv, tp=(L.n_kv + 7) // 8 * 8,
                      k_row=s.kv_dim // 2, k_head=s.hd // 2, v_row=s.kv_dim // 2, v_head=s.hd // 2, N=N,
                      q_tok=s.hd * s.n_head, q_head=s.hd, m_row=n_pad // 2, has_mask=1, H_kv=s.n_head_kv)
    assert s.n_head * N * d.tp >= 1 << 24
    want = np.zeros(N * s.n_head * s.hd, np.float32)
    O.kco_flash_attn_f16(L.get("qr", np.float32), L.get("k_cache", np.uint16), L.get("v_cache", np.uint16), L.mask,
                         want, C.byref(d), np.float32(1.0 / s.hd ** 0.5))
    assert kq.rel_diff(L.get("attn", np.float32), want) < 2e-6
    be.close()
    L.free()


def test_kept_graph_is_launched_again_for_new_inputs():
    shape, N, p0 = gg.LayerShape(), 8, 100
    note(f"ggml graph reuse: N={N}, p0={p0}")
    L = Layer(shape, N, p0, seed=500)
    graph_be, eager_be = kc.GgmlBackend(graphs=1), kc.GgmlBackend(graphs=0)
    nodes = kc.GgmlNodes(L.g.nodes)  # the node array built once
    for trial in range(3):
        L.set_x(600 + trial)  # new values at the same addresses
        graph_be.compute(nodes)
        got = L.get("out", np.float32)
        kc.synchronize()
        eager_be.compute(L.g.nodes)
        want = L.get("out", np.float32)
        assert np.array_equal(kq.bits(got), kq.bits(want)), trial
        if trial:
            assert not np.array_equal(kq.bits(got), kq.bits(prev)), "the output follows the input"
        prev = got
    st = graph_be.stats()
    assert (st["computes"], st["graphs_recorded"], st["graphs_reused"]) == (3, 1, 2)
    # the same node array with one src link moved (the attention norm's MUL now reads the FFN norm's
    # weight): recorded again, not the kept graph launched
    mul = next(t for t in L.g.nodes if t.op == kc.GGML_OP["mul"] and
               C.addressof(t.src[1].contents) == C.addressof(L.t["attn_norm"]))
    mul.src[1] = C.pointer(L.t["ffn_norm"])
    graph_be.compute(nodes)
    got = L.get("out", np.float32)
    kc.synchronize()
    eager_be.compute(L.g.nodes)
    assert np.array_equal(kq.bits(got), kq.bits(L.get("out", np.float32)))
    assert not np.array_equal(kq.bits(got), kq.bits(prev))
    st = graph_be.stats()
    assert (st["computes"], st["graphs_recorded"], st["graphs_reused"]) == (4, 2, 2)
    graph_be.compute(nodes)  # and that graph kept in turn
    assert graph_be.stats()["graphs_reused"] == 3
    # another node list (the attention of one more token): recorded again
    L2 = Layer(shape, N, p0 + 1, seed=500)
    graph_be.compute(L2.g.nodes)
    assert graph_be.stats()["graphs_recorded"] == 3
    for b in (graph_be, eager_be):
        b.close()
    L.free()
    L2.free()


SHARED = [
    ("decode", gg.LayerShape(), 1, 40, {}, ()),
    ("decode, roped q and k graph outputs", gg.LayerShape(), 1, 40, {}, ("qr", "kr")),
    ("decode, qwen3 q / k norm", gg.LayerShape(n_embd=1024, n_head=8, n_head_kv=2, head_dim=128, neox=True,
                                              qk_norm=True), 1, 70, {}, ()),
    ("decode, qwen3, normed q graph output", gg.LayerShape(n_embd=1024, n_head=8, n_head_kv=2, head_dim=128, neox=True,
                                                           qk_norm=True), 1, 70, {}, ("qn",)),
    ("batch of 8", gg.LayerShape(), 8, 100, {}, ()),
    ("batch of 64 (MFMA matmuls, masked attention)", gg.LayerShape(), 64, 64, dict(attn_tokens=64), ()),
]


@pytest.mark.parametrize("graphs", [1, 0])
@pytest.mark.parametrize("case", SHARED, ids=[c[0] for c in SHARED])
def test_layer_with_shared_memory_equals_distinct_memory(case, graphs):
    """The layer with its nodes placed as ggml's allocator places them (freed memory reused best
    fit, ROPE / RMS_NORM / MUL / ADD in place over the parent they read last) against the same layer
    with a block of its own per tensor: the layer output and both caches bit-identical. With the
    memory shared, a cache of quantized inputs keyed by data pointer hands the o projection another
    tensor's slots, and fused launches whose workgroups write one tensor while others read its
    in-place parent race; both are what this checks."""
    name, shape, N, p0, cfg, outs = case
    note(f"ggml layer, shared memory: {name}, graphs={graphs}")
    got = {}
    for share in (True, False):
        L = Layer(shape, N, p0, seed=1300 + N, share=share, outputs=outs)
        if share:
            assert L.t["cur"].data == L.t["norm"].data
            assert (L.t["qr"].data == L.t["q"].data) == (shape.qk_norm == 0 or "qn" not in outs)
            if N == 64:
                assert L.t["attn"].data == L.t["cur"].data  # the attention output on the normed rows
        be = kc.GgmlBackend(graphs=graphs, **cfg)
        be.compute(L.g.nodes)
        kc.synchronize()
        got[share] = [L.get("out", np.float32).view(np.uint32), L.get("k_cache", np.uint16),
                      L.get("v_cache", np.uint16)] + [L.get(n, np.float32).view(np.uint32) for n in outs]
        be.close()
        L.free()
    for a, b, what in zip(got[True], got[False], ("out", "k_cache", "v_cache") + outs):
        assert np.array_equal(a, b), what


def test_profile_times_calls_and_launches():
    """GGML_KERNELCORE_PROFILE (ggml-kernelcore.cpp:331-346, 400-415, 1033-1035): with 1 each call's
    compute, recording and run times add up in the stats; with 2 every launch is also timed on the
    device (one by one), per kernel name and MUL_MAT weight shape, and the results are those of the
    untimed backend bit for bit."""
    L = Layer(gg.LayerShape(), 1, 40, seed=1700)
    plain = kc.GgmlBackend(graphs=1)
    plain.compute(L.g.nodes)
    want = L.get("out", np.float32)
    assert plain.stats()["compute_ms"] == 0.0  # profile off: nothing timed
    plain.close()
    be1 = kc.GgmlBackend(graphs=1, profile=1)
    for _ in range(3):
        be1.compute(L.g.nodes)
    st = be1.stats()
    assert st["graphs_recorded"] == 1 and st["graphs_reused"] == 2
    assert st["compute_ms"] > 0 and st["run_ms"] > 0 and st["record_ms"] > 0
    assert st["record_ms"] + st["run_ms"] <= st["compute_ms"] * 1.001 + 1e-3
    assert be1.profile() == {}
    be1.close()
    be2 = kc.GgmlBackend(graphs=1, profile=2)
    for _ in range(2):
        be2.compute(L.g.nodes)
    assert np.array_equal(kq.bits(L.get("out", np.float32)), kq.bits(want))
    st, prof = be2.stats(), be2.profile()
    assert st["graphs_recorded"] == 0 and st["computes"] == 2
    names, _ = kc.ggml_graph_plan(L.g.nodes)
    s = L.s
    assert sum(n for n, _ in prof.values()) == 2 * len([n for n in names if n not in "[]"])
    assert prof[f"decode_norm_matvec {s.q_dim}x{s.n_embd}"][0] == 2
    assert prof[f"decode_norm_swiglu {s.n_ff}x{s.n_embd}"][0] == 2
    assert all(ms > 0 for _, ms in prof.values())
    be2.close()
    L.free()


def test_unclaimed_node_is_refused_before_any_launch():
    L = Layer(gg.LayerShape(), 9, 10, seed=700)  # 9 tokens: attention beyond attn_tokens
    be = kc.GgmlBackend()
    out_before = L.get("out", np.float32)
    with pytest.raises(kc.KcError) as e:
        be.compute(L.g.nodes)
    assert e.value.name == "UnsupportedOperation"
    assert np.array_equal(kq.bits(L.get("out", np.float32)), kq.bits(out_before))
    assert be.stats()["computes"] == 0
    be.close()
    L.free()


# ---- a whole decoder through the backend against the model driver ---------------------------------

LLAMA = dict(n_layer=2, n_embd=512, n_head=8, n_head_kv=2, head_dim=64, n_ff=1024, n_vocab=1024, norm_eps=1e-5,
             rope_theta=500000.0, rope_neox=0, qk_norm=0, max_ctx=256, max_batch=128)
QWEN = dict(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, head_dim=128, n_ff=768, n_vocab=1536, norm_eps=1e-6,
            rope_theta=1000000.0, rope_neox=1, qk_norm=1, max_ctx=256, max_batch=128)
LAYER_IDS = dict(attn_norm=3, wq=4, wk=5, wv=6, wo=7, ffn_norm=8, wg=9, wu=10, wd=11, q_norm=12, k_norm=13)


class BackendDecoder:
    """The model's weights in the backend's buffers (kcWeightSetTensor) and its KV caches; step(tokens)
    builds llama.cpp's graph for those tokens at the current position and runs kcGgmlGraphCompute."""

    def __init__(self, cfg, weights, be, share=False):
        self.cfg, self.be, self.share = cfg, be, share
        self.s = gg.LayerShape.of_model(cfg, cfg["max_ctx"])
        self.bufs = []
        wg = gg.Graph(self._alloc)
        self.W = {"layers": [gg.layer_weights(wg, self.s) for _ in range(cfg["n_layer"])],
                  "output_norm": wg.leaf("f32", [self.s.n_embd], buffer="weights"),
                  "output": wg.leaf("q6k", [self.s.n_embd, self.s.n_vocab], buffer="weights")}
        self.keep = wg
        for l, lw in enumerate(self.W["layers"]):
            for name, tid in LAYER_IDS.items():
                if name in lw:
                    self._set(lw[name], weights[(tid, l)])
            for c in ("k_cache", "v_cache"):
                kc.call("kcMemset", lw[c].data, 0, self.s.kv_dim * self.s.kv_size * 2)
        self._set(self.W["output_norm"], weights[(1, -1)])
        self._set(self.W["output"], weights[(2, -1)])
        self.embd = oracle.dequant(O, "q4k", weights[(0, -1)], cfg["n_vocab"], cfg["n_embd"]).reshape(
            cfg["n_vocab"], cfg["n_embd"])
        self.pos = 0

    def _alloc(self, nbytes, type_, ne):
        if type_ in ("q4k", "q6k"):
            nbytes = kc.weight_alloc_size(type_, ne[1], ne[0])
        b = kc.Buffer(nbytes)
        self.bufs.append(b)
        return b.ptr

    def _set(self, t, data):
        names = {v: k for k, v in kc.GGML_TYPE.items()}
        qt = names[t.type]
        if qt in ("q4k", "q6k"):
            kc.weight_set(qt, t.ne[1], t.ne[0], t.data, data)
        else:
            a = np.ascontiguousarray(data)
            kc.call("kcMemcpy", t.data, a.ctypes.data, a.nbytes, kc.HOST_TO_DEVICE)

    def step(self, tokens):
        N, p0 = len(tokens), self.pos
        n_kv = p0 + N
        step_bufs = len(self.bufs)
        g = gg.Graph(self._alloc)
        io, _, _, logits = gg.decoder(g, self.s, self.cfg["n_layer"], N, n_kv, weights=self.W)
        if self.share:  # the step's nodes placed as ggml's allocator places them
            gg.share_memory(g, lambda n: self._alloc(n, "f32", [n // 4]))
        put = lambda t, a: kc.call("kcMemcpy", t.data, np.ascontiguousarray(a).ctypes.data, a.nbytes,
                                   kc.HOST_TO_DEVICE)
        put(io["x"], self.embd[np.asarray(tokens)].astype(np.float32))
        pos = np.arange(p0, p0 + N, dtype=np.int32)
        put(io["pos"], pos)
        put(io["kv_idx"], pos.astype(np.int64))
        m = np.full((N, io["mask"].ne[0]), -np.inf, np.float16)
        for i in range(N):
            m[i, :p0 + i + 1] = 0.0
        put(io["mask"], m)
        self.be.compute(g.nodes)
        out = np.empty(self.s.n_vocab, np.float32)  # the last token's logits
        kc.call("kcMemcpy", out.ctypes.data, logits.data, out.nbytes, kc.DEVICE_TO_HOST)
        for b in self.bufs[step_bufs:]:
            b.free()
        del self.bufs[step_bufs:]
        self.pos += N
        return out

    def free(self):
        for b in self.bufs:
            b.free()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / np.linalg.norm(b)


@pytest.mark.parametrize("share", [False, True], ids=["distinct-memory", "shared-memory"])
@pytest.mark.parametrize("name,cfg", [("llama", LLAMA), ("qwen3", QWEN)])
def test_decoder_graph_matches_the_model_driver(name, cfg, share):
    """Two layers, the output norm and the head as llama.cpp's graph through kcGgmlGraphCompute,
    against kcModelForward and the oracle model on the same weights (N(0, 0.02) quantized as ggml
    does): a 20-token prompt in steps of up to 8 tokens (the backend's attention batch), then 4
    single tokens. The paths sum attention in different orders, and a per-32 activation that sits
    on a rounding tie flips one 8-bit value on an ulp of difference: in the Qwen3 case the second
    decode step is such a step (the oracle itself moves by 2.7e-3 when its attention output is
    perturbed by one ulp; the driver lands there, the backend not). So the bar is the model tests'
    -- 1e-2 relative L2 on the logits, the q8 activation noise -- and the same greedy token;
    typical steps agree to 2e-7. shared-memory: each step's nodes placed as ggml's allocator
    places them (gg.share_memory)."""
    from tests.model_weights import quantized_weights
    note(f"ggml decoder vs model driver: {name}")
    w = quantized_weights(cfg, 11)
    m = kc.Model(**cfg)
    for (tid, layer), data in w.items():
        m.set_tensor(tid, layer, data)
    be = kc.GgmlBackend()
    d = BackendDecoder(cfg, w, be, share=share)
    o = OracleModel(cfg, w)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg["n_vocab"], 20).astype(np.int32)
    want = m.forward(prompt)
    ref = o.forward(prompt)
    for i in range(0, 20, 8):
        got = d.step(prompt[i:i + 8])
    note(f"  prompt: rel L2 {rel_l2(got, want):.2e} (vs the oracle: backend {rel_l2(got, ref):.2e}, "
         f"driver {rel_l2(want, ref):.2e})")
    assert rel_l2(got, want) < 1e-2 and rel_l2(got, ref) < 1e-2 and int(np.argmax(got)) == int(np.argmax(want))
    for step in range(4):
        t = int(np.argmax(want))
        want = m.forward([t])
        ref = o.forward([t])
        got = d.step([t])
        note(f"  decode {step}: rel L2 {rel_l2(got, want):.2e} (vs the oracle: backend {rel_l2(got, ref):.2e}, "
             f"driver {rel_l2(want, ref):.2e})")
        assert rel_l2(got, want) < 1e-2 and rel_l2(got, ref) < 1e-2 and int(np.argmax(got)) == int(np.argmax(want))
    st = be.stats()
    assert st["computes"] == 7 and st["graphs_recorded"] == 7  # every step a new node list (n_kv grows)
    be.close()
    d.free()
    m.close()
