"""ggml-shaped graphs of kcGgmlTensor descriptors (include/kernelcore/ggml_backend.h), to drive the
backend core from Python (its tests and the bench): tensors follow ggml's conventions (ne[0] the
fastest dimension, nb in bytes, views share their source's memory), ops get ggml's result shapes
and op_params layout, and `finish` fills the use counts and output flags a ggml_cgraph would carry.

`llama_layer` builds one transformer layer the way llama.cpp's graph does with flash attention
on (the attention block: RMS_NORM + MUL, MUL_MAT q/k/v, RESHAPE, ROPE, SET_ROWS of k and v into
the fp16 KV cache, VIEWs of the cache, PERMUTE of q, FLASH_ATTN_EXT, MUL_MAT o, ADD; the FFN:
RMS_NORM + MUL, MUL_MAT gate/up, GLU SWIGLU, MUL_MAT down, ADD) -- the node order of
/root/reference/docs/cuda_cpu_poc_plan.md:1156-1158 and llm/llm_model.cpp:287-360.

With no allocator every tensor gets a distinct fake address (for plans, which never touch
memory); with one (called with the ggml byte size, type and ne), every non-view tensor gets the
memory it returns. `Graph.share_memory` then places the computed nodes as ggml's graph allocator
does (ggml-alloc.c: freed tensors' memory reused best-fit, elementwise ops run in place over a parent
whose last use they are), so that tests see the aliasing a llama.cpp build hands the backend."""
import ctypes as C
import struct

import kernelcore_amd as kc

SIZE = {"f32": 4, "f16": 2, "i32": 4, "i64": 8}
BLOCK = {"q4k": (256, 144), "q6k": (256, 210)}


def f32bits(v):
    return struct.unpack("<i", struct.pack("<f", float(v)))[0]


def packed_nb(type_, ne):
    blck, size = BLOCK.get(type_, (1, SIZE.get(type_, 4)))
    nb = [size, size * (ne[0] // blck)]
    for d in range(2, 4):
        nb.append(nb[-1] * ne[d - 1])
    return nb


class Graph:
    def __init__(self, alloc=None):
        self.alloc = alloc
        self.fake = 1 << 20
        self.nodes = []
        self.keep = []
        self.srcs = {}  # id(tensor) -> [src tensors]
        self.view_of = {}  # id(view) -> (base tensor, byte offset): ggml's view_src and view_offs

    def _memory(self, nbytes, type_, ne):
        if self.alloc is None:
            p = self.fake
            self.fake += (nbytes + 255) // 256 * 256 + 256
            return p
        return self.alloc(nbytes, type_, ne)

    def tensor(self, op, type_, ne, srcs=(), params=(), nb=None, data=None, buffer="other", view=False,
               compute=False, view_src=None):
        ne = list(ne) + [1] * (4 - len(ne))
        nb = list(nb) if nb is not None else packed_nb(type_, ne)
        t = kc.GgmlTensor()
        t.op, t.type = kc.GGML_OP[op], kc.GGML_TYPE[type_]
        for d in range(4):
            t.ne[d], t.nb[d] = ne[d], nb[d]
        nbytes = nb[3] * ne[3]
        t.data = data if data is not None else self._memory(max(nbytes, 4), type_, ne)
        for i, s in enumerate(srcs):
            if s is not None:
                t.src[i] = C.pointer(s)
        for i, p in enumerate(params):
            t.op_params[i] = p
        t.buffer, t.view, t.compute = kc.GGML_BUFFER[buffer], int(view), int(compute)
        self.keep.append(t)
        self.srcs[id(t)] = [s for s in srcs if s is not None]
        if view:  # the base is never itself a view (ggml folds view chains into view_src)
            base = self.view_of.get(id(view_src or srcs[0]), (view_src or srcs[0], 0))[0]
            self.view_of[id(t)] = (base, t.data - base.data)
        return t

    def leaf(self, type_, ne, buffer="other"):
        return self.tensor("none", type_, ne, buffer=buffer)

    def node(self, *a, **k):
        t = self.tensor(*a, compute=True, **k)
        self.nodes.append(t)
        return t

    # ---- ops (ggml result shapes and op_params) ----
    def rms_norm(self, x, eps):
        return self.node("rms_norm", "f32", x.ne, [x], [f32bits(eps)])

    def mul(self, a, b):
        return self.node("mul", "f32", a.ne, [a, b])

    def add(self, a, b):
        return self.node("add", "f32", a.ne, [a, b])

    def mul_mat(self, w, x):
        return self.node("mul_mat", "f32", [w.ne[1], x.ne[1], x.ne[2], x.ne[3]], [w, x])

    def reshape(self, t, ne):
        return self.node("reshape", _tname(t), ne, [t], data=t.data, buffer=_bname(t), view=True)

    def view(self, t, ne, nb, offset=0):
        return self.node("view", _tname(t), ne, [t], nb=list(nb), data=t.data + offset, buffer=_bname(t), view=True)

    def permute(self, t, axes):
        ne, nb = [0] * 4, [0] * 4
        for i, a in enumerate(axes):
            ne[a], nb[a] = t.ne[i], t.nb[i]
        return self.node("permute", _tname(t), ne, [t], nb=nb, data=t.data, buffer=_bname(t), view=True)

    def rope(self, x, pos, n_dims, neox, freq_base, ff=None, p15=0, freq_scale=1.0, ext_factor=0.0,
             attn_factor=1.0):
        params = [0, n_dims, 2 if neox else 0, 0, 0, f32bits(freq_base), f32bits(freq_scale), f32bits(ext_factor),
                  f32bits(attn_factor), f32bits(32.0), f32bits(1.0)] + [0] * 4 + [p15]
        return self.node("rope", "f32", x.ne, [x, pos, ff], params)

    def set_rows(self, dst, src, idx):
        return self.node("set_rows", _tname(dst), dst.ne, [src, idx], nb=list(dst.nb), data=dst.data,
                         buffer=_bname(dst), view=True, view_src=dst)

    def flash_attn_ext(self, q, k, v, mask, scale, max_bias=0.0, softcap=0.0):
        return self.node("flash_attn_ext", "f32", [v.ne[0], q.ne[2], q.ne[1], q.ne[3]], [q, k, v, mask],
                         [f32bits(scale), f32bits(max_bias), f32bits(softcap)])

    def swiglu(self, g, u, op=2, swapped=0):
        return self.node("glu", "f32", g.ne, [g, u], [op, swapped])

    def finish(self, outputs=()):
        """Use counts (how many nodes read each node) and output flags, as ggml_cgraph keeps them."""
        uses = {}
        for t in self.nodes:
            for s in self.srcs[id(t)]:
                uses[id(s)] = uses.get(id(s), 0) + 1
        for t in self.nodes:
            t.uses = uses.get(id(t), 0)
        for t in outputs:
            t.output = 1
        return self.nodes


INPLACE_OPS = ("add", "mul", "rms_norm", "rope")  # ggml_op_can_inplace, for the ops built here


def share_memory(g, alloc, align=64, inplace_views=True):
    """Places g's computed non-view nodes (g.finish first) in one arena as ggml_gallocr does: nodes in
    order; a node of an op that can run in place takes the memory of a parent whose last remaining
    use it is (not an output, the same layout, no view of it left); else the best-fitting freed
    block, else new memory at the end; a tensor's memory is freed after its last reader (and the last
    reader of its views) ran, outputs never. inplace_views: a parent that is a view of offset 0 (a
    RESHAPE of a MUL_MAT output) is taken over too, with its base (the variant that shares the most
    memory). alloc(nbytes) gives the arena; views then follow their bases. Leaves keep their memory.
    Returns the arena size."""
    base_of = lambda t: g.view_of.get(id(t), (t, 0))[0]
    children, views = {}, {}
    for t in g.nodes:
        if t.view:
            b = base_of(t)
            views[id(b)] = views.get(id(b), 0) + 1
        for s in g.srcs[id(t)]:
            children[id(s)] = children.get(id(s), 0) + 1
    addr, live, free, top = {}, set(), [], 0  # free: [offset, size] blocks, merged when adjacent
    nbytes = lambda t: (max(t.nb[3] * t.ne[3], 4) + align - 1) // align * align
    layout = lambda t: (t.type, tuple(t.ne), tuple(t.nb))
    owner = {}  # id(node) -> the node whose block it holds (itself, or an in-place parent's)

    def release(t):
        if t.output or id(t) not in live:
            return
        live.discard(id(t))
        free.append([addr[id(t)], nbytes(owner[id(t)])])
        free.sort()
        merged = []
        for b in free:
            if merged and merged[-1][0] + merged[-1][1] == b[0]:
                merged[-1][1] += b[1]
            else:
                merged.append(b)
        free[:] = merged

    def in_place(t):
        if kc_op_name(t) not in INPLACE_OPS:
            return None
        for p in g.srcs[id(t)]:
            q = base_of(p)
            if id(q) not in live or q.output or layout(p) != layout(t) or children.get(id(p), 0) != 1:
                continue
            if not p.view and not views.get(id(p), 0):
                return p
            if p.view and inplace_views and views.get(id(q), 0) == 1 and not children.get(id(q), 0) and \
                    p.data == q.data:
                return q
        return None

    for t in g.nodes:
        if not t.view:
            q = in_place(t)
            if q is not None:  # t takes over q's block; q is never freed
                live.discard(id(q))
                addr[id(t)], owner[id(t)] = addr[id(q)], owner[id(q)]
            else:
                n = nbytes(t)
                fits = [b for b in free if b[1] >= n]
                if fits:
                    b = min(fits, key=lambda b: b[1])
                    addr[id(t)] = b[0]
                    b[0] += n
                    b[1] -= n
                    if not b[1]:
                        free.remove(b)
                else:
                    addr[id(t)] = top
                    top += n
                owner[id(t)] = t
            live.add(id(t))
        for s in g.srcs[id(t)]:
            children[id(s)] -= 1
            if children[id(s)]:
                continue
            if s.view:
                b = base_of(s)
                views[id(b)] -= 1
                if not views[id(b)] and not children.get(id(b), 0):
                    release(b)
            elif not views.get(id(s), 0):
                release(s)
    arena = alloc(max(top, 4))
    for t in g.nodes:
        if not t.view:
            t.data = arena + addr[id(t)]
    for t in g.nodes:  # views follow their bases (in node order: a base comes before its views)
        if t.view:
            b, o = g.view_of[id(t)]
            t.data = b.data + o
    return top


def kc_op_name(t):
    return {v: k for k, v in kc.GGML_OP.items()}[t.op]


def _tname(t):
    return {v: k for k, v in kc.GGML_TYPE.items()}[t.type]


def _bname(t):
    return {v: k for k, v in kc.GGML_BUFFER.items()}[t.buffer]


class LayerShape:
    def __init__(self, n_embd=512, n_head=8, n_head_kv=2, n_ff=1024, kv_size=512, eps=1e-5, base=500000.0,
                 neox=False, wq="q4k", wk="q4k", wv="q6k", wo="q4k", wg="q4k", wu="q4k", wd="q6k", freq_factors=False,
                 head_dim=None, qk_norm=False, n_vocab=0):
        self.n_embd, self.n_head, self.n_head_kv, self.n_ff = n_embd, n_head, n_head_kv, n_ff
        self.hd = head_dim or n_embd // n_head
        self.q_dim = self.hd * n_head
        self.kv_dim = self.hd * n_head_kv
        self.kv_size, self.eps, self.base, self.neox = kv_size, eps, base, neox
        self.types = dict(wq=wq, wk=wk, wv=wv, wo=wo, wg=wg, wu=wu, wd=wd)
        self.freq_factors, self.qk_norm, self.n_vocab = freq_factors, qk_norm, n_vocab

    @classmethod
    def of_model(cls, cfg, kv_size):
        """The shape of a kc.Model config dict (n_layer, n_embd, n_head, ...)."""
        return cls(n_embd=cfg["n_embd"], n_head=cfg["n_head"], n_head_kv=cfg["n_head_kv"], n_ff=cfg["n_ff"],
                   kv_size=kv_size, eps=cfg["norm_eps"], base=cfg["rope_theta"], neox=bool(cfg["rope_neox"]),
                   head_dim=cfg["head_dim"], qk_norm=bool(cfg["qk_norm"]), n_vocab=cfg["n_vocab"])


def inputs(g, s, n_tokens, n_kv):
    """The graph inputs of a step over n_tokens tokens attending over n_kv cache rows: the token
    embeddings (GET_ROWS runs on the CPU backend, which hands its output over), the positions, the
    cache rows the new keys go to, and the f16 causal mask (rows padded to an even count)."""
    N = n_tokens
    t = {"x": g.leaf("f32", [s.n_embd, N]), "pos": g.leaf("i32", [N]), "kv_idx": g.leaf("i64", [N]),
         "mask": g.leaf("f16", [(n_kv + 1) // 2 * 2, N])}
    t["ff"] = g.leaf("f32", [s.hd // 2]) if s.freq_factors else None
    return t


def layer_weights(g, s):
    """One layer's weights (the backend's weight buffers) and its fp16 K / V caches (its KV buffers)."""
    t = {}
    for name, (rows, k) in dict(wq=(s.q_dim, s.n_embd), wk=(s.kv_dim, s.n_embd), wv=(s.kv_dim, s.n_embd),
                                wo=(s.n_embd, s.q_dim), wg=(s.n_ff, s.n_embd), wu=(s.n_ff, s.n_embd),
                                wd=(s.n_embd, s.n_ff)).items():
        t[name] = g.leaf(s.types[name], [k, rows], buffer="weights")
    t["attn_norm"] = g.leaf("f32", [s.n_embd], buffer="weights")
    t["ffn_norm"] = g.leaf("f32", [s.n_embd], buffer="weights")
    if s.qk_norm:
        t["q_norm"] = g.leaf("f32", [s.hd], buffer="weights")
        t["k_norm"] = g.leaf("f32", [s.hd], buffer="weights")
    t["k_cache"] = g.leaf("f16", [s.kv_dim, s.kv_size], buffer="kv")
    t["v_cache"] = g.leaf("f16", [s.kv_dim, s.kv_size], buffer="kv")
    return t


def layer(g, s, x, io, w, n_tokens, n_kv, last_only=False):
    """One transformer layer on x (a [n_embd, N] tensor) in llama.cpp's order; returns its nodes.
    last_only: the output-row selection of the last layer (llama.cpp's GET_ROWS of the output rows,
    which the CPU backend runs; here a view of the last row): after the attention projection only
    the last token's row continues through the residual ADD and the FFN."""
    N, t = n_tokens, dict(w)
    t["norm"] = g.rms_norm(x, s.eps)
    t["cur"] = g.mul(t["norm"], w["attn_norm"])
    t["q"] = g.mul_mat(w["wq"], t["cur"])
    t["k"] = g.mul_mat(w["wk"], t["cur"])
    t["v"] = g.mul_mat(w["wv"], t["cur"])
    t["q3"] = g.reshape(t["q"], [s.hd, s.n_head, N])
    t["k3"] = g.reshape(t["k"], [s.hd, s.n_head_kv, N])
    q3, k3 = t["q3"], t["k3"]
    if s.qk_norm:  # Qwen3: RMS norm of each head's q and k with their own weights, before RoPE
        t["qn"] = g.mul(g.rms_norm(q3, s.eps), w["q_norm"])
        t["kn"] = g.mul(g.rms_norm(k3, s.eps), w["k_norm"])
        q3, k3 = t["qn"], t["kn"]
    t["qr"] = g.rope(q3, io["pos"], s.hd, s.neox, s.base, io["ff"])
    t["kr"] = g.rope(k3, io["pos"], s.hd, s.neox, s.base, io["ff"])
    t["kr2"] = g.reshape(t["kr"], [s.kv_dim, N])
    t["k_set"] = g.set_rows(w["k_cache"], t["kr2"], io["kv_idx"])
    t["v_set"] = g.set_rows(w["v_cache"], t["v"], io["kv_idx"])
    row = s.kv_dim * 2
    t["k_view"] = g.view(t["k_set"], [s.hd, n_kv, s.n_head_kv, 1], [2, row, s.hd * 2, row * n_kv])
    t["v_view"] = g.view(t["v_set"], [s.hd, n_kv, s.n_head_kv, 1], [2, row, s.hd * 2, row * n_kv])
    t["q_perm"] = g.permute(t["qr"], [0, 2, 1, 3])
    t["attn"] = g.flash_attn_ext(t["q_perm"], t["k_view"], t["v_view"], io["mask"], 1.0 / s.hd ** 0.5)
    t["attn2"] = g.reshape(t["attn"], [s.q_dim, N])
    t["o"] = g.mul_mat(w["wo"], t["attn2"])
    o, res = t["o"], x
    if last_only and N > 1:
        row = s.n_embd * 4
        o = t["o_last"] = g.view(t["o"], [s.n_embd, 1], [4, row, row, row], (N - 1) * row)
        res = t["x_last"] = g.view(x, [s.n_embd, 1], [4, row, row, row], (N - 1) * row)
    t["ffn_inp"] = g.add(o, res)
    t["norm2"] = g.rms_norm(t["ffn_inp"], s.eps)
    t["cur2"] = g.mul(t["norm2"], w["ffn_norm"])
    t["gate"] = g.mul_mat(w["wg"], t["cur2"])
    t["up"] = g.mul_mat(w["wu"], t["cur2"])
    t["act"] = g.swiglu(t["gate"], t["up"])
    t["down"] = g.mul_mat(w["wd"], t["act"])
    t["out"] = g.add(t["down"], t["ffn_inp"])
    return t


def llama_layer(g, s, n_tokens, n_kv):
    """One layer over n_tokens new tokens whose keys go to the cache rows given by `kv_idx`,
    attending over the first n_kv rows of the cache. Returns the named tensors (leaves and nodes)."""
    io = inputs(g, s, n_tokens, n_kv)
    w = layer_weights(g, s)
    t = layer(g, s, io["x"], io, w, n_tokens, n_kv)
    t.update(io)
    g.finish(outputs=[t["out"]])
    return t


def decoder(g, s, n_layer, n_tokens, n_kv, weights=None):
    """n_layer layers, the output norm and the head (the last token's logits, [n_vocab, 1]: the last
    layer keeps only the output row after its attention, as llama.cpp does); weights: an optional
    dict of layer_weights ("layers") and the "output_norm" / "output" leaves to build the step over
    existing weights and caches. Returns (io, weights, layers, logits)."""
    io = inputs(g, s, n_tokens, n_kv)
    if weights is None:
        weights = {"layers": [layer_weights(g, s) for _ in range(n_layer)],
                   "output_norm": g.leaf("f32", [s.n_embd], buffer="weights"),
                   "output": g.leaf("q6k", [s.n_embd, s.n_vocab], buffer="weights")}
    x, layers = io["x"], []
    for l in range(n_layer):
        t = layer(g, s, x, io, weights["layers"][l], n_tokens, n_kv, last_only=l == n_layer - 1)
        layers.append(t)
        x = t["out"]
    norm = g.rms_norm(x, s.eps)
    cur = g.mul(norm, weights["output_norm"])
    logits = g.mul_mat(weights["output"], cur)
    g.finish(outputs=[logits])
    return io, weights, layers, logits
