"""A float64 textbook Llama / Qwen3 forward, written from the architecture's mathematics and not
from the oracle's code: test infrastructure that pins oracle/model.py (OracleModel).

It shares no code with the oracle or the GPU driver. The weights are dequantized here with ggml's
block formulas in float64 (dequantize_row_q4_K / q6_K, restated vectorised), and every operation
runs on exact float64 activations: no 8-bit activation quantization, no fp16 KV cache, no fused
kernels, no KV cache at all (causal attention over the whole sequence at once). What it computes,
per token t of the sequence and layer l (the reference's decode step, llm/llm_model.cpp:287-360,
in the ggml graph order of docs/cuda_cpu_poc_plan.md:1156-1158):

    h   = rmsnorm(x) * attn_norm                 rmsnorm(v) = v / sqrt(mean(v^2) + eps)
    q, k, v = Wq h, Wk h, Wv h
    (Qwen3) q, k = per-head rmsnorm(q) * q_norm, rmsnorm(k) * k_norm
    q, k = rope(q, t), rope(k, t)                NORM pairs (2i, 2i+1), NEOX pairs (i, i + D/2),
                                                 angle t * base^(-2i/D) / freq_factor[i]
    a_h = sum_s<=t softmax_s(q_h . k_{g(h),s} / sqrt(D)) v_{g(h),s},   g(h) = h // (H / H_kv)
    x   = x + Wo a
    x   = x + Wdown (silu(Wgate h2) * Wup h2),   h2 = rmsnorm(x) * ffn_norm
    logits = Wout (rmsnorm(x) * output_norm)

Differences from OracleModel are therefore the 8-bit activation and fp16 cache rounding only,
which the 1e-2 relative-L2 bar of the north star covers; a wiring mistake (a head mapping, a
swapped norm, a dropped residual, a rotated pair) moves the logits far more."""
from __future__ import annotations

import numpy as np

Q4K, Q6K, F32, F16 = 12, 14, 0, 1


def _f16(b):
    return np.ascontiguousarray(b).view(np.float16).astype(np.float64).reshape(-1)


def dequant_q4k(blocks):
    """[nblk, 144] uint8 -> [nblk, 256] float64 (ggml dequantize_row_q4_K)."""
    b = blocks.reshape(-1, 144)
    d, dmin = _f16(b[:, 0:2]), _f16(b[:, 2:4])
    sc = b[:, 4:16].astype(np.int64)
    qs = b[:, 16:144].astype(np.int64)
    out = np.empty((b.shape[0], 256))
    for j in range(8):
        if j < 4:
            s, m = sc[:, j] & 63, sc[:, j + 4] & 63
        else:
            s = (sc[:, j + 4] & 0xF) | ((sc[:, j - 4] >> 6) << 4)
            m = (sc[:, j + 4] >> 4) | ((sc[:, j] >> 6) << 4)
        q = (qs[:, 32 * (j // 2):32 * (j // 2) + 32] >> (4 * (j % 2))) & 0xF
        out[:, 32 * j:32 * j + 32] = (d * s)[:, None] * q - (dmin * m)[:, None]
    return out


def dequant_q6k(blocks):
    """[nblk, 210] uint8 -> [nblk, 256] float64 (ggml dequantize_row_q6_K)."""
    b = blocks.reshape(-1, 210)
    ql, qh = b[:, 0:128].astype(np.int64), b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    d = _f16(b[:, 208:210])
    out = np.empty((b.shape[0], 256))
    for n in range(2):
        for quad in range(4):
            l = np.arange(32)
            byte = ql[:, 64 * n + l + (32 if quad in (1, 3) else 0)]
            lo = (byte >> 4) if quad >= 2 else (byte & 0xF)
            hi = (qh[:, 32 * n + l] >> (2 * quad)) & 3
            s = sc[:, 8 * n + l // 16 + 2 * quad]
            out[:, 128 * n + 32 * quad + l] = d[:, None] * s * ((lo | (hi << 4)) - 32)
    return out


def matrix(raw, qtype, rows, k):
    """A weight matrix [rows, k] in float64 from its ggml bytes."""
    if qtype == F32:
        return np.asarray(raw, np.float64).reshape(rows, k)
    if qtype == F16:
        return np.ascontiguousarray(raw).view(np.float16).astype(np.float64).reshape(rows, k)
    deq = dequant_q4k if qtype == Q4K else dequant_q6k
    return deq(np.ascontiguousarray(raw, np.uint8)).reshape(rows, k)


def rmsnorm(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def rope(x, pos, base, ff, neox):
    """x [n, heads, D] at positions pos [n]."""
    D = x.shape[-1]
    i = np.arange(D // 2)
    ang = pos[:, None].astype(np.float64) * base ** (-2.0 * i / D) / ff[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    y = x.copy()
    if neox:
        a, b = x[..., : D // 2], x[..., D // 2:]
        y[..., : D // 2], y[..., D // 2:] = a * c - b * s, a * s + b * c
    else:
        a, b = x[..., 0::2], x[..., 1::2]
        y[..., 0::2], y[..., 1::2] = a * c - b * s, a * s + b * c
    return y


def q8_round_trip(x, block):
    """The values an 8-bit activation block stands for: per `block` values d = max|x| / 127 and
    q = x / d rounded half away from zero (tests/test_llm_kernels.cpp's quantizeQ8x4 / Q8K
    definition), returned as q * d in float64."""
    xb = x.reshape(-1, block)
    d = np.abs(xb).max(axis=1, keepdims=True) / 127.0
    with np.errstate(divide="ignore", invalid="ignore"):
        t = np.where(d > 0, xb / d, 0.0)
    q = np.clip(np.sign(t) * np.floor(np.abs(t) + 0.5), -127, 127)
    return (q * d).reshape(x.shape)


class Model64:
    """cfg: the kcModelConfig fields as a dict; tensors[(id, layer)] = raw bytes or floats (the
    layout kcModelSetTensor takes; layer -1 for the global ones); types[(id, layer)] overrides a
    matrix's default type as in OracleModel.

    forward(tokens) appends tokens at the current position (one call = one llama.cpp ubatch) and
    returns the last token's logits. q8=True also models where the reference's path rounds: every
    K-quant product reads its input as 8-bit blocks (32 values for one token, 256 for a batch; an
    F16 matrix reads the float input), the KV cache holds fp16 values, and a batch's last layer
    continues after the attention projection with its last row only. q8=False is the exact
    model."""

    DEFAULT = {0: Q4K, 1: F32, 2: Q6K, 3: F32, 4: Q4K, 5: Q4K, 6: Q6K, 7: Q4K, 8: F32, 9: Q4K, 10: Q4K, 11: Q6K,
               12: F32, 13: F32}

    def __init__(self, cfg, tensors, types=None, q8=False):
        self.c = cfg
        self.t = tensors
        self.types = dict(types or {})
        self.q8 = q8
        self._m = {}
        self.pos = 0
        self.kc = [np.zeros((0, cfg["n_head_kv"], cfg["head_dim"])) for _ in range(cfg["n_layer"])]
        self.vc = [np.zeros((0, cfg["n_head_kv"], cfg["head_dim"])) for _ in range(cfg["n_layer"])]

    def qtype(self, tid, layer):
        return self.types.get((tid, layer), self.DEFAULT[tid])

    def mat(self, tid, layer, rows, k):
        key = (tid, layer)
        if key not in self._m:
            self._m[key] = matrix(self.t[key], self.qtype(tid, layer), rows, k)
        return self._m[key]

    def vec(self, tid, layer=-1):
        return np.asarray(self.t[(tid, layer)], np.float64)

    def proj(self, x, tid, layer, rows, k, block):
        """x [n, k] times the matrix's transpose; with q8, a K-quant matrix sees 8-bit x."""
        if self.q8 and self.qtype(tid, layer) in (Q4K, Q6K):
            x = q8_round_trip(x, block)
        return x @ self.mat(tid, layer, rows, k).T

    def ffn(self, x, l, block):
        c = self.c
        E, F = c["n_embd"], c["n_ff"]
        h2 = rmsnorm(x, self.vec(8, l), float(c["norm_eps"]))
        gt = self.proj(h2, 9, l, F, E, block)
        up = self.proj(h2, 10, l, F, E, block)
        return self.proj(gt / (1.0 + np.exp(-gt)) * up, 11, l, E, F, block)

    def forward(self, tokens):
        c = self.c
        n, p0 = len(tokens), self.pos
        E, H, Hkv, D, V = c["n_embd"], c["n_head"], c["n_head_kv"], c["head_dim"], c["n_vocab"]
        eps = float(c["norm_eps"])
        G = H // Hkv
        blk = 32 if n == 1 else 256
        ff = np.asarray(self.t.get((14, -1), np.ones(D // 2)), np.float64)
        pos = np.arange(p0, p0 + n)
        x = self.mat(0, -1, V, E)[np.asarray(tokens)]
        for l in range(c["n_layer"]):
            h = rmsnorm(x, self.vec(3, l), eps)
            q = self.proj(h, 4, l, H * D, E, blk).reshape(n, H, D)
            k = self.proj(h, 5, l, Hkv * D, E, blk).reshape(n, Hkv, D)
            v = self.proj(h, 6, l, Hkv * D, E, blk).reshape(n, Hkv, D)
            if c["qk_norm"]:
                q = rmsnorm(q, self.vec(12, l), eps)
                k = rmsnorm(k, self.vec(13, l), eps)
            q = rope(q, pos, float(c["rope_theta"]), ff, c["rope_neox"])
            k = rope(k, pos, float(c["rope_theta"]), ff, c["rope_neox"])
            if self.q8:  # the cache holds fp16 values
                k = k.astype(np.float16).astype(np.float64)
                v = v.astype(np.float16).astype(np.float64)
            self.kc[l] = np.concatenate([self.kc[l], k])
            self.vc[l] = np.concatenate([self.vc[l], v])
            T = p0 + n
            visible = np.arange(T)[None, :] <= pos[:, None]  # query i sees positions <= p0 + i
            att = np.empty((n, H, D))
            for hh in range(H):
                g = hh // G
                s = q[:, hh, :] @ self.kc[l][:, g, :].T / np.sqrt(D)
                s = np.where(visible, s, -np.inf)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                att[:, hh, :] = (p / p.sum(axis=1, keepdims=True)) @ self.vc[l][:, g, :]
            o = self.proj(att.reshape(n, H * D), 7, l, E, H * D, blk)
            if self.q8 and n > 1 and l == c["n_layer"] - 1:
                # llama.cpp's output-row selection: the last layer's FFN on the last row only
                x = x[n - 1:] + o[n - 1:]
                x = x + self.ffn(x, l, 32)
            else:
                x = x + o
                x = x + self.ffn(x, l, blk)
        self.pos += n
        hf = rmsnorm(x[-1:], self.vec(1), eps)
        return self.proj(hf, 2, -1, V, E, 32)[0]


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))
