"""CPU oracle of the decode driver (test infrastructure only).

Composes the C restatements in oracle/kc_oracle.c into the transformer step the GPU driver
(kernelcore_amd/csrc/model.cpp) runs, in the op order of the reference's ggml backend graph
(docs/cuda_cpu_poc_plan.md:1158; dispatch ggml-kernelcore.cpp:555-589): one token takes per-32
activations and the matvecs, a batch per-256 activations and the matmuls, and the last layer of
a batch continues after the attention projection with the last token only (llama.cpp's output-row
selection). Only tests/ import this module.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import FaDims, dequant, lib, matmul_f16, quantize_q8x4, quantize_q8k

Q4K, Q6K, F32, F16 = 12, 14, 0, 1
BB = {Q4K: 144, Q6K: 210}


def shapes(cfg):
    """tensor id -> (qtype, rows, k), the same table as kcModelTensorInfo."""
    E, Q, KV, F, V, hd = (cfg["n_embd"], cfg["n_head"] * cfg["head_dim"], cfg["n_head_kv"] * cfg["head_dim"],
                          cfg["n_ff"], cfg["n_vocab"], cfg["head_dim"])
    return {0: (Q4K, V, E), 1: (F32, 1, E), 2: (Q6K, V, E), 3: (F32, 1, E), 4: (Q4K, Q, E), 5: (Q4K, KV, E),
            6: (Q6K, KV, E), 7: (Q4K, E, Q), 8: (F32, 1, E), 9: (Q4K, F, E), 10: (Q4K, F, E), 11: (Q6K, E, F),
            12: (F32, 1, hd), 13: (F32, 1, hd)}


class OracleModel:
    def __init__(self, cfg, tensors, threads=0, types=None):
        """tensors[(id, layer)] = raw ggml bytes (uint8) or float32 arrays; global ids use layer -1;
        (14, -1), when present, holds the RoPE frequency factors. types[(id, layer)] = Q4K / Q6K
        overrides a matrix's default type (a GGUF Q4_K_M file mixes them); F16 (per-layer matrices,
        row-major halves) multiplies the f32 activations instead of the quantized ones, as the
        reference's MUL_MAT dispatch does (ggml-kernelcore.cpp:559-566). threads > 0 runs the
        matvecs, matmuls and attention with the vectorised, threaded forms (kc_oracle_simd.c:
        bit-identical results, rows or (query, head) pairs split over threads) -- the full-size
        GPU tests and the bench's CPU baseline."""
        self.cfg = cfg
        self.t = tensors
        self.types = dict(types or {})
        self.L = lib()
        self.threads = threads
        self.pos = 0
        kvd = cfg["n_head_kv"] * cfg["head_dim"]
        self.kc = [np.zeros(cfg["max_ctx"] * kvd, np.uint16) for _ in range(cfg["n_layer"])]
        self.vc = [np.zeros(cfg["max_ctx"] * kvd, np.uint16) for _ in range(cfg["n_layer"])]

    # ---- kernels --------------------------------------------------------------------------------
    def w(self, tid, layer=-1):
        return self.t[(tid, layer)]

    def qt(self, tid, layer=-1):
        return self.types.get((tid, layer), shapes(self.cfg)[tid][0])

    def matvec(self, tid, layer, slot, rows, k, xf=None):
        qt = self.qt(tid, layer)
        if qt == F16:
            return matmul_f16(self.L, self.w(tid, layer).view(np.uint16), xf, rows, k, 1)[0]
        nb = k // 32
        y = np.zeros(rows, np.float32)
        xq = np.ascontiguousarray(slot[:nb * 8])
        xd = np.ascontiguousarray(slot[nb * 8:nb * 10].view(np.float32))
        if self.threads > 0:
            fn = self.L.kco_matvec_q6k_q8_simd if qt == Q6K else self.L.kco_matvec_q4k_q8_simd
            fn(self.w(tid, layer), xq, xd, y, rows, k, self.threads)
        else:
            fn = self.L.kco_matvec_q6k_q8 if qt == Q6K else self.L.kco_matvec_q4k_q8
            fn(self.w(tid, layer), xq, xd, y, rows, k)
        return y

    def matmul(self, tid, layer, slots, rows, k, n, xf=None):
        qt = self.qt(tid, layer)
        if qt == F16:
            return matmul_f16(self.L, self.w(tid, layer).view(np.uint16), xf, rows, k, n)
        y = np.zeros(rows * n, np.float32)
        if self.threads > 0:
            fn = self.L.kco_matmul_q6k_q8k_simd if qt == Q6K else self.L.kco_matmul_q4k_q8k_simd
            fn(self.w(tid, layer), slots, y, rows, k, n, self.threads)
        else:
            fn = self.L.kco_matmul_q6k_q8k if qt == Q6K else self.L.kco_matmul_q4k_q8k
            fn(self.w(tid, layer), slots, y, rows, k, n)
        return y.reshape(n, rows)

    def rope(self, x, n_head, pos):
        c = self.cfg
        y = np.zeros_like(x)
        ff = np.ascontiguousarray(self.t.get((14, -1), np.ones(c["head_dim"] // 2, np.float32)), np.float32)
        self.L.kco_rope_ggml(np.ascontiguousarray(x, np.float32), y, np.asarray(pos, np.int32), ff, c["head_dim"], n_head,
                             len(pos), np.log2(np.float32(c["rope_theta"])), int(c["rope_neox"]))
        return y

    def attention(self, l, q, n, p0):
        c = self.cfg
        H, Hkv, D = c["n_head"], c["n_head_kv"], c["head_dim"]
        T = p0 + n
        tp = (T + 7) // 8 * 8
        mask = np.zeros(n * tp, np.float16)
        if n > 1:
            mask[:] = -np.inf
            for i in range(n):
                mask[i * tp:i * tp + p0 + i + 1] = 0.0
        d = FaDims(H=H, T=T, D=D, group=H // Hkv, tp=tp, k_row=Hkv * D // 2, k_head=D // 2, v_row=Hkv * D // 2,
                   v_head=D // 2, N=n, q_tok=H * D, q_head=D, m_row=tp // 2, has_mask=int(n > 1), H_kv=Hkv)
        out = np.zeros(n * H * D, np.float32)
        args = (np.ascontiguousarray(q, np.float32), self.kc[l], self.vc[l], mask.view(np.uint16), out, C.byref(d),
                np.float32(1.0 / np.sqrt(np.float32(D))))
        if self.threads > 0:
            self.L.kco_flash_attn_f16_mt(*args, self.threads)
        else:
            self.L.kco_flash_attn_f16(*args)
        return out.reshape(n, H * D)

    def set_rows(self, l, k, v, p0):
        c = self.cfg
        kvd = c["n_head_kv"] * c["head_dim"]
        n = k.shape[0]
        idx = np.arange(p0, p0 + n, dtype=np.int64)
        for cache, src in ((self.kc[l], k), (self.vc[l], v)):
            self.L.kco_set_rows_f16(np.ascontiguousarray(src, np.float32).reshape(-1), idx, cache, kvd // 2, n, kvd,
                                    kvd // 2, c["max_ctx"])

    def residual(self, x, y):
        """The residual stream's ADD (tests plant mistakes here by overriding it)."""
        return x + y

    # ---- one row, per-32 path ---------------------------------------------------------------------
    def _norm32(self, x, wt):
        E = x.size
        nb = E // 32
        slot = np.zeros(nb * 11, np.int32)
        self.L.kco_sumsq_part(x, slot, E, 1)
        y = np.zeros(E, np.float32)
        self.L.kco_norm_mul_q8(x, wt, y, slot, E, 1, np.float32(self.cfg["norm_eps"]))
        return slot, y

    def _ffn_one(self, l, x):
        c = self.cfg
        slot, y = self._norm32(x, self.w(8, l))
        g = self.matvec(9, l, slot, c["n_ff"], c["n_embd"], y)
        u = self.matvec(10, l, slot, c["n_ff"], c["n_embd"], y)
        s = np.zeros(c["n_ff"], np.float32)
        q = np.zeros(c["n_ff"] // 32 * 11, np.int32)
        self.L.kco_silu_mul_q8f(g, u, s, q, c["n_ff"], 1)
        return self.matvec(11, l, q, c["n_embd"], c["n_ff"], s)

    def _head(self, x):
        c = self.cfg
        slot, _ = self._norm32(x, self.w(1))
        return self.matvec(2, -1, slot, c["n_vocab"], c["n_embd"])

    def _qkv_post(self, l, q, k, n, p0):
        c = self.cfg
        hd = c["head_dim"]
        if c["qk_norm"]:
            qn = np.zeros_like(q)
            kn = np.zeros_like(k)
            self.L.kco_rms_norm(np.ascontiguousarray(q.reshape(-1)), self.w(12, l), qn.reshape(-1), hd,
                                c["n_head"] * n, np.float32(c["norm_eps"]))
            self.L.kco_rms_norm(np.ascontiguousarray(k.reshape(-1)), self.w(13, l), kn.reshape(-1), hd,
                                c["n_head_kv"] * n, np.float32(c["norm_eps"]))
            q, k = qn, kn
        pos = np.arange(p0, p0 + n, dtype=np.int32)
        qr = self.rope(q.reshape(-1), c["n_head"], pos).reshape(n, -1)
        kr = self.rope(k.reshape(-1), c["n_head_kv"], pos).reshape(n, -1)
        return qr, kr

    def forward(self, tokens):
        c = self.cfg
        n = len(tokens)
        p0 = self.pos
        E, Q, KV = c["n_embd"], c["n_head"] * c["head_dim"], c["n_head_kv"] * c["head_dim"]
        emb = np.ascontiguousarray(self.w(0)).reshape(c["n_vocab"], -1)  # ggml rows of the embedding
        et = "q6k" if self.qt(0) == Q6K else "q4k"
        x = np.concatenate([dequant(self.L, et, emb[t], 1, E) for t in tokens]).astype(np.float32)
        eps = np.float32(c["norm_eps"])
        down = None
        if n == 1:
            x = x.reshape(-1).copy()
            for l in range(c["n_layer"]):
                if l > 0:
                    x = self.residual(x, down)
                slot, xn = self._norm32(x, self.w(3, l))
                q = self.matvec(4, l, slot, Q, E, xn)
                k = self.matvec(5, l, slot, KV, E, xn)
                v = self.matvec(6, l, slot, KV, E, xn)
                qr, kr = self._qkv_post(l, q.reshape(1, -1), k.reshape(1, -1), 1, p0)
                self.set_rows(l, kr, v.reshape(1, -1), p0)
                att = self.attention(l, qr, 1, p0).reshape(-1)
                xq, xd = quantize_q8x4(self.L, att)
                aslot = np.concatenate([xq, xd.view(np.int32), np.zeros(Q // 32, np.int32)])
                o = self.matvec(7, l, aslot, E, Q, att)
                x = self.residual(x, o)
                down = self._ffn_one(l, x)
            x = self.residual(x, down)
            logits = self._head(x)
        else:
            nsb, nb = E // 256, E // 32
            for l in range(c["n_layer"]):
                if l > 0:
                    x = self.residual(x, down)
                sq = np.zeros(n * nb * 11, np.int32)
                self.L.kco_sumsq_part(np.ascontiguousarray(x.reshape(-1)), sq, E, n)
                slots = np.zeros(n * nsb * 85, np.int32)
                y = np.zeros(n * E, np.float32)
                self.L.kco_norm_mul_q8k(np.ascontiguousarray(x.reshape(-1)), self.w(3, l), y, slots, sq, E, n, eps)
                q = self.matmul(4, l, slots, Q, E, n, y)
                k = self.matmul(5, l, slots, KV, E, n, y)
                v = self.matmul(6, l, slots, KV, E, n, y)
                qr, kr = self._qkv_post(l, q, k, n, p0)
                self.set_rows(l, kr, v, p0)
                att = self.attention(l, qr.reshape(-1), n, p0)
                aslots = np.zeros(n * Q // 256 * 85, np.int32)
                self.L.kco_quantize_cols_k(np.ascontiguousarray(att.reshape(-1)), aslots, Q, n)
                o = self.matmul(7, l, aslots, E, Q, n, att)
                if l + 1 < c["n_layer"]:
                    x = self.residual(x, o)
                    sq = np.zeros(n * nb * 11, np.int32)
                    self.L.kco_sumsq_part(np.ascontiguousarray(x.reshape(-1)), sq, E, n)
                    self.L.kco_norm_mul_q8k(np.ascontiguousarray(x.reshape(-1)), self.w(8, l), y, slots, sq, E, n, eps)
                    g = self.matmul(9, l, slots, c["n_ff"], E, n, y)
                    u = self.matmul(10, l, slots, c["n_ff"], E, n, y)
                    s = np.zeros(n * c["n_ff"], np.float32)
                    fslots = np.zeros(n * c["n_ff"] // 256 * 85, np.int32)
                    self.L.kco_silu_mul_q8k(np.ascontiguousarray(g.reshape(-1)), np.ascontiguousarray(u.reshape(-1)), s,
                                            fslots, c["n_ff"], n)
                    down = self.matmul(11, l, fslots, E, c["n_ff"], n, s)
                else:
                    x = self.residual(x[n - 1], o[n - 1]).astype(np.float32)
                    down = self._ffn_one(l, x)
            x = self.residual(x, down)
            logits = self._head(x)
        self.pos += n
        return logits
