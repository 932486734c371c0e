"""kcModelLoadGguf on the GPU: synthetic model files (tests/gguf_writer.py, the llama.cpp layout)
with mixed Q4_K / Q6_K matrices as in a Q4_K_M file (and F16 attn_v, as some Qwen3 files carry), RoPE frequency factors, and a tied head.
The loaded model must give the same logits, bit for bit, as the same weights set through
kcModelSetTensorTyped, and meet the oracle's bar (1e-2 relative L2) with the same per-tensor types
(the reference loader: llm/gguf_model.cpp:51-106)."""
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
from oracle.model import F16, F32, Q4K, Q6K, OracleModel, shapes
from tests import gguf_writer as gw
from tests.model_weights import random_weights

pytestmark = pytest.mark.gpu

LLAMA = dict(n_layer=2, n_embd=512, n_head=8, n_head_kv=2, head_dim=64, n_ff=1024, n_vocab=1024, norm_eps=1e-5,
             rope_theta=500000.0, rope_neox=0, qk_norm=0, max_ctx=256, max_batch=128)
QWEN = dict(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, head_dim=128, n_ff=768, n_vocab=1536, norm_eps=1e-6,
            rope_theta=1000000.0, rope_neox=1, qk_norm=1, max_ctx=256, max_batch=128)


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / np.linalg.norm(b)


def mixed_types(cfg, rng, same_gate_up=True):
    """A Q4_K_M-like mix: attn_v / ffn_down Q6_K or Q4_K per layer, some q / o matrices Q6_K, the
    embedding Q6_K and the head Q4_K."""
    t = {(0, -1): Q6K, (2, -1): Q4K}
    for l in range(cfg["n_layer"]):
        for tid in (4, 5, 6, 7, 9, 11):
            t[(tid, l)] = Q6K if rng.integers(0, 2) else Q4K
        t[(10, l)] = t[(9, l)] if same_gate_up else (Q4K if t[(9, l)] == Q6K else Q6K)
    return t


def all_types(cfg, types):
    full = {}
    for tid, (qt, _, _) in shapes(cfg).items():
        if qt == F32:
            continue
        for layer in ([-1] if tid in (0, 2) else range(cfg["n_layer"])):
            full[(tid, layer)] = types.get((tid, layer), qt)
    return full


def run_pair(m_a, m_b, o, prompt, steps, cfg):
    a, b, lo = m_a.forward(prompt), m_b.forward(prompt), o.forward(prompt)
    assert np.array_equal(a, b)
    assert rel_l2(a, lo) < 1e-2, rel_l2(a, lo)
    for _ in range(steps):
        t = int(np.argmax(lo))
        a, b, lo = m_a.forward([t]), m_b.forward([t]), o.forward([t])
        assert np.array_equal(a, b)
        assert rel_l2(a, lo) < 1e-2, rel_l2(a, lo)
    want = []
    for _ in range(4):
        want.append(int(np.argmax(lo)))
        lo = o.forward([want[-1]])
    assert list(m_a.generate(4)) == want


@pytest.mark.parametrize("name,cfg,arch,tied,n_prompt,f16_v", [("llama", LLAMA, "llama", False, 70, False),
                                                               ("qwen3", QWEN, "qwen3", True, 40, False),
                                                               ("qwen3-f16-v", QWEN, "qwen3", True, 40, True)])
def test_load_gguf_matches_set_tensor_and_oracle(tmp_path, name, cfg, arch, tied, n_prompt, f16_v):
    rng = np.random.default_rng(21)
    types = mixed_types(cfg, rng)
    if f16_v:  # F16 attn_v in every layer (matmul_f16 of the f32 activations)
        for l in range(cfg["n_layer"]):
            types[(6, l)] = F16
    w = random_weights(cfg, 13, types)
    if tied:  # the head is the embedding matrix, in its type
        w[(2, -1)] = w[(0, -1)]
        types[(2, -1)] = types[(0, -1)]
    if not tied:  # Llama-3-style RoPE frequency factors
        w[(14, -1)] = rng.uniform(0.5, 4.0, cfg["head_dim"] // 2).astype(np.float32)
    path = str(tmp_path / f"{name}.gguf")
    gw.model_gguf(path, arch, cfg, w, {k: v for k, v in types.items()}, tied=tied)
    note(f"gguf {name}: loading {path}")
    m_file = kc.Model.load_gguf(path, cfg["max_ctx"], cfg["max_batch"])
    m_set = kc.Model(**cfg)
    full = all_types(cfg, types)
    for (tid, layer), data in w.items():
        qt = full.get((tid, layer))
        m_set.set_tensor(tid, layer, data, None if qt is None else qt)
    for (tid, layer), qt in full.items():  # the loader recorded every matrix's type
        assert m_file.tensor_info(tid, max(layer, 0))[0] == qt
    o = OracleModel(cfg, w, types=full)
    prompt = rng.integers(0, cfg["n_vocab"], n_prompt).astype(np.int32)
    run_pair(m_file, m_set, o, prompt, 3, cfg)
    note(f"gguf {name}: file == typed set_tensor == oracle bar")
    m_file.close()
    m_set.close()


def test_load_gguf_gate_up_types_differ(tmp_path):
    """A layer whose gate and up differ in type decodes through the unfused kernels: same bar."""
    cfg = dict(LLAMA, n_layer=1)
    rng = np.random.default_rng(5)
    types = mixed_types(cfg, rng, same_gate_up=False)
    w = random_weights(cfg, 17, types)
    path = str(tmp_path / "mix.gguf")
    gw.model_gguf(path, "llama", cfg, w, types)
    m = kc.Model.load_gguf(path, cfg["max_ctx"], cfg["max_batch"])
    o = OracleModel(cfg, w, types=all_types(cfg, types))
    prompt = np.arange(3, 40, dtype=np.int32)
    lg, lo = m.forward(prompt), o.forward(prompt)
    assert rel_l2(lg, lo) < 1e-2
    for _ in range(3):
        t = int(np.argmax(lo))
        lg, lo = m.forward([t]), o.forward([t])
        assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    m.close()


def test_load_gguf_shape_mismatch(tmp_path):
    cfg = dict(LLAMA, n_layer=1)
    w = random_weights(cfg, 3)
    w[(4, 0)] = w[(4, 0)][: w[(4, 0)].size // 2]  # attn_q with half its rows
    path = str(tmp_path / "bad.gguf")
    types = {k: v for k, v in all_types(cfg, {}).items()}
    gw.model_gguf(path, "llama", cfg, w, types, extra_kv=())
    # the writer takes the shape from the config; rewrite attn_q's rows in the directory
    blob = bytearray(open(path, "rb").read())
    name = b"blk.0.attn_q.weight"
    i = blob.index(name) + len(name) + 4 + 8  # n_dims, ne[0]
    blob[i:i + 8] = (cfg["n_head"] * cfg["head_dim"] // 2).to_bytes(8, "little")
    open(path, "wb").write(bytes(blob))
    with pytest.raises(kc.KcError) as e:
        kc.Model.load_gguf(path, cfg["max_ctx"], cfg["max_batch"])
    assert "blk.0.attn_q.weight: shape" in str(e.value)
