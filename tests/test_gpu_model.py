"""The decode driver end to end on the GPU against the CPU oracle model (oracle/model.py), at small
Llama- and Qwen3-shaped configs with random K-quant weights. Bar: logits
within 1e-2 relative L2 of the oracle for the prompt (batch path: per-256 activations, matmuls,
causal attention) and for single decode steps (per-32 activations, matvecs); greedy tokens from
the graph-replayed generate agree with the oracle's argmax chain."""
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
from oracle.model import OracleModel
from tests.model_weights import random_weights

pytestmark = pytest.mark.gpu

LLAMA = dict(n_layer=2, n_embd=512, n_head=8, n_head_kv=2, head_dim=64, n_ff=1024, n_vocab=1024, norm_eps=1e-5,
             rope_theta=500000.0, rope_neox=0, qk_norm=0, max_ctx=256, max_batch=128)
QWEN = dict(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, head_dim=128, n_ff=768, n_vocab=1536, norm_eps=1e-6,
            rope_theta=1000000.0, rope_neox=1, qk_norm=1, max_ctx=256, max_batch=128)


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / np.linalg.norm(b)


def build(cfg, seed):
    w = random_weights(cfg, seed)
    m = kc.Model(**cfg)
    for (tid, layer), data in w.items():
        m.set_tensor(tid, layer, data)
    return m, OracleModel(cfg, w)


# prompt lengths below 64 run the column-tiled matmul, 64 and above the MFMA matmul; the second
# chunk continues the prompt at a nonzero position (causal attention over cache + chunk)
@pytest.mark.parametrize("name,cfg,n_prompt,n_chunk", [("llama", LLAMA, 37, 0), ("qwen3", QWEN, 37, 0),
                                                       ("llama", LLAMA, 100, 24), ("qwen3", QWEN, 90, 64)])
def test_model_prompt_decode_generate(name, cfg, n_prompt, n_chunk):
    note(f"model {name}: building")
    m, o = build(cfg, 7)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, cfg["n_vocab"], n_prompt + n_chunk).astype(np.int32)
    note(f"model {name}: prompt of {n_prompt} + {n_chunk}")
    for part in (prompt[:n_prompt], prompt[n_prompt:]):
        if part.size == 0:
            continue
        lg = m.forward(part)
        lo = o.forward(part)
        assert np.all(np.isfinite(lg))
        assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
        note(f"model {name}: chunk of {part.size} rel L2 {rel_l2(lg, lo):.2e}")
    for step in range(3):  # single tokens: the decode path
        t = int(rng.integers(0, cfg["n_vocab"]))
        lg = m.forward([t])
        lo = o.forward([t])
        assert rel_l2(lg, lo) < 1e-2, (step, rel_l2(lg, lo))
    note(f"model {name}: decode rel L2 {rel_l2(lg, lo):.2e}")
    assert m.position() == prompt.size + 3
    # greedy generation through the captured graph vs the oracle's argmax chain
    gen = m.generate(6)
    want = []
    logits = lo
    for _ in range(6):
        tok = int(np.argmax(logits))
        want.append(tok)
        logits = o.forward([tok])
    assert list(gen) == want
    assert m.position() == prompt.size + 3 + 5
    m.close()


def test_model_generate_matches_forward_loop():
    """The graph replays and eager single-token forwards give the same tokens and positions."""
    cfg = dict(LLAMA, n_layer=1)
    m1, _ = build(cfg, 11)
    m2, _ = build(cfg, 11)
    prompt = np.arange(10, 30, dtype=np.int32)
    l1 = m1.forward(prompt)
    l2 = m2.forward(prompt)
    assert np.array_equal(l1, l2)
    gen = m1.generate(8)
    toks = []
    logits = l2
    for _ in range(8):
        t = int(np.argmax(logits))
        toks.append(t)
        logits = m2.forward([t])
    assert list(gen) == toks
    m1.close()
    m2.close()


def test_model_argument_validation():
    cfg = dict(LLAMA, n_layer=1)
    L = kc.lib()
    import ctypes as C
    bad = kc.ModelConfig(**dict(cfg, n_embd=500))
    h = C.c_void_p()
    assert kc.ERRORS[L.kcModelCreate(C.byref(bad), C.byref(h))] == "InvalidValue"
    m = kc.Model(**cfg)
    with pytest.raises(kc.KcError):  # weights not set
        m.forward([1, 2, 3])
    qt, rows, k, nbytes = m.tensor_info("wv", 0)
    assert (qt, rows, k) == (14, 128, 512) and nbytes == 128 * 2 * 210
    with pytest.raises(kc.KcError):  # wrong size
        m.set_tensor("wv", 0, np.zeros(nbytes - 1, np.uint8))
    m.close()


@pytest.mark.parametrize("name,cfg,n_prompt,n_chunk", [("llama", LLAMA, 100, 24), ("qwen3", QWEN, 90, 64),
                                                       ("llama", LLAMA, 65, 32)])
def test_model_prompt_attention_kernels_agree(name, cfg, n_prompt, n_chunk):
    """The prompt's attention with the query heads of a KV head in one workgroup (attn_path 3, the
    default when its grid fills the GPU) against one query head per workgroup (2) and the oracle:
    prompts and a continuing chunk whose last query tile holds a single query (65: a key block
    reaching past the context, whose cache rows were never written)."""
    w = random_weights(cfg, 7)
    prompt = np.random.default_rng(3).integers(0, cfg["n_vocab"], n_prompt + n_chunk).astype(np.int32)
    got = {}
    for ap in (2, 3):
        kc.set_option("attn_path", ap)
        try:
            m = kc.Model(**cfg)
            for (tid, layer), data in w.items():
                m.set_tensor(tid, layer, data)
            got[ap] = [m.forward(prompt[:n_prompt]), m.forward(prompt[n_prompt:])]
            m.close()
        finally:
            kc.set_option("attn_path", 0)
    o = OracleModel(cfg, w)
    for i, part in enumerate((prompt[:n_prompt], prompt[n_prompt:])):
        lo = o.forward(part)
        note(f"attention kernels {name} {n_prompt}+{n_chunk} part {i}: rel L2 {rel_l2(got[3][i], lo):.2e}, "
             f"kernels {rel_l2(got[3][i], got[2][i]):.2e}")
        assert rel_l2(got[3][i], lo) < 1e-2
        assert rel_l2(got[3][i], got[2][i]) < 1e-6  # (the same products and sums: equal in practice)


@pytest.mark.parametrize("head_dim,n_head,n_head_kv", [(128, 4, 2), (64, 8, 1), (128, 2, 2)])
def test_qwen3_prompt_norms_fused_bit_identical(head_dim, n_head, n_head_kv):
    """A Qwen3 prompt's per-head q / k norms inside the RoPE + cache-store launch (the default)
    against the three launches (option qk_fuse = 1): the same logits and the same cache bits, for a
    prompt and a continuing chunk (70 tokens: the last workgroups hold part of 64 head rows; one KV
    head: a workgroup's 64 k rows span 64 tokens)."""
    cfg = dict(QWEN, head_dim=head_dim, n_head=n_head, n_head_kv=n_head_kv)
    w = random_weights(cfg, 17)
    prompt = np.random.default_rng(4).integers(0, cfg["n_vocab"], 70 + 33).astype(np.int32)
    got = {}
    for fuse in (1, 0):
        kc.set_option("qk_fuse", fuse)
        try:
            m = kc.Model(**cfg)
            for (tid, layer), data in w.items():
                m.set_tensor(tid, layer, data)
            lg = [m.forward(prompt[:70]), m.forward(prompt[70:])]
            caches = [m.read_cache(li, which, 0, len(prompt)) for li in range(cfg["n_layer"]) for which in (0, 1)]
            got[fuse] = (lg, caches)
            m.close()
        finally:
            kc.set_option("qk_fuse", 0)
    for a, b in zip(got[0][0], got[1][0]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for a, b in zip(got[0][1], got[1][1]):
        assert np.array_equal(a, b)
    lo = OracleModel(cfg, w).forward(prompt[:70])
    assert rel_l2(got[0][0][0], lo) < 1e-2


@pytest.mark.parametrize("n_embd", [256, 768, 3072, 4096])
def test_prompt_add_norm_register_form_bit_identical(n_embd):
    """The prompt's residual add + RMS norm + per-256 quantization with each row's values kept in
    registers (the default up to four values per thread) against the LDS form (option addnorm_lds
    = 1): the same logits and the same cache bits for a prompt and a continuing chunk (256 and 768
    values: workgroups with wavefronts past the row's end)."""
    cfg = dict(LLAMA, n_embd=n_embd, n_head=n_embd // 64, n_head_kv=2, n_ff=512, n_vocab=512)
    w = random_weights(cfg, 23)
    prompt = np.random.default_rng(6).integers(0, cfg["n_vocab"], 70 + 33).astype(np.int32)
    got = {}
    for lds in (1, 0):
        kc.set_option("addnorm_lds", lds)
        try:
            m = kc.Model(**cfg)
            for (tid, layer), data in w.items():
                m.set_tensor(tid, layer, data)
            lg = [m.forward(prompt[:70]), m.forward(prompt[70:])]
            caches = [m.read_cache(li, which, 0, len(prompt)) for li in range(cfg["n_layer"]) for which in (0, 1)]
            got[lds] = (lg, caches)
            m.close()
        finally:
            kc.set_option("addnorm_lds", 0)
    for a, b in zip(got[0][0], got[1][0]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for a, b in zip(got[0][1], got[1][1]):
        assert np.array_equal(a, b)
    lo = OracleModel(cfg, w).forward(prompt[:70])
    assert rel_l2(got[0][0][0], lo) < 1e-2


@pytest.mark.parametrize("cfg", [LLAMA, QWEN], ids=["llama", "qwen3"])
def test_prompt_without_int8_slots_bit_identical(cfg):
    """A prompt whose quantizers write only the matrix-core operand layout (the default: no int8
    slots where no product reads them) against one whose products convert the int8 slots themselves
    (option prefill_act = 1): the same logits and cache bits, for a 70-token prompt (slots skipped)
    and a 33-token continuation (under 64 columns: slots written and read)."""
    w = random_weights(cfg, 29)
    prompt = np.random.default_rng(8).integers(0, cfg["n_vocab"], 70 + 33).astype(np.int32)
    got = {}
    for act in (1, 0):
        kc.set_option("prefill_act", act)
        try:
            m = kc.Model(**cfg)
            for (tid, layer), data in w.items():
                m.set_tensor(tid, layer, data)
            lg = [m.forward(prompt[:70]), m.forward(prompt[70:])]
            caches = [m.read_cache(li, which, 0, len(prompt)) for li in range(cfg["n_layer"]) for which in (0, 1)]
            got[act] = (lg, caches)
            m.close()
        finally:
            kc.set_option("prefill_act", 0)
    for a, b in zip(got[0][0], got[1][0]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for a, b in zip(got[0][1], got[1][1]):
        assert np.array_equal(a, b)


def test_model_3b_shape_two_layers():
    """Two layers at the full Llama-3.2-3B widths (3072 / 24 heads / 8 KV heads / 8192 FFN / 128256
    vocab): an 8-token prompt and two decode steps against the oracle."""
    cfg = dict(n_layer=2, n_embd=3072, n_head=24, n_head_kv=8, head_dim=128, n_ff=8192, n_vocab=128256,
               norm_eps=1e-5, rope_theta=500000.0, rope_neox=0, qk_norm=0, max_ctx=64, max_batch=16)
    note("model 3b-shape: building")
    m, o = build(cfg, 21)
    prompt = np.random.default_rng(5).integers(0, cfg["n_vocab"], 8).astype(np.int32)
    lg, lo = m.forward(prompt), o.forward(prompt)
    assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    note(f"model 3b-shape: prompt rel L2 {rel_l2(lg, lo):.2e}")
    for _ in range(2):
        t = int(np.argmax(lo))
        lg, lo = m.forward([t]), o.forward([t])
        assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    m.close()


def test_model_qwen3_8b_shape_two_layers():
    """Two layers at the Qwen3-8B widths (4096 / 32 heads / 8 KV heads / 12288 FFN / 151936 vocab,
    per-head q/k RMS norm, NEOX RoPE): a 70-token prompt (the MFMA matmuls, K split for o and down)
    and two decode steps against the oracle."""
    cfg = dict(n_layer=2, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=12288, n_vocab=151936,
               norm_eps=1e-6, rope_theta=1000000.0, rope_neox=1, qk_norm=1, max_ctx=128, max_batch=80)
    note("model 8b-shape: building")
    m, o = build(cfg, 23)
    prompt = np.random.default_rng(6).integers(0, cfg["n_vocab"], 70).astype(np.int32)
    lg, lo = m.forward(prompt), o.forward(prompt)
    assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    note(f"model 8b-shape: prompt rel L2 {rel_l2(lg, lo):.2e}")
    for _ in range(2):
        t = int(np.argmax(lo))
        lg, lo = m.forward([t]), o.forward([t])
        assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    m.close()


def test_model_prefill_on_the_wide_tile_matmul():
    """matmul_path = 7: the model's grouped prefill matmuls (q/k/v and gate/up in one launch, K
    split for o and down) on the wide-tile MFMA kernel, a 70-token prompt at the Qwen3-8B widths
    (two layers) against the oracle."""
    cfg = dict(n_layer=2, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=12288, n_vocab=151936,
               norm_eps=1e-6, rope_theta=1000000.0, rope_neox=1, qk_norm=1, max_ctx=128, max_batch=80)
    kc.set_option("matmul_path", 7)
    try:
        m, o = build(cfg, 23)
        prompt = np.random.default_rng(6).integers(0, cfg["n_vocab"], 70).astype(np.int32)
        lg, lo = m.forward(prompt), o.forward(prompt)
        note(f"model 8b-shape, wide-tile matmul: prompt rel L2 {rel_l2(lg, lo):.2e}")
        assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
        m.close()
    finally:
        kc.set_option("matmul_path", 0)


@pytest.mark.parametrize("name,cfg", [("llama", LLAMA), ("qwen3", QWEN)])
def test_model_unfused_decode_path(name, cfg):
    """decode_path = 1 runs the one-kernel-per-reference-op decode step (add_sumsq, norm_mul_q8,
    the matvecs, rope, set_rows, attention, quantize_q8x4, silu_mul_q8): same oracle bar."""
    kc.set_option("decode_path", 1)
    try:
        m, o = build(cfg, 5)
        prompt = np.arange(3, 3 + 21, dtype=np.int32)
        lg, lo = m.forward(prompt), o.forward(prompt)
        for _ in range(3):
            t = int(np.argmax(lo))
            lg, lo = m.forward([t]), o.forward([t])
            assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
        gen = m.generate(4)
        want = []
        for _ in range(4):
            want.append(int(np.argmax(lo)))
            lo = o.forward([want[-1]])
        assert list(gen) == want
        m.close()
    finally:
        kc.set_option("decode_path", 0)


def test_model_fused_matvecs_unfused_attention():
    """decode_path = 2: the fused matvec kernels with the one-op-per-kernel attention."""
    kc.set_option("decode_path", 2)
    try:
        m, o = build(LLAMA, 5)
        prompt = np.arange(3, 3 + 21, dtype=np.int32)
        lg, lo = m.forward(prompt), o.forward(prompt)
        for _ in range(3):
            t = int(np.argmax(lo))
            lg, lo = m.forward([t]), o.forward([t])
            assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
        m.close()
    finally:
        kc.set_option("decode_path", 0)


@pytest.mark.parametrize("name,cfg", [("llama", LLAMA), ("qwen3", QWEN)])
def test_model_attention_merge_forms_agree(name, cfg):
    """The decode step merges the split attention's chunk partials with one wavefront per 64
    outputs (cross-lane quantization); decode_path = 3 runs the first form, one workgroup per KV
    head with one thread per block of 32. Same operations in the same order: the logits agree bit
    for bit, over steps that cross a chunk boundary (positions 100..139, chunks of 64)."""
    m0, o = build(cfg, 11)
    m3, _ = build(cfg, 11)
    prompt = np.arange(5, 5 + 100, dtype=np.int32)
    a, b = m0.forward(prompt), m3.forward(prompt)
    assert np.array_equal(a, b)
    lo = o.forward(prompt)
    try:
        for step in range(40):
            t = int(np.argmax(a))
            kc.set_option("decode_path", 0)
            a = m0.forward([t])
            kc.set_option("decode_path", 3)
            b = m3.forward([t])
            kc.set_option("decode_path", 0)
            assert np.array_equal(a, b), (step, float(np.max(np.abs(a - b))))
            if step < 3:  # and the oracle's bar on the first steps
                lo = o.forward([t])
                assert rel_l2(a, lo) < 1e-2, rel_l2(a, lo)
    finally:
        kc.set_option("decode_path", 0)
    note(f"model {name}: the two merge forms agree over 40 steps")
    m0.close()
    m3.close()


def test_model_long_context_split_attention():
    """A cache too large for the one-workgroup attention's LDS scores (max_ctx 12288 with 4 query
    heads per KV head) takes the split-context attention and its merge kernel."""
    cfg = dict(LLAMA, n_layer=1, max_ctx=12288)
    m, o = build(cfg, 9)
    prompt = np.arange(40, 40 + 70, dtype=np.int32)  # 70 positions: two chunks of 64
    lg, lo = m.forward(prompt), o.forward(prompt)
    for _ in range(3):
        t = int(np.argmax(lo))
        lg, lo = m.forward([t]), o.forward([t])
        assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    m.close()


@pytest.mark.parametrize("name,cfg,f16", [
    ("llama-f16-v", LLAMA, [(6, 0), (6, 1)]),                                      # F16 attn_v (a Qwen3 GGUF case)
    ("qwen3-f16-mixed", QWEN, [(6, 0), (7, 0), (9, 0), (10, 0), (11, 0), (4, 1)]),  # every matrix kind
])
def test_model_f16_matrices(name, cfg, f16):
    """F16 per-layer matrices (kcModelSetTensorTyped with KC_QTYPE_F16): matmul_f16 of the f32
    activations in the prompt (MFMA kernel), the single-token steps and the graph-replayed generate
    (unfused decode, per-row kernel), against the oracle with the same types."""
    from oracle.model import F16
    note(f"model {name}: building")
    types = {t: F16 for t in f16}
    w = random_weights(cfg, 23, types)
    m = kc.Model(**cfg)
    for (tid, layer), data in w.items():
        m.set_tensor(tid, layer, data, "f16" if (tid, layer) in types else None)
    for t in f16:
        qt, rows, k, nbytes = m.tensor_info(t[0], t[1])
        assert qt == 1 and nbytes == rows * k * 2
    o = OracleModel(cfg, w, types=types)
    prompt = np.random.default_rng(9).integers(0, cfg["n_vocab"], 40).astype(np.int32)
    lg, lo = m.forward(prompt), o.forward(prompt)
    assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    note(f"model {name}: prompt rel L2 {rel_l2(lg, lo):.2e}")
    for _ in range(3):
        t = int(np.argmax(lo))
        lg, lo = m.forward([t]), o.forward([t])
        assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    want = []
    for _ in range(5):
        want.append(int(np.argmax(lo)))
        lo = o.forward([want[-1]])
    assert list(m.generate(5)) == want
    m.close()


def test_model_f16_rejected_for_global_matrices():
    cfg = dict(LLAMA, n_layer=1)
    m = kc.Model(**cfg)
    _, rows, k, _ = m.tensor_info("output")
    with pytest.raises(kc.KcError):
        m.set_tensor("output", -1, np.zeros(rows * k * 2, np.uint8), "f16")
    m.close()


def test_model_llama2_ffn_width_decodes_fused():
    """n_ff 11008 (Llama-2-7B): 43 super-blocks, 11 groups of 4 -- a prime above the wavefront cap of
    the down-projection matvec. The plan keeps the fused single-token path (8 wavefronts, uneven
    shares) and the decode matches the oracle."""
    cfg = dict(n_layer=1, n_embd=512, n_head=8, n_head_kv=8, head_dim=64, n_ff=11008, n_vocab=1024, norm_eps=1e-5,
               rope_theta=10000.0, rope_neox=0, qk_norm=0, max_ctx=64, max_batch=16)
    assert kc.plan_decode(**cfg) == 1
    note("model n_ff 11008: building")
    m, o = build(cfg, 31)
    prompt = np.random.default_rng(8).integers(0, cfg["n_vocab"], 9).astype(np.int32)
    lg, lo = m.forward(prompt), o.forward(prompt)
    assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    for _ in range(3):
        t = int(np.argmax(lo))
        lg, lo = m.forward([t]), o.forward([t])
        assert rel_l2(lg, lo) < 1e-2, rel_l2(lg, lo)
    gen = m.generate(4)
    want, logits = [], lo
    for _ in range(4):
        want.append(int(np.argmax(logits)))
        logits = o.forward([want[-1]])
    assert list(gen) == want
    m.close()
