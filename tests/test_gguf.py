"""The GGUF reader (include/kernelcore/gguf.h) on the CPU: files written by tests/gguf_writer.py
(the llama.cpp layout) read back value for value, and corrupt files rejected with InvalidValue
instead of a read past the map. The reference reader's behaviour it keeps (llm/gguf.cpp:87-141):
versions >= 2, general.alignment (32 by default), tensors of unknown block size listed with 0
bytes. kcModelLoadGguf's checks that run before any GPU work are here too."""
import struct

import numpy as np
import pytest

import kernelcore_amd as kc
from tests import gguf_writer as gw


def _kv():
    return [("general.architecture", gw.STR, "llama"), ("k.u8", gw.U8, 200), ("k.i8", gw.I8, -100),
            ("k.u16", gw.U16, 60000), ("k.i16", gw.I16, -30000), ("k.u32", gw.U32, 4000000000),
            ("k.i32", gw.I32, -2000000000), ("k.f32", gw.F32V, 1.5), ("k.bool", gw.BOOL, True),
            ("k.u64", gw.U64, 2**40 + 3), ("k.i64", gw.I64, -(2**40)), ("k.f64", gw.F64, 0.1),
            ("k.str", gw.STR, "héllo"), ("k.arr_i32", gw.ARR, (gw.I32, [1, -2, 3])),
            ("k.arr_str", gw.ARR, (gw.STR, ["a", "bc", ""]))]


def _tensors(rng):
    return [("a.f32", gw.GGML_F32, (5, 3), rng.standard_normal(15).astype(np.float32).tobytes()),
            ("b.q4k", gw.GGML_Q4_K, (512, 2), rng.integers(0, 256, 2 * 2 * 144, dtype=np.uint8).tobytes()),
            ("c.q6k", gw.GGML_Q6_K, (256, 3, 1), rng.integers(0, 256, 3 * 210, dtype=np.uint8).tobytes()),
            ("d.q8_0", 8, (64,), rng.integers(0, 256, 2 * 34, dtype=np.uint8).tobytes())]


@pytest.mark.parametrize("alignment,version", [(32, 3), (64, 3), (32, 2)])
def test_gguf_round_trip(tmp_path, alignment, version):
    rng = np.random.default_rng(1)
    path = str(tmp_path / "t.gguf")
    tensors = _tensors(rng)
    gw.write_gguf(path, _kv(), tensors, alignment=alignment, version=version)
    g = kc.Gguf(path)
    try:
        assert g.version() == (version, alignment)
        assert g.str("general.architecture") == "llama"
        assert g.num("k.u8") == 200 and g.num("k.i8") == -100 and g.num("k.u16") == 60000
        assert g.num("k.i16") == -30000 and g.num("k.u32") == 4000000000 and g.num("k.i32") == -2000000000
        assert g.num("k.f32") == 1.5 and g.num("k.bool") == 1 and g.num("k.u64") == 2**40 + 3
        assert g.num("k.i64") == -(2**40) and g.num("k.f64") == 0.1
        assert g.str("k.str") == "héllo"
        assert g.array("k.arr_i32") == (3, gw.I32) and g.array("k.arr_str") == (3, gw.STR)
        assert g.tensor_names() == [t[0] for t in tensors]
        for name, gt, ne, data in tensors:
            t, shape, raw = g.tensor(name)
            assert t == gt and shape == tuple(ne)
            assert raw.tobytes() == data
        with pytest.raises(kc.KcError):
            g.num("k.str")  # a string is not numeric
        with pytest.raises(kc.KcError):
            g.str("missing.key")
        with pytest.raises(kc.KcError):
            g.tensor("missing.tensor")
    finally:
        g.close()


def test_gguf_unknown_type_listed_without_bytes(tmp_path):
    path = str(tmp_path / "u.gguf")
    gw.write_gguf(path, [("general.architecture", gw.STR, "x")], [("u", 99, (8,), b"\0" * 16)])
    g = kc.Gguf(path)
    try:
        t, shape, raw = g.tensor("u")
        assert t == 99 and shape == (8,) and raw.size == 0
    finally:
        g.close()


def _expect_invalid(path, needle):
    with pytest.raises(kc.KcError) as e:
        kc.Gguf(path)
    assert e.value.name == "InvalidValue"
    assert needle in str(e.value), str(e.value)


def test_gguf_rejects_corrupt_files(tmp_path):
    rng = np.random.default_rng(2)
    path = str(tmp_path / "ok.gguf")
    gw.write_gguf(path, _kv(), _tensors(rng))
    blob = open(path, "rb").read()
    bad = str(tmp_path / "bad.gguf")
    # every truncation of the header and of the data section
    for cut in list(range(24, 400, 7)) + [len(blob) - 1, len(blob) - 100]:
        open(bad, "wb").write(blob[:cut])
        with pytest.raises(kc.KcError):
            kc.Gguf(bad)
    open(bad, "wb").write(b"GGUX" + blob[4:])
    _expect_invalid(bad, "magic")
    open(bad, "wb").write(blob[:4] + struct.pack("<I", 1) + blob[8:])
    _expect_invalid(bad, "version")
    open(bad, "wb").write(blob[:8] + struct.pack("<Q", 2**40) + blob[16:])
    _expect_invalid(bad, "implausible")
    # a tensor offset past the end of the file: rewrite the last tensor's offset
    name = b"d.q8_0"
    i = blob.rindex(name) + len(name) + 4 + 8 + 4  # n_dims, ne[0], type
    open(bad, "wb").write(blob[:i] + struct.pack("<Q", 2**30) + blob[i + 8:])
    _expect_invalid(bad, "past the end")
    with pytest.raises(kc.KcError):
        kc.Gguf(str(tmp_path / "does_not_exist.gguf"))


def test_load_gguf_rejects_before_gpu_work(tmp_path):
    """Architecture and hyperparameter checks fail before the model (and the GPU) is touched."""
    path = str(tmp_path / "m.gguf")
    gw.write_gguf(path, [("general.architecture", gw.STR, "gpt2")], [])
    with pytest.raises(kc.KcError) as e:
        kc.Model.load_gguf(path, 64, 8)
    assert "architecture gpt2 not supported" in str(e.value)
    gw.write_gguf(path, [("general.architecture", gw.STR, "llama"), ("llama.block_count", gw.U32, 2)], [])
    with pytest.raises(kc.KcError) as e:
        kc.Model.load_gguf(path, 64, 8)
    assert "missing hyperparameters" in str(e.value)
    kv = [("general.architecture", gw.STR, "llama")] + [(f"llama.{k}", gw.U32, v) for k, v in
                                                         (("block_count", 1), ("embedding_length", 256),
                                                          ("feed_forward_length", 256),
                                                          ("attention.head_count", 2),
                                                          ("rope.dimension_count", 64))]
    gw.write_gguf(path, kv, [])
    with pytest.raises(kc.KcError) as e:
        kc.Model.load_gguf(path, 64, 8)
    assert "partial rotary" in str(e.value)
    gw.write_gguf(path, kv[:-1], [])
    with pytest.raises(kc.KcError) as e:
        kc.Model.load_gguf(path, 64, 8)
    assert "token_embd" in str(e.value)


@pytest.mark.parametrize("key,value,vt", [("block_count", 1e12, "F64"), ("embedding_length", float("nan"), "F64"),
                                          ("attention.head_count", 2.5, "F64"), ("feed_forward_length", 0, "U32"),
                                          ("attention.head_count_kv", -3, "I32"),
                                          ("attention.key_length", float("inf"), "F64"),
                                          ("attention.head_count", 2**40, "U64")])
def test_load_gguf_rejects_out_of_range_hyperparameters(tmp_path, key, value, vt):
    """Counts read as doubles must be whole numbers in [1, 2^31 - 1] before they become ints."""
    path = str(tmp_path / "h.gguf")
    good = {"block_count": 1, "embedding_length": 256, "feed_forward_length": 256, "attention.head_count": 2}
    kv = [("general.architecture", gw.STR, "llama")]
    for k, v in good.items():
        if k != key:
            kv.append((f"llama.{k}", gw.U32, v))
    kv.append((f"llama.{key}", getattr(gw, vt), value))
    gw.write_gguf(path, kv, [])
    with pytest.raises(kc.KcError) as e:
        kc.Model.load_gguf(path, 64, 8)
    assert e.value.name == "InvalidValue"
    assert "whole number" in str(e.value), str(e.value)


def test_load_gguf_rejects_non_finite_epsilon(tmp_path):
    path = str(tmp_path / "e.gguf")
    kv = [("general.architecture", gw.STR, "llama")] + [
        (f"llama.{k}", gw.U32, v) for k, v in (("block_count", 1), ("embedding_length", 256),
                                              ("feed_forward_length", 256), ("attention.head_count", 2))]
    kv.append(("llama.attention.layer_norm_rms_epsilon", gw.F64, float("nan")))
    gw.write_gguf(path, kv, [])
    with pytest.raises(kc.KcError) as e:
        kc.Model.load_gguf(path, 64, 8)
    assert "positive finite" in str(e.value)
