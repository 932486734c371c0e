"""Host-only checks of the MUL_MAT dispatcher (include/kernelcore/mul_mat.h): the backend switches
read from the environment as the reference's backend reads them
(integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp:46-53, 81-86), and the nodes
it refuses before any launch. No GPU: a refused node returns before touching the device, and a
recording allocates nothing until its first accepted node."""
import pytest

import kernelcore_amd as kc

DUMMY = 0x1000  # never dereferenced: every node below is refused first


def env(monkeypatch, **vals):
    for name in ("MATVEC_COLS", "Q8K", "TILE", "ROW_BLOCK"):
        monkeypatch.delenv(f"GGML_KERNELCORE_{name}", raising=False)
    for name, v in vals.items():
        monkeypatch.setenv(f"GGML_KERNELCORE_{name}", v)
    return kc.mul_mat_config_from_env()


def test_defaults(monkeypatch):
    assert env(monkeypatch) == {"matvec_cols": 0, "q8k": 1, "tile": 8, "row_block": 8}


@pytest.mark.parametrize("var,value,field,want", [
    ("MATVEC_COLS", "1", "matvec_cols", 1), ("MATVEC_COLS", "true", "matvec_cols", 0),
    ("MATVEC_COLS", "0", "matvec_cols", 0),
    ("Q8K", "0", "q8k", 0), ("Q8K", "no", "q8k", 1), ("Q8K", "1", "q8k", 1),
    ("TILE", "4", "tile", 4), ("TILE", "16", "tile", 8), ("TILE", "x", "tile", 8),
    ("ROW_BLOCK", "12", "row_block", 12), ("ROW_BLOCK", "0", "row_block", 1), ("ROW_BLOCK", "-5", "row_block", 1),
])
def test_environment_switches(monkeypatch, var, value, field, want):
    assert env(monkeypatch, **{var: value})[field] == want


@pytest.mark.parametrize("bad", [dict(tile=5), dict(tile=0), dict(row_block=0)])
def test_recording_rejects_bad_switches(bad):
    with pytest.raises(kc.KcError) as e:
        kc.MulMatRecording(**bad)
    assert e.value.name == "InvalidValue"


@pytest.mark.parametrize("node,why", [
    (dict(wtype=13), "weight type"),
    (dict(w=None), "null"), (dict(x=None), "null"), (dict(y=None), "null"),
    (dict(rows=12), "rows"), (dict(rows=0), "rows"),
    (dict(k=300), "k must"), (dict(k=0), "k must"), (dict(wtype="f16", k=7), "k must"),
    (dict(ncols=0), "ncols"), (dict(ncols=1 << 31), "ncols"),
    (dict(x_col_bytes=4 * 512 - 4), "x_col_bytes"), (dict(x_col_bytes=4 * 512 + 2), "x_col_bytes"),
    (dict(wtype="f16", x_col_bytes=4 * 512 + 64), "contiguous"),
])
def test_refused_nodes(node, why):
    a = dict(wtype="q4k", w=DUMMY, rows=16, k=512, x=DUMMY, ncols=3, y=DUMMY, x_col_bytes=4 * 512)
    a.update(node)
    rec = kc.MulMatRecording()
    with pytest.raises(kc.KcError) as e:
        rec.mul_mat(a["wtype"], a["w"], a["rows"], a["k"], a["x"], a["ncols"], a["y"], x_col_bytes=a["x_col_bytes"])
    assert e.value.name == "InvalidValue" and why in str(e.value), str(e.value)
    rec.close()


@pytest.mark.parametrize("kind,args,why", [
    ("norm", dict(n=300), "multiple of 256"), ("norm", dict(rows=0), "rows positive"),
    ("norm", dict(n=4096, rows=4096), "2^24"), ("norm", dict(x=None), "null"), ("norm", dict(a=DUMMY), "one of a / b"),
    ("swiglu", dict(n=100), "multiple of 256"), ("swiglu", dict(cols=0), "cols positive"), ("swiglu", dict(u=None), "null"),
])
def test_refused_fused_producers(kind, args, why):
    rec = kc.MulMatRecording()
    with pytest.raises(kc.KcError) as e:
        if kind == "norm":
            a = dict(x=DUMMY, w=DUMMY, y=DUMMY, n=1024, rows=2, eps=1e-5, a=None, b=None)
            a.update(args)
            rec.fused_norm(a["x"], a["w"], a["y"], a["n"], a["rows"], a["eps"], a=a["a"], b=a["b"])
        else:
            a = dict(g=DUMMY, u=DUMMY, y=DUMMY, n=1024, cols=2)
            a.update(args)
            rec.fused_swiglu(a["g"], a["u"], a["y"], a["n"], a["cols"])
    assert e.value.name == "InvalidValue" and why in str(e.value), str(e.value)
    rec.close()
