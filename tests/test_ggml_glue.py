"""The ggml glue (kernelcore_amd/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp) on the CPU: it compiles
(against tests/ggml_stub, a test-only stand-in of the ggml API it uses: llama.cpp is not in this
image), exports the reference backend's entry points (integrations/llama.cpp/ggml/include/
ggml-kernelcore.h:15-17, ggml-kernelcore.cpp:1025-1054), fills every vtable slot the reference
fills (:213-225, :234-246, :272-281, :301-310, :794-811, :968-984, :998-1003) with a callback that
reaches the libkernelcore_amd entry behind it, and answers the registry / device / buffer-type calls
a llama.cpp build makes at start-up -- here without a GPU, where kcInit fails and the backend
claims nothing."""
import os
import re
import subprocess

import pytest

import kernelcore_amd as kc
from tests import glue

SRC = open(glue.GLUE_SRC).read()


def test_glue_compiles_warning_free(tmp_path):
    out = subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
                          "-Wno-missing-field-initializers", f"-I{glue.STUB}",
                          f"-I{os.path.join(kc.ROOT, 'kernelcore_amd', 'ggml', 'include')}",
                          f"-I{os.path.join(kc.ROOT, 'include')}", glue.GLUE_SRC], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr


def test_glue_exports_the_reference_entry_points():
    syms = subprocess.run(["nm", "-D", "--defined-only", glue.LIB_PATH], capture_output=True, text=True,
                          check=True).stdout
    for name in ("ggml_backend_kernelcore_init", "ggml_backend_is_kc", "ggml_backend_kernelcore_reg",
                 "ggml_backend_init"):  # the last: GGML_BACKEND_DL_IMPL
        assert re.search(rf" T {name}$", syms, re.M), name
    hdr = open(os.path.join(kc.ROOT, "kernelcore_amd", "ggml", "include", "ggml-kernelcore.h")).read()
    for decl in ("ggml_backend_t     ggml_backend_kernelcore_init(void)", "bool               ggml_backend_is_kc(ggml_backend_t backend)",
                 "ggml_backend_reg_t ggml_backend_kernelcore_reg(void)"):
        assert decl in hdr


def body(fn):
    """The source of the glue's function fn (its braces matched)."""
    m = re.search(rf"^[\w:<>\s\*&]*?(?<!\w){re.escape(fn)}\((?:[^()]|\([^()]*\))*\)\s*(?:const\s*)?\{{", SRC, re.M)
    assert m, fn
    i, depth = m.end(), 1
    while depth:
        depth += {"{": 1, "}": -1}.get(SRC[i], 0)
        i += 1
    return SRC[m.start():i]


def vtable(name):
    """{slot: callback or 'nullptr'} of the glue's vtable initializer `name`."""
    m = re.search(rf"const ggml_backend_\w+ {name} = \{{(.*?)\n\}};", SRC, re.S)
    assert m, name
    return dict(re.findall(r"/\* \.(\w+)\s*= \*/ (\w+)", m.group(1)))


# Every slot the reference fills (ggml-kernelcore.cpp lines cited), and the libkernelcore_amd entries
# the glue's callback must reach (through the helpers it calls).
REFERENCE_SLOTS = {
    "buffer_i": (":213-225", {"free_buffer": ["kcFree"], "get_base": [], "memset_tensor": ["kcWeightMemsetTensor", "kcMemset"],
                              "set_tensor": ["kcWeightSetTensor", "kcMemcpy"], "get_tensor": ["kcWeightGetTensor", "kcMemcpy"],
                              "clear": ["kcMemset"]}),
    "kv_buffer_i": (":234-246", {"free_buffer": ["kcFree"], "get_base": [], "memset_tensor": ["kcMemset"],
                                 "set_tensor": ["kcMemcpy"], "get_tensor": ["kcMemcpy"], "clear": ["kcMemset"]}),
    "buft_i": (":272-281", {"get_name": [], "alloc_buffer": ["kcMalloc"], "get_alignment": [],
                            "get_alloc_size": ["kcWeightAllocSize"], "is_host": []}),
    "kv_buft_i": (":301-310", {"get_name": [], "alloc_buffer": ["kcMalloc"], "get_alignment": [], "get_alloc_size": [],
                               "is_host": []}),
    "backend_i": (":794-811", {"get_name": [], "free": ["kcGgmlBackendDestroy", "kcStreamDestroy"],
                               "graph_compute": ["kcGgmlGraphCompute"]}),
    "device_i": (":968-984", {"get_name": [], "get_description": [], "get_memory": ["kcDeviceGetMemoryInfo"],
                              "get_type": [], "get_props": ["kcDeviceGetMemoryInfo"],
                              "init_backend": ["kcStreamCreate", "kcGgmlBackendCreate"], "get_buffer_type": [],
                              "get_host_buffer_type": ["kcGgmlOffersKvBuffer"], "supports_op": ["kcGgmlSupportsOp"],
                              "supports_buft": []}),
    "reg_i": (":998-1003", {"get_name": [], "get_device_count": [], "get_device": [], "get_proc_address": []}),
}
HELPERS = {"alloc_buffer": "alloc_buffer", "free": "~BackendCtx", "get_props": "dev_get_memory",
           "init_backend": "ggml_backend_kernelcore_init"}


def reaches(fn, entry, seen=None):
    """Whether fn's body, or a glue function it calls, names entry."""
    seen = seen or set()
    if fn in seen:
        return False
    seen.add(fn)
    b = body(fn)
    if entry in b:
        return True
    for callee in set(re.findall(r"\b([a-z_][a-z_0-9]*)\(", b)) - {fn}:
        if re.search(rf"^[\w:<>\s\*&]*\b{callee}\(", SRC, re.M) and callee not in ("if", "for", "while", "switch", "return",
                                                                                   "sizeof", "static_cast"):
            try:
                if reaches(callee, entry, seen):
                    return True
            except AssertionError:
                pass
    return False


@pytest.mark.parametrize("table", list(REFERENCE_SLOTS))
def test_every_reference_slot_is_filled_and_reaches_its_kc_entry(table):
    where, slots = REFERENCE_SLOTS[table]
    filled = vtable(table)
    for slot, entries in slots.items():
        fn = filled.get(slot)
        assert fn and fn != "nullptr", f"{table}.{slot} (reference {where})"
        for entry in entries:
            start = fn
            if slot == "free" and table == "backend_i":
                start = "~BackendCtx"
            assert reaches(start, entry) or reaches(HELPERS.get(slot, fn), entry), f"{table}.{slot}: {fn} -> {entry}"


def test_the_kept_graph_entry_points_exist_in_the_library():
    L = kc.lib()
    for name in ("kcGgmlGraphCompute", "kcGgmlSupportsOp", "kcGgmlOffersKvBuffer", "kcWeightMemsetTensor",
                 "kcDeviceGetMemoryInfo", "kcGgmlBackendGetProfile"):
        assert hasattr(L, name)


def test_startup_calls_without_a_device():
    """What llama.cpp asks at start-up (ggml_backend_dev_get_props etc.): one ACCEL device named
    Kernelcore; with no GPU (kcInit fails here) memory 0 / 0 and mmap allowed (nothing is claimed),
    the weights' buffer type offered, the KV one not, and no op supported."""
    i = glue.info()
    assert (i["reg"], i["name"], i["devices"], glue.DEVICE_TYPES[i["type"]]) == ("Kernelcore", "Kernelcore", 1, "ACCEL")
    assert i["dl_init"] and i["api_version"] >= 1
    if kc.lib().kcGetDeviceCount is not None and i["memory_total"] == 0:
        assert i["mmap_support"]
        assert glue.buft(1) is None
        assert glue.lib().kcgt_supports_mul_mat(12, 3072, 3072, 1, 0) == 0
    w = glue.buft(0)
    assert w == dict(name="Kernelcore", alignment=64, is_host=False, supported=True)


@pytest.mark.parametrize("type_,ne0,ne1", [(12, 3072, 3072), (14, 3072, 128256), (12, 256, 8), (14, 768, 40),
                                            (0, 3072, 7), (1, 130, 24), (12, 3072, 7)])
def test_alloc_size_is_the_stream_for_kquant_weights(type_, ne0, ne1):
    """get_alloc_size (:259-266): a 2-D K-quant weight of whole 8-row groups takes its stream
    (kcWeightAllocSize; at least its ggml bytes), anything else its ggml bytes."""
    got = glue.lib().kcgt_alloc_size(0, type_, ne0, ne1)
    bb = {12: 144, 14: 210}.get(type_)
    nbytes = ne0 // 256 * bb * ne1 if bb else ne0 * ne1 * (4 if type_ == 0 else 2)
    if bb and ne1 % 8 == 0:
        assert got == max(kc.stream_bytes({12: "q4k", 14: "q6k"}[type_], ne1, ne0), nbytes)
    else:
        assert got == nbytes
