"""Python bindings of libkernelcore_amd.so (the kc* C ABI in include/kernelcore/kc.h).

The library is the product: HIP kernels for gfx950 plus the kc* runtime in C++. This module is a
thin ctypes layer for tests and benchmarks; it holds no compute of its own and never falls back
to a CPU path. If the shared library is missing it raises, and on a machine without a GPU
``kcInit`` returns an error that surfaces as ``KcError``.

Struct layouts mirror include/kernelcore/llm_kernels.h (which keeps the field order of the
reference's llm/llm_kernels.hpp).
"""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libkernelcore_amd.so")
HEADERS = [os.path.join(ROOT, "include", "kernelcore", n) for n in ("kc.h", "llm_kernels.h", "model.h", "gguf.h",
                                                                                   "mul_mat.h", "weights.h",
                                                                                   "ggml_backend.h")]

ERRORS = ["Success", "NotInitialized", "InvalidValue", "InvalidDevice", "OutOfMemory", "InvalidPointer",
          "InvalidResourceHandle", "UnsupportedOperation", "InvalidKernelImage", "KernelNotFound",
          "DynamicCodeBlocked", "LaunchFailure", "KernelFault", "ContextPoisoned", "NotReady", "InternalError"]
ERR = {name: i for i, name in enumerate(ERRORS)}
HOST_TO_DEVICE, DEVICE_TO_HOST, DEVICE_TO_DEVICE, HOST_TO_HOST = range(4)
QTYPE = {"q4k": 12, "q6k": 14, "f16": 1}
BLOCK_BYTES = {"q4k": 144, "q6k": 210}

_p = C.c_void_p
_i = C.c_int
_f = C.c_float


class KcError(RuntimeError):
    def __init__(self, fn, code, detail):
        self.code = code
        self.name = ERRORS[code] if 0 <= code < len(ERRORS) else f"error {code}"
        super().__init__(f"{fn}: {self.name}" + (f" ({detail})" if detail else ""))


# ---- argument structs (include/kernelcore/llm_kernels.h) -----------------------------------------

def _struct(name, fields):
    return type(name, (C.Structure,), {"_fields_": fields})


VectorAddArgs = _struct("VectorAddArgs", [("a", _p), ("b", _p), ("out", _p), ("count", _i)])
QuantizeArgs = _struct("QuantizeArgs", [("x", _p), ("xq", _p), ("xd", _p), ("count", _i)])
MatvecQ4Q8Args = _struct("MatvecQ4Q8Args", [("qw", _p), ("xq", _p), ("xd", _p), ("y", _p), ("dims", _p),
                                            ("rows", _i), ("k", _i)])
MatmulKQ8Args = _struct("MatmulKQ8Args", [("qw", _p), ("xq", _p), ("y", _p), ("dims", _p), ("rows", _i), ("k", _i),
                                          ("ncols", _i), ("row_block", _i)])
MatmulF16Args = _struct("MatmulF16Args", [("qw", _p), ("x", _p), ("y", _p), ("dims", _p), ("rows", _i), ("k", _i),
                                          ("ncols", _i)])
QuantizeColsArgs = _struct("QuantizeColsArgs", [("x", _p), ("q", _p), ("dims", _p), ("k", _i), ("ncols", _i)])
RmsNormArgs = _struct("RmsNormArgs", [("x", _p), ("w", _p), ("y", _p), ("n", _i), ("rows", _i), ("eps", _f)])
MulRowsArgs = _struct("MulRowsArgs", [("x", _p), ("w", _p), ("y", _p), ("n", _i), ("count", _i)])
RopeGgmlArgs = _struct("RopeGgmlArgs", [("x", _p), ("y", _p), ("pos", _p), ("ff", _p), ("dims", _p), ("head_dim", _i),
                                        ("n_head", _i), ("n_tokens", _i), ("log2_base", _f), ("neox", C.c_bool)])
AddSumsqFArgs = _struct("AddSumsqFArgs", [("a", _p), ("b", _p), ("out", _p), ("q", _p), ("dims", _p), ("n", _i),
                                          ("rows", _i)])
SumsqPartArgs = _struct("SumsqPartArgs", [("x", _p), ("q", _p), ("dims", _p), ("n", _i), ("rows", _i)])
NormMulQ8Args = _struct("NormMulQ8Args", [("x", _p), ("w", _p), ("y", _p), ("q", _p), ("dims", _p), ("n", _i),
                                          ("rows", _i), ("eps", _f)])
AddNormQ8FArgs = _struct("AddNormQ8FArgs", [("a", _p), ("b", _p), ("x", _p), ("w", _p), ("y", _p), ("q", _p),
                                            ("dims", _p), ("n", _i), ("rows", _i), ("eps", _f)])
SiluMulQ8FArgs = _struct("SiluMulQ8FArgs", [("g", _p), ("u", _p), ("y", _p), ("q", _p), ("dims", _p), ("n", _i),
                                            ("cols", _i)])
SiluMulArgs = _struct("SiluMulArgs", [("g", _p), ("u", _p), ("out", _p), ("count", _i)])
SetRowsF16Args = _struct("SetRowsF16Args", [("src", _p), ("idx", _p), ("dst", _p), ("dims", _p), ("pairs", _i),
                                            ("rows", _i), ("src_row", _i), ("dst_row", _i), ("dst_rows", _i)])
FaDims = _struct("FaDims", [(n, _i) for n in ("H", "T", "D", "group", "tp", "k_row", "k_head", "v_row", "v_head",
                                              "N", "q_tok", "q_head", "m_row", "has_mask", "H_kv")])
FaScoresArgs = _struct("FaScoresArgs", [("q", _p), ("k", _p), ("mask", _p), ("s", _p), ("dims", _p), ("d", FaDims),
                                        ("scale", _f)])
FaMaxArgs = _struct("FaMaxArgs", [("s", _p), ("m", _p), ("dims", _p), ("d", FaDims)])
FaExpArgs = _struct("FaExpArgs", [("s", _p), ("m", _p), ("dims", _p), ("d", FaDims)])
FaValuesArgs = _struct("FaValuesArgs", [("p", _p), ("v", _p), ("out", _p), ("dims", _p), ("d", FaDims)])
FlashAttnArgs = _struct("FlashAttnArgs", [("q", _p), ("k", _p), ("v", _p), ("mask", _p), ("out", _p), ("dims", _p),
                                          ("d", FaDims), ("scale", _f)])
FlashDecodeArgs = _struct("FlashDecodeArgs", [("q", _p), ("k", _p), ("v", _p), ("mask", _p), ("out", _p),
                                             ("part", _p), ("dims", _p), ("d", FaDims), ("scale", _f)])
GetRowsKquantArgs = _struct("GetRowsKquantArgs", [("qw", _p), ("ids", _p), ("y", _p), ("qtype", _i), ("rows", _i),
                                                  ("k", _i), ("n", _i)])
QuantizeKquantArgs = _struct("QuantizeKquantArgs", [("x", _p), ("blocks", _p), ("qtype", _i), ("rows", _i), ("k", _i)])
FillNormalArgs = _struct("FillNormalArgs", [("y", _p), ("n", C.c_longlong), ("seed", C.c_ulonglong), ("mean", _f),
                                            ("stdev", _f)])
KquantRepackArgs = _struct("KquantRepackArgs", [("src", _p), ("dst", _p), ("qtype", _i), ("rows", _i), ("k", _i)])
DeviceProperties = _struct("DeviceProperties", [("name", C.c_char * 128), ("worker_count", C.c_uint),
                                                ("performance_workers", C.c_uint), ("total_memory", C.c_size_t),
                                                ("is_hardware_gpu", C.c_bool), ("guard_pages", C.c_bool),
                                                ("large_pages", C.c_bool), ("kernel_stack_bytes", C.c_size_t)])
ModelConfig = _struct("ModelConfig", [("n_layer", _i), ("n_embd", _i), ("n_head", _i), ("n_head_kv", _i),
                                      ("head_dim", _i), ("n_ff", _i), ("n_vocab", _i), ("norm_eps", _f),
                                      ("rope_theta", _f), ("rope_neox", _i), ("qk_norm", _i), ("max_ctx", _i),
                                      ("max_batch", _i)])
TENSORS = {"token_embd": 0, "output_norm": 1, "output": 2, "attn_norm": 3, "wq": 4, "wk": 5, "wv": 6, "wo": 7,
           "ffn_norm": 8, "w_gate": 9, "w_up": 10, "w_down": 11, "q_norm": 12, "k_norm": 13, "rope_freqs": 14}
KernelEntry = _struct("KernelEntry", [("name", C.c_char_p), ("validate", _p), ("launch", _p), ("chunkable", _i)])

# ---- library ----------------------------------------------------------------------------------------

_LIB = None


def build(jobs: int = 8) -> None:
    """Compiles libkernelcore_amd.so for gfx950 (make -C kernelcore_amd)."""
    subprocess.run(["make", "-s", "-C", HERE, f"-j{jobs}"], check=True)


def declared_symbols():
    """Every function the public headers declare with KC_API."""
    names = set()
    for h in HEADERS:
        text = open(h).read()
        for m in re.finditer(r"KC_API\s+[^;(]*?\b(kc\w+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def lib():
    """The loaded library; raises if it was not built (there is no fallback)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() or make -C kernelcore_amd")
        L = C.CDLL(LIB_PATH)
        for name in declared_symbols():
            getattr(L, name).restype = _i
        for name in ("kcGetErrorString", "kcCodegenName", "kcGetLastErrorDetail"):
            getattr(L, name).restype = C.c_char_p
        L.kcMalloc.argtypes = [C.POINTER(_p), C.c_size_t]
        L.kcFree.argtypes = [_p]
        L.kcMemcpy.argtypes = [_p, _p, C.c_size_t, _i]
        L.kcMemset.argtypes = [_p, _i, C.c_size_t]
        L.kcLaunchKernel.argtypes = [C.c_char_p, _p, _p]
        L.kcLaunchKernelChunked.argtypes = [C.c_char_p, _p, C.c_uint, C.c_int64, _p]
        L.kcKquantStreamBytes.argtypes = [_i, _i, _i, C.POINTER(C.c_size_t)]
        L.kcEventElapsedTime.argtypes = [C.POINTER(_f), _p, _p]
        for n in ("kcEventRecord", "kcStreamWaitEvent"):
            getattr(L, n).argtypes = [_p, _p]
        L.kcSetKernelOption.argtypes = [C.c_char_p, _i]
        L.kcGetKernelOption.argtypes = [C.c_char_p, C.POINTER(_i)]
        L.kcModelCreate.argtypes = [C.POINTER(ModelConfig), C.POINTER(_p)]
        L.kcModelDestroy.argtypes = [_p]
        L.kcModelPlanDecode.argtypes = [C.POINTER(ModelConfig), C.POINTER(_i)]
        L.kcModelTensorInfo.argtypes = [_p, _i, _i, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i), C.POINTER(C.c_size_t)]
        L.kcModelSetTensor.argtypes = [_p, _i, _i, _p, C.c_size_t]
        L.kcModelSetTensorTyped.argtypes = [_p, _i, _i, _i, _p, C.c_size_t]
        L.kcModelLoadGguf.argtypes = [C.c_char_p, _i, _i, C.POINTER(_p)]
        L.kcGgufOpen.argtypes = [C.c_char_p, C.POINTER(_p)]
        L.kcGgufClose.argtypes = [_p]
        L.kcGgufVersion.argtypes = [_p, C.POINTER(_i), C.POINTER(_i)]
        L.kcGgufGetNum.argtypes = [_p, C.c_char_p, C.POINTER(C.c_double)]
        L.kcGgufGetStr.argtypes = [_p, C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t)]
        L.kcGgufGetArray.argtypes = [_p, C.c_char_p, C.POINTER(C.c_int64), C.POINTER(_i)]
        L.kcGgufTensorCount.argtypes = [_p, C.POINTER(_i)]
        L.kcGgufTensorName.argtypes = [_p, _i, C.POINTER(C.c_char_p)]
        L.kcGgufTensorInfo.argtypes = [_p, C.c_char_p, C.POINTER(_i), C.POINTER(_i), C.POINTER(C.c_int64),
                                       C.POINTER(C.c_size_t), C.POINTER(_p)]
        L.kcModelForward.argtypes = [_p, _p, _i, _p]
        L.kcModelGenerate.argtypes = [_p, _i, _p]
        L.kcModelPosition.argtypes = [_p, C.POINTER(_i)]
        L.kcModelReset.argtypes = [_p]
        L.kcModelReadCache.argtypes = [_p, _i, _i, _i, _i, _p]
        L.kcModelStream.argtypes = [_p, C.POINTER(_p)]
        L.kcMulMatConfigFromEnv.argtypes = [C.POINTER(MulMatConfig)]
        L.kcMulMatConfigFromEnv.restype = None
        L.kcMulMatRecordingCreate.argtypes = [C.POINTER(_p), C.POINTER(MulMatConfig), _p]
        L.kcMulMatRecordingReset.argtypes = [_p]
        L.kcMulMatRecordingDestroy.argtypes = [_p]
        L.kcMulMat.argtypes = [_p, C.POINTER(MulMatNode), C.POINTER(MulMatPlan)]
        L.kcWeightAllocSize.argtypes = [_i, _i, _i, C.POINTER(C.c_size_t)]
        L.kcWeightSetTensor.argtypes = [_i, _i, _i, _p, _p, C.c_size_t, C.c_size_t, _p]
        L.kcWeightGetTensor.argtypes = [_i, _i, _i, _p, _p, C.c_size_t, C.c_size_t, _p]
        L.kcWeightMemsetTensor.argtypes = [_i, _i, _i, _p, _i, C.c_size_t, C.c_size_t, _p]
        L.kcDeviceGetMemoryInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        L.kcGgmlBackendGetProfile.argtypes = [_p, _p, _i, C.POINTER(_i)]
        L.kcMulMatFusedNorm.argtypes = [_p, C.POINTER(MulMatNormNode), C.POINTER(MulMatPlan)]
        L.kcMulMatFusedSwiglu.argtypes = [_p, C.POINTER(MulMatSwigluNode), C.POINTER(MulMatPlan)]
        L.kcGgmlConfigFromEnv.argtypes = [C.POINTER(GgmlConfig)]
        L.kcGgmlConfigFromEnv.restype = None
        L.kcGgmlSupportsOp.argtypes = [C.POINTER(GgmlConfig), C.POINTER(GgmlTensor)]
        L.kcGgmlOffersKvBuffer.argtypes = [C.POINTER(GgmlConfig)]
        L.kcGgmlGraphPlan.argtypes = [C.POINTER(GgmlConfig), _p, _i, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t),
                                      C.POINTER(C.c_size_t)]
        L.kcGgmlBackendCreate.argtypes = [C.POINTER(_p), C.POINTER(GgmlConfig), _p]
        L.kcGgmlBackendDestroy.argtypes = [_p]
        L.kcGgmlGraphCompute.argtypes = [_p, _p, _i]
        L.kcGgmlBackendGetStats.argtypes = [_p, C.POINTER(GgmlStats)]
        L.kcGetErrorString.argtypes = [_i]
        L.kcCodegenName.argtypes = [_i]
        _LIB = L
    return _LIB


def check(fn, code):
    if code != 0:
        raise KcError(fn, code, lib().kcGetLastErrorDetail().decode(errors="replace"))


def call(fn, *args):
    """Calls kc<fn>(*args) and raises KcError on failure."""
    check(fn, getattr(lib(), fn)(*args))


def status(fn, *args):
    """Calls kc<fn>(*args) and returns the error name ("Success", "InvalidValue", ...)."""
    return ERRORS[getattr(lib(), fn)(*args)]


def stream_bytes(qtype, rows, k):
    n = C.c_size_t()
    call("kcKquantStreamBytes", QTYPE[qtype], rows, k, C.byref(n))
    return n.value


class Buffer:
    """A kcMalloc allocation with numpy transfers."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = _p()
        call("kcMalloc", C.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    @classmethod
    def of(cls, array):
        a = np.ascontiguousarray(array)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, array, offset=0):
        a = np.ascontiguousarray(array)
        if a.nbytes:
            call("kcMemcpy", self.ptr + offset, a.ctypes.data, a.nbytes, HOST_TO_DEVICE)

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        if out.nbytes:
            call("kcMemcpy", out.ctypes.data, self.ptr + offset, out.nbytes, DEVICE_TO_HOST)
        return out

    def at(self, offset):
        return self.ptr + offset

    def free(self):
        if self.ptr:
            lib().kcFree(self.ptr)
            self.ptr = None


def init():
    call("kcInit")


def launch(name, args, stream=None):
    check(f"kcLaunchKernel({name})", lib().kcLaunchKernel(name.encode(), C.byref(args), stream))


def launch_status(name, args, stream=None):
    return ERRORS[lib().kcLaunchKernel(name.encode(), C.byref(args), stream)]


def synchronize():
    call("kcDeviceSynchronize")


def set_option(name, value):
    call("kcSetKernelOption", name.encode(), value)


def device_properties():
    p = DeviceProperties()
    call("kcGetDeviceProperties", C.byref(p), 0)
    return p


# ---- typed helpers over the built-in kernels ---------------------------------------------------------

def repack(qtype, blocks: Buffer, rows, k, stream=None):
    """ggml blocks (rows x k/256, device) -> a new weight-stream Buffer."""
    out = Buffer(stream_bytes(qtype, rows, k))
    launch("repack_kquant", KquantRepackArgs(blocks.ptr, out.ptr, QTYPE[qtype], rows, k), stream)
    return out


def upload_weights(qtype, blocks_np, rows, k):
    """Uploads raw ggml block bytes and repacks them on the GPU; returns the stream Buffer."""
    raw = Buffer.of(np.ascontiguousarray(blocks_np, np.uint8))
    try:
        return repack(qtype, raw, rows, k)
    finally:
        raw.free()


def plan_decode(**cfg):
    """kcModelPlanDecode (host only): 1 when single tokens take the fused kernels, else 0; raises
    KcError (InvalidValue) for a config the driver rejects."""
    c = ModelConfig(**cfg)
    fused = _i()
    call("kcModelPlanDecode", C.byref(c), C.byref(fused))
    return fused.value


WEIGHT_TYPES = {"f32": 0, "f16": 1, "q4k": 12, "q6k": 14}


def weight_alloc_size(qtype, rows, k):
    """kcWeightAllocSize (host only): device bytes of a rows x k weight of qtype."""
    n = C.c_size_t()
    call("kcWeightAllocSize", WEIGHT_TYPES.get(qtype, qtype), rows, k, C.byref(n))
    return n.value


def weight_set(qtype, rows, k, dst, data, offset=0, stream=None):
    """kcWeightSetTensor: host bytes (a numpy array) at `offset` of the tensor's ggml form into dst."""
    a = np.ascontiguousarray(data)
    call("kcWeightSetTensor", WEIGHT_TYPES.get(qtype, qtype), rows, k, dst, a.ctypes.data, offset, a.nbytes, stream)


def weight_memset(qtype, rows, k, dst, value, offset, size, stream=None):
    """kcWeightMemsetTensor: bytes [offset, offset + size) of the tensor's ggml form set to value."""
    call("kcWeightMemsetTensor", WEIGHT_TYPES.get(qtype, qtype), rows, k, dst, value, offset, size, stream)


def device_memory():
    """kcDeviceGetMemoryInfo: (free, total) HBM bytes."""
    f, t = C.c_size_t(), C.c_size_t()
    call("kcDeviceGetMemoryInfo", C.byref(f), C.byref(t))
    return f.value, t.value


def weight_get(qtype, rows, k, src, offset, size, stream=None):
    """kcWeightGetTensor: bytes [offset, offset + size) of the tensor's ggml form (uint8 array)."""
    out = np.zeros(size, np.uint8)
    call("kcWeightGetTensor", WEIGHT_TYPES.get(qtype, qtype), rows, k, src, out.ctypes.data, offset, size, stream)
    return out


class MulMatConfig(C.Structure):
    """kcMulMatConfig (include/kernelcore/mul_mat.h): the backend's switches."""
    _fields_ = [("matvec_cols", _i), ("q8k", _i), ("tile", _i), ("row_block", _i)]


class MulMatNode(C.Structure):
    """kcMulMatNode: one MUL_MAT node (weights w: rows x k of wtype; input x: ncols columns)."""
    _fields_ = [("wtype", _i), ("w", _p), ("rows", _i), ("k", _i), ("x", _p), ("ncols", C.c_longlong),
                ("x_col_bytes", C.c_size_t), ("y", _p)]


class MulMatNormNode(C.Structure):
    """kcMulMatNormNode: [ADD +] RMS_NORM + MUL, quantized for the MUL_MATs reading y."""
    _fields_ = [("a", _p), ("b", _p), ("x", _p), ("w", _p), ("y", _p), ("n", _i), ("rows", _i), ("eps", _f)]


class MulMatSwigluNode(C.Structure):
    """kcMulMatSwigluNode: SWIGLU, quantized for the MUL_MATs reading y."""
    _fields_ = [("g", _p), ("u", _p), ("y", _p), ("n", _i), ("cols", _i)]


class MulMatPlan(C.Structure):
    """kcMulMatPlan: what a node recorded."""
    _fields_ = [("quantizer", C.c_char * 24), ("input_reused", _i), ("kernel", C.c_char * 24), ("launches", _i),
                ("k256", _i)]

    def as_dict(self):
        return {"quantizer": self.quantizer.decode(), "input_reused": bool(self.input_reused),
                "kernel": self.kernel.decode(), "launches": self.launches, "k256": bool(self.k256)}


def mul_mat_config_from_env():
    """kcMulMatConfigFromEnv (host only): the reference's defaults and GGML_KERNELCORE_* overrides."""
    c = MulMatConfig()
    lib().kcMulMatConfigFromEnv(C.byref(c))
    return {"matvec_cols": c.matvec_cols, "q8k": c.q8k, "tile": c.tile, "row_block": c.row_block}


class MulMatRecording:
    """A kcMulMat recording: MUL_MAT nodes dispatched as the reference's ggml backend does, inputs
    quantized once per recording (include/kernelcore/mul_mat.h)."""

    def __init__(self, stream=None, **cfg):
        c = None
        if cfg:
            base = mul_mat_config_from_env()
            base.update(cfg)
            c = MulMatConfig(**base)
        h = _p()
        call("kcMulMatRecordingCreate", C.byref(h), C.byref(c) if c is not None else None, stream)
        self.h = h

    def reset(self):
        call("kcMulMatRecordingReset", self.h)

    def mul_mat(self, wtype, w, rows, k, x, ncols, y, x_col_bytes=None):
        """Records one node; returns its plan as a dict. wtype: "q4k", "q6k" or "f16" (or the id)."""
        wt = {"q4k": 12, "q6k": 14, "f16": 1}.get(wtype, wtype)
        node = MulMatNode(wt, w, rows, k, x, ncols, x_col_bytes if x_col_bytes is not None else 4 * k, y)
        plan = MulMatPlan()
        call("kcMulMat", self.h, C.byref(node), C.byref(plan))
        return plan.as_dict()

    def fused_norm(self, x, w, y, n, rows, eps, a=None, b=None):
        """[x = a + b;] y = rms_norm(x) * w, its slots registered for the next MUL_MATs; the plan."""
        plan = MulMatPlan()
        call("kcMulMatFusedNorm", self.h, C.byref(MulMatNormNode(a, b, x, w, y, n, rows, eps)), C.byref(plan))
        return plan.as_dict()

    def fused_swiglu(self, g, u, y, n, cols):
        """y = silu(g) * u, its slots registered for the next MUL_MATs; the plan."""
        plan = MulMatPlan()
        call("kcMulMatFusedSwiglu", self.h, C.byref(MulMatSwigluNode(g, u, y, n, cols)), C.byref(plan))
        return plan.as_dict()

    def close(self):
        if self.h:
            call("kcMulMatRecordingDestroy", self.h)
            self.h = None


# ---- the ggml backend core (include/kernelcore/ggml_backend.h) --------------------------------------

GGML_OP = {"none": 0, "reshape": 1, "view": 2, "permute": 3, "transpose": 4, "mul_mat": 5, "add": 6, "rms_norm": 7,
           "mul": 8, "rope": 9, "glu": 10, "set_rows": 11, "flash_attn_ext": 12, "other": 13}
GGML_TYPE = {"f32": 0, "f16": 1, "q4k": 12, "q6k": 14, "i32": 26, "i64": 27}
GGML_BUFFER = {"other": 0, "weights": 1, "kv": 2}


class GgmlTensor(C.Structure):
    """kcGgmlTensor: one ggml tensor as the backend core reads it."""


GgmlTensor._fields_ = [("op", _i), ("type", _i), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("data", _p),
                       ("src", C.POINTER(GgmlTensor) * 5), ("op_params", C.c_int32 * 16), ("buffer", _i),
                       ("compute", _i), ("output", _i), ("view", _i), ("uses", _i)]


class GgmlConfig(C.Structure):
    """kcGgmlConfig: the backend's switches."""
    _fields_ = [("mul_mat", MulMatConfig), ("disabled", _i), ("matmul_only", _i), ("attn", _i), ("attn_tokens", _i),
                ("concurrent", _i), ("graphs", _i), ("profile", _i)]


class GgmlStats(C.Structure):
    """kcGgmlStats: what a backend's graph_compute calls did."""
    _fields_ = [("computes", C.c_longlong), ("graphs_recorded", C.c_longlong), ("graphs_reused", C.c_longlong),
                ("launches", C.c_longlong), ("compute_ms", C.c_double), ("record_ms", C.c_double), ("run_ms", C.c_double)]


class GgmlProfileEntry(C.Structure):
    """kcGgmlProfileEntry: one launch name's device time (profile = 2)."""
    _fields_ = [("name", C.c_char * 64), ("launches", C.c_longlong), ("ms", C.c_double)]


_MM_KEYS = ("matvec_cols", "q8k", "tile", "row_block")


def ggml_config(**over):
    """kcGgmlConfigFromEnv (host only) with the given switches overridden: a GgmlConfig."""
    c = GgmlConfig()
    lib().kcGgmlConfigFromEnv(C.byref(c))
    for k, v in over.items():
        if k in _MM_KEYS:
            setattr(c.mul_mat, k, int(v))
        else:
            setattr(c, k, int(v))
    return c


def ggml_config_dict(c):
    d = {k: getattr(c.mul_mat, k) for k in _MM_KEYS}
    d.update({k: getattr(c, k) for k, _ in GgmlConfig._fields_[1:]})
    return d


def _node_array(nodes):
    arr = (C.POINTER(GgmlTensor) * max(1, len(nodes)))(*[C.pointer(t) for t in nodes])
    return arr


class GgmlNodes:
    """A node list converted once to the array kcGgmlGraphCompute reads (a caller that computes the
    same graph every step passes this instead of rebuilding the array each time, as ggml's own
    cgraph node array is passed)."""

    def __init__(self, nodes):
        self.n = len(nodes)
        self.arr = _node_array(nodes)


def ggml_supports_op(t, **cfg):
    """kcGgmlSupportsOp: whether the backend claims t (host logic only)."""
    return bool(lib().kcGgmlSupportsOp(C.byref(ggml_config(**cfg)), C.byref(t)))


def ggml_offers_kv_buffer(**cfg):
    return bool(lib().kcGgmlOffersKvBuffer(C.byref(ggml_config(**cfg))))


def ggml_graph_plan(nodes, **cfg):
    """kcGgmlGraphPlan: the launch names graph_compute would make for nodes, and its scratch ints
    (no device needed)."""
    arr = _node_array(nodes)
    need, ints = C.c_size_t(), C.c_size_t()
    c = ggml_config(**cfg)
    call("kcGgmlGraphPlan", C.byref(c), arr, len(nodes), None, 0, C.byref(need), C.byref(ints))
    buf = C.create_string_buffer(need.value)
    call("kcGgmlGraphPlan", C.byref(c), arr, len(nodes), buf, need.value, None, None)
    return buf.value.decode().split(), ints.value


class GgmlBackend:
    """A kcGgmlBackend: graph_compute over descriptor lists on one stream."""

    def __init__(self, stream=None, **cfg):
        h = _p()
        call("kcGgmlBackendCreate", C.byref(h), C.byref(ggml_config(**cfg)), stream)
        self.h = h

    def compute(self, nodes):
        if isinstance(nodes, GgmlNodes):
            call("kcGgmlGraphCompute", self.h, nodes.arr, nodes.n)
        else:
            call("kcGgmlGraphCompute", self.h, _node_array(nodes), len(nodes))

    def stats(self):
        s = GgmlStats()
        call("kcGgmlBackendGetStats", self.h, C.byref(s))
        return {k: getattr(s, k) for k, _ in GgmlStats._fields_}

    def profile(self):
        """kcGgmlBackendGetProfile: {launch name: (launches, ms)} of profile = 2."""
        n = _i()
        call("kcGgmlBackendGetProfile", self.h, None, 0, C.byref(n))
        arr = (GgmlProfileEntry * max(1, n.value))()
        call("kcGgmlBackendGetProfile", self.h, arr, n.value, C.byref(n))
        return {arr[i].name.decode(): (arr[i].launches, arr[i].ms) for i in range(n.value)}

    def close(self):
        if self.h:
            call("kcGgmlBackendDestroy", self.h)
            self.h = None


class Model:
    """The decode driver (include/kernelcore/model.h)."""

    def __init__(self, **cfg):
        self.cfg = ModelConfig(**cfg)
        h = _p()
        call("kcModelCreate", C.byref(self.cfg), C.byref(h))
        self.h = h

    def tensor_info(self, tensor, layer=-1):
        qt, rows, k, nb = _i(), _i(), _i(), C.c_size_t()
        call("kcModelTensorInfo", self.h, TENSORS.get(tensor, tensor), layer, C.byref(qt), C.byref(rows), C.byref(k),
             C.byref(nb))
        return qt.value, rows.value, k.value, nb.value

    def set_tensor(self, tensor, layer, data, qtype=None):
        """Raw ggml blocks (or floats); qtype "q4k" / "q6k" picks a matrix's type (default: the
        tensor's default type)."""
        a = np.ascontiguousarray(data)
        t = TENSORS.get(tensor, tensor)
        if qtype is None:
            call("kcModelSetTensor", self.h, t, layer, a.ctypes.data, a.nbytes)
        else:
            call("kcModelSetTensorTyped", self.h, t, layer, QTYPE.get(qtype, qtype), a.ctypes.data, a.nbytes)

    @classmethod
    def load_gguf(cls, path, max_ctx, max_batch):
        """kcModelLoadGguf: a model (and its config) from a GGUF file."""
        self = cls.__new__(cls)
        h = _p()
        call("kcModelLoadGguf", os.fsencode(path), max_ctx, max_batch, C.byref(h))
        self.h = h
        n_vocab = _i()
        call("kcModelTensorInfo", h, 0, 0, None, C.byref(n_vocab), None, None)
        self.cfg = ModelConfig(n_vocab=n_vocab.value)
        return self

    def forward(self, tokens, want_logits=True):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros(self.cfg.n_vocab, np.float32) if want_logits else None
        call("kcModelForward", self.h, t.ctypes.data, t.size, out.ctypes.data if want_logits else None)
        return out

    def generate(self, steps):
        out = np.zeros(steps, np.int32)
        call("kcModelGenerate", self.h, steps, out.ctypes.data)
        return out

    def position(self):
        p = _i()
        call("kcModelPosition", self.h, C.byref(p))
        return p.value

    def read_cache(self, layer, which, pos0, n):
        """fp16 bits (uint16) of positions [pos0, pos0 + n) of a layer's k (which 0) or v (1) cache."""
        kvd = self.cfg.n_head_kv * self.cfg.head_dim
        out = np.zeros(max(n, 1) * kvd, np.uint16)
        call("kcModelReadCache", self.h, layer, which, pos0, n, out.ctypes.data)
        return out[: n * kvd]

    def reset(self):
        call("kcModelReset", self.h)

    def stream(self):
        s = _p()
        call("kcModelStream", self.h, C.byref(s))
        return s

    def close(self):
        if self.h:
            lib().kcModelDestroy(self.h)
            self.h = None


class Gguf:
    """A GGUF file opened read-only (include/kernelcore/gguf.h)."""

    def __init__(self, path):
        h = _p()
        call("kcGgufOpen", os.fsencode(path), C.byref(h))
        self.h = h

    def version(self):
        v, a = _i(), _i()
        call("kcGgufVersion", self.h, C.byref(v), C.byref(a))
        return v.value, a.value

    def num(self, key):
        v = C.c_double()
        call("kcGgufGetNum", self.h, key.encode(), C.byref(v))
        return v.value

    def str(self, key):
        p, n = C.c_char_p(), C.c_size_t()
        call("kcGgufGetStr", self.h, key.encode(), C.byref(p), C.byref(n))
        return C.string_at(p, n.value).decode()

    def array(self, key):
        n, t = C.c_int64(), _i()
        call("kcGgufGetArray", self.h, key.encode(), C.byref(n), C.byref(t))
        return n.value, t.value

    def tensor_names(self):
        n = _i()
        call("kcGgufTensorCount", self.h, C.byref(n))
        out = []
        for i in range(n.value):
            p = C.c_char_p()
            call("kcGgufTensorName", self.h, i, C.byref(p))
            out.append(p.value.decode())
        return out

    def tensor(self, name):
        """(ggml type, shape ne[:n_dims], the tensor's bytes as a uint8 array copied out of the map)"""
        t, nd, nb, data = _i(), _i(), C.c_size_t(), _p()
        ne = (C.c_int64 * 4)()
        call("kcGgufTensorInfo", self.h, name.encode(), C.byref(t), C.byref(nd), ne, C.byref(nb), C.byref(data))
        raw = np.frombuffer(C.string_at(data, nb.value), np.uint8).copy() if nb.value else np.zeros(0, np.uint8)
        return t.value, tuple(ne[i] for i in range(nd.value)), raw

    def close(self):
        if self.h:
            lib().kcGgufClose(self.h)
            self.h = None
