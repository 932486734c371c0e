"""ctypes access to the Kernelcore ggml glue (kernelcore_amd/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp)
built with the test-only ggml stand-in of tests/ggml_stub (libkcggml_glue_test.so, made by
__graft_entry__.build()): the entry points of tests/ggml_stub/glue_driver.cpp."""
import ctypes as C
import os

import kernelcore_amd as kc

HERE = os.path.dirname(os.path.abspath(__file__))
GLUE_SRC = os.path.join(kc.ROOT, "kernelcore_amd", "ggml", "src", "ggml-kernelcore", "ggml-kernelcore.cpp")
STUB = os.path.join(HERE, "ggml_stub")
LIB_PATH = os.path.join(STUB, "libkcggml_glue_test.so")
_LIB = None

_p, _i, _s, _ll = C.c_void_p, C.c_int, C.c_size_t, C.c_longlong


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (make -C tests/ggml_stub)")
        kc.lib()  # the runtime the glue links, loaded first (one kc runtime per process)
        L = C.CDLL(LIB_PATH)
        L.kcgt_info.argtypes = [C.c_char_p, C.c_char_p, C.c_char_p, _i, C.POINTER(_i), C.POINTER(_i), C.POINTER(_s),
                                C.POINTER(_s), C.POINTER(_i), C.POINTER(_i), C.POINTER(_i)]
        L.kcgt_buft.argtypes = [_i, C.c_char_p, _i, C.POINTER(_s), C.POINTER(_i), C.POINTER(_i)]
        L.kcgt_alloc_size.argtypes = [_i, _i, _ll, _ll]
        L.kcgt_alloc_size.restype = _s
        L.kcgt_supports_mul_mat.argtypes = [_i, _ll, _ll, _ll, _i]
        L.kcgt_buffer_ops.argtypes = [_i, _i, _ll, _ll, _p, _p, _i, _s, _s, _p, _i, _p, _p]
        L.kcgt_graph_compute.argtypes = [_p, _p, _i, _p, _i, _i]
        _LIB = L
    return _LIB


def info():
    n = 256
    reg, dev, desc = C.create_string_buffer(n), C.create_string_buffer(n), C.create_string_buffer(n)
    count, typ, mmap, api, dl = _i(), _i(), _i(), _i(), _i()
    free, total = _s(), _s()
    assert lib().kcgt_info(reg, dev, desc, n, C.byref(count), C.byref(typ), C.byref(free), C.byref(total), C.byref(mmap),
                           C.byref(api), C.byref(dl)) == 0
    return dict(reg=reg.value.decode(), name=dev.value.decode(), description=desc.value.decode(), devices=count.value,
                type=typ.value, memory_free=free.value, memory_total=total.value, mmap_support=bool(mmap.value),
                api_version=api.value, dl_init=bool(dl.value))


def buft(kind):
    """kind 0: the weights' buffer type, 1: the KV caches' (None when the device offers none)."""
    name, align, host, sup = C.create_string_buffer(64), _s(), _i(), _i()
    if not lib().kcgt_buft(kind, name, 64, C.byref(align), C.byref(host), C.byref(sup)):
        return None
    return dict(name=name.value.decode(), alignment=align.value, is_host=bool(host.value), supported=bool(sup.value))


DEVICE_TYPES = {0: "CPU", 1: "GPU", 2: "IGPU", 3: "ACCEL"}
