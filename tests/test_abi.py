"""CPU checks of the C ABI: the library loads, exports every symbol the headers declare, and the
calls that need no GPU behave as the reference's runtime does (include/kernelcore/api.hpp,
src/runtime.cpp:209-252)."""
import ctypes as C
import subprocess
import sys

import pytest

import kernelcore_amd as kc


def test_library_exports_every_declared_symbol():
    L = kc.lib()
    declared = kc.declared_symbols()
    assert len(declared) >= 40
    missing = [n for n in declared if not hasattr(L, n)]
    assert missing == []


def test_library_has_gfx950_code_object():
    # the offload bundle of the fat binary names its target triple
    data = open(kc.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_error_strings_keep_reference_values():
    L = kc.lib()
    for code, name in enumerate(kc.ERRORS):
        assert L.kcGetErrorString(code).decode() == name
    assert L.kcCodegenName(4).decode() == "hip"
    assert L.kcCodegenName(0).decode() == "auto"


def test_calls_before_init_return_not_initialized():
    # A fresh process: the runtime is process-wide.
    code = (
        "import ctypes as C, kernelcore_amd as kc\n"
        "L = kc.lib()\n"
        "p = C.c_void_p()\n"
        "print(L.kcMalloc(C.byref(p), 16), L.kcGetDeviceCount(C.byref(C.c_int())),"
        " L.kcStreamCreate(C.byref(C.c_void_p())), L.kcFree(None))\n"
    )
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=kc.ROOT, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["1", "1", "1", "1"]  # NotInitialized


def test_stream_bytes_layout_math():
    # 16-row tiles x groups of 4 super-blocks; exact ggml size when both divide.
    assert kc.stream_bytes("q4k", 3072, 3072) == 3072 * 12 * 144
    assert kc.stream_bytes("q6k", 128256, 3072) == 128256 * 12 * 210
    assert kc.stream_bytes("q4k", 8, 256) == 16 * 4 * 144  # padded rows and super-blocks
    assert kc.stream_bytes("q6k", 40, 768) == 48 * 4 * 210
    L = kc.lib()
    n = C.c_size_t()
    assert L.kcKquantStreamBytes(12, 8, 100, C.byref(n)) == kc.ERR["InvalidValue"]
    assert L.kcKquantStreamBytes(13, 8, 256, C.byref(n)) == kc.ERR["InvalidValue"]


def test_kernel_options_are_validated():
    assert kc.status("kcSetKernelOption", b"no_such_option", 1) == "InvalidValue"
    kc.set_option("matvec_waves", 2)
    v = C.c_int()
    kc.call("kcGetKernelOption", b"matvec_waves", C.byref(v))
    assert v.value == 2
    kc.set_option("matvec_waves", 0)


def test_codegen_cpu_paths_are_unsupported():
    L = kc.lib()
    assert kc.ERRORS[L.kcSetKernelCodegen(1)] == "UnsupportedOperation"
    assert kc.ERRORS[L.kcSetKernelCodegen(9)] == "InvalidValue"
    assert L.kcSetKernelCodegen(4) == 0
    cg = C.c_int()
    assert L.kcGetKernelCodegen(C.byref(cg)) == 0 and cg.value == 4
    assert L.kcSetKernelCodegen(0) == 0


STRUCTS = ["VectorAddArgs", "QuantizeArgs", "MatvecQ4Q8Args", "MatmulKQ8Args", "MatmulF16Args", "QuantizeColsArgs",
           "RmsNormArgs", "MulRowsArgs", "RopeGgmlArgs", "AddSumsqFArgs", "SumsqPartArgs", "NormMulQ8Args",
           "AddNormQ8FArgs", "SiluMulQ8FArgs",
           "SiluMulArgs", "SetRowsF16Args", "FaDims", "FaScoresArgs", "FaMaxArgs", "FaExpArgs", "FaValuesArgs",
           "KquantRepackArgs", "GetRowsKquantArgs", "QuantizeKquantArgs", "FillNormalArgs", "FlashAttnArgs", "FlashDecodeArgs",
           "DeviceProperties",
           "MulMatConfig", "MulMatNode", "MulMatPlan", "MulMatNormNode", "MulMatSwigluNode", "GgmlTensor",
           "GgmlConfig", "GgmlStats", "GgmlProfileEntry"]


def test_struct_layouts_match_the_c_header(tmp_path):
    """ctypes mirrors against what gcc makes of include/kernelcore/llm_kernels.h."""
    lines = ["#include <stdio.h>", "#include <stddef.h>", "#include <kernelcore/llm_kernels.h>",
             "#include <kernelcore/mul_mat.h>", "#include <kernelcore/ggml_backend.h>", "int main(void) {"]
    for s in STRUCTS:
        cls = getattr(kc, s)
        lines.append(f'printf("{s} %zu\\n", sizeof(kc{s}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{s}.{f} %zu\\n", offsetof(kc{s}, {f}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{kc.ROOT}/include", str(src), "-o", str(exe)], check=True)
    want = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    for s in STRUCTS:
        cls = getattr(kc, s)
        assert int(want[s]) == C.sizeof(cls), s
        for f, _ in cls._fields_:
            assert int(want[f"{s}.{f}"]) == getattr(cls, f).offset, f"{s}.{f}"


def test_cpp_shim_compiles_reference_style_calls(tmp_path):
    """C++ written against the reference's api.hpp (kc::Error results, default arguments,
    llm:: argument structs with their defaults) compiles against include/kernelcore/api.hpp."""
    src = tmp_path / "shim.cpp"
    src.write_text(r'''
#include <kernelcore/api.hpp>
#include <kernelcore/kernels.hpp>
kc::Error f(const int* qw, const int* xq, const float* xd, float* y) {
    if (kc::Error e = kcInit(); e != kc::Error::Success) return e;
    llm::MatvecQ4Q8Args a{qw, xq, xd, y, nullptr, 8, 256};
    llm::MatmulKQ8Args m{qw, xq, y, nullptr, 8, 256, 3};
    static_assert(sizeof(m) == 48);
    if (m.row_block != 8) return kc::Error::InternalError;
    kcStream_t s = nullptr;
    (void)kcLaunchKernelChunked("matvec_q4k_q8", &a, 4);
    (void)kcMemcpy(y, xd, 4, kc::CopyKind::DeviceToDevice);
    kc::DeviceProperties p;
    (void)kcGetDeviceProperties(&p, 0);
    (void)kc::kernels::launchVectorAdd(xd, xd, y, 1);
    return kcLaunchKernel("matvec_q4k_q8", &a, s);
}
''')
    subprocess.run(["g++", "-std=c++20", "-fsyntax-only", f"-I{kc.ROOT}/include", str(src)], check=True)
