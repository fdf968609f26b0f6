"""Host-side checks that need no GPU: the C ABI library loads and exports every
function include/omhip.h declares, the headers compile as C and C++23, the
caching pool behaves (fake device), and bench.py refuses more than one GPU."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "omhip.h")
LIB = os.path.join(ROOT, "omnimatchdeeplearningtool_amd", "libomhip.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(omHip\w+)\s*\(", text)))


def test_header_declares_the_hot_path():
    names = declared_functions()
    for must in ("omHipMatmul", "omHipMatmulTransB", "omHipBatchedMatmul", "omHipConv2d", "omHipConv2dBiasBnAct",
                 "omHipBatchNorm2d", "omHipReLU", "omHipAddBias", "omHipMatmulF16", "omHipMatmulBF16", "omHipInit",
                 "omHipMalloc", "omHipFree", "omHipCopyH2D", "omHipCopyD2H"):
        assert must in names
    assert len(names) >= 45


@pytest.mark.skipif(not os.path.exists(LIB), reason="libomhip.so not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


@pytest.mark.skipif(not os.path.exists(LIB), reason="libomhip.so not built")
def test_python_signatures_cover_header():
    import omnimatchdeeplearningtool_amd as om
    sigs = set(om._SIGS) | {"omHipGetLastError"}
    assert set(declared_functions()) == sigs


def header_parameter_kinds():
    """name -> parameter kinds ('ptr', 'i', 'll', 'sz', 'f') of every declaration in omhip.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for name, params in re.findall(r"\b(omHip\w+)\s*\(([^)]*)\)\s*;", text):
        kinds = []
        for p in params.split(","):
            p = " ".join(p.split())
            if not p or p == "void":
                continue
            t = re.sub(r"\b\w+$", "", p).strip()   # drop the parameter name
            kinds.append("ptr" if "*" in t else "ll" if t == "long long" else "sz" if t == "size_t"
                         else "f" if t == "float" else "i" if t == "int" else t)
        out[name] = kinds
    return out


def test_python_argtypes_match_header():
    """Every ctypes signature the package binds has the header's parameter count and kinds, so a
    call never passes an int where the C function reads a pointer, a float or a 64-bit size."""
    import omnimatchdeeplearningtool_amd as om

    def kind(t):
        if t in (ctypes.c_void_p, ctypes.c_char_p) or issubclass(t, ctypes._Pointer):
            return "ptr"
        return {ctypes.c_int: "i", ctypes.c_longlong: "ll", ctypes.c_size_t: "sz", ctypes.c_float: "f"}[t]

    decl = header_parameter_kinds()
    assert len(decl) >= 90
    wrong = {n: ([kind(t) for t in args], decl[n]) for n, args in om._SIGS.items()
             if [kind(t) for t in args] != decl[n]}
    assert not wrong, wrong


def test_headers_compile_as_c_and_cpp23(tmp_path):
    c_src = tmp_path / "c.c"
    c_src.write_text('#include "omhip.h"\nint main(void){ int (*f)(int) = omHipInit; (void)f; return 0; }\n')
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{ROOT}/include", "-c", str(c_src), "-o",
                    str(tmp_path / "c.o")], check=True)
    cpp = tmp_path / "b.cpp"
    cpp.write_text('#include "omhip_backend.hpp"\nint main(){ auto f = &om::HIPBackend::matmul; (void)f; return 0; }\n')
    subprocess.run(["g++", "-std=c++23", "-Wall", "-Werror", f"-I{ROOT}/include", "-c", str(cpp), "-o",
                    str(tmp_path / "b.o")], check=True)


def test_caching_pool(tmp_path):
    exe = tmp_path / "pool"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-pthread", "-fsanitize=address,undefined",
                    os.path.join(ROOT, "tests", "cpp", "test_caching_pool.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout


def test_gemm_plan_partials_fit_the_fixed_scratch(tmp_path):
    """Every split-K plan's partial sums fit omHipGemmStridedBatchedNoAlloc's fixed array."""
    exe = tmp_path / "plan"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-Werror", os.path.join(ROOT, "tests", "cpp", "test_gemm_plan.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], stdout=subprocess.PIPE,
                       stderr=subprocess.PIPE, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
