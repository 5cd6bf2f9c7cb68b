"""CPU checks of the C-ABI boundary: the library loads, exports every symbol
the headers declare, keeps the reference Tensor layout, and -- with no GPU
present -- fails loudly (NULL / error) instead of computing on the CPU."""
import ctypes
import os
import re
import subprocess

import pytest

import tinytorch_amd

ROOT = tinytorch_amd.ROOT
HEADERS = [os.path.join(ROOT, "include", h)
           for h in ("tensor.h", "autograd.h", "tt_hip.h", "tt_data.h")]


def test_every_header_is_checked():
    assert sorted(os.listdir(os.path.join(ROOT, "include"))) == sorted(
        os.path.basename(h) for h in HEADERS)


def declared_functions(path):
    src = open(path).read()
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    src = re.sub(r"//[^\n]*", " ", src)
    src = re.sub(r"#[^\n]*", " ", src)
    src = re.sub(r"typedef struct \w+ \{.*?\} \w+;", " ", src, flags=re.S)
    names = re.findall(r"\b([A-Za-z_]\w*)\s*\([^;{}]*\)\s*;", src)
    return sorted(set(n for n in names if n not in ("if", "while", "for", "sizeof")))


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_headers_parse():
    names = declared_functions(HEADERS[0])
    assert "tt_conv2d" in names and "tt_sgemm_rowmajor" in names and len(names) == 23


def test_every_declared_symbol_is_exported():
    syms = exported(tinytorch_amd.LIB_PATH)
    missing = [n for h in HEADERS for n in declared_functions(h) if n not in syms]
    assert not missing, f"declared but not exported: {missing}"


def test_python_signatures_cover_headers():
    have = {name for name, _, _ in tinytorch_amd.SIGNATURES}
    missing = [n for h in HEADERS for n in declared_functions(h) if n not in have]
    assert not missing, f"no ctypes signature for: {missing}"
    tinytorch_amd.lib()  # every declared signature resolves


def test_reference_symbols_all_present():
    """Every function of the reference headers (include/tensor.h:20-50,
    include/autograd.h:14-48) plus tt_sgemm_rowmajor (src/gemm.c:569)."""
    ref_names = """tt_new tt_fromdata tt_retain tt_release tt_data tt_numel tt_ndim tt_shape
    tt_strides tt_add tt_mul tt_addscalar tt_mulscalar tt_matmul tt_matmul_fast tt_matmul_omp
    tt_relu tt_softmax tt_reshape tt_conv2d tt_maxpool2d tt_avgpool2d tt_sgemm_rowmajor
    ag_leaf ag_add ag_mul ag_addscalar ag_mulscalar ag_matmul ag_relu ag_softmax ag_padones
    ag_reshape ag_conv2d ag_maxpool2d ag_avgpool2d ag_value ag_grad ag_requires_grad
    ag_backward ag_backward_from ag_release ag_retain""".split()
    syms = exported(tinytorch_amd.LIB_PATH)
    assert [n for n in ref_names if n not in syms] == []


class CTensor(ctypes.Structure):
    # the reference layout (include/tensor.h:10-17) followed by the appended fields
    _fields_ = [("data", ctypes.POINTER(ctypes.c_float)), ("shape", ctypes.POINTER(ctypes.c_long)),
                ("strides", ctypes.POINTER(ctypes.c_long)), ("ndim", ctypes.c_int),
                ("numel", ctypes.c_long), ("refcount", ctypes.c_int),
                ("dev", ctypes.c_void_p), ("valid", ctypes.c_int)]


def test_tensor_prefix_layout():
    """The first six fields sit where the reference's ctypes mirror reads them."""
    assert CTensor.shape.offset == 8 and CTensor.strides.offset == 16
    assert CTensor.ndim.offset == 24 and CTensor.numel.offset == 32
    assert CTensor.refcount.offset == 40 and CTensor.dev.offset == 48


def test_pybind_module_imports():
    import importlib
    import sys
    sys.path.insert(0, os.path.join(ROOT, "build"))
    try:
        m = importlib.import_module("tinytorch_pybind")
    finally:
        sys.path.pop(0)
    for meth in ("leaf", "value", "grad", "backward", "add", "mul", "addscalar", "mulscalar",
                 "matmul", "relu", "softmax", "padones", "reshape", "conv2d", "maxpool2d",
                 "avgpool2d", "__add__", "__mul__", "softmax_ce", "sgd_step", "detach"):
        assert hasattr(m.Node, meth), meth
    for meth in ("sgd_momentum", "adam", "step", "t"):
        assert hasattr(m.Optim, meth), meth


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU device node is present")
def test_no_gpu_fails_loudly():
    """Without a GPU every entry point reports failure; nothing runs on the CPU."""
    L = tinytorch_amd.lib()
    assert L.tth_available() == 0
    with pytest.raises(RuntimeError):
        tinytorch_amd.require_gpu()
    shp = (ctypes.c_long * 2)(2, 3)
    assert not L.tt_new(shp, 2)
    data = (ctypes.c_float * 6)(*range(6))
    assert not L.tt_fromdata(data, shp, 2)
    C = (ctypes.c_float * 4)()
    A = (ctypes.c_float * 4)(1, 2, 3, 4)
    assert L.tt_sgemm_rowmajor(2, 2, 2, A, A, C, 1) != 0
    assert not L.tth_malloc(16)


def test_hostile_shapes_rejected_before_any_device_call():
    """reference tests/test_ops.py:303-332: huge / zero / negative dims -> NULL."""
    L = tinytorch_amd.lib()
    for dims in ((2**40, 2**40), (2**62, 2), (2**21, 2**21), (2**40,), (-3, 4), (0, 4)):
        arr = (ctypes.c_long * len(dims))(*dims)
        assert not L.tt_new(arr, len(dims))
    big = (ctypes.c_long * 2)(2**40, 2**40)
    assert not L.tt_fromdata(None, big, 2)
    nine = (ctypes.c_long * 9)(*([1] * 9))
    assert not L.tt_new(nine, 9)


REF_INCLUDE = "/root/reference/include"


def prototypes(path):
    """name -> (return type, [parameter types]) with parameter names and
    whitespace normalised away."""
    src = open(path).read()
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    src = re.sub(r"//[^\n]*", " ", src)
    src = re.sub(r"#[^\n]*", " ", src)
    src = re.sub(r"typedef struct \w+ \{.*?\} \w+;", " ", src, flags=re.S)
    out = {}
    for ret, name, params in re.findall(
            r"([A-Za-z_][\w\s\*]*?)\s*\b([A-Za-z_]\w*)\s*\(([^;{}()]*)\)\s*;", src):
        ret = re.sub(r"\s+", " ", ret.replace("*", " * ")).strip().split(" ")
        ret = " ".join(t for t in ret if t not in ("typedef", "extern", '"C"', "{", "}"))
        types = []
        for p in params.split(","):
            p = re.sub(r"\s+", " ", p.replace("*", " * ")).strip()
            if not p or p == "void":
                continue
            toks = p.split(" ")
            if len(toks) > 1 and re.fullmatch(r"[A-Za-z_]\w*", toks[-1]) and toks[-1] not in (
                    "int", "long", "float", "double", "char", "size_t"):
                toks = toks[:-1]  # drop the parameter name
            types.append(" ".join(toks))
        out[name] = (ret, types)
    return out


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference headers not present")
@pytest.mark.parametrize("header", ["tensor.h", "autograd.h"])
def test_prototypes_match_reference(header):
    """Every reference prototype (include/tensor.h:20-50, include/autograd.h:
    14-48) is declared here with the same return and parameter types."""
    ref = prototypes(os.path.join(REF_INCLUDE, header))
    ours = prototypes(os.path.join(ROOT, "include", header))
    assert len(ref) >= 20
    diff = {n: (ref[n], ours.get(n)) for n in ref if ours.get(n) != ref[n]}
    assert not diff, diff


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference headers not present")
def test_tensor_struct_prefix_matches_reference():
    """The Tensor struct keeps the reference's fields, types and order as its
    prefix (include/tensor.h:10-17)."""
    def fields(path):
        src = re.sub(r"/\*.*?\*/", " ", open(path).read(), flags=re.S)
        body = re.search(r"typedef struct Tensor \{(.*?)\} Tensor;", src, flags=re.S).group(1)
        return [re.sub(r"\s+", " ", f.replace("*", " * ")).strip()
                for f in body.split(";") if f.strip()]
    ref = fields(os.path.join(REF_INCLUDE, "tensor.h"))
    ours = fields(os.path.join(ROOT, "include", "tensor.h"))
    assert ours[:len(ref)] == ref


@pytest.mark.skipif(not os.path.isdir("/root/reference/src"), reason="reference sources not present")
def test_sgemm_rowmajor_prototype_matches_reference():
    """tt_sgemm_rowmajor (reference src/gemm.c:569, exported without a header)."""
    src = open("/root/reference/src/gemm.c").read()
    m = re.search(r"\bint\s+tt_sgemm_rowmajor\s*\(([^)]*)\)", src)
    assert m
    ref_decl = "int tt_sgemm_rowmajor(" + m.group(1) + ");"
    tmp = os.path.join(ROOT, "build", "_ref_sgemm_proto.h")
    os.makedirs(os.path.dirname(tmp), exist_ok=True)
    with open(tmp, "w") as f:
        f.write(ref_decl)
    assert prototypes(os.path.join(ROOT, "include", "tensor.h"))["tt_sgemm_rowmajor"] == \
        prototypes(tmp)["tt_sgemm_rowmajor"]
