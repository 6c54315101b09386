"""The C ABI library loads on the CPU and exports every function include/*.h declares.
No compute calls (there may be no GPU here)."""
import ctypes
import os
import re

from scmp_kernels_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in os.listdir(inc):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(inc, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(scmp_\w+)\s*\(", text, re.M):
            names.add(m.group(1))
    return names


def test_header_declares_entry_points():
    names = _declared()
    assert {"scmp_sc_gemm", "scmp_quantize", "scmp_build_stream_tables"} <= names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(_lib.EXPORTS) == _declared()


def test_abi_version_and_error_string():
    lib = _lib.load()
    assert lib.scmp_abi_version() == 3
    assert isinstance(lib.scmp_last_error(), bytes)


def test_struct_layouts_match_header_order():
    # ctypes structures follow the C declaration order of include/scmp_hip.h
    hdr = open(os.path.join(ROOT, "include", "scmp_hip.h")).read()
    for cname, pyt in (("scmp_quant_args", _lib.QuantArgs), ("scmp_epilogue", _lib.Epilogue),
                       ("scmp_gemm_args", _lib.GemmArgs)):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (cname, cname), hdr, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            decl = re.sub(r"^(const\s+)?\w+\s*", "", decl)
            fields += [f.strip().lstrip("*").strip() for f in decl.split(",")]
        assert fields == [f[0] for f in pyt._fields_], (cname, fields)


def test_argument_checks_fail_before_any_device_call():
    """Argument validation of the class-run entry points returns SCMP_E_ARG with a message,
    before touching the device (runs without a GPU)."""
    lib = _lib.load()
    dummy = ctypes.c_void_p(16)          # never dereferenced: the checks reject first
    rc = lib.scmp_permute_code_columns(None, 4, 16, dummy, 16, dummy, 16, None)
    assert rc == -1 and b"null" in lib.scmp_last_error()
    rc = lib.scmp_permute_code_columns(dummy, 4, 16, dummy, 20, dummy, 24, None)
    assert rc == -1 and b"multiple of 16" in lib.scmp_last_error()
    g = _lib.GemmArgs()
    g.ca = g.cb = g.lut = g.y = dummy.value
    g.N, g.M, g.D, g.batch = 8, 8, 64, 1
    g.lda = g.ldb = 64
    g.JP, g.ldy = 64, 8
    g.epi.kind = _lib.EPI_ROWCOL
    g.impl = _lib.GEMM_MFMA_FP4
    g.nclass = 2
    g.group_class = dummy.value
    g.chunk = 16                          # chunked accumulation and class runs do not mix
    assert lib.scmp_sc_gemm(g, None) == -1 and b"group_class" in lib.scmp_last_error()
    g.chunk = 0
    g.d_class = dummy.value               # nor per-d classes and class runs
    assert lib.scmp_sc_gemm(g, None) == -1 and b"group_class" in lib.scmp_last_error()
    g.d_class = None
    g.impl = _lib.GEMM_MFMA               # class runs are an FP4-kernel layout
    assert lib.scmp_sc_gemm(g, None) == -1 and b"group_class" in lib.scmp_last_error()
