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
    assert lib.scmp_abi_version() == 2
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
