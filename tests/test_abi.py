"""The C-ABI boundary: libxpose.so loads without a GPU and exports every
function include/xpose.h declares (no compute call is made)."""
import ctypes as C
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(path):
    """Names of the functions a C header declares: `<type> name(` at the start
    of a statement, comments removed."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    names = []
    for stmt in text.split(";"):
        stmt = stmt.strip()
        if stmt.startswith(("#", "typedef", "struct", "enum")) or "{" in stmt:
            stmt = stmt.split("}")[-1].strip()
        m = re.match(r"^(?:const\s+)?[A-Za-z_][\w\s\*]*?[\s\*](xp_\w+)\s*\(", stmt)
        if m:
            names.append(m.group(1))
    return names


def test_header_declares_the_entry_points():
    names = declared_functions(os.path.join(ROOT, "include", "xpose.h"))
    assert len(names) == len(set(names)), "duplicate declaration"
    # the boundary's main groups are all present
    for n in ("xp_init", "xp_mv_int4", "xp_attention_decode", "xp_topk4_harvest",
              "xp_session_create", "xp_session_decode_step", "xp_batch_create", "xp_draw"):
        assert n in names, n
    assert len(names) > 80


def test_library_exports_every_declared_function(xh):
    lib = C.CDLL(xh.LIB_PATH)
    names = declared_functions(os.path.join(ROOT, "include", "xpose.h"))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared in xpose.h but not exported: {missing}"
