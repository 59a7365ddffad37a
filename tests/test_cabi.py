"""The C-ABI library loads without a GPU and exports every entry point include/*.h declares."""
import ctypes as C
import os
import re

import eureka_moe as em

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    names = set()
    for f in os.listdir(os.path.join(ROOT, "include")):
        if f.endswith(".h"):
            src = open(os.path.join(ROOT, "include", f)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names |= set(re.findall(r"\b(llb_\w+)\s*\(", src))
    return names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(em.LIB_PATH)
    names = declared()
    assert len(names) >= 20
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_prototypes_cover_the_header():
    assert declared() <= set(em._SIGS), sorted(declared() - set(em._SIGS))


def test_load_raises_without_library(tmp_path):
    try:
        em.load(str(tmp_path / "nope.so"))
    except em.LlbError as e:
        assert "no fallback" in str(e)
    else:
        raise AssertionError("load() must fail loudly")
