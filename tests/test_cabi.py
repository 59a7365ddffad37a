"""The C-ABI library loads without a GPU and exports every entry point include/*.h declares."""
import ctypes as C
import os
import re

import pytest

import eureka_moe as em

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    names = set()
    for f in os.listdir(os.path.join(ROOT, "include")):
        if f.endswith(".h"):
            src = open(os.path.join(ROOT, "include", f)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            # macros and header-only static inline wrappers (llb_backend_hip.h) are not library symbols
            src = re.sub(r"#define(?:[^\n]*\\\n)*[^\n]*", "", src)
            src = re.sub(r"static inline [^{]*\{[^}]*\}", "", src)
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


# ---- the layer entry points refuse what they cannot run, before any device call, and name the rule
DUMMY = 0x10000  # a nonzero address that the checks below never reach


def _layer(**kw):
    s = em.SHAPES["c2"]
    d = dict(dm=s.dm, ne=s.ne, nk=s.nk, ef=s.ef, sf=s.sf, fx=s.fx, fsg=s.fsg, fsu=s.fsu, fsd=s.fsd, pad=0,
             router=DUMMY, shgate=DUMMY, G=DUMMY, U=DUMMY, D=DUMMY, SG=DUMMY, SU=DUMMY, SD=DUMMY)
    d.update(kw)
    L = em.MoeLayer()
    for k, v in d.items():
        setattr(L, k, v)
    return L


def _forward(lib, L, T=1, sb=1 << 30, tier=em.EXACT, bufs=DUMMY):
    return lib.llb_moe_hip_forward(C.byref(L), T, bufs, 0, bufs, bufs, bufs, bufs, sb, tier)


@pytest.mark.parametrize("change,rule", [
    (dict(dm=2000), "multiples of 256"), (dict(ef=300), "multiples of 256"), (dict(nk=64), "nk"),
    (dict(nk=0), "nk"), (dict(ne=2048), "ne <= 1024"), (dict(fx=em.SHAPES["c2"].fx & ~15 | 7), "expert formats"),
    (dict(router=0), "null weights"), (dict(D=0), "null weights"), (dict(dm=16384), "router"),
    (dict(sf=300), "shared expert"), (dict(SD=0), "shared expert"), (dict(fsg=em.Q8_0, fsu=em.Q8_0), "shared gate/up"),
])
def test_forward_refuses_each_rule(change, rule):
    lib = em.load()
    rc = _forward(lib, _layer(**change))
    assert rc == -1 and rule in lib.llb_hip_last_error().decode(), (rc, lib.llb_hip_last_error())


def test_forward_refuses_buffers_tier_and_scratch():
    lib = em.load()
    L = _layer()
    assert _forward(lib, L, bufs=0) == -1 and b"null buffer" in lib.llb_hip_last_error()
    assert _forward(lib, L, tier=7) == -1 and b"tier" in lib.llb_hip_last_error()
    need = lib.llb_moe_hip_scratch_bytes(C.byref(L), 1, em.EXACT)
    assert need > 0
    assert _forward(lib, L, sb=need - 1) == -3 and b"scratch" in lib.llb_hip_last_error()
    assert _forward(lib, L, T=0) == 0  # nothing to do: no device call
    rc = lib.llb_moe_hip_forward_norm(C.byref(L), 1, DUMMY, 0, DUMMY, 1e-6, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY, DUMMY,
                                      1 << 30, em.EXACT)
    assert rc == -1 and b"input-step" in lib.llb_hip_last_error()


def test_fused_path_is_refused():
    """the fused one-launch layer hung the GPU and its cause is not shown: asking for it is an error"""
    lib = em.load()
    assert lib.llb_moe_hip_set_fused(1) == -1
    assert b"disabled" in lib.llb_hip_last_error() and b"hung" in lib.llb_hip_last_error()
    assert lib.llb_moe_hip_set_fused(0) == 0


def test_forward_static_refuses_before_touching_a_device():
    """llb_moe_hip_forward_static's argument checks (the f16 tier, a streamed layer, a scratch need past the
    static array) answer before any device call, so they run here without a GPU"""
    lib = C.CDLL(em.LIB_PATH)
    f = lib.llb_moe_hip_forward_static
    f.restype = C.c_int
    f.argtypes = em._SIGS["llb_moe_hip_forward_static"][1]
    lib.llb_hip_last_error.restype = C.c_char_p
    lib.llb_moe_hip_scratch_bytes.restype = C.c_size_t
    lib.llb_moe_hip_scratch_bytes.argtypes = [C.POINTER(em.MoeLayer), C.c_uint32, C.c_int]
    s = em.SHAPES["c1"]
    L = em.MoeLayer(s.dm, s.ne, s.nk, s.ef, s.sf, s.fx, s.fsg, s.fsu, s.fsd)
    assert f(None, 1, 0, 0, 0, 0, 0, em.EXACT) == -1
    assert f(C.byref(L), 1, 0, 0, 0, 0, 0, em.F16) == -1 and b"f16" in lib.llb_hip_last_error()
    assert lib.llb_moe_hip_scratch_bytes(C.byref(L), 4096, em.EXACT) > em.STATIC_SCRATCH_BYTES
    assert f(C.byref(L), 4096, 0, 0, 0, 0, 0, em.EXACT) == -1 and b"static array" in lib.llb_hip_last_error()
    L.res = 2  # LLB_MOE_RES_STREAM
    assert f(C.byref(L), 1, 0, 0, 0, 0, 0, em.EXACT) == -1 and b"streamed" in lib.llb_hip_last_error()
