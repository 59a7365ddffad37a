"""ctypes access to the CPU oracle (oracle/libmoe_oracle.so) -- test infrastructure only.

Builds host copies of the same synthetic layers the product generates on the device (the same
hash streams and quantizers), and runs the oracle's layer functions on them.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle", "libmoe_oracle.so")
REF = os.path.join(ROOT, "oracle", "_ref", "libref_q35.so")
REF_Q4DP = os.path.join(ROOT, "oracle", "_ref", "libref_q4dp.so")

F32, Q8_0, Q4_K, Q6_K, Q5_K = 0, 1, 3, 4, 9
BLOCK = {F32: (4, 1), Q8_0: (34, 32), Q4_K: (144, 256), Q6_K: (210, 256), Q5_K: (176, 256)}
ST_ROUTER, ST_SHGATE, ST_G, ST_U, ST_D, ST_SG, ST_SU, ST_SD, ST_H2, ST_X1, ST_BIAS = range(11)
W_SIGMA = 0.02


def row_bytes(fm, cols):
    b, n = BLOCK[fm]
    return cols // n * b


class MoLayer(C.Structure):
    _fields_ = [("dm", C.c_uint32), ("ne", C.c_uint32), ("nk", C.c_uint32), ("ef", C.c_uint32), ("sf", C.c_uint32),
                ("fg", C.c_uint32), ("fu", C.c_uint32), ("fd", C.c_uint32),
                ("fsg", C.c_uint32), ("fsu", C.c_uint32), ("fsd", C.c_uint32),
                ("router", C.c_void_p), ("shgate", C.c_void_p), ("G", C.c_void_p), ("U", C.c_void_p),
                ("D", C.c_void_p), ("SG", C.c_void_p), ("SU", C.c_void_p), ("SD", C.c_void_p),
                ("router_bias", C.c_void_p)]


P = C.c_void_p
_SIGS = {
    "mo_f16": (C.c_float, [C.c_uint32]),
    "mo_f32_to_f16": (C.c_uint16, [C.c_float]),
    "mo_row_bytes": (C.c_uint64, [C.c_uint32, C.c_uint32]),
    "mo_deq_row": (C.c_int, [C.c_uint32, P, C.c_uint32, P]),
    "mo_quant_row": (C.c_int, [C.c_uint32, P, C.c_uint32, P]),
    "mo_gauss": (C.c_float, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float]),
    "mo_gauss_fill": (None, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, P]),
    "mo_gen_rows": (C.c_int, [C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32, C.c_float, P]),
    "mo_cdepth": (C.c_uint32, [C.c_uint32]),
    "mo_tuned": (C.c_int, [C.c_uint32, C.c_uint32]),
    "mo_dot_stride": (C.c_float, [C.c_uint32, P, C.c_uint32, P]),
    "mo_dot_tree": (C.c_float, [C.c_uint32, P, C.c_uint32, P]),
    "mo_gemv_row": (C.c_float, [C.c_uint32, P, C.c_uint32, P]),
    "mo_exp": (C.c_float, [C.c_float]),
    "mo_silu_mul": (C.c_float, [C.c_float, C.c_float]),
    "mo_router": (None, [C.POINTER(MoLayer), P, P, P]),
    "mo_topk": (None, [P, C.c_uint32, C.c_uint32, C.c_float, P, P, P]),
    "mo_group": (None, [P, C.c_uint32, C.c_uint32, C.c_uint32, P, P, P]),
    "mo_moe_exact": (C.c_int, [C.POINTER(MoLayer), C.c_uint32, P, P, P, P, P, P, C.c_int]),
    "mo_moe_exact_act": (C.c_int, [C.POINTER(MoLayer), C.c_uint32, P, P, P]),
    "mo_moe_q8": (C.c_int, [C.POINTER(MoLayer), C.c_uint32, P, P, P, P, P, P, C.c_int]),
    "mo_moe_f64": (C.c_int, [C.POINTER(MoLayer), C.c_uint32, P, P, P]),
    "mo_q8_1": (None, [P, C.c_uint32, P, P, P]),
    "mo_dot_q8": (C.c_float, [C.c_uint32, P, C.c_uint32, P, P, P]),
    "mo_rmsnorm_add": (C.c_float, [P, P, P, C.c_float, C.c_uint32, P, P]),
    "mo_sigmoid": (C.c_float, [C.c_float]),
    "mo_renorm": (None, [P, C.c_uint32]),
    "mo_combine": (C.c_float, [P, P, C.c_uint32, C.c_int, C.c_float, C.c_float, C.c_float]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE):
            raise RuntimeError(f"{ORACLE} missing: run `make -C oracle`")
        _lib = C.CDLL(ORACLE)
        for n, (r, a) in _SIGS.items():
            f = getattr(_lib, n)
            f.restype, f.argtypes = r, a
    return _lib


def ref_q4dp():
    """The reference's q8 CPU twin, tools/q4dp/q4dp_ref.h, compiled by oracle/Makefile (None if not built)."""
    if not os.path.exists(REF_Q4DP):
        return None
    r = C.CDLL(REF_Q4DP)
    r.ref_q8x_c.restype, r.ref_q8x_c.argtypes = None, [P, P, P, C.c_uint32]
    r.ref_sb_c.restype = C.c_float
    r.ref_sb_c.argtypes = [P, P, P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int]
    r.ref_row_c.restype, r.ref_row_c.argtypes = C.c_float, [P, C.c_uint32, P, P, C.c_uint32, C.c_int]
    return r


def ref_lib():
    """The reference's own tools/qwen35_engine.c compiled by oracle/Makefile (None if not built)."""
    if not os.path.exists(REF):
        return None
    r = C.CDLL(REF)
    r.ref_half_to_float.restype, r.ref_half_to_float.argtypes = C.c_float, [C.c_uint]
    r.ref_dot_fmt.restype, r.ref_dot_fmt.argtypes = C.c_float, [C.c_int, P, C.c_int, P]
    r.ref_deq_row.restype, r.ref_deq_row.argtypes = None, [C.c_int, P, C.c_int, P]
    for n in ("ref_hf_exp", "ref_hf_silu", "ref_hf_sigmoid"):
        getattr(r, n).restype, getattr(r, n).argtypes = C.c_float, [C.c_float]
    r.ref_rms_norm.restype, r.ref_rms_norm.argtypes = None, [P, P, P, C.c_int, C.c_float]
    return r


def rmsnorm_add(x, z, w, eps):
    """mo_rmsnorm_add over the rows of x, z ([T][n] f32): (x1, h2, s per row)"""
    x, z, w = (np.ascontiguousarray(a, np.float32) for a in (x, z, w))
    T, n = x.shape
    x1, h2, s = np.zeros_like(x), np.zeros_like(x), np.zeros(T, np.float32)
    for t in range(T):
        xt, zt, x1t, h2t = x[t].copy(), z[t].copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
        s[t] = lib().mo_rmsnorm_add(ptr(xt), ptr(zt), ptr(w), eps, n, ptr(x1t), ptr(h2t))
        x1[t], h2[t] = x1t, h2t
    return x1, h2, s


def ptr(a):
    """The address of a (None for None). The caller must hold a for as long as the address is used:
    ptr(temporary) can dangle before the call that receives it runs."""
    return a.ctypes.data if a is not None else None


def gen_rows(fm, seed, stream, r0, nr, cols, sigma=W_SIGMA):
    out = np.zeros(nr * row_bytes(fm, cols), np.uint8)
    assert lib().mo_gen_rows(fm, seed, stream, r0, nr, cols, sigma, ptr(out)) == 0
    return out


def gauss(seed, stream, i0, n, sigma=1.0):
    out = np.empty(n, np.float32)
    lib().mo_gauss_fill(seed, stream, i0, n, sigma, ptr(out))
    return out


def deq(fm, row, cols):
    out = np.empty(cols, np.float32)
    assert lib().mo_deq_row(fm, ptr(row), cols, ptr(out)) == 0
    return out


class HostLayer:
    """Host copy of a synthetic layer. experts=None: every expert; else only those (others zero)."""

    def __init__(self, shape, seed=0, layer=0, experts=None, bias=None):
        self.bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        s, L = shape, layer * 16
        self.shape = s
        self.router = gen_rows(F32, seed, L + ST_ROUTER, 0, s.ne, s.dm).view(np.float32)
        rbg, rbu, rbd = row_bytes(s.fg, s.dm), row_bytes(s.fu, s.dm), row_bytes(s.fd, s.ef)
        self.G = np.zeros(s.ne * s.ef * rbg, np.uint8)
        self.U = np.zeros(s.ne * s.ef * rbu, np.uint8)
        self.D = np.zeros(s.ne * s.dm * rbd, np.uint8)
        self.have = set()
        self.seed, self.layer = seed, layer
        self.add_experts(range(s.ne) if experts is None else experts)
        self.shgate = self.SG = self.SU = self.SD = None
        if s.sf:
            self.shgate = gen_rows(F32, seed, L + ST_SHGATE, 0, 1, s.dm).view(np.float32)
            self.SG = gen_rows(s.fsg, seed, L + ST_SG, 0, s.sf, s.dm)
            self.SU = gen_rows(s.fsu, seed, L + ST_SU, 0, s.sf, s.dm)
            self.SD = gen_rows(s.fsd, seed, L + ST_SD, 0, s.dm, s.sf)
        self._mk()

    def add_experts(self, experts):
        s, L = self.shape, self.layer * 16
        rbg, rbu, rbd = row_bytes(s.fg, s.dm), row_bytes(s.fu, s.dm), row_bytes(s.fd, s.ef)
        for e in sorted(set(int(x) for x in experts) - self.have):
            # generated in place (the rows of expert e of each stack)
            for buf, fm, st, nr, cols, rb in ((self.G, s.fg, ST_G, s.ef, s.dm, rbg), (self.U, s.fu, ST_U, s.ef, s.dm, rbu),
                                              (self.D, s.fd, ST_D, s.dm, s.ef, rbd)):
                assert lib().mo_gen_rows(fm, self.seed, L + st, e * nr, nr, cols, W_SIGMA,
                                         buf.ctypes.data + e * nr * rb) == 0
            self.have.add(e)

    def _mk(self):
        s = self.shape
        self.desc = MoLayer(s.dm, s.ne, s.nk, s.ef, s.sf, s.fg, s.fu, s.fd, s.fsg, s.fsu, s.fsd,
                            ptr(self.router), ptr(self.shgate), ptr(self.G), ptr(self.U), ptr(self.D),
                            ptr(self.SG), ptr(self.SU), ptr(self.SD), ptr(self.bias))

    def route(self, h2):
        """ids, wt, sgo per token, the exact tier's routing."""
        s = self.shape
        T = h2.shape[0]
        ids = np.zeros((T, s.nk), np.uint32)
        wt = np.zeros((T, s.nk), np.float32)
        sgo = np.zeros(T, np.float32)
        lg = np.zeros(s.ne, np.float32)
        sg = np.zeros(1, np.float32)
        for t in range(T):
            h = np.ascontiguousarray(h2[t])
            lib().mo_router(C.byref(self.desc), ptr(h), ptr(lg), ptr(sg))
            lib().mo_topk(ptr(lg), s.ne, s.nk, float(sg[0]), ptr(ids[t]), ptr(wt[t]), sgo[t:].ctypes.data)
        return ids, wt, sgo

    def run(self, h2, x1=None, tier="exact", nthreads=1):
        s = self.shape
        h2 = np.ascontiguousarray(h2, np.float32)
        T = h2.shape[0]
        ids, _, _ = self.route(h2)
        self.add_experts(np.unique(ids))
        self._mk()
        y = np.zeros((T, s.dm), np.float32)
        ids = np.zeros((T, s.nk), np.uint32)
        wt = np.zeros((T, s.nk), np.float32)
        sgo = np.zeros(T, np.float32)
        f = lib().mo_moe_exact if tier == "exact" else lib().mo_moe_q8
        x1c = np.ascontiguousarray(x1, np.float32) if x1 is not None else None
        assert f(C.byref(self.desc), T, ptr(h2), ptr(x1c), ptr(y), ptr(ids), ptr(wt), ptr(sgo), nthreads) == 0
        return y, ids, wt, sgo

    def f64(self, h2, ids):
        s = self.shape
        T = h2.shape[0]
        y = np.zeros((T, s.dm), np.float64)
        h2c = np.ascontiguousarray(h2, np.float32)  # held while the oracle reads them
        idc = np.ascontiguousarray(ids, np.uint32)
        assert lib().mo_moe_f64(C.byref(self.desc), T, ptr(h2c), ptr(idc), ptr(y)) == 0
        return y


def inputs(shape, seed, T, layer=0):
    h2 = gauss(seed, layer * 16 + ST_H2, 0, T * shape.dm).reshape(T, shape.dm)
    x1 = gauss(seed, layer * 16 + ST_X1, 0, T * shape.dm).reshape(T, shape.dm)
    return h2, x1


def err_metrics(y, ref):
    """max relative error (max |y - ref| / max |ref|), norm-relative error, cosine similarity."""
    y = np.asarray(y, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    d = np.abs(y - r)
    return dict(max_rel=float(d.max() / max(np.abs(r).max(), 1e-30)),
                rel=float(np.linalg.norm(y - r) / max(np.linalg.norm(r), 1e-30)),
                cos=float(np.dot(y, r) / max(np.linalg.norm(y) * np.linalg.norm(r), 1e-30)))
