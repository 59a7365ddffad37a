"""eureka_moe -- Python host side of the MI355X MoE FFN backend.

A thin ctypes mirror of the C ABI in include/llb_moe_hip.h (the drop-in boundary for the reference's
llb_moe_run, host/llb_host.c:622-724, and pf_moe, host/llb_pf.h:286-389). It loads the in-tree
libeureka_moe.so built by __graft_entry__.build(); there is no fallback: without the library
every entry point raises.

Layers are described by the same fields llb_moe_run reads from a layer's table row
(host/llb_host.c:623-627): d_model, expert count, top-k, expert ff, shared ff, the formats word
(gate | up << 4 | down << 8 | fused << 12) and the device addresses of the router, the shared
gate row and the expert stacks.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(HERE), "libeureka_moe.so")

F32, Q8_0, Q4_K, Q6_K, Q5_K = 0, 1, 3, 4, 9
EXACT, Q8, F16 = 0, 1, 2
BLOCK = {F32: (4, 1), Q8_0: (34, 32), Q4_K: (144, 256), Q6_K: (210, 256), Q5_K: (176, 256)}


def row_bytes(fm, cols):
    """LLB_FM_RB (host/llb_formats.h:16)."""
    b, n = BLOCK[fm]
    return cols // n * b


class LlbError(RuntimeError):
    pass


class MoeLayer(C.Structure):
    """llb_moe_layer (include/llb_moe_hip.h)."""
    _fields_ = [("dm", C.c_uint32), ("ne", C.c_uint32), ("nk", C.c_uint32), ("ef", C.c_uint32), ("sf", C.c_uint32),
                ("fx", C.c_uint32), ("fsg", C.c_uint32), ("fsu", C.c_uint32), ("fsd", C.c_uint32), ("pad", C.c_uint32),
                ("router", C.c_uint64), ("shgate", C.c_uint64), ("G", C.c_uint64), ("U", C.c_uint64), ("D", C.c_uint64),
                ("SG", C.c_uint64), ("SU", C.c_uint64), ("SD", C.c_uint64), ("router_bias", C.c_uint64),
                ("PG", C.c_uint64), ("PU", C.c_uint64), ("PD", C.c_uint64),
                ("PSG", C.c_uint64), ("PSU", C.c_uint64), ("PSD", C.c_uint64),
                ("res", C.c_uint32), ("own", C.c_uint32), ("stream", C.c_uint64)]


_SIGS = {
    "llb_hip_init": (C.c_int, [C.c_int]),
    "llb_hip_last_error": (C.c_char_p, []),
    "llb_hip_set_stream": (C.c_int, [C.c_void_p]),
    "llb_hip_alloc_zero": (C.c_uint64, [C.c_size_t]),
    "llb_hip_free": (C.c_int, [C.c_uint64]),
    "llb_hip_zero": (C.c_int, [C.c_uint64, C.c_size_t]),
    "llb_hip_copy": (C.c_int, [C.c_uint64, C.c_uint64, C.c_size_t]),
    "llb_hip_write": (C.c_int, [C.c_uint64, C.c_void_p, C.c_size_t]),
    "llb_hip_read": (C.c_int, [C.c_void_p, C.c_uint64, C.c_size_t]),
    "llb_hip_sync": (C.c_int, []),
    "llb_hip_mem_info": (C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "llb_hip_module_load": (C.c_int, [C.c_char_p, C.POINTER(C.c_uint64)]),
    "llb_hip_module_function": (C.c_int, [C.c_uint64, C.c_char_p, C.POINTER(C.c_void_p)]),
    "llb_hip_launch": (C.c_int, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                 C.POINTER(C.c_void_p), C.c_uint32]),
    "llb_hip_launch3": (C.c_int, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                  C.POINTER(C.c_void_p), C.c_uint32]),
    "llb_hip_host_alloc": (C.c_int, [C.c_size_t, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)]),
    "llb_hip_host_free": (C.c_int, [C.c_void_p]),
    "llb_hip_copy_h2d_async": (C.c_int, [C.c_uint64, C.c_void_p, C.c_size_t]),
    "llb_hip_graph_begin": (C.c_int, []),
    "llb_hip_graph_end": (C.c_int, [C.POINTER(C.c_uint64)]),
    "llb_hip_graph_launch": (C.c_int, [C.c_uint64]),
    "llb_hip_graph_free": (C.c_int, [C.c_uint64]),
    "llb_moe_table_check": (C.c_int, [C.POINTER(C.c_uint32), C.c_uint32, C.c_uint32, C.c_uint64]),
    "llb_moe_layer_from_table": (C.c_int, [C.POINTER(C.c_uint32), C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64,
                                           C.c_uint64, C.POINTER(MoeLayer)]),
    "llb_moe_run_table": (C.c_int, [C.POINTER(C.c_uint32), C.c_uint32, C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64,
                                    C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64,
                                    C.c_uint64, C.c_uint64, C.c_size_t, C.c_int]),
    "llb_moe_hip_scratch_bytes": (C.c_size_t, [C.POINTER(MoeLayer), C.c_uint32, C.c_int]),
    "llb_moe_hip_forward": (C.c_int, [C.POINTER(MoeLayer), C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64,
                                      C.c_uint64, C.c_uint64, C.c_size_t, C.c_int]),
    "llb_moe_hip_forward_static": (C.c_int, [C.POINTER(MoeLayer), C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64,
                                             C.c_uint64, C.c_uint64, C.c_int]),
    "llb_moe_hip_forward_norm": (C.c_int, [C.POINTER(MoeLayer), C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64,
                                           C.c_float, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64,
                                           C.c_uint64, C.c_size_t, C.c_int]),
    "llb_moe_hip_set_fused": (C.c_int, [C.c_int]),
    "llb_moe_hip_set_q8_gemm": (C.c_int, [C.c_int]),
    "llb_moe_hip_q8_gemm": (C.c_int, []),
    "llb_moe_hip_set_group_scan": (C.c_int, [C.c_int]),
    "llb_moe_hip_set_lean_topk": (C.c_int, [C.c_int]),
    "llb_moe_hip_lean_topk": (C.c_int, []),
    "llb_moe_hip_group_scan": (C.c_int, []),
    "llb_moe_hip_group_scratch_bytes": (C.c_size_t, [C.c_uint32, C.c_uint32]),
    "llb_moe_hip_pack_bytes": (C.c_size_t, [C.POINTER(MoeLayer)]),
    "llb_gguf_open": (C.c_void_p, [C.c_char_p]),
    "llb_gguf_close": (None, [C.c_void_p]),
    "llb_gguf_count": (C.c_uint64, [C.c_void_p]),
    "llb_gguf_find": (C.c_int, [C.c_void_p, C.c_char_p]),
    "llb_gguf_tensor_at": (C.c_int, [C.c_void_p, C.c_uint64, C.c_char_p, C.c_size_t, C.POINTER(C.c_uint64),
                                     C.POINTER(C.c_uint64), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                     C.POINTER(C.c_uint64)]),
    "llb_moe_hip_load_layer": (C.c_int, [C.c_void_p, C.c_uint32, C.c_int, C.POINTER(MoeLayer)]),
    "llb_moe_hip_unload_layer": (C.c_int, [C.POINTER(MoeLayer)]),
    "llb_moe_table_from_gguf": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint32), C.c_uint32, C.POINTER(C.c_uint32)]),
    "llb_moe_hip_residency": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(MoeLayer), C.c_uint32,
                                        C.POINTER(C.c_int), C.POINTER(C.c_uint64)]),
    "llb_moe_hip_pack": (C.c_int, [C.POINTER(MoeLayer), C.c_uint64, C.c_size_t]),
    "llb_moe_hip_status": (C.c_int, [C.c_uint64, C.POINTER(MoeLayer), C.c_uint32]),
    "llb_moe_hip_topk": (C.c_int, [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64,
                                   C.c_uint64, C.c_uint64]),
    "llb_moe_hip_group": (C.c_int, [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64,
                                    C.c_uint64, C.c_size_t]),
    "llb_moe_hip_q8_1": (C.c_int, [C.c_uint64, C.c_uint32, C.c_uint64, C.c_uint64]),
    "llb_moe_hip_rmsnorm_add": (C.c_int, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_uint32, C.c_uint32,
                                          C.c_uint64, C.c_uint64]),
    "llb_moe_hip_dequant": (C.c_int, [C.c_uint32, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint64]),
    "llb_moe_hip_exp": (C.c_int, [C.c_uint64, C.c_uint64, C.c_uint64]),
    "llb_moe_hip_timing": (C.c_int, [C.c_int]),
    "llb_hip_spin": (C.c_int, [C.c_uint32]),
    "llb_moe_hip_timing_read": (C.c_int, [C.POINTER(C.c_double), C.POINTER(C.c_long), C.c_int]),
    "llb_moe_hip_stage_name": (C.c_char_p, [C.c_int]),
    "llb_moe_hip_gen_gauss": (C.c_int, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_uint64]),
    "llb_moe_hip_gen_rows": (C.c_int, [C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32,
                                       C.c_float, C.c_uint64]),
}


def load(path=LIB_PATH):
    """The C-ABI library with prototypes set. Raises if it is not built: there is no CPU path."""
    if not os.path.exists(path):
        raise LlbError(f"{path} is missing: run __graft_entry__.build() (the HIP path has no fallback)")
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


class Device:
    """The backend contract over one GPU, with allocation tracking."""

    def __init__(self, device=0, lib=None):
        self.lib = lib or load()
        self.check(self.lib.llb_hip_init(device))
        self._live = []

    def check(self, rc):
        if rc != 0:
            raise LlbError(f"rc {rc}: {self.lib.llb_hip_last_error().decode()}")
        return rc

    def alloc(self, nbytes):
        p = self.lib.llb_hip_alloc_zero(int(nbytes))
        if p == 0:
            raise LlbError(f"alloc {nbytes}: {self.lib.llb_hip_last_error().decode()}")
        self._live.append(p)
        return p

    def free(self, p):
        if p in self._live:
            self._live.remove(p)
            self.check(self.lib.llb_hip_free(p))

    def free_all(self):
        for p in list(self._live):
            self.free(p)

    def write(self, p, arr):
        a = np.ascontiguousarray(arr)
        self.check(self.lib.llb_hip_write(p, a.ctypes.data, a.nbytes))

    def upload(self, arr):
        a = np.ascontiguousarray(arr)
        p = self.alloc(max(a.nbytes, 4))
        self.write(p, a)
        return p

    def read(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        self.check(self.lib.llb_hip_read(out.ctypes.data, p, out.nbytes))
        return out

    def sync(self):
        self.check(self.lib.llb_hip_sync())

    def set_stream(self, handle):
        self.check(self.lib.llb_hip_set_stream(C.c_void_p(handle) if handle else None))

    def timing(self, on):
        self.check(self.lib.llb_moe_hip_timing(1 if on else 0))

    def timing_read(self):
        """{stage name: (mean us, count)} of the stages timed since timing(True)."""
        us = (C.c_double * 16)()
        n = (C.c_long * 16)()
        k = self.lib.llb_moe_hip_timing_read(us, n, 16)
        return {self.lib.llb_moe_hip_stage_name(i).decode(): (us[i], n[i]) for i in range(k) if n[i]}

    def capture(self, fn):
        """fn's launches recorded as a graph: returns a handle for replay()."""
        self.check(self.lib.llb_hip_graph_begin())
        try:
            fn()
        finally:
            h = C.c_uint64()
            self.check(self.lib.llb_hip_graph_end(C.byref(h)))
        return h.value

    def replay(self, handle):
        self.check(self.lib.llb_hip_graph_launch(handle))

    def mem_info(self):
        f, t = C.c_size_t(), C.c_size_t()
        self.check(self.lib.llb_hip_mem_info(C.byref(f), C.byref(t)))
        return f.value, t.value


# ---------------------------------------------------------------- layer shapes (benchmark workloads)

class Shape:
    def __init__(self, dm, ne, nk, ef, sf, fg, fu, fd, fsg=Q4_K, fsu=Q4_K, fsd=Q6_K, fused=False):
        self.dm, self.ne, self.nk, self.ef, self.sf = dm, ne, nk, ef, sf
        self.fg, self.fu, self.fd, self.fsg, self.fsu, self.fsd, self.fused = fg, fu, fd, fsg, fsu, fsd, fused

    @property
    def fx(self):
        return self.fg | self.fu << 4 | self.fd << 8 | (int(self.fused) << 12) | 1 << 13

    def stack_bytes(self):
        g = self.ne * self.ef * row_bytes(self.fg, self.dm)
        u = self.ne * self.ef * row_bytes(self.fu, self.dm)
        d = self.ne * self.dm * row_bytes(self.fd, self.ef)
        return g, u, d

    def expert_bytes(self):
        """bytes of one routed expert (gate + up + down)."""
        return sum(self.stack_bytes()) // self.ne

    def shared_bytes(self):
        if not self.sf:
            return 0
        return self.sf * (row_bytes(self.fsg, self.dm) + row_bytes(self.fsu, self.dm)) + self.dm * row_bytes(self.fsd, self.sf)


STATIC_SCRATCH_BYTES = 16 << 20  # LLB_MOE_STATIC_SCRATCH_BYTES (llb_moe_hip.h)

SHAPES = {
    # config 1: 128 experts top-8, ef 768, Q8_0, no shared expert
    "c1": Shape(2048, 128, 8, 768, 0, Q8_0, Q8_0, Q8_0),
    # config 2: Qwen3.5-35B-A3B-like: 256 experts top-8, ef 512, Q4_K gate/up, Q6_K down, shared 512
    "c2": Shape(2048, 256, 8, 512, 512, Q4_K, Q4_K, Q6_K),
    # config 4 variant (ii): config 1's layer with Q4_K gate/up and Q6_K down
    "c1k": Shape(2048, 128, 8, 768, 0, Q4_K, Q4_K, Q6_K),
    # config 5: 512 experts top-10, ef 512, shared 512
    "c5": Shape(2048, 512, 10, 512, 512, Q4_K, Q4_K, Q6_K),
}

# hash streams of a layer's tensors: stream = layer * 16 + slot
ST_ROUTER, ST_SHGATE, ST_G, ST_U, ST_D, ST_SG, ST_SU, ST_SD, ST_H2, ST_X1, ST_BIAS = range(11)
W_SIGMA = 0.02


def zipf_bias(ne, seed, s=1.1):
    """Expert-load skew of the batched-decode workload: b_e = log z_e, z proportional to rank^-s over a seeded expert
    permutation (ranks 1..ne), as f32"""
    rank = np.empty(ne, np.int64)
    rank[np.random.default_rng(seed).permutation(ne)] = np.arange(1, ne + 1)
    return (-s * np.log(rank.astype(np.float64))).astype(np.float32)


class Layer:
    """A synthetic MoE layer resident in HBM, generated on the device from (seed, layer)."""

    def __init__(self, dev, shape, seed=0, layer=0, bias=None):
        self.dev, self.shape, self.seed, self.layer = dev, shape, seed, layer
        s, L = shape, layer * 16
        lib = dev.lib
        self.router = dev.alloc(s.ne * s.dm * 4)
        dev.check(lib.llb_moe_hip_gen_rows(F32, seed, L + ST_ROUTER, 0, s.ne, s.dm, W_SIGMA, self.router))
        gb, ub, db = s.stack_bytes()
        self.G = dev.alloc(gb)
        self.U = dev.alloc(ub)
        self.D = dev.alloc(db)
        dev.check(lib.llb_moe_hip_gen_rows(s.fg, seed, L + ST_G, 0, s.ne * s.ef, s.dm, W_SIGMA, self.G))
        dev.check(lib.llb_moe_hip_gen_rows(s.fu, seed, L + ST_U, 0, s.ne * s.ef, s.dm, W_SIGMA, self.U))
        dev.check(lib.llb_moe_hip_gen_rows(s.fd, seed, L + ST_D, 0, s.ne * s.dm, s.ef, W_SIGMA, self.D))
        self.shgate = self.SG = self.SU = self.SD = 0
        if s.sf:
            self.shgate = dev.alloc(s.dm * 4)
            dev.check(lib.llb_moe_hip_gen_rows(F32, seed, L + ST_SHGATE, 0, 1, s.dm, W_SIGMA, self.shgate))
            self.SG = dev.alloc(s.sf * row_bytes(s.fsg, s.dm))
            self.SU = dev.alloc(s.sf * row_bytes(s.fsu, s.dm))
            self.SD = dev.alloc(s.dm * row_bytes(s.fsd, s.sf))
            dev.check(lib.llb_moe_hip_gen_rows(s.fsg, seed, L + ST_SG, 0, s.sf, s.dm, W_SIGMA, self.SG))
            dev.check(lib.llb_moe_hip_gen_rows(s.fsu, seed, L + ST_SU, 0, s.sf, s.dm, W_SIGMA, self.SU))
            dev.check(lib.llb_moe_hip_gen_rows(s.fsd, seed, L + ST_SD, 0, s.dm, s.sf, W_SIGMA, self.SD))
        self.bias = dev.upload(np.asarray(bias, np.float32)) if bias is not None else 0
        self.desc = MoeLayer(s.dm, s.ne, s.nk, s.ef, s.sf, s.fx, s.fsg, s.fsu, s.fsd, 0, self.router, self.shgate,
                             self.G, self.U, self.D, self.SG, self.SU, self.SD, self.bias)

        self.packed = 0

    def pack(self):
        """packed copies of the stacks for the f16 tier (llb_moe_hip_pack); returns the bytes used."""
        n = self.dev.lib.llb_moe_hip_pack_bytes(C.byref(self.desc))
        if not n:
            raise LlbError("llb_moe_hip_pack_bytes: layer cannot be packed")
        self.unpack()
        self.packed = self.dev.alloc(n)
        self.dev.check(self.dev.lib.llb_moe_hip_pack(C.byref(self.desc), self.packed, n))
        return n

    def unpack(self):
        """drop the packed copies (the f16 tier reads the GGUF stacks again)."""
        if self.packed:
            self.dev.free(self.packed)
        self.packed = 0
        for f in ("PG", "PU", "PD", "PSG", "PSU", "PSD"):
            setattr(self.desc, f, 0)

    def free(self):
        for p in (self.router, self.shgate, self.G, self.U, self.D, self.SG, self.SU, self.SD, self.bias, self.packed):
            if p:
                self.dev.free(p)


class Runner:
    """Buffers for T tokens through llb_moe_hip_forward."""

    def __init__(self, dev, shape, T, tier=EXACT):
        self.dev, self.shape, self.T, self.tier = dev, shape, T, tier
        s = shape
        self.h2 = dev.alloc(T * s.dm * 4)
        self.x1 = dev.alloc(T * s.dm * 4)
        self.y = dev.alloc(T * s.dm * 4)
        self.ids = dev.alloc(T * s.nk * 4)
        self.wt = dev.alloc(T * s.nk * 4)
        probe = MoeLayer(s.dm, s.ne, s.nk, s.ef, s.sf, s.fx, s.fsg, s.fsu, s.fsd)
        self.scratch_bytes = dev.lib.llb_moe_hip_scratch_bytes(C.byref(probe), T, tier)
        self.scratch = dev.alloc(self.scratch_bytes)

    def gen_inputs(self, seed, layer=0, residual=True):
        lib, s = self.dev.lib, self.shape
        self.dev.check(lib.llb_moe_hip_gen_gauss(seed, layer * 16 + ST_H2, 0, self.T * s.dm, 1.0, self.h2))
        if residual:
            self.dev.check(lib.llb_moe_hip_gen_gauss(seed, layer * 16 + ST_X1, 0, self.T * s.dm, 1.0, self.x1))

    def forward(self, layer, residual=True):
        self.dev.check(self.dev.lib.llb_moe_hip_forward(C.byref(layer.desc), self.T, self.h2, self.x1 if residual else 0,
                                                        self.y, self.ids, self.wt, self.scratch, self.scratch_bytes,
                                                        self.tier))

    def status(self, layer):
        """raises if a fused launch on this runner's scratch had a phase wait time out."""
        self.dev.check(self.dev.lib.llb_moe_hip_status(self.scratch, C.byref(layer.desc), self.T))

    def outputs(self):
        s = self.shape
        return (self.dev.read(self.y, (self.T, s.dm), np.float32), self.dev.read(self.ids, (self.T, s.nk), np.uint32),
                self.dev.read(self.wt, (self.T, s.nk), np.float32))

    def free(self):
        for p in (self.h2, self.x1, self.y, self.ids, self.wt, self.scratch):
            self.dev.free(p)
