"""A GGUF v3 writer for tests (test infrastructure): the metadata and tensor-table layout of the GGUF
format (a public file format; the reader under test is eureka-engine_amd/csrc/llb_moe_gguf.cpp), and a
synthetic MoE layer's tensors named as llama.cpp's qwen MoE models name them, with the bytes of
eureka_moe.Layer(dev, shape, seed, layer) (oracle_lib.gen_rows: the device generator's bytes)."""
import struct

import numpy as np

import eureka_moe as em
import oracle_lib as ol

GGML = {em.F32: 0, em.Q8_0: 8, em.Q4_K: 12, em.Q5_K: 13, em.Q6_K: 14}
_KV_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, ty, val):
    out = _str(key) + struct.pack("<I", ty)
    if ty == 8:
        return out + _str(val)
    if ty == 9:
        et, items = val
        out += struct.pack("<IQ", et, len(items))
        for it in items:
            out += _str(it) if et == 8 else struct.pack(_KV_FMT[et], it)
        return out
    return out + struct.pack(_KV_FMT[ty], val)


def write(path, tensors, alignment=32, extra_kv=()):
    """tensors: [(name, ggml_type, dims (ne0 fastest), bytes)]; returns {name: absolute offset}"""
    kvs = [("general.architecture", 8, "qwen35moe"), ("general.alignment", 4, alignment),
           ("tokenizer.ggml.tokens", 9, (8, ["a", "bb", "ccc"])), ("qwen35moe.expert_count", 4, 8),
           ("qwen35moe.rope.freq_base", 6, 1e6), ("general.tags", 9, (4, [1, 2, 3]))]
    extra = list(extra_kv)
    kvs = [k for k in kvs if k[0] not in {e[0] for e in extra}] + extra  # extra_kv replaces a default key
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs))
    for k in kvs:
        head += _kv(*k)
    rel, off = [], 0
    for name, ty, dims, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        rel.append(off)
        head += _str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", ty, off)
        off += len(data)
    data0 = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data0 - len(head)))
        pos = 0
        for (name, ty, dims, data), r in zip(tensors, rel):
            f.write(b"\0" * (r - pos))
            f.write(data)
            pos = r + len(data)
    return {t[0]: data0 + r for t, r in zip(tensors, rel)}


def layer_tensors(shape, seed, layer, blk=None):
    """the tensors of eureka_moe.Layer(dev, shape, seed, layer) as GGUF blk.<blk>.* entries"""
    s, L = shape, layer * 16
    blk = layer if blk is None else blk
    rows = lambda fm, st, nr, cols: ol.gen_rows(fm, seed, L + st, 0, nr, cols).tobytes()  # noqa: E731
    t = [(f"blk.{blk}.ffn_gate_inp.weight", 0, (s.dm, s.ne), rows(em.F32, em.ST_ROUTER, s.ne, s.dm)),
         (f"blk.{blk}.ffn_gate_exps.weight", GGML[s.fg], (s.dm, s.ef, s.ne), rows(s.fg, em.ST_G, s.ne * s.ef, s.dm)),
         (f"blk.{blk}.ffn_up_exps.weight", GGML[s.fu], (s.dm, s.ef, s.ne), rows(s.fu, em.ST_U, s.ne * s.ef, s.dm)),
         (f"blk.{blk}.ffn_down_exps.weight", GGML[s.fd], (s.ef, s.dm, s.ne), rows(s.fd, em.ST_D, s.ne * s.dm, s.ef))]
    if s.sf:
        t += [(f"blk.{blk}.ffn_gate_inp_shexp.weight", 0, (s.dm,), rows(em.F32, em.ST_SHGATE, 1, s.dm)),
              (f"blk.{blk}.ffn_gate_shexp.weight", GGML[s.fsg], (s.dm, s.sf), rows(s.fsg, em.ST_SG, s.sf, s.dm)),
              (f"blk.{blk}.ffn_up_shexp.weight", GGML[s.fsu], (s.dm, s.sf), rows(s.fsu, em.ST_SU, s.sf, s.dm)),
              (f"blk.{blk}.ffn_down_shexp.weight", GGML[s.fsd], (s.sf, s.dm), rows(s.fsd, em.ST_SD, s.dm, s.sf))]
    return t
