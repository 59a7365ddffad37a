"""The GGUF reader (llb_gguf_open / find / tensor_at in eureka-engine_amd/csrc/llb_moe_gguf.cpp; the
reference's llb_gg_tensor, host/llb_gguf.c:854-865) on files written by tests/gguf_io.py: every tensor's
name, absolute offset, bytes, ggml type and dims read back as written, with metadata of every value kind
(strings, arrays of strings and of numbers) skipped; malformed files are refused with a named error, and
random corruption of a valid header never crashes the reader. Host code only: no device needed."""
import ctypes as C
import os

import numpy as np
import pytest

import eureka_moe as em
import gguf_io

lib = em.load()
SMALL = em.Shape(2048, 16, 4, 256, 256, em.Q4_K, em.Q4_K, em.Q6_K)


def read_table(path):
    g = lib.llb_gguf_open(path.encode())
    assert g, lib.llb_hip_last_error()
    out = {}
    try:
        name = C.create_string_buffer(256)
        off, nb, nd = C.c_uint64(), C.c_uint64(), C.c_uint32()
        ty = C.c_uint32()
        dims = (C.c_uint64 * 4)()
        for i in range(lib.llb_gguf_count(g)):
            assert lib.llb_gguf_tensor_at(g, i, name, 256, C.byref(off), C.byref(nb), C.byref(ty), C.byref(nd), dims) == 0
            out[name.value.decode()] = (off.value, nb.value, ty.value, tuple(dims[:nd.value]))
            assert lib.llb_gguf_find(g, name.value) == i
        assert lib.llb_gguf_find(g, b"blk.0.no_such.weight") == -1
    finally:
        lib.llb_gguf_close(g)
    return out


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_tensor_table_round_trip(tmp_path, alignment):
    ts = gguf_io.layer_tensors(SMALL, seed=4, layer=0) + gguf_io.layer_tensors(SMALL, seed=4, layer=1, blk=3)
    path = str(tmp_path / "m.gguf")
    offs = gguf_io.write(path, ts, alignment=alignment)
    tab = read_table(path)
    raw = open(path, "rb").read()
    assert len(tab) == len(ts)
    for name, ty, dims, data in ts:
        off, nb, gty, gd = tab[name]
        assert (off, nb, gty, gd) == (offs[name], len(data), ty, tuple(dims))
        assert off % alignment == 0 and raw[off:off + nb] == data


def _expect_refused(path, why):
    g = lib.llb_gguf_open(path.encode())
    if g:
        lib.llb_gguf_close(g)
    assert not g, why
    assert lib.llb_hip_last_error().startswith(b"gguf:")


def test_malformed_files_refused(tmp_path):
    ts = gguf_io.layer_tensors(SMALL, seed=4, layer=0)[:2]
    good = str(tmp_path / "good.gguf")
    gguf_io.write(good, ts)
    raw = bytearray(open(good, "rb").read())
    cases = {
        "bad magic": b"GGUG" + raw[4:],
        "version 1": raw[:4] + (1).to_bytes(4, "little") + raw[8:],
        "huge tensor count": raw[:8] + (1 << 40).to_bytes(8, "little") + raw[16:],
        "truncated header": raw[:100],
        "truncated data": raw[:-10],
        "empty": b"",
    }
    for why, data in cases.items():
        p = str(tmp_path / "bad.gguf")
        open(p, "wb").write(bytes(data))
        _expect_refused(p, why)
    assert not lib.llb_gguf_open(str(tmp_path / "missing.gguf").encode())
    # a tensor offset past the end, and one not on the alignment
    for shift in (1 << 40, 3):
        p = str(tmp_path / "off.gguf")
        gguf_io.write(p, ts)
        d = bytearray(open(p, "rb").read())
        tab_name = ts[1][0].encode()
        i = d.index(tab_name) + len(tab_name)
        nd = int.from_bytes(d[i:i + 4], "little")
        o = i + 4 + 8 * nd + 4
        d[o:o + 8] = (int.from_bytes(d[o:o + 8], "little") + shift).to_bytes(8, "little")
        open(p, "wb").write(bytes(d))
        _expect_refused(p, f"offset + {shift}")


def test_header_corruption_never_crashes(tmp_path):
    ts = gguf_io.layer_tensors(SMALL, seed=4, layer=0)[:2]
    good = str(tmp_path / "good.gguf")
    offs = gguf_io.write(good, ts)
    raw = bytes(open(good, "rb").read())
    head = min(offs.values())
    rng = np.random.default_rng(0)
    p = str(tmp_path / "fuzz.gguf")
    for _ in range(400):
        d = bytearray(raw)
        for _ in range(rng.integers(1, 6)):
            d[rng.integers(0, head)] = rng.integers(0, 256)
        open(p, "wb").write(bytes(d))
        g = lib.llb_gguf_open(p.encode())
        if g:  # a corruption the format allows: the table must still lie inside the file
            n = lib.llb_gguf_count(g)
            off, nb = C.c_uint64(), C.c_uint64()
            for i in range(n):
                assert lib.llb_gguf_tensor_at(g, i, None, 0, C.byref(off), C.byref(nb), None, None, None) == 0
                assert off.value + nb.value <= len(d)
            lib.llb_gguf_close(g)


def test_load_layer_checks_without_device(tmp_path):
    """type / size mismatches against the layer's formats are refused before any allocation"""
    ts = gguf_io.layer_tensors(SMALL, seed=4, layer=0)
    p = str(tmp_path / "m.gguf")
    gguf_io.write(p, ts)
    g = lib.llb_gguf_open(p.encode())
    try:
        s = SMALL
        wrong = em.MoeLayer(s.dm, s.ne, s.nk, s.ef, s.sf, em.Q8_0 | em.Q8_0 << 4 | s.fd << 8, s.fsg, s.fsu, s.fsd)
        assert lib.llb_moe_hip_load_layer(g, 0, 0, C.byref(wrong)) != 0
        assert b"ffn_gate_exps" in lib.llb_hip_last_error()
        missing = em.MoeLayer(s.dm, s.ne, s.nk, s.ef, s.sf, s.fx, s.fsg, s.fsu, s.fsd)
        assert lib.llb_moe_hip_load_layer(g, 7, 0, C.byref(missing)) != 0
        assert b"not found" in lib.llb_hip_last_error()
        assert lib.llb_moe_hip_load_layer(g, 0, 5, C.byref(missing)) != 0
    finally:
        lib.llb_gguf_close(g)
