"""llb_moe_hip_residency: llb_moe_load's choice of where the routed experts live (host/llb_host.c:532-545),
run on the CPU with the capacities given through LLB_MOE_VRAM / LLB_MOE_RAM. The expert bytes are the
stacks' sizes in the file; device is chosen when they fit the free device memory less 0.75 GiB, host when
they fit MemAvailable less 4 GiB, stream otherwise; LLB_MOE_EXPERTS forces a mode (an unknown value is
ignored, as in the reference); and the one "moe:" line on stderr names the choice and where each capacity
came from."""
import ctypes as C

import pytest

import eureka_moe as em
import gguf_io

lib = em.load()
SMALL = em.Shape(2048, 16, 4, 256, 256, em.Q4_K, em.Q4_K, em.Q6_K)
RV, RR = 3 << 28, 4 << 30
GIB = 1 << 30


@pytest.fixture
def model(tmp_path):
    ts = gguf_io.layer_tensors(SMALL, seed=4, layer=0) + gguf_io.layer_tensors(SMALL, seed=4, layer=1, blk=3)
    p = str(tmp_path / "m.gguf")
    gguf_io.write(p, ts)
    tot = sum(len(d) for n, _, _, d in ts if "_exps." in n)
    g = lib.llb_gguf_open(p.encode())
    assert g
    yield g, tot
    lib.llb_gguf_close(g)


def _layers(fx=None):
    s = SMALL
    L = (em.MoeLayer * 2)()
    for i in range(2):
        L[i] = em.MoeLayer(s.dm, s.ne, s.nk, s.ef, s.sf, s.fx if fx is None else fx, s.fsg, s.fsu, s.fsd)
    return (C.c_uint32 * 2)(0, 3), L


def _choose(g, monkeypatch, vram=None, ram=None, experts=None, fx=None):
    for k, v in (("LLB_MOE_VRAM", vram), ("LLB_MOE_RAM", ram), ("LLB_MOE_EXPERTS", experts)):
        if v is None:
            monkeypatch.delenv(k, raising=False)
        else:
            monkeypatch.setenv(k, str(v))
    blk, L = _layers(fx)
    mode, nb = C.c_int(-1), C.c_uint64()
    rc = lib.llb_moe_hip_residency(g, blk, L, 2, C.byref(mode), C.byref(nb))
    return rc, mode.value, nb.value


def test_expert_bytes_are_the_stacks(model, monkeypatch):
    g, tot = model
    rc, _, nb = _choose(g, monkeypatch, vram=0, ram=0)
    assert rc == 0 and nb == tot


@pytest.mark.parametrize("dv,dr,want", [
    (0, 0, 0),      # exactly tot + 0.75 GiB of VRAM: device
    (-1, 0, 1),     # one byte short of VRAM, RAM exactly tot + 4 GiB: host
    (-1, -1, 2),    # short of both: stream
    (GIB, -1, 0),   # plenty of VRAM wins whatever the RAM
])
def test_thresholds(model, monkeypatch, capfd, dv, dr, want):
    g, tot = model
    rc, mode, _ = _choose(g, monkeypatch, vram=tot + RV + dv, ram=tot + RR + dr)
    assert rc == 0 and mode == want
    err = capfd.readouterr().err
    names = ["device (VRAM)", "host (pinned, device-mapped RAM)", "stream (mmapped GGUF, the k experts copied per token)"]
    line = [l for l in err.splitlines() if l.startswith("moe: ")]
    assert len(line) == 1, err
    assert line[0].startswith(f"moe: 2 layers, experts {tot / GIB:.2f} GiB -> {names[want]} [free VRAM ")
    assert "(LLB_MOE_VRAM)" in line[0] and "(LLB_MOE_RAM)" in line[0]


@pytest.mark.parametrize("forced,want", [("device", 0), ("host", 1), ("stream", 2)])
def test_forced_mode(model, monkeypatch, forced, want):
    g, tot = model
    for vram, ram in ((0, 0), (1 << 50, 1 << 50)):
        rc, mode, _ = _choose(g, monkeypatch, vram=vram, ram=ram, experts=forced)
        assert rc == 0 and mode == want


def test_unknown_forced_value_is_ignored(model, monkeypatch):
    g, tot = model
    rc, mode, _ = _choose(g, monkeypatch, vram=0, ram=tot + RR, experts="gpu")
    assert rc == 0 and mode == 1


def test_ram_defaults_to_memavailable(model, monkeypatch, capfd):
    g, tot = model
    avail = 0
    for ln in open("/proc/meminfo"):
        if ln.startswith("MemAvailable:"):
            avail = int(ln.split()[1]) * 1024
    rc, mode, _ = _choose(g, monkeypatch, vram=0)
    assert rc == 0 and mode == (1 if tot + RR <= avail else 2)
    line = [l for l in capfd.readouterr().err.splitlines() if l.startswith("moe: ")][0]
    assert "(LLB_MOE_VRAM)" in line and "(LLB_MOE_RAM)" not in line


def test_mismatched_layer_is_refused(model, monkeypatch):
    g, _ = model
    rc, mode, _ = _choose(g, monkeypatch, vram=0, ram=0, fx=em.Q8_0 | em.Q8_0 << 4 | SMALL.fd << 8)
    assert rc != 0 and mode == -1
    assert b"ffn_gate_exps" in lib.llb_hip_last_error()


def test_null_arguments_refused(model):
    g, _ = model
    blk, L = _layers()
    mode = C.c_int()
    assert lib.llb_moe_hip_residency(None, blk, L, 2, C.byref(mode), None) != 0
    assert lib.llb_moe_hip_residency(g, blk, L, 0, C.byref(mode), None) != 0
    assert lib.llb_moe_hip_residency(g, blk, L, 2, None, None) != 0
