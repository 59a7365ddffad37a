"""llb_moe_table_from_gguf: the table rows a qwen35moe GGUF implies, against the reference's own sidecar
writer (tools/gguf2pack.c, built from its source into oracle/_ref by oracle/Makefile) run on the same file:
every word of every row equal, for separate and fused gate / up stacks, K-quant and Q8_0 experts, and a
trailing nextn block that both leave out. The rows then decode (llb_moe_layer_from_table) to the layer's
shape and formats. Host code only."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import eureka_moe as em
import gguf_io

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
G2P = os.path.join(ROOT, "oracle", "_ref", "gguf2pack")
lib = em.load()

# a small but complete qwen35moe backbone: d_model 256, 2 heads of 64, 1 kv head, SSM with 2 groups of
# state 16, inner 128, time-step rank 4, conv kernel 4; every second layer full attention
D, H, KVH, HD = 256, 2, 1, 64
S, NG, INNER, TR, KC = 16, 2, 128, 4, 4
KD, VD = S * NG, INNER
CONV, VHD = 2 * KD + VD, INNER // TR
BYTES = {0: (4, 1), 1: (2, 1), 8: (34, 32), 11: (110, 256), 12: (144, 256), 13: (176, 256), 14: (210, 256),
         23: (136, 256), 30: (2, 1), 42: (18, 64), 142: (34, 128)}


def _t(name, ty, dims):
    bb, be = BYTES[ty]
    n = int(np.prod(dims))
    return (name, ty, tuple(dims), bytes(n // be * bb))


def model(nl, ne, nk, ef, sf, gty, dty, fused=False, mtp=0, types=None):
    """types: {tensor name without "blk.N.": ggml type} overrides for the trunk (every layer)"""
    kv = [("qwen35moe.block_count", 4, nl + mtp), ("qwen35moe.attention.head_count", 4, H),
          ("qwen35moe.attention.head_count_kv", 4, KVH), ("qwen35moe.embedding_length", 4, D),
          ("qwen35moe.attention.key_length", 4, HD), ("qwen35moe.expert_feed_forward_length", 4, ef),
          ("qwen35moe.expert_shared_feed_forward_length", 4, sf), ("qwen35moe.context_length", 4, 4096),
          ("qwen35moe.attention.layer_norm_rms_epsilon", 6, 1e-6), ("qwen35moe.full_attention_interval", 4, 2),
          ("qwen35moe.ssm.conv_kernel", 4, KC), ("qwen35moe.ssm.state_size", 4, S),
          ("qwen35moe.ssm.group_count", 4, NG), ("qwen35moe.ssm.time_step_rank", 4, TR),
          ("qwen35moe.ssm.inner_size", 4, INNER), ("qwen35moe.expert_used_count", 4, nk),
          ("qwen35moe.expert_count", 4, ne)]
    if mtp:
        kv.append(("qwen35moe.nextn_predict_layers", 4, mtp))
    ts = [_t("token_embd.weight", 0, (D, 3)), _t("output_norm.weight", 0, (D,))]
    for i in range(nl + mtp):
        b = f"blk.{i}."
        ts += [_t(b + "attn_norm.weight", 0, (D,)), _t(b + "post_attention_norm.weight", 0, (D,))]
        ts += [_t(b + "ffn_gate_inp.weight", 0, (D, ne)), _t(b + "ffn_gate_inp_shexp.weight", 0, (D,))]
        ts += [_t(b + "ffn_gate_shexp.weight", 12, (D, sf)), _t(b + "ffn_up_shexp.weight", 12, (D, sf)),
               _t(b + "ffn_down_shexp.weight", 14, (sf, D))]
        if (i + 1) % 2 == 0:
            ts += [_t(b + "attn_q.weight", 0, (D, 2 * HD * H)), _t(b + "attn_k.weight", 0, (D, HD * KVH)),
                   _t(b + "attn_v.weight", 0, (D, HD * KVH)), _t(b + "attn_output.weight", 0, (HD * H, D)),
                   _t(b + "attn_q_norm.weight", 0, (HD,)), _t(b + "attn_k_norm.weight", 0, (HD,))]
        else:
            ts += [_t(b + "attn_qkv.weight", 0, (D, 2 * KD + VD)), _t(b + "attn_gate.weight", 0, (D, VD)),
                   _t(b + "ssm_conv1d.weight", 0, (KC, CONV)), _t(b + "ssm_dt.bias", 0, (TR,)),
                   _t(b + "ssm_a", 0, (TR,)), _t(b + "ssm_beta.weight", 0, (D, TR)),
                   _t(b + "ssm_alpha.weight", 0, (D, TR)), _t(b + "ssm_norm.weight", 0, (VHD,)),
                   _t(b + "ssm_out.weight", 0, (VD, D))]
        if fused:
            ts.append(_t(b + "ffn_gate_up_exps.weight", gty, (D, 2 * ef, ne)))
        else:
            ts += [_t(b + "ffn_gate_exps.weight", gty, (D, ef, ne)), _t(b + "ffn_up_exps.weight", gty, (D, ef, ne))]
        ts.append(_t(b + "ffn_down_exps.weight", dty, (ef, D, ne)))
    if types:
        ts = [_t(n, types.get(n.split(".", 2)[2] if n.startswith("blk.") else n, ty), dims) if
              (n.split(".", 2)[2] if n.startswith("blk.") else n) in types else (n, ty, dims, data)
              for n, ty, dims, data in ts]
    return ts, kv


CASES = {"kquants": dict(nl=2, ne=8, nk=2, ef=256, sf=256, gty=12, dty=14),
         "q8_fused": dict(nl=3, ne=16, nk=4, ef=512, sf=256, gty=8, dty=8, fused=True),
         "q5_nextn": dict(nl=2, ne=8, nk=3, ef=256, sf=512, gty=13, dty=12, mtp=1),
         # the other trunk formats the reference's writer places (Q3_K, IQ4_XS, Q2_0, PQ2_0, F16;
         # tools/gguf2pack.c:377-379)
         "trunk_types": dict(nl=2, ne=8, nk=2, ef=256, sf=256, gty=12, dty=14,
                             types={"ffn_gate_shexp.weight": 11, "ffn_up_shexp.weight": 23,
                                    "ffn_down_shexp.weight": 42, "attn_qkv.weight": 142, "attn_gate.weight": 1,
                                    "attn_q.weight": 11, "attn_k.weight": 23})}


def _ours(path, cap=8):
    g = lib.llb_gguf_open(path.encode())
    assert g, lib.llb_hip_last_error()
    try:
        tab, nl = (C.c_uint32 * (32 * cap))(), C.c_uint32()
        rc = lib.llb_moe_table_from_gguf(g, tab, cap, C.byref(nl))
        assert rc == 0, lib.llb_hip_last_error()
        return np.frombuffer(tab, np.uint32)[:32 * nl.value].reshape(nl.value, 32).copy()
    finally:
        lib.llb_gguf_close(g)


@pytest.mark.parametrize("case", sorted(CASES))
def test_table_rows_match_the_reference_sidecar(tmp_path, case):
    if not os.path.exists(G2P):
        pytest.skip("oracle/_ref/gguf2pack is not built (make -C oracle ref; needs the reference tree)")
    ts, kv = model(**CASES[case])
    path = str(tmp_path / "m.gguf")
    gguf_io.write(path, ts, alignment=32, extra_kv=kv)
    out = tmp_path / "side"
    r = subprocess.run([G2P, path, "--sidecar-only", str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    ref = np.fromfile(out / "table.bin", np.uint32).reshape(-1, 32)
    ours = _ours(path)
    assert ours.shape == ref.shape and np.array_equal(ours, ref), (ours ^ ref).nonzero()


@pytest.mark.parametrize("case", sorted(c for c in CASES if "types" not in CASES[c]))
def test_table_rows_decode_to_the_layer(tmp_path, case):
    c = CASES[case]
    ts, kv = model(**c)
    path = str(tmp_path / "m.gguf")
    gguf_io.write(path, ts, alignment=32, extra_kv=kv)
    rows = _ours(path)
    assert rows.shape[0] == c["nl"]
    fm = {8: em.Q8_0, 12: em.Q4_K, 13: em.Q5_K, 14: em.Q6_K}
    for w in rows:
        L = em.MoeLayer()
        w32 = (C.c_uint32 * 32)(*w.tolist())
        assert lib.llb_moe_layer_from_table(w32, D, 1 << 20, 1 << 30, 2 << 30, 3 << 30, C.byref(L)) == 0, \
            lib.llb_hip_last_error()
        assert (L.ne, L.nk, L.ef, L.sf) == (c["ne"], c["nk"], c["ef"], c["sf"])
        assert L.fx & 15 == fm[c["gty"]] and L.fx >> 4 & 15 == fm[c["gty"]] and L.fx >> 8 & 15 == fm[c["dty"]]
        assert bool(L.fx >> 12 & 1) == bool(c.get("fused")) and (L.fsg, L.fsu, L.fsd) == (em.Q4_K, em.Q4_K, em.Q6_K)
        assert L.router == (1 << 20) + (w[21] & 0x0FFFFFFF) and L.shgate == (1 << 20) + (w[22] & 0x0FFFFFFF)


def test_refuses_a_layer_without_its_stacks(tmp_path):
    ts, kv = model(**CASES["kquants"])
    ts = [t for t in ts if t[0] != "blk.1.ffn_down_exps.weight"]
    path = str(tmp_path / "m.gguf")
    gguf_io.write(path, ts, alignment=32, extra_kv=kv)
    g = lib.llb_gguf_open(path.encode())
    try:
        tab, nl = (C.c_uint32 * 256)(), C.c_uint32()
        assert lib.llb_moe_table_from_gguf(g, tab, 8, C.byref(nl)) != 0
        assert b"stacks" in lib.llb_hip_last_error()
    finally:
        lib.llb_gguf_close(g)


def _edit(ts, name, ty=None, dims=None):
    out = []
    for t in ts:
        if t[0] == name:
            t = _t(name, t[1] if ty is None else ty, t[2] if dims is None else dims)
        out.append(t)
    return out


D_, NE_, EF_ = D, CASES["kquants"]["ne"], CASES["kquants"]["ef"]
BAD = {
    "duplicate": lambda ts: ts + [_t("blk.0.ssm_a", 0, (TR,))],
    "router_q8": lambda ts: _edit(ts, "blk.0.ffn_gate_inp.weight", ty=8),
    "router_shape": lambda ts: _edit(ts, "blk.1.ffn_gate_inp.weight", dims=(D_, NE_ + 1)),
    "shgate_shape": lambda ts: _edit(ts, "blk.0.ffn_gate_inp_shexp.weight", dims=(D_, 2)),
    "gate_experts": lambda ts: _edit(ts, "blk.0.ffn_gate_exps.weight", dims=(D_, EF_, NE_ - 1)),
    "down_rows": lambda ts: _edit(ts, "blk.1.ffn_down_exps.weight", dims=(EF_, 2 * D_, NE_)),
    "up_f32": lambda ts: _edit(ts, "blk.1.ffn_up_exps.weight", ty=0),
    "up_q3k": lambda ts: _edit(ts, "blk.1.ffn_up_exps.weight", ty=11),
    # BF16 anywhere: no format code (the reference's writer has no registry entry for it and does not finish)
    "norm_bf16": lambda ts: _edit(ts, "blk.0.attn_norm.weight", ty=30),
    "embd_bf16": lambda ts: _edit(ts, "token_embd.weight", ty=30),
}


@pytest.mark.parametrize("bad", sorted(BAD))
def test_refuses_what_the_reference_sidecar_refuses(tmp_path, bad):
    """the reference's sidecar writer dies on these files (duplicate names, a router or shared gate that is
    not F32 of its shape, expert stacks of the wrong shape or format); the table builder refuses them too"""
    ts, kv = model(**CASES["kquants"])
    path = str(tmp_path / "m.gguf")
    gguf_io.write(path, BAD[bad](ts), alignment=32, extra_kv=kv)
    g = lib.llb_gguf_open(path.encode())
    assert g, lib.llb_hip_last_error()
    try:
        tab, nl = (C.c_uint32 * 256)(), C.c_uint32()
        assert lib.llb_moe_table_from_gguf(g, tab, 8, C.byref(nl)) != 0
        assert lib.llb_hip_last_error().startswith(b"table: ")
    finally:
        lib.llb_gguf_close(g)
    if os.path.exists(G2P):
        r = subprocess.run([G2P, path, "--sidecar-only", str(tmp_path / "side")], capture_output=True, text=True,
                           timeout=120)
        assert r.returncode != 0, r.stdout
