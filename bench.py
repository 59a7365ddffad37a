"""Benchmark of the MoE FFN hot path on one MI355X (headline metric: MoE layer us/token at
decode + prefill tok/s, each against the HBM / MFMA roofline).

Default workload (single-token decode): the Qwen3.5-35B-A3B-like layer -- hidden 2048, 256 experts,
top-8, expert ff 512, shared expert 512, gate/up Q4_K, down Q6_K -- decoding one token through
40 independently seeded layers resident in HBM (about 21 GB of expert stacks, far past the caches).
A step = one token through the 40 layers; value = microseconds per token-layer.

  python bench.py [--steps K] [--warmup W] [--layers L] [--config c2] [--tier exact|q8] [--no-cpu]
                  [--legs q8,batched,prefill,prefill_k,c5,rmsnorm,residency]
  python bench.py --copy-calib          (the PMC byte-counter calibration copies only)
  python bench.py --traffic-from DIR    (profiles/traffic.json from rocprofv3 FETCH_SIZE / WRITE_SIZE passes)
"""
import argparse
import subprocess
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "eureka-engine_amd"), os.path.join(ROOT, "tests")]

import numpy as np  # noqa: E402

import eureka_moe as em  # noqa: E402

HBM_PEAK_GBS = 8000.0


def measured_traffic(workload, stage, applies=True):
    """HBM bytes per launch of a stage's kernel, as rocprofv3 FETCH_SIZE / WRITE_SIZE passes measured it
    (calibrated against a copy of known size): profiles/traffic.json. None when not measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)[workload][stage] if applies else None
    except (OSError, KeyError, ValueError):
        return None


def traffic_source():
    """where roofline.traffic comes from: it is not measured in this run (PMC counters need their own
    rocprofv3 passes), so the line names the file and the commit its passes were made at"""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            at = json.load(f).get("commit", "unrecorded")
    except (OSError, ValueError):
        return None
    return f"profiles/traffic.json (rocprofv3 FETCH_SIZE / WRITE_SIZE passes at commit {at}), not this run"


# kernel (rocprofv3 name prefix) -> (workload, stage) for the PMC passes run with --legs prefill,prefill_k;
# the GEMM's first template argument is the weight format (1 Q8_0, 3 Q4_K, 4 Q6_K), its second the mode
TRAFFIC_KERNELS = {
    "k_router<": ("c2_decode", "route"),
    "k_gu_dec<": ("c2_decode", "gate_up"),
    "k_dn_dec<": ("c2_decode", "down"),
    "k_moe_gemm3<1u, 0u, true>": ("c1_prefill_2048", "gate_up"),
    "k_moe_gemm3<1u, 1u, true>": ("c1_prefill_2048", "down"),
    "k_moe_gemm3<3u, 0u, true>": ("c1k_prefill_2048", "gate_up"),
    "k_moe_gemm3<4u, 1u, true>": ("c1k_prefill_2048", "down"),
}


def _counter_means(d, counter, prefix=None):
    """mean value of `counter` per dispatch for each kernel in a rocprofv3 --pmc csv directory."""
    import csv
    import glob
    fs = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not fs:
        raise SystemExit(f"bench.py: no counter_collection.csv under {d}")
    acc = {}
    for f in fs:
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] != counter:
                continue
            name = r["Kernel_Name"].removeprefix("void ").removeprefix("__amd_rocclr_")
            key = next((k for k in (prefix or TRAFFIC_KERNELS) if name.startswith(k)), None)
            if key is None:
                continue
            # a dispatch's counter can be split over rows (one per XCD / instance): sum by dispatch first
            acc.setdefault(key, {}).setdefault(r["Dispatch_Id"], 0.0)
            acc[key][r["Dispatch_Id"]] += float(r["Counter_Value"])
    return {k: sum(v.values()) / len(v) for k, v in acc.items()}


def traffic_from(d):
    """profiles/traffic.json from DIR/{pmc,cal}_{FETCH_SIZE,WRITE_SIZE}: per-launch HBM bytes of each stage
    kernel, each counter scaled by what it reads for the --copy-calib copies (256 MiB each)."""
    cal_kib = (256 << 20) / 1024
    cf = _counter_means(os.path.join(d, "cal_FETCH_SIZE"), "FETCH_SIZE", ["copyBuffer"])["copyBuffer"]
    cw = _counter_means(os.path.join(d, "cal_WRITE_SIZE"), "WRITE_SIZE", ["copyBuffer"])["copyBuffer"]
    ff, wf = cal_kib / cf, cal_kib / cw
    fe = _counter_means(os.path.join(d, "pmc_FETCH_SIZE"), "FETCH_SIZE")
    wr = _counter_means(os.path.join(d, "pmc_WRITE_SIZE"), "WRITE_SIZE")
    out = {"method": "rocprofv3 --pmc FETCH_SIZE, then --pmc WRITE_SIZE (KiB per dispatch, averaged over "
                     "dispatches); bytes = FETCH_SIZE * fetch_factor * 1024 + WRITE_SIZE * write_factor * 1024, "
                     "the factors from 256 MiB device-to-device copies (bench.py --copy-calib) profiled the same way",
           "fetch_factor": round(ff, 4), "write_factor": round(wf, 4),
           "calibration_kib": {"fetch": cf, "write": cw}, "kib_per_dispatch": {}}
    try:
        out["commit"] = subprocess.run(["git", "-C", ROOT, "rev-parse", "--short", "HEAD"], capture_output=True,
                                       text=True, timeout=10).stdout.strip() or "unrecorded"
    except (OSError, subprocess.SubprocessError):
        out["commit"] = "unrecorded"
    # kernels the passes did not see keep their earlier figures (a pass may cover decode or prefill only)
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            old = json.load(f)
        for k, v in old.get("kib_per_dispatch", {}).items():
            if k in TRAFFIC_KERNELS and k not in fe:
                out["kib_per_dispatch"][k] = v
                wl, st = TRAFFIC_KERNELS[k]
                out.setdefault(wl, {})[st] = old[wl][st]
    except (OSError, KeyError, ValueError):
        pass
    for k, (wl, st) in TRAFFIC_KERNELS.items():
        if k in fe and k in wr:
            out.setdefault(wl, {})[st] = int(round((fe[k] * ff + wr[k] * wf) * 1024))
            out["kib_per_dispatch"][k] = {"fetch": round(fe[k], 1), "write": round(wr[k], 1)}
    with open(os.path.join(ROOT, "profiles", "traffic.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


def stage_bytes(shape, T=1, shared_in_gu=True):
    """algorithmic HBM bytes per launch of each stage for T = 1 decode (every selected expert distinct).
    shared_in_gu: the one-token decode kernels read the shared expert's gate / up rows in the gate / up
    launch (k_gu_dec); the general path reads them in the router launch."""
    s = shape
    rbg, rbu, rbd = em.row_bytes(s.fg, s.dm), em.row_bytes(s.fu, s.dm), em.row_bytes(s.fd, s.ef)
    route = s.ne * s.dm * 4
    gate_up = s.nk * s.ef * (rbg + rbu)
    down = s.nk * s.dm * rbd
    if s.sf:
        sgu = s.sf * (em.row_bytes(s.fsg, s.dm) + em.row_bytes(s.fsu, s.dm))
        route += s.dm * 4
        if shared_in_gu:
            gate_up += sgu
        else:
            route += sgu
        down += s.dm * em.row_bytes(s.fsd, s.sf)
    return {"route": route, "gate_up": gate_up, "down": down}


MFMA_F16_PEAK_TFS = 2500.0


MFMA_I8_PEAK_TOPS = 5000.0


def prefill(dev, shape, T, layers, steps, warmup, name="", tier=None, graph=False):
    """T-token chunks through `layers` resident layers on the f16 MFMA tier (stacks packed once,
    outside the timer) or the q8 tier: tokens/s, and the gate/up kernel's rate (algorithmic flops
    2 T nk dm ef x 2 per launch over its HIP-event time) against the f16 MFMA peak (f16 tier) or the
    int8 MFMA peak (q8 tier, whose products run on v_dot4 rather than the matrix cores)."""
    tier = em.F16 if tier is None else tier
    Ls = [em.Layer(dev, shape, seed=1, layer=100 + i) for i in range(layers)]
    if tier == em.F16:
        for L in Ls:
            L.pack()
    run = em.Runner(dev, shape, T, tier=tier)
    run.gen_inputs(1)
    dev.sync()

    def step():
        for L in Ls:
            run.forward(L)

    for _ in range(max(1, warmup)):  # eager first: the f16 tier makes its side stream on first use
        step()
    dev.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    dev.sync()
    wall_eager = time.perf_counter() - t0
    wall = wall_eager
    launch = "eager"
    if graph:  # the same launches replayed as one graph a step (as the decode line runs)
        try:
            gs = dev.capture(step)
            dev.replay(gs)
            dev.sync()
            t0 = time.perf_counter()
            for _ in range(steps):
                dev.replay(gs)
            dev.sync()
            wall = time.perf_counter() - t0
            dev.check(dev.lib.llb_hip_graph_free(gs))
            launch = "one HIP graph a step"
        except em.LlbError as e:  # keep the eager figure, and say why
            launch = f"eager (graph capture failed: {e})"
    dev.timing(1)
    dev.check(dev.lib.llb_hip_spin(20000))
    for L in Ls:
        run.forward(L)
    st = dev.timing_read()
    dev.timing(False)
    gu_us = st["gate_up"][0]
    flops = 2.0 * T * shape.nk * shape.dm * shape.ef * 2
    ach = flops / (gu_us * 1e-6) / 1e12
    wbytes = shape.ne * shape.ef * (em.row_bytes(shape.fg, shape.dm) + em.row_bytes(shape.fu, shape.dm))
    run.free()
    for L in Ls:
        L.free()
    us_layer = wall / (steps * layers) * 1e6
    q8_mfma = tier != em.F16 and dev.lib.llb_moe_hip_q8_gemm() == 1
    wgbs = wbytes / (gu_us * 1e-6) / 1e9
    if tier == em.F16 or q8_mfma:
        peak = MFMA_F16_PEAK_TFS if tier == em.F16 else MFMA_I8_PEAK_TOPS
        kern = "gate_up GEMM (f16 MFMA)" if tier == em.F16 else "gate_up GEMM (int8 MFMA on q8_1 activations)"
        roof = {"bound": "mfma", "kernel": kern, "achieved": round(ach, 1), "peak": peak,
                "unit": "TFLOP/s" if tier == em.F16 else "TOP/s", "frac": round(ach / peak, 4)}
    else:
        # per-slot v_dot4 GEMVs use no matrix core: priced as a weight stream (every expert's gate / up
        # bytes once a launch) against HBM
        roof = {"bound": "hbm", "kernel": "gate_up (int8 v_dot4 GEMVs on q8_1 activations, per slot)",
                "achieved": round(wgbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(wgbs / HBM_PEAK_GBS, 4),
                "int8_tops": round(ach, 2)}
    roof.update({"traffic": measured_traffic(f"{name}_prefill_{T}", "gate_up", tier == em.F16),
                 "traffic_source": traffic_source(),
                 "kernel_us": round(gu_us, 2), "weight_gbs": round(wgbs, 1)})
    return {"tokens_per_s": round(T / (us_layer * 1e-6), 1), "us_per_layer_chunk": round(us_layer, 2), "T": T,
            "layers": layers, "launch": launch,
            "eager_us_per_layer_chunk": round(wall_eager / (steps * layers) * 1e6, 2),
            "stages_us": {k: round(v[0], 2) for k, v in st.items()}, "roofline": roof}


def batched(dev, shape, T, layers, steps, warmup, tier):
    """config 3: T tokens a step through `layers` layers with the Zipf(1.1) router bias"""
    Ls = [em.Layer(dev, shape, seed=3, layer=200 + i, bias=em.zipf_bias(shape.ne, 3 + i)) for i in range(layers)]
    if tier == em.F16:
        for L in Ls:
            L.pack()
    run = em.Runner(dev, shape, T, tier=tier)
    run.gen_inputs(3)
    for _ in range(warmup):
        for L in Ls:
            run.forward(L)
    dev.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        for L in Ls:
            run.forward(L)
    dev.sync()
    wall = time.perf_counter() - t0
    dev.timing(1)
    dev.check(dev.lib.llb_hip_spin(20000))
    for L in Ls:
        run.forward(L)
    st = dev.timing_read()
    dev.timing(False)
    ids = dev.read(run.ids, (T, shape.nk), np.uint32)
    uniq = int(np.unique(ids).size)
    hist = np.bincount(ids.ravel(), minlength=shape.ne)
    load = {"tokens_per_expert_top10": sorted(hist.tolist(), reverse=True)[:10], "experts_hit": uniq,
            "experts_with_20_or_more": int((hist >= 20).sum()), "experts_unused": int((hist == 0).sum())}
    run.free()
    for L in Ls:
        L.free()
    us = wall / (steps * layers) * 1e6
    byts = uniq * shape.expert_bytes() + shape.ne * shape.dm * 4 + shape.shared_bytes()
    return {"us_per_layer": round(us, 2), "us_per_token_layer": round(us / T, 3), "T": T,
            "unique_experts_last_layer": uniq, "expert_load_last_layer": load, "algorithmic_bytes_last_layer": byts,
            "stages_us": {k: round(v[0], 2) for k, v in st.items()},
            "hbm_frac_last_layer": round(byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def rmsnorm_leg(dev, n, steps=50):
    """llb_moe_hip_rmsnorm_add (the router's input step): microseconds a call for one decode row, and
    HBM bytes / time for a 2048-row chunk (x, z read, x1, h2 written: 16 bytes a column a row)"""
    out = {}
    for T in (1, 2048):
        bufs = [dev.alloc(T * n * 4) for _ in range(4)]
        w = dev.alloc(n * 4)
        dev.check(dev.lib.llb_moe_hip_gen_gauss(0, 900, 0, T * n, 1.0, bufs[0]))
        dev.check(dev.lib.llb_moe_hip_gen_gauss(0, 901, 0, T * n, 1.0, bufs[1]))
        dev.check(dev.lib.llb_moe_hip_gen_gauss(0, 902, 0, n, 1.0, w))
        call = lambda: dev.check(dev.lib.llb_moe_hip_rmsnorm_add(bufs[0], bufs[1], w, 1e-6, T, n, bufs[2], bufs[3]))  # noqa: E731
        call()
        dev.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            call()
        dev.sync()
        us = (time.perf_counter() - t0) / steps * 1e6
        for b in bufs + [w]:
            dev.free(b)
        if T == 1:
            out["us_per_call_T1"] = round(us, 2)
        else:
            gbs = 16.0 * T * n / (us * 1e-6) / 1e9
            out["T2048"] = {"us": round(us, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    out["config"] = f"n = {n}, eps 1e-6, back-to-back eager calls (the T = 1 figure includes launch)"
    return out


def residency_leg(dev, shape, tokens=16):
    """GGUF expert stacks (llb_moe_hip_load_layer) in each residency mode on one layer of `shape`: the
    file is written from a device-generated layer (the same bytes), then per mode the load time (file to
    placement: GB/s of expert stacks) and eager exact-tier decode microseconds a token-layer."""
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gguf_io
    s = shape
    L = em.Layer(dev, s, seed=6, layer=0)
    gb, ub, db = s.stack_bytes()
    rd = lambda p, n: dev.read(p, (n,), np.uint8).tobytes()  # noqa: E731
    ts = [("blk.0.ffn_gate_inp.weight", 0, (s.dm, s.ne), rd(L.router, s.ne * s.dm * 4)),
          ("blk.0.ffn_gate_exps.weight", gguf_io.GGML[s.fg], (s.dm, s.ef, s.ne), rd(L.G, gb)),
          ("blk.0.ffn_up_exps.weight", gguf_io.GGML[s.fu], (s.dm, s.ef, s.ne), rd(L.U, ub)),
          ("blk.0.ffn_down_exps.weight", gguf_io.GGML[s.fd], (s.ef, s.dm, s.ne), rd(L.D, db))]
    if s.sf:
        ts += [("blk.0.ffn_gate_inp_shexp.weight", 0, (s.dm,), rd(L.shgate, s.dm * 4)),
               ("blk.0.ffn_gate_shexp.weight", gguf_io.GGML[s.fsg], (s.dm, s.sf), rd(L.SG, s.sf * em.row_bytes(s.fsg, s.dm))),
               ("blk.0.ffn_up_shexp.weight", gguf_io.GGML[s.fsu], (s.dm, s.sf), rd(L.SU, s.sf * em.row_bytes(s.fsu, s.dm))),
               ("blk.0.ffn_down_shexp.weight", gguf_io.GGML[s.fsd], (s.sf, s.dm), rd(L.SD, s.dm * em.row_bytes(s.fsd, s.sf)))]
    L.free()
    out = {}
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as td:
        path = os.path.join(td, "layer.gguf")
        gguf_io.write(path, ts)
        g = dev.lib.llb_gguf_open(path.encode())
        assert g, dev.lib.llb_hip_last_error()
        run = em.Runner(dev, s, 1, tier=em.EXACT)
        for mode, name in ((0, "device"), (1, "host"), (2, "stream")):
            desc = em.MoeLayer(s.dm, s.ne, s.nk, s.ef, s.sf, s.fx, s.fsg, s.fsu, s.fsd)
            t0 = time.perf_counter()
            dev.check(dev.lib.llb_moe_hip_load_layer(g, 0, mode, C.byref(desc)))
            dev.sync()
            load_s = time.perf_counter() - t0

            class Lo:
                pass
            lo = Lo()
            lo.desc = desc
            run.gen_inputs(7)
            run.forward(lo)
            dev.sync()
            t0 = time.perf_counter()
            for _ in range(tokens):
                run.forward(lo)
            dev.sync()
            us = (time.perf_counter() - t0) / tokens * 1e6
            dev.check(dev.lib.llb_moe_hip_unload_layer(C.byref(desc)))
            out[name] = {"load_s": round(load_s, 3), "load_gbs": round((gb + ub + db) / load_s / 1e9, 2),
                         "decode_us_per_token_layer": round(us, 1)}
        run.free()
        dev.lib.llb_gguf_close(g)
    out["config"] = (f"one {s.ne}-expert layer ({(gb + ub + db) / 1e9:.2f} GB of expert stacks) from a GGUF on the "
                     f"box's local disk (page cache warm after the write); eager exact-tier decode, {tokens} tokens")
    return out


def hbm_copy_leg(dev, nbytes=1 << 30, reps=20):
    """achievable HBM bandwidth: device-to-device copies of 1 GiB (read + write bytes over wall time, one sync
    around the batch), beside the 8 TB/s datasheet peak the roofline fractions use"""
    src, dst = dev.alloc(nbytes), dev.alloc(nbytes)
    dev.check(dev.lib.llb_hip_copy(dst, src, nbytes))
    dev.sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        dev.check(dev.lib.llb_hip_copy(dst, src, nbytes))
    dev.sync()
    dt = time.perf_counter() - t0
    dev.free(src)
    dev.free(dst)
    gbs = 2 * nbytes * reps / dt / 1e9
    return {"gbs": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
            "config": f"{reps} device-to-device copies of {nbytes >> 20} MiB (hipMemcpyAsync), read + write bytes"}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(shape, seconds=12.0, threads=1):
    """the CPU oracle's exact layer on tokens of layer 0 (experts generated first, outside the timer): one
    thread, and with threads > 1 also the rows-parallel OpenMP variant on the same tokens. Returns
    (single, threaded or None)."""
    import oracle_lib as ol
    hl = ol.HostLayer(shape, seed=0, layer=0, experts=[])
    n, spent, spent_mt, t = 0, 0.0, 0.0, 0
    while spent < seconds and n < 64:
        h2 = ol.gauss(0, ol.ST_H2, t * shape.dm, shape.dm).reshape(1, shape.dm)
        ids, _, _ = hl.route(h2)
        hl.add_experts(np.unique(ids))
        hl._mk()
        for nt in ((1, threads) if threads > 1 else (1,)):
            y = np.zeros((1, shape.dm), np.float32)
            i2, w2, s2 = np.zeros((1, shape.nk), np.uint32), np.zeros((1, shape.nk), np.float32), np.zeros(1, np.float32)
            t0 = time.perf_counter()
            rc = ol.lib().mo_moe_exact(C.byref(hl.desc), 1, ol.ptr(h2), None, ol.ptr(y), ol.ptr(i2), ol.ptr(w2),
                                       ol.ptr(s2), nt)
            dt = time.perf_counter() - t0
            assert rc == 0
            if nt == 1:
                spent += dt
            else:
                spent_mt += dt
        n += 1
        t += 1

    def rec(sec, nt):
        return {"value": sec / n * 1e6, "unit": "us/token-layer", "cores": nt, "kind": "port",
                "sample": f"{n} decode tokens of one {shape.ne}-expert layer through the oracle's exact tier "
                          f"(oracle/moe_oracle.c, -O2 -ffp-contract=off, {nt} thread{'s' if nt > 1 else ''}"
                          f"{', OpenMP over rows' if nt > 1 else ''}); expert generation outside the timer; "
                          f"host CPU {cpu_model()}, {os.cpu_count()} logical CPUs visible"}
    return rec(spent, 1), (rec(spent_mt, threads) if threads > 1 else None)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--tier", default="exact", choices=["exact", "q8"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--q8-gemm", action="store_true", help="the q8 tier's int8-MFMA GEMM (llb_moe_hip_set_q8_gemm)")
    ap.add_argument("--group-scan", action="store_true", help="histogram + scan dispatch (llb_moe_hip_set_group_scan)")
    ap.add_argument("--lean-topk", action="store_true", help="the decode's lean top-k (llb_moe_hip_set_lean_topk)")
    ap.add_argument("--eager", dest="graph", action="store_false", help="launch per layer instead of a graph")
    ap.add_argument("--no-prefill", dest="prefill", action="store_false", help="skip the prefill leg")
    ap.add_argument("--prefill-config", default="c1")
    ap.add_argument("--prefill-T", type=int, default=2048)
    ap.add_argument("--no-c5", dest="c5", action="store_false",
                    help="skip the config-5 leg (48 resident 512-expert layers, 1 + 512 tokens a launch)")
    ap.add_argument("--legs", default="q8,step,batched,prefill,prefill_k,prefill_q8,c5,rmsnorm,residency,copy",
                    help="legs after the decode line: q8 (the int8 tier's decode), step (the decode step with the "
                         "input step, two calls or one), batched (config 3), prefill (c1), "
                         "prefill_k (c1k), prefill_q8 (c1 on the q8 tier), c5, rmsnorm, residency (GGUF stacks in each "
                         "residency mode), copy "
                         "(achievable HBM bandwidth)")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="only write profiles/traffic.json from the PMC csv directories under DIR and exit")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only run three 256 MiB device-to-device copies (the PMC byte-counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the MoE path is not sharded across GPUs); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.traffic_from:
        traffic_from(args.traffic_from)
        return
    legs = set(args.legs.split(",")) if args.legs else set()
    if not args.prefill:
        legs -= {"batched", "prefill", "prefill_k", "prefill_q8"}
    if not args.c5:
        legs.discard("c5")
    if args.copy_calib:
        dev = em.Device(0)
        n = 256 << 20
        src, dst = dev.alloc(n), dev.alloc(n)
        for _ in range(3):
            dev.check(dev.lib.llb_hip_copy(dst, src, n))
        dev.sync()
        print(json.dumps({"copy_calib_bytes": 3 * n}), flush=True)
        return

    shape = em.SHAPES[args.config]
    tier = em.EXACT if args.tier == "exact" else em.Q8
    dev = em.Device(0)
    dev.check(dev.lib.llb_moe_hip_set_q8_gemm(1 if args.q8_gemm else 0))
    dev.check(dev.lib.llb_moe_hip_set_group_scan(1 if args.group_scan else 0))
    dev.check(dev.lib.llb_moe_hip_set_lean_topk(1 if args.lean_topk else 0))
    layers = [em.Layer(dev, shape, seed=0, layer=i) for i in range(args.layers)]
    T = 1
    h2 = dev.alloc(args.layers * shape.dm * 4)
    x1 = dev.alloc(args.layers * shape.dm * 4)
    for i in range(args.layers):
        dev.check(dev.lib.llb_moe_hip_gen_gauss(0, i * 16 + em.ST_H2, 0, shape.dm, 1.0, h2 + i * shape.dm * 4))
        dev.check(dev.lib.llb_moe_hip_gen_gauss(0, i * 16 + em.ST_X1, 0, shape.dm, 1.0, x1 + i * shape.dm * 4))
    y = dev.alloc(args.layers * shape.dm * 4)
    ids = dev.alloc(args.layers * shape.nk * 4)
    wt = dev.alloc(args.layers * shape.nk * 4)
    sb = dev.lib.llb_moe_hip_scratch_bytes(C.byref(layers[0].desc), T, tier)
    sc = dev.alloc(sb)
    dev.sync()

    def step():
        for i, L in enumerate(layers):
            dev.check(dev.lib.llb_moe_hip_forward(C.byref(L.desc), T, h2 + i * shape.dm * 4, x1 + i * shape.dm * 4,
                                                  y + i * shape.dm * 4, ids + i * shape.nk * 4, wt + i * shape.nk * 4,
                                                  sc, sb, tier))

    run = step
    if args.graph:
        g = dev.capture(step)  # one token through every layer as one HIP graph (llb_graph_begin / end)
        run = lambda: dev.replay(g)  # noqa: E731
    for _ in range(args.warmup):
        run()
    dev.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    dev.sync()
    wall = time.perf_counter() - t0
    us_layer = wall / (args.steps * args.layers) * 1e6

    # one more pass over the layers with HIP events around each stage, queued behind a bounded stall
    # so the kernels run back to back: each stage interval is one kernel (route: its four tree rows)
    nl = min(args.layers, 64)
    sub = lambda: [dev.check(dev.lib.llb_moe_hip_forward(  # noqa: E731
        C.byref(layers[i].desc), T, h2 + i * shape.dm * 4, x1 + i * shape.dm * 4, y + i * shape.dm * 4,
        ids + i * shape.nk * 4, wt + i * shape.nk * 4, sc, sb, tier)) for i in range(nl)]
    dev.timing(1)
    dev.check(dev.lib.llb_hip_spin(20000))  # the host queues every launch while the GPU is held
    sub()
    stages = dev.timing_read()
    dev.timing(False)

    # the int8 tier (expert products on q8_1 activations, llb_mx_*'s arithmetic) on the same layers and
    # tokens, one graph a step
    q8_us = None
    if "q8" in legs and tier == em.EXACT:
        def step_q8():
            for i, L in enumerate(layers):
                dev.check(dev.lib.llb_moe_hip_forward(C.byref(L.desc), T, h2 + i * shape.dm * 4, x1 + i * shape.dm * 4,
                                                      y + i * shape.dm * 4, ids + i * shape.nk * 4, wt + i * shape.nk * 4,
                                                      sc8, sb8, em.Q8))
        sb8 = dev.lib.llb_moe_hip_scratch_bytes(C.byref(layers[0].desc), T, em.Q8)
        sc8 = dev.alloc(sb8)
        run8 = step_q8
        if args.graph:
            g8 = dev.capture(step_q8)
            run8 = lambda: dev.replay(g8)  # noqa: E731
        for _ in range(args.warmup):
            run8()
        dev.sync()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            run8()
        dev.sync()
        q8_us = (time.perf_counter() - t0) / (args.steps * args.layers) * 1e6
        dev.free(sc8)

    # a whole decode step per layer: the input step (x1 = x + z, h2 = rmsnorm(x1) w) then the layer, each
    # layer's input the previous layer's output, one HIP graph a step; two calls a layer, and the input
    # step inside the router launch (llb_moe_hip_forward_norm)
    step_us = None
    if "step" in legs and tier == em.EXACT:
        z = dev.alloc(shape.dm * 4)
        wn = dev.alloc(shape.dm * 4)
        xin = dev.alloc(shape.dm * 4)
        dev.check(dev.lib.llb_moe_hip_gen_gauss(1, em.ST_X1, 0, shape.dm, 1.0, z))
        dev.check(dev.lib.llb_moe_hip_gen_gauss(1, em.ST_H2, 0, shape.dm, 1.0, xin))
        dev.check(dev.lib.llb_moe_hip_gen_gauss(2, 0, 0, shape.dm, 0.1, wn))
        dm4 = shape.dm * 4

        def chain(fused):
            def f():
                for i, L in enumerate(layers):
                    xi = xin if i == 0 else y + (i - 1) * dm4
                    a = (C.byref(L.desc), T)
                    tail = (y + i * dm4, ids + i * shape.nk * 4, wt + i * shape.nk * 4, sc, sb, tier)
                    if fused:
                        dev.check(dev.lib.llb_moe_hip_forward_norm(*a, xi, z, wn, 1e-6, x1 + i * dm4, h2 + i * dm4, *tail))
                    else:
                        dev.check(dev.lib.llb_moe_hip_rmsnorm_add(xi, z, wn, 1e-6, T, shape.dm, x1 + i * dm4, h2 + i * dm4))
                        dev.check(dev.lib.llb_moe_hip_forward(*a, h2 + i * dm4, x1 + i * dm4, *tail))
            return f
        step_us = {}
        for nm, fused in (("two_calls", False), ("input_step_in_router", True)):
            fn = chain(fused)
            gs = dev.capture(fn) if args.graph else None
            runs = (lambda: dev.replay(gs)) if args.graph else fn
            for _ in range(args.warmup):
                runs()
            dev.sync()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                runs()
            dev.sync()
            step_us[nm] = round((time.perf_counter() - t0) / (args.steps * args.layers) * 1e6, 3)
            if gs:
                dev.check(dev.lib.llb_hip_graph_free(gs))
        for p_ in (z, wn, xin):
            dev.free(p_)

    # the one-token exact decode runs k_router / k_gu_dec / k_dn_dec for dm = 2048 layers
    sbytes = stage_bytes(shape, shared_in_gu=(tier == em.EXACT and shape.dm == 2048))
    dom = max(("gate_up", "down"), key=lambda k: stages.get(k, (0, 0))[0])
    dom_us = stages[dom][0]
    ach = sbytes[dom] / (dom_us * 1e-6) / 1e9
    layer_bytes = sum(sbytes.values())
    out = {
        "metric": f"moe_layer_us_per_token_decode_{args.config}",
        "value": round(us_layer, 3),
        "unit": "us/token-layer",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32" if tier == em.EXACT else "int8",
        "data": "synthetic: weights N(0,0.02) quantized on the device by this project's quantizers, x N(0,1)",
        "variants": {"q8_gemm": args.q8_gemm, "group_scan": args.group_scan, "lean_topk": args.lean_topk},
        "config": {"workload": f"{args.config} decode, 1 token through {args.layers} resident layers, {args.tier} tier"
                                f"{', one HIP graph a step' if args.graph else ', eager launches'}",
                   "dm": shape.dm, "ne": shape.ne, "nk": shape.nk, "ef": shape.ef, "sf": shape.sf,
                   "formats": {"gate": shape.fg, "up": shape.fu, "down": shape.fd}},
        "layer_gbs": round(layer_bytes / (us_layer * 1e-6) / 1e9, 1),
        "layer_frac_hbm": round(layer_bytes / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "stages_us": {k: round(v[0], 3) for k, v in stages.items()},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(f"{args.config}_decode", dom, args.tier == "exact"),
                     "traffic_source": traffic_source(),
                     "bytes_per_launch": sbytes[dom], "kernel_us": round(dom_us, 3)},
    }
    if step_us is not None:
        out["decode_step_with_input"] = dict(us_per_token_layer=step_us, config=(
            f"{args.config} decode, 1 token a layer through {args.layers} layers, each layer's input step "
            f"(llb_rmsnorm_add, eps 1e-6) then the layer, the next layer's input its output; exact tier"
            f"{', one HIP graph a step' if args.graph else ''}"))
    if q8_us is not None:
        out["decode_q8_tier"] = {"us_per_token_layer": round(q8_us, 3),
                                 "config": f"{args.config} decode, the int8 tier (q8_1 activations, v_dot4), same layers "
                                           f"and tokens{', one HIP graph a step' if args.graph else ''}"}
    if "batched" in legs:
        b3 = {}
        for tn, tv in (("f16", em.F16), ("exact", em.EXACT)):
            b3[tn] = batched(dev, em.SHAPES["c1"], 64, 4, max(2, args.steps // 4), 1, tv)
        out["batched_c3"] = b3
    for L in layers:
        L.free()
    layers.clear()
    if "prefill" in legs:
        pshape = em.SHAPES[args.prefill_config]
        out["prefill"] = prefill(dev, pshape, args.prefill_T, 4, max(2, args.steps // 4), 1, args.prefill_config,
                                 graph=args.graph)
        out["prefill"]["config"] = f"{args.prefill_config} layer, {args.prefill_T}-token chunk, f16 MFMA tier, packed stacks"
    if "prefill_q8" in legs:
        # the q8 tier (the reference's LLB_PREFILL=fast numerics: q8_1 activations, integer block dots)
        out["prefill_q8"] = prefill(dev, em.SHAPES[args.prefill_config], args.prefill_T, 2, max(2, args.steps // 8), 1,
                                    args.prefill_config, tier=em.Q8, graph=args.graph)
        out["prefill_q8"]["config"] = (f"{args.prefill_config} layer, {args.prefill_T}-token chunk, q8 tier "
                                       f"(q8_1 activations, v_dot4 block dots), GGUF stacks")
    if "prefill_k" in legs:
        # the same layer shape with Q4_K gate / up and Q6_K down weight tiles
        out["prefill_k_quants"] = prefill(dev, em.SHAPES["c1k"], args.prefill_T, 4, max(2, args.steps // 4), 1, "c1k",
                                          graph=args.graph)
        out["prefill_k_quants"]["config"] = f"c1k layer (Q4_K gate/up, Q6_K down), {args.prefill_T}-token chunk, f16 MFMA tier, packed stacks"
    if "c5" in legs:
        # config 5: one decode token and a 512-token chunk in one launch, Zipf(1.1) routing, 48 resident
        # layers (512 experts, top-10, ~1 GB each) cycled layer by layer
        c5 = batched(dev, em.SHAPES["c5"], 513, 48, 2, 1, em.F16)
        c5["tokens_per_s"] = round(513 / (c5["us_per_layer"] * 1e-6), 1)
        c5["config"] = "c5: 48 layers x 512 experts top-10 (Q4_K gate/up, Q6_K down, shared expert), 1 + 512 tokens a launch, f16 tier, packed stacks"
        out["c5_mixed"] = c5
    if "residency" in legs:
        out["residency_gguf"] = residency_leg(dev, shape)
    if "rmsnorm" in legs:
        out["rmsnorm_add"] = rmsnorm_leg(dev, shape.dm)
    if "copy" in legs:
        out["hbm_copy"] = hbm_copy_leg(dev)
    if not args.no_cpu:
        # and the rows-parallel variant on the box's CPU share (OMP_NUM_THREADS, 16 on the GPU boxes)
        nt = max(1, min(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1), 64))
        out["cpu_baseline"], mt = cpu_baseline(shape, threads=nt)
        if mt:
            out["cpu_baseline_threads"] = mt
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
