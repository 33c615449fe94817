"""Benchmark of the ternary x int8 GEMM path on one MI355X.

Default workload (one step): the full linear set of one FastConformer layer at T=338 frames, d_model=1024, every
GEMM on synthetic resident inputs with its epilogue: FF1 up 1024->4096 (SiLU) and down 4096->1024 (AddScaled 0.5),
stacked q|k|v 1024->3072, pos 1024->1024 on 2T-1=675 rows, out-proj 1024->1024 (AddScaled 1), conv pointwise1
1024->2048 and pointwise2 1024->1024 (AddScaled 1), FF2 up/down. Trits P(0)=0.4, P(+-1)=0.3; per-output-channel f16
scales in [0.01, 0.05]; activations N(0,1) quantized per token (group = K). value = ternary x int8 GEMM TOPS
(2*M*N*K per GEMM, zeros counted) over the timed steps.

Each step is replayed from a HIP graph captured once (the launches of a real encoder step are captured the same
way), so the timed region holds device work only. Prints one JSON line. Extra keys: "roofline" for the dominant kernel (HIP-event time per launch on the launch
stream), "cpu_baseline" (the AVX-512 VNNI restatement on the host cores, bounded sample), "details" (the M=338 and
M=8192 FFN-up GEMM alone, group = K and 128).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, TOP/s
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, GB/s


def layer_shapes(t: int):
    """(name, M, K, N, epilogue kind, alpha) of one layer's linear set (encoder.rs:79-94,138-293,582-630)."""
    return [
        ("ff1_up", t, 1024, 4096, 1, 0.0),
        ("ff1_down", t, 4096, 1024, 2, 0.5),
        ("qkv", t, 1024, 3072, 0, 0.0),
        ("pos", 2 * t - 1, 1024, 1024, 0, 0.0),
        ("o_proj", t, 1024, 1024, 2, 1.0),
        ("pw1", t, 1024, 2048, 0, 0.0),
        ("pw2", t, 1024, 1024, 2, 1.0),
        ("ff2_up", t, 1024, 4096, 1, 0.0),
        ("ff2_down", t, 4096, 1024, 2, 0.5),
    ]


def cpu_info():
    """The host CPU as /proc/cpuinfo and lscpu name it: model name, vendor family / model / stepping (on AMD, family
    26 is Zen 5 and 25 is Zen 3/4), logical CPUs, and whether AVX-512 VNNI is present."""
    info = {"logical_cpus": os.cpu_count()}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k in ("model name", "vendor_id", "cpu family", "model", "stepping") and k.replace(" ", "_") not in info:
                    info[k.replace(" ", "_")] = v
                if k == "flags" and "avx512_vnni_flag" not in info:
                    info["avx512_vnni"] = "avx512_vnni" in v.split()
                    info["avx512_vnni_flag"] = True
                if line.strip() == "" and "model_name" in info:
                    break
    except OSError:
        pass
    info.pop("avx512_vnni_flag", None)
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core"):
                info["lscpu_" + k.strip().lower().replace(" ", "_").replace("(s)", "s")] = v.strip()
    except (OSError, ValueError):
        pass
    return info


def algo_bytes(m, k, n, group, int32_out=False):
    """2-bit weights + f32 weight scales + int8 activations + f32 activation scales (+ gsum) + f32 output."""
    ng = k // group
    b = n * k / 4 + n * ng * 4 + m * k + m * ng * 8 + m * n * 4
    return b + (m * n * 4 if int32_out else 0)


class Gemm:
    """One GEMM with resident synthetic operands."""

    def __init__(self, vx, synth, dev, name, m, k, n, ep, alpha, group, cfg, role, int32_out=False):
        import torch

        self.name, self.m, self.k, self.n, self.group = name, m, k, n, group
        trits = synth.synth_trits(synth.workload_seed(cfg, role), n, k)
        s16 = synth.synth_channel_scales_f16(synth.workload_seed(cfg, role + 1), n, k // group)
        x = synth.synth_normal(synth.workload_seed(cfg, role + 2), m * k).reshape(m, k)
        self.w = vx.TernaryMatrix.from_packed(synth.pack_rows(trits), s16, n, k, group)
        self.xa = vx.QuantAct.quantize(torch.from_numpy(x).to(dev), group)
        self.y = torch.zeros((m, n), dtype=torch.float32, device=dev)
        # int32 output: the exact sums of each group beside y (with one group, the int32 accumulators)
        self.gs = torch.zeros((k // group, m, n), dtype=torch.int32, device=dev) if int32_out else None
        self.ep = {0: vx.Epilogue.Store, 1: vx.Epilogue.Silu}.get(ep) or vx.Epilogue.AddScaled(alpha)
        self.vx = vx
        self.ops = 2.0 * m * n * k
        self.bytes = algo_bytes(m, k, n, group, int32_out)
        self.host = (trits, s16, x)

    def run(self):
        self.vx.gemm_ep(self.w, self.xa, self.y, None, self.ep, self.gs)


def capture(torch, fn, reps=1):
    """A HIP graph (torch.cuda.CUDAGraph) replaying `fn` `reps` times: the step is launched back to back by the
    device, without Python or launch overhead between kernels."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm (first-call work happens outside the capture)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    torch.cuda.synchronize()
    return g


def time_launches(torch, gemms, reps, replays=5):
    """Average device time per launch of each GEMM: a graph of `reps` launches replayed `replays` times, timed
    with HIP events on the replay stream."""
    out = {}
    st = torch.cuda.current_stream()
    for g in gemms:
        graph = capture(torch, g.run, reps)
        graph.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(replays):
            graph.replay()
        b.record(st)
        torch.cuda.synchronize()
        out[g.name] = a.elapsed_time(b) * 1e-3 / (reps * replays)
        del graph
    return out


def traffic_of(g):
    """HBM bytes per launch of a GEMM of the step, from the committed rocprofv3 --pmc summary
    (profiles/tgemm_traffic.json: FETCH_SIZE and WRITE_SIZE of the GEMM's kernel in the default bench run, each
    scaled by the same counter's reading for a plain copy of known size); None when absent or for another shape."""
    path = os.path.join(ROOT, "profiles", "tgemm_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    shape = f"{g.m}x{g.k}x{g.n}:G{g.group}:ep{g.ep.kind}"
    for e in t.get("entries", []):
        if e.get("shape") == shape:
            return e.get("traffic_bytes")
    return None


def roofline_of(g, sec):
    t_mfma = g.ops / (PEAK_INT8_TOPS * 1e12)
    t_hbm = g.bytes / (PEAK_HBM_GBS * 1e9)
    if t_mfma >= t_hbm:
        a = g.ops / sec / 1e12
        return {"bound": "mfma", "achieved": round(a, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                "frac": round(a / PEAK_INT8_TOPS, 4)}
    a = g.bytes / sec / 1e9
    return {"bound": "hbm", "achieved": round(a, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(a / PEAK_HBM_GBS, 4)}


def cpu_baseline(gemms, budget_s=10.0):
    """The reference's AVX-512 VNNI kernel (C restatement, oracle/vnni_baseline.c) with gemm_ep's row-block split
    on the host cores, over the same layer's GEMMs, repeated until about `budget_s` of CPU work."""
    from oracle import oracle

    if not oracle.lib().or_have_vnni():
        return None
    threads = min(os.cpu_count() or 1, 16)
    prepared = []
    for g in gemms:
        trits, s16, x = g.host
        ws = oracle.f16_to_f32(s16)
        q, xs, gsum = oracle.quantize(x, g.group)
        wq, sq = oracle.quad16_pack(trits, ws, g.group)
        y = np.zeros((g.m, g.n), np.float32)
        prepared.append((g, wq, sq, q, xs, gsum, y))

    def one_pass():
        for g, wq, sq, q, xs, gsum, y in prepared:
            oracle.gemm_ep_vnni(wq, sq, g.n, g.k, g.group, q, xs, gsum, y, g.ep.kind, g.ep.alpha, threads=threads)

    one_pass()  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        one_pass()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 1000:
            break
    ops = sum(g.ops for g in gemms) * reps
    cpu = cpu_info()
    return {"value": round(ops / el / 1e12, 4), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"{reps} passes of the same layer's {len(gemms)} GEMMs (T=338), {el:.1f} s, "
                      f"{threads} threads of {cpu.get('logical_cpus')} logical CPUs "
                      f"({cpu.get('lscpu_model_name') or cpu.get('model_name', '?')}, family {cpu.get('cpu_family', '?')} "
                      f"model {cpu.get('model', '?')}), AVX-512 VNNI restatement of kernels/x86.rs with gemm_ep's "
                      f"block split"}


ENC_WORKLOADS = [  # (name, log-mel frames at 10 ms, segments): 27.04 s -> T=338, 60 s -> T=750, 32 x 10 s -> T=125
    ("t338_27s", 2704, 1),
    ("t750_60s", 6000, 1),
    ("b32x10s_t125", 1000, 32),
]


def encoder_setup(synth, n_layers=24):
    """The 24-layer encoder with random ternary weights (synth.synth_layer) and random subsampling weights."""
    from voxrt_amd import encoder as E

    enc = E.Encoder(n_layers=n_layers)
    params = [synth.synth_layer(i) for i in range(n_layers)]
    for i, p in enumerate(params):
        enc.set_layer(i, p)
    sp = synth.synth_subsampling()
    enc.set_subsampling(sp)
    return enc, params, sp


def encoder_rtfx(torch, synth, enc, dev, reps=5, only=None):
    """Device time of encoder forwards from log-mel features (subsampling + 24 layers, each frame count replayed
    from its hipGraph), as RTFx = audio seconds / encoder seconds. Several segments of one length go through one
    batched forward (each segment's output equals its own forward); "sequential_ms" times the same segments one
    forward at a time."""
    out = {}
    for name, t_in, nseg in ENC_WORKLOADS:
        if only and name != only:
            continue
        feats = torch.from_numpy(synth.synth_normal(synth.workload_seed(4, t_in & 0xFF), nseg * t_in * 128)
                                 .reshape(nseg, t_in, 128)).to(dev)

        def run(y):
            if nseg == 1:
                enc.forward_feats(feats[0], out=y[0])
            else:
                enc.forward_feats_batch(feats, out=y)

        y = torch.empty((nseg, enc.out_frames(t_in), enc.d), dtype=torch.float32, device=dev)
        run(y)  # first call: workspace, graph capture
        run(y)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run(y)
        e1.record()
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) * 1e-3 / reps
        audio = t_in * nseg / 100.0
        out[name] = {"frames": enc.out_frames(t_in), "segments": nseg, "audio_s": audio, "ms": round(sec * 1e3, 3),
                     "rtfx": round(audio / sec, 1)}
        if nseg > 1:
            y1 = enc.forward_feats(feats[0])
            torch.cuda.synchronize()
            e0.record()
            for s in range(nseg):
                enc.forward_feats(feats[s], out=y1)
            e1.record()
            torch.cuda.synchronize()
            out[name]["sequential_ms"] = round(e0.elapsed_time(e1), 3)
            del y1
        del y
    return out


def clip_batch_tops(torch, vx, synth, dev, params, reps=3, group=None):
    """64 short clips (25 + lcg % 164 frames each, 2-15 s) concatenated to M rows of per-token int8 activations
    through the linear layers of all 24 layers (ff1 up/down, q|k|v, out, pw1, pw2, ff2 up/down; the position
    projection depends on each clip's length and is left out). group None: one group (per-output-channel scales,
    G = K); 128: the model's 128-column groups. Returns the aggregate TOPS of one pass over the 192 GEMMs."""
    lens = 25 + synth.Lcg(synth.workload_seed(2, 0)).take(64) % 164
    m = int(lens.sum())
    names = ("ff1_w1", "ff1_w2", "qkv", "o", "pw1", "pw2", "ff2_w1", "ff2_w2")
    acts = {}
    for k in (1024, 4096):
        x = torch.from_numpy(synth.synth_normal(synth.workload_seed(2, k >> 10), m * k).reshape(m, k)).to(dev)
        acts[k] = vx.QuantAct.quantize(x, group or k)
        del x
    work, ops, ys = [], 0.0, {}
    for p in params:
        for n in names:
            q, s16 = p["linears"][n]
            out, inp = s16.shape[0], s16.shape[1] * 128
            if group:
                w = vx.TernaryMatrix.from_packed(q, s16, out, inp, group)
            else:
                w = vx.TernaryMatrix.from_packed(q, np.ascontiguousarray(s16[:, :1]), out, inp, inp)
            if out not in ys:  # one output buffer per width: the GEMMs run one after another
                ys[out] = torch.empty((m, out), dtype=torch.float32, device=dev)
            work.append((w, acts[inp], ys[out]))
            ops += 2.0 * m * out * inp

    def step():
        for w, a, y in work:
            vx.gemm_ep(w, a, y, None, vx.Epilogue.Store)

    graph = capture(torch, step)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / reps
    del graph, work, acts, ys
    torch.cuda.empty_cache()
    return {"clips": 64, "rows": m, "gemms": 192, "group": group or "K", "ms": round(sec * 1e3, 3),
            "tops": round(ops / sec / 1e12, 1),
            "pct_int8_peak": round(100 * ops / sec / 1e12 / PEAK_INT8_TOPS, 1)}


def cpu_single_core(synth, kernel="vnni"):
    """The reference's per-core CPU GEMM protocol (tests/x86_bench.rs:31-72): FF shapes 4096x1024 and 1024x4096,
    n = 376 tokens, trits lcg % 3 - 1 and x = (lcg % 2001)/100 - 10 from seed 1, f16 scales 0.02, group 128, a
    256-row slice through one x86 range kernel on one thread, best of 5; GMAC/s per core, as bench/README.md:122-123
    quotes (AVX-512 VNNI 337-359, AVX2 178-181 on a Zen 5 core). kernel: "vnni" (x86.rs:46-154) or "avx2"
    (x86.rs:163-290), both restated in oracle/."""
    from oracle import oracle

    if kernel == "vnni" and not oracle.lib().or_have_vnni():
        return None
    if kernel == "avx2" and not oracle.lib().or_have_avx2():
        return None
    rng = synth.Lcg(1)
    out_rates = {}
    for out, inp in ((4096, 1024), (1024, 4096)):
        n, rows = 376, 256
        trits = (rng.take(out * inp) % 3).astype(np.int8).reshape(out, inp) - 1
        ws = np.full((out, inp // 128), np.float32(np.float16(0.02)), np.float32)
        xf = ((rng.take(n * inp) % 2001).astype(np.float32) / np.float32(100.0) - np.float32(10.0)).reshape(n, inp)
        q, xs, gsum = oracle.quantize(xf, 128)
        wq, sq = oracle.quad16_pack(trits.astype(np.int8), ws, 128)
        y = np.zeros((n, out), np.float32)
        best = float("inf")
        for _ in range(5):
            t0 = time.perf_counter()
            if kernel == "vnni":
                oracle.gemm_vnni_range(wq, sq, out, inp, 128, q, xs, gsum, y, 0, rows, 0, n)
            else:
                oracle.gemm_avx2_range(wq, sq, out, inp, 128, True, q, xs, gsum, y, 0, rows, 0, n)
            best = min(best, time.perf_counter() - t0)
        out_rates[f"{out}x{inp}"] = round(rows * inp * n / best / 1e9, 1)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    name = {"vnni": "AVX-512 VNNI", "avx2": "AVX2"}[kernel]
    return {"gmac_per_s_per_core": out_rates, "threads": 1, "cpu": model, "logical_cpus": os.cpu_count(),
            "protocol": f"x86_bench.rs: n=376, 256-row slice, best of 5, {name} restatement"}


class Gemv:
    """One decoder-style GEMV (gemm_single, kernels/mod.rs:285-316): int8 rows [out, 640] with f32 scales in
    128-column groups, one token, bias; operands as the kernels.rs:271-316 grid draws them, resident on the device."""

    def __init__(self, vx, synth, dev, out, inp=640):
        import torch

        rng = synth.Lcg(out)
        rows = (rng.take(out * inp) % 255).astype(np.uint8).view(np.int8).reshape(out, inp)
        scales = ((rng.take(out * inp // 128) % 100).astype(np.float32) / np.float32(1000.0)
                  + np.float32(0.001)).astype(np.float32).reshape(out, inp // 128)
        x = ((rng.take(inp) % 2001).astype(np.float32) / np.float32(100.0) - np.float32(10.0)).reshape(1, inp)
        self.name, self.vx = f"gemv_{out}x{inp}", vx
        self.w = vx.TernaryMatrix.from_i8_rows(rows, scales, out, inp, 128)
        self.x = vx.QuantAct.quantize(torch.from_numpy(x).to(dev), 128)
        self.bias = torch.from_numpy((rng.take(out) % 100).astype(np.float32)).to(dev)
        self.y = torch.zeros((1, out), dtype=torch.float32, device=dev)
        self.bytes = out * inp + out * (inp // 128) * 4 + inp + 8 * (inp // 128) + out * 8

    def run(self):
        self.vx.gemm_single(self.w, self.x, self.y, self.bias)


def attention_us(torch, dev, reps=10):
    """The int8 attention core of one layer alone (8 heads, head_dim 128; q|k|v and the relative rows N(0,1)):
    microseconds per call at T = 338 and 750, and the MAC rate over its 3072*T^2 MACs (Q.K, Q.R band, P.V)."""
    from voxrt_amd import encoder as E

    out = {}
    for t in (338, 750):
        r = np.random.default_rng(t)
        qkv = torch.from_numpy(r.standard_normal((t, 3072)).astype(np.float32)).to(dev)
        rel = torch.from_numpy(r.standard_normal((2 * t - 1, 1024)).astype(np.float32)).to(dev)
        bu = torch.from_numpy((0.1 * r.standard_normal((8, 128))).astype(np.float32)).to(dev)
        bv = torch.from_numpy((0.1 * r.standard_normal((8, 128))).astype(np.float32)).to(dev)
        ctx = torch.empty((t, 1024), dtype=torch.float32, device=dev)
        ws = torch.empty(max(E.attention_ws_bytes(t, 1024, 8), 1), dtype=torch.uint8, device=dev)
        graph = capture(torch, lambda: E.attention_core(qkv, rel, 8, bu, bv, ctx=ctx, ws=ws), reps)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(3):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (3 * reps)
        del graph
        out[f"t{t}"] = {"us": round(us, 2), "gmac_per_s": round(3072 * t * t / us * 1e-3, 1)}
    return out


def cpu_encoder_rtfx(params, sp, synth, budget_s=30.0):
    """The CPU int8 encoder restatement (oracle: VNNI GEMMs on all threads, glue parallel like the reference's
    rayon loops) timed on the host cores: subsampling + 24 layers, weights unpacked and Quad16-packed beforehand
    (load time). Stops after the budget; reports what it timed."""
    from oracle import oracle as orc

    threads = min(os.cpu_count() or 1, 16)
    orc.set_threads(threads)
    layers = []
    for p in params:
        lp = {n: (orc.unpack_rows(q, s.shape[1] * 128), orc.f16_to_f32(s)) for n, (q, s) in p["linears"].items()}
        lp["norms"] = p["norms"]
        lp["bias_u"], lp["bias_v"] = p["bias_u"], p["bias_v"]
        lp["dw_t"], lp["dw_bias"] = orc.fold_bn(p["dw"], **p["bn"])
        layers.append(orc.pack_layer_quad16(lp))
    out = {}
    spent = 0.0
    for name, t_in, nseg in ENC_WORKLOADS:
        if spent > budget_s:
            break
        feats = synth.synth_normal(synth.workload_seed(4, t_in & 0xFF), t_in * 128).reshape(t_in, 128)
        t0 = time.perf_counter()
        done = 0
        for _ in range(nseg):
            x = orc.subsampling(feats, sp)
            t = x.shape[0]
            pos = orc.rel_pos_table(t, 1024)
            for lp in layers:
                x = orc.conformer_layer(x, pos, lp, heads=8, threads=threads)
            done += 1
            if time.perf_counter() - t0 + spent > budget_s:
                break
        sec = (time.perf_counter() - t0) / done
        spent += sec * done
        out[name] = {"segments_timed": done, "ms_per_segment": round(sec * 1e3, 1),
                     "rtfx": round(t_in / 100.0 / sec, 1)}
    orc.set_threads(1)
    return {"threads": threads, "kind": "port", "by_workload": out,
            "note": "C restatement of the reference's int8 Encoder::forward (encoder.rs:816-856): GEMMs through the "
                    "AVX-512 VNNI restatement on all threads; LayerNorm, softmax, GLU/depthwise conv and the f32 "
                    "subsampling as plain C loops parallel over rows (the reference vectorizes these with NEON/AVX2 "
                    "helpers), so the reference's own CPU encoder is faster and x_vs_cpu is an upper bound. For "
                    "context, the reference publishes 104-105x real time end to end (frontend + encoder + decoder) "
                    "on 16 Zen 5 threads (README.md:62-67)."}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-details", action="store_true")
    ap.add_argument("--no-encoder", action="store_true", help="skip the 24-layer encoder RTFx leg")
    ap.add_argument("--encoder-only", action="store_true",
                    help="only the 24-layer encoder RTFx leg (prints its JSON and exits)")
    ap.add_argument("--encoder-workload", choices=[w[0] for w in ENC_WORKLOADS],
                    help="with --encoder-only: time this workload alone (for kernel traces)")
    ap.add_argument("--gemm", type=int, nargs=4, metavar=("M", "K", "N", "G"),
                    help="run only this GEMM (Store epilogue), 6 eager launches: for counter collection")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only run a plain 256 MiB device copy 5 times (the counter calibration of the traffic figure)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the ternary GEMM path shards by "
              f"independent clips with no collective, so a multi-GPU figure is N independent copies of this one",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calib:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes": src.numel() * 4, "dispatches": 5}), flush=True)
        return

    import voxrt_amd as vx
    from voxrt_amd import synth

    vx.kernels.check(vx.lib().vx_init(0))
    dev = torch.device("cuda:0")
    if args.gemm:
        m, k, n, grp = args.gemm
        g = Gemm(vx, synth, dev, "gemm", m, k, n, 0, 0.0, grp, 2, 1)
        for _ in range(6):
            g.run()
        torch.cuda.synchronize()
        print(json.dumps({"gemm": f"{m}x{k}x{n}:G{grp}", "launches": 6, "ops_per_launch": g.ops}), flush=True)
        return
    if args.encoder_only:
        enc, eparams, esp = encoder_setup(synth)
        out = {"encoder": encoder_rtfx(torch, synth, enc, dev, only=args.encoder_workload)}
        enc.free()
        if not args.no_cpu:
            out["encoder_cpu"] = cpu_encoder_rtfx(eparams, esp, synth)
        print(json.dumps(out), flush=True)
        return
    T = 338
    gemms = [Gemm(vx, synth, dev, name, m, k, n, ep, a, k, 1, 16 * i + 1)
             for i, (name, m, k, n, ep, a) in enumerate(layer_shapes(T))]

    def step():
        for g in gemms:
            g.run()

    graph = capture(torch, step)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = e0.elapsed_time(e1) * 1e-3
    ops = sum(g.ops for g in gemms)
    value = ops * args.steps / gpu_s / 1e12
    del graph

    per = time_launches(torch, gemms, 20)
    # the roofline kernel: the slowest launch of the step (the FFN up- and down-projections take about the same
    # time, so it may be either); every GEMM's own roofline entry is in details
    dom = max(gemms, key=lambda g: per[g.name])
    roof = roofline_of(dom, per[dom.name])
    roof["kernel"] = f"ternary GEMM {dom.name}: M={dom.m} K={dom.k} N={dom.n} G={dom.group} (small-token kernel)"
    roof["traffic"] = traffic_of(dom)

    details = {"per_gemm_us": {g.name: round(per[g.name] * 1e6, 2) for g in gemms},
               "roofline_per_gemm": {g.name: dict(roofline_of(g, per[g.name]), traffic=traffic_of(g)) for g in gemms}}
    if not args.no_details:
        extra = []
        for name, m, k, n, grp in [("ffn_up_t338_gK", 338, 1024, 4096, 1024), ("ffn_up_t338_g128", 338, 1024, 4096, 128),
                                   ("ffn_up_m8192_gK", 8192, 1024, 4096, 1024),
                                   ("ffn_up_m8192_g128", 8192, 1024, 4096, 128),
                                   ("ffn_down_m8192_gK", 8192, 4096, 1024, 4096),
                                   ("ffn_down_m8192_g128", 8192, 4096, 1024, 128)]:
            extra.append(Gemm(vx, synth, dev, name, m, k, n, 0, 0.0, grp, 0, 1))
        # the single-GEMM workload's literal output: int32 accumulators plus fp32 dequant (one group, Store)
        for name, m in [("int32_out_t338_gK", 338), ("int32_out_m8192_gK", 8192)]:
            extra.append(Gemm(vx, synth, dev, name, m, 1024, 4096, 0, 0.0, 1024, 0, 1, int32_out=True))
        pe = time_launches(torch, extra, 10)
        for g in extra:
            s = pe[g.name]
            details[g.name] = {"us": round(s * 1e6, 2), "tops": round(g.ops / s / 1e12, 1),
                               "pct_int8_peak": round(100 * g.ops / s / 1e12 / PEAK_INT8_TOPS, 1),
                               "hbm_gbs": round(g.bytes / s / 1e9, 0)}
            if g.gs is not None:
                details[g.name]["output"] = "int32 [1][M][N] + fp32 [M][N]"
        del extra
    cpu = None if args.no_cpu else cpu_baseline(gemms)
    details["host_cpu"] = cpu_info()
    if not args.no_cpu and not args.no_details:
        details["cpu_vnni_single_core"] = cpu_single_core(synth, "vnni")
        details["cpu_avx2_single_core"] = cpu_single_core(synth, "avx2")
    if not args.no_encoder:
        enc, eparams, esp = encoder_setup(synth)
        details["encoder"] = encoder_rtfx(torch, synth, enc, dev)
        enc.free()
        if not args.no_details:
            details["clip_batch_24_layers"] = clip_batch_tops(torch, vx, synth, dev, eparams)
            details["clip_batch_24_layers_g128"] = clip_batch_tops(torch, vx, synth, dev, eparams, group=128)
            details["attention_core"] = attention_us(torch, dev)
            gv = [Gemv(vx, synth, dev, out) for out in (8198, 2560)]
            tg = time_launches(torch, gv, 50)
            details["gemv_single_token"] = {g.name: {"us": round(tg[g.name] * 1e6, 2),
                                                    "gb_per_s": round(g.bytes / tg[g.name] / 1e9, 0)} for g in gv}
            del gv
        if not args.no_cpu:
            ce = cpu_encoder_rtfx(eparams, esp, synth)
            details["encoder_cpu"] = ce
            for k, v in ce["by_workload"].items():
                if k in details["encoder"]:
                    details["encoder"][k]["x_vs_cpu"] = round(details["encoder"][k]["rtfx"] / v["rtfx"], 1)

    line = {
        "metric": "ternary x int8 GEMM TOPS (one FastConformer layer's linear set at T=338)",
        "value": round(value, 2), "unit": "TOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(gpu_s / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "layer_linear_set_t338", "T": T, "d_model": 1024, "ffn": 4096, "group": "K",
                   "gemms": [f"{n}:{m}x{k}x{nn}" for n, m, k, nn, _, _ in layer_shapes(T)],
                   "pct_int8_peak": round(100 * value / PEAK_INT8_TOPS, 2), "wall_s": round(wall, 3)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "details": details,
    }
    if "encoder" in details:
        line["config"]["encoder_rtfx_t338"] = details["encoder"]["t338_27s"]["rtfx"]
        if "encoder_cpu" in details and "t338_27s" in details["encoder_cpu"]["by_workload"]:
            line["config"]["encoder_cpu_rtfx_t338"] = details["encoder_cpu"]["by_workload"]["t338_27s"]["rtfx"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
