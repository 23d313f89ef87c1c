#!/usr/bin/env python
"""Decode-time state path of the hybrid Gated-DeltaNet / attention Qwen3.6-27B engine on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--workload all|step|gdn-layer|attn-layer|
                     verify-step|prefill|conv-prefill|mlp-layer]
                    [--profile-family gdn|gdn1|attn|attn1|verify|conv|copy|prefill|mlp]

Default (``--workload all``): one JSON line whose top level is the headline workload — the batch-8 decode
step at 4096 positions per user: 48 Gated-DeltaNet layers (conv1d update + L2-norm + gated delta rule on
fp32 [8, 48, 128, 128] states, in place) and 16 attention layers (append of one token's K/V into block-64
pages + paged GQA decode, 24 q heads / 4 KV heads x 256, over a shared 2048-page pool through per-user
random block tables), replayed as one HIP graph that also advances every user's position — and whose
``configs`` key holds the other workloads, each with its own roofline and CPU baseline:
  gdn-layer     one GDN layer, batch 1 (96 layers' distinct buffers rotate, 627 MB per loop)
  attn-layer    one attention layer at 32768 positions, batch 1 (4 layers' distinct pools rotate)
  verify-step   MTP verify at batch 1, 8192 positions, 4 tokens, 64 layers + acceptance by slot
  prefill       chunked gated delta rule over 8192 tokens + the paged K/V fill (two prompts rotate)
  conv-prefill  the prompt conv with its carry over 8192 tokens (the prefill -> decode handoff)
  mlp-layer     the MLP half of one layer at one row, weights streamed as MXFP4 (gate | up) and MXINT8 (down)
Inputs are seeded synthetic tensors resident in HBM before the timed region.

Timing: K timed replays (``--steps``) bracketed by synchronisation, each replay between its own pair of HIP
events on the replay stream (the length rewind that keeps the context fixed runs between replays, outside
the events); ``ms_per_step`` is their mean. A second pass of max(K, 200) replays gives the median, p10 and
p90. SCLK, MCLK and power are sampled during it. value = algorithmic bytes / ms_per_step (GB/s).
roofline = the dominant kernel's per-launch algorithmic bytes / its average launch time (HIP events around
back-to-back launches on the stream they run on). cpu_baseline = the CPU oracle on a bounded sample of the
same workload on the host's cores (and on one thread), median of >= 5 runs after one warm-up.

``--profile-family`` launches one kernel family back to back (for rocprofv3 counter runs) and exits.
"""
import argparse
import ctypes
import glob
import json
import os
import statistics
import sys
import threading
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "tt-qwen-resident_amd"))

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
METRIC = "decode-step state-path µs and achieved HBM GB/s (% of peak) at batch 1/8"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


# ------------------------------------------------------------------------------------------------ telemetry


class Telemetry:
    """Samples the GPU's current SCLK / MCLK (pp_dpm_sclk / pp_dpm_mclk, the starred level) and power
    (hwmon power1_average or power1_input) from sysfs every 20 ms while active."""

    def __init__(self):
        self.card = None
        for c in sorted(glob.glob("/sys/class/drm/card*/device")):
            if os.path.exists(os.path.join(c, "pp_dpm_sclk")):
                self.card = c
                break
        self.samples = []
        self._stop = threading.Event()
        self._t = None

    @staticmethod
    def _dpm(path):
        try:
            with open(path) as f:
                for line in f:
                    if "*" in line:
                        return float(line.split(":")[1].strip().rstrip("*").strip().lower().replace("mhz", ""))
        except (OSError, ValueError, IndexError):
            return None
        return None

    def _power(self):
        for name in ("power1_average", "power1_input"):
            for p in glob.glob(os.path.join(self.card, "hwmon", "hwmon*", name)):
                try:
                    with open(p) as f:
                        return float(f.read()) / 1e6
                except (OSError, ValueError):
                    pass
        return None

    def sample(self):
        if self.card is None:
            return
        self.samples.append((self._dpm(os.path.join(self.card, "pp_dpm_sclk")),
                             self._dpm(os.path.join(self.card, "pp_dpm_mclk")), self._power()))  # fmt: skip

    def __enter__(self):
        self.samples = []
        self._stop.clear()

        def run():
            while not self._stop.is_set():
                self.sample()
                time.sleep(0.02)

        self._t = threading.Thread(target=run, daemon=True)
        self._t.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._t.join()

    def summary(self):
        if self.card is None:
            return dict(available=False)

        def stats(i):
            v = [s[i] for s in self.samples if s[i] is not None]
            return dict(mean=round(statistics.mean(v), 1), max=round(max(v), 1)) if v else None

        return dict(samples=len(self.samples), sclk_mhz=stats(0), mclk_mhz=stats(1), power_w=stats(2))


# ------------------------------------------------------------------------------------------------ timing


def capture(torch, fn):
    """fn recorded into a HIP graph on a side stream (run once eagerly first, so every buffer exists)."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    return g


def capture_calls(torch, make_calls):
    """C-ABI launches (pre-built argument tuples) recorded into a HIP graph on a side stream: make_calls(stream)
    returns the (entry, args) list; the launches run once eagerly first."""
    from qwen36_state._lib import lib

    L = lib()
    s = torch.cuda.Stream()
    fns = [(getattr(L, name), args) for name, args in make_calls(ctypes.c_void_p(s.cuda_stream))]
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f, a in fns:
            assert f(*a) == 0, L.qs_last_error()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for f, a in fns:
            f(*a)
    torch.cuda.synchronize()
    return g


def replay_times(torch, replay, n, between=None):
    """Per-replay times (ms): each replay between its own pair of HIP events on the current stream (the
    stream the graphs launch on); ``between`` (untimed) runs after each replay's end event. Synchronised on
    both sides."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in evs:
        e0.record()
        replay()
        e1.record()
        if between is not None:
            between()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return [e0.elapsed_time(e1) for e0, e1 in evs], wall


SETTLE_MS = 150.0  # untimed replays before a per-workload line's timed replays (its first replays run slower)


def timed(torch, args, replay, between=None, tel=None, settle_ms=0.0):
    """W untimed replays (then more, untimed, until settle_ms of wall time have passed: the per-workload lines
    settle the clocks this way, the headline step keeps exactly W), K timed replays (the contract's step count)
    and a statistics pass of max(K, 200) replays with telemetry. Returns (ms mean over K, stats dict)."""
    for _ in range(args.warmup):
        replay()
        if between is not None:
            between()
    if settle_ms > 0:
        torch.cuda.synchronize()
        t_end = time.perf_counter() + settle_ms / 1e3
        while time.perf_counter() < t_end:
            for _ in range(8):
                replay()
                if between is not None:
                    between()
            torch.cuda.synchronize()
    ts, wall = replay_times(torch, replay, args.steps, between)
    n = max(args.steps, 200)
    if tel is not None:
        with tel:
            st, _ = replay_times(torch, replay, n, between)
    else:
        st, _ = replay_times(torch, replay, n, between)
    q = statistics.quantiles(st, n=10)
    stats = dict(replays=n, median_ms=round(statistics.median(st), 5), p10_ms=round(q[0], 5),
                 p90_ms=round(q[-1], 5), timed_wall_s=round(wall, 4))  # fmt: skip
    return statistics.mean(ts), stats


def kernel_time(torch, make_calls, reps):
    """Average ms of one launch: reps x len(calls) back-to-back C-ABI launches (pre-built argument tuples)
    captured into a HIP graph on a side stream, replayed once untimed and once between HIP events on that
    stream, so no host work sits between the launches. make_calls(stream) returns the (entry, args) list."""
    from qwen36_state._lib import lib

    L = lib()
    s = torch.cuda.Stream()
    fns = [(getattr(L, name), args) for name, args in make_calls(ctypes.c_void_p(s.cuda_stream))]
    with torch.cuda.stream(s):
        for f, a in fns:
            assert f(*a) == 0, L.qs_last_error()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(reps):
            for f, a in fns:
                f(*a)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        e0.record(s)
        g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * len(fns))


def gdn_call(d, B, ws, stream, out, z=None, norm_w=None):
    """The fused GDN decode (z, norm_w: with the gated RMSNorm epilogue) as a (name, args) C-ABI call."""
    from qwen36_state.ops import CONV_K, DK, DV, NK, NV

    return "qs_gdn_decode_fused", (
        _p(d["x"]), _p(d["conv_state"]), _p(d["taps"]), _p(d["g"]), _p(d["beta"]), _p(d["state"]), _p(out),
        ctypes.c_void_p(0), _p(z), NV * DV, _p(norm_w), _p(ws), ctypes.c_void_p(0), B, NK, NV, DK, DV, CONV_K,
        ctypes.c_float(DK**-0.5), ctypes.c_float(1e-6),
        stream,
    )  # fmt: skip


def gdn_epilogue_times(torch, layers, B, ws, reps):
    """The GDN mixer's gated RMSNorm epilogue (model.py:274-275) two ways, per layer (ms): fused into the decode
    launch (z, norm_w given) and as the unfused pair (the decode launch, then qs_gdn_gated_norm on its bf16 o).
    Seeded z rows [B, NV DV] and norm_w [DV] per layer; the layers' states advance while timing (their values
    do not change the work)."""
    from qwen36_state.ops import DV, EPS, NV

    gen = torch.Generator(device="cuda:0").manual_seed(5)
    zs = [torch.randn(B, NV * DV, generator=gen, device="cuda:0").bfloat16() for _ in layers]
    nw = 1 + 0.1 * torch.randn(DV, generator=gen, device="cuda:0")
    outs = [torch.empty(B, NV, DV, dtype=torch.bfloat16, device="cuda:0") for _ in layers]
    fused = kernel_time(torch, lambda st: [gdn_call(d, B, ws, st, o, z, nw) for d, o, z in zip(layers, outs, zs)],
                        reps)  # fmt: skip

    def pair(st):
        calls = []
        for d, o, z in zip(layers, outs, zs):
            calls.append(gdn_call(d, B, ws, st, o))
            calls.append(("qs_gdn_gated_norm", (_p(o), _p(z), _p(nw), _p(o), B * NV, DV, ctypes.c_float(EPS), st)))
        return calls

    return fused, 2 * kernel_time(torch, pair, reps)


def attn_call(d, table, lens, B, T, pps, ws, stream, out):
    from qwen36_state.ops import HD, NKV, NQ

    return "qs_paged_gqa_decode", (
        _p(d["q"]), _p(d["k_new"]), _p(d["v_new"]), _p(d["k_cache"]), _p(d["v_cache"]), _p(table), _p(lens),
        _p(out), _p(ws), B, T, NQ, NKV, HD, 64, table.shape[1], d["k_cache"].shape[0], pps,
        ctypes.c_float(d["scale"]), ctypes.c_void_p(0), stream,
    )  # fmt: skip


def roofline(name, nbytes, ms, traffic_key=None, flops=None):
    """The roofline object of one kernel family; ``traffic`` is the measured HBM bytes per launch of
    profiles/pmc_traffic.json under ``traffic_key`` (default: the family's name; ``False``: none measured at
    this shape, reported as null)."""
    achieved = nbytes / (ms * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(REPO, "profiles", "pmc_traffic.json")
    if traffic_key is not False and os.path.exists(tf):
        with open(tf) as f:
            traffic = json.load(f).get(traffic_key or name, {}).get("hbm_bytes_per_launch")
    out = dict(kernel=name, bound="hbm", achieved=round(achieved, 1), peak=PEAK_HBM_GBS, unit="GB/s",
               frac=round(achieved / PEAK_HBM_GBS, 4), traffic=traffic, bytes_per_launch=nbytes,
               us_per_launch=round(ms * 1e3, 2))  # fmt: skip
    if flops is not None:
        out["mfma"] = dict(tflops=round(flops / (ms * 1e-3) / 1e12, 1), peak=PEAK_BF16_TFLOPS,
                           frac=round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4))  # fmt: skip
    return out


def entry(workload, nbytes, ms, stats, dom, extra=None):
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = dict(value=round(gbs, 1), unit="GB/s", us_per_step=round(ms * 1e3, 2), frac_of_peak=round(gbs / PEAK_HBM_GBS, 4),
               median_us=round(stats["median_ms"] * 1e3, 2), p10_us=round(stats["p10_ms"] * 1e3, 2),
               p90_us=round(stats["p90_ms"] * 1e3, 2), replays=stats["replays"], workload=workload,
               bytes_per_step=nbytes, roofline=dom)  # fmt: skip
    if extra:
        out.update(extra)
    return out


# ------------------------------------------------------------------------------------------------ CPU baseline


def cpu_threads():
    try:
        share = len(os.sched_getaffinity(0))
    except AttributeError:
        share = os.cpu_count() or 1
    return max(1, min(share, 16))


def cpu_time(torch, fn, reps=5):
    """Median seconds of fn over reps runs after one warm-up, on the host's cores and on one thread."""
    out = {}
    for threads in (cpu_threads(), 1):
        torch.set_num_threads(threads)
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        out[threads] = statistics.median(ts)
    torch.set_num_threads(cpu_threads())
    return out


def cpu_entry(torch, nbytes, t, unit_note, reps=5):
    """cpu_baseline dict from {threads: seconds per unit of work} scaled to the workload's bytes."""
    n = cpu_threads()
    return dict(value=round(nbytes / t[n] / 1e9, 3), unit="GB/s", cores=n, kind="port",
                os_cpu_count=os.cpu_count(), torch_threads=n, one_thread_value=round(nbytes / t[1] / 1e9, 3),
                ms=round(t[n] * 1e3, 2), one_thread_ms=round(t[1] * 1e3, 2), sample=unit_note + f" (median of {reps} "
                "after a warm-up)")  # fmt: skip


def _oracle():
    sys.path.insert(0, REPO)
    from oracle import state_path as O

    return O


def cpu_step(torch, step):
    """2 GDN + 1 attention layers of the batch-8 step at the real shapes, scaled to 48 + 16 layers."""
    O = _oracle()
    from qwen36_state.ops import DK, DV, NK, NV

    gl, al = step.gdn_layers(), step.attn_layers()
    gdn = [{k: v.cpu() for k, v in step.layer[l].items() if torch.is_tensor(v)} for l in gl[:2]]
    a = {k: v.cpu() for k, v in step.layer[al[0]].items() if torch.is_tensor(v)}
    table, lens = step.block_table.cpu(), step.lens.cpu() + 1
    scale = step.layer[al[0]]["scale"]

    def run():
        for d in gdn:
            O.gdn_decode(d["x"].float(), d["conv_state"].float(), d["taps"].float(), d["g"], d["beta"], d["state"],
                         NK, NV, DK, DV)  # fmt: skip
        O.paged_append(a["k_cache"], a["v_cache"], a["k_new"], a["v_new"], table, lens - 1)
        O.gqa_decode(a["q"], a["k_cache"], a["v_cache"], table, lens, scale)

    t = cpu_time(torch, run)
    # per step: 24 x (2 GDN layers) + 16 x (1 attention layer), the GDN / attention split measured separately
    t_g = cpu_time(torch, lambda: [O.gdn_decode(d["x"].float(), d["conv_state"].float(), d["taps"].float(), d["g"],
                                                d["beta"], d["state"], NK, NV, DK, DV) for d in gdn])  # fmt: skip
    scaled = {n: len(gl) / 2 * t_g[n] + len(al) * (t[n] - t_g[n]) for n in t}
    return cpu_entry(torch, step.bytes_per_step(), scaled,
                     f"2 GDN + 1 attention layers of the batch-{step.B} step at {step.ctx} positions, scaled to "
                     f"{len(gl)} + {len(al)} layers")  # fmt: skip


# ------------------------------------------------------------------------------------------------ workloads


def bench_step(args, torch, tel, batch=None, pps=None):
    from qwen36_state.decode import StatePathStep, layer_bytes

    batch = args.batch if batch is None else batch
    pps = args.pps if pps is None else pps
    log(f"building the {args.layers}-layer step: batch {batch}, {args.ctx} positions")
    step = StatePathStep.synthetic(batch, args.ctx, args.layers, device="cuda:0", pages_per_split=pps)
    gl, al = step.gdn_layers(), step.attn_layers()
    step.step()
    step.rewind()
    g = step.capture()
    ms, stats = timed(torch, args, g.replay, between=step.rewind, tel=tel)
    nbytes = step.bytes_per_step()
    log(f"step: {ms * 1e3:.1f} µs mean, {stats['median_ms'] * 1e3:.1f} µs median, {nbytes / ms / 1e6:.0f} GB/s")
    lens1 = step.lens + 1  # the lengths the step's attention layers see
    t_gdn = kernel_time(torch, lambda st: [gdn_call(step.layer[l], step.B, step.gdn_ws, st, step.layer[l]["o"])
                                           for l in gl], args.kernel_reps)  # fmt: skip
    t_att = kernel_time(torch, lambda st: [attn_call(step.layer[l], step.block_table, lens1, step.B, 1, step.pps,
                                                     step.attn_ws, st, step.layer[l]["o"]) for l in al],
                        args.kernel_reps)  # fmt: skip
    b_gdn, b_att = layer_bytes(batch, args.ctx), layer_bytes(batch, args.ctx, attn=True)
    kern = {"gdn_decode_fused": (t_gdn, b_gdn, len(gl)), "paged_gqa_decode": (t_att, b_att, len(al))}
    for k, (t, b, n) in kern.items():
        log(f"{k}: {t * 1e3:.2f} µs per launch, {b / t / 1e6:.0f} GB/s, {n} launches per step")
    dom = max(kern, key=lambda k: kern[k][0] * kern[k][2])
    t_fused, t_pair = gdn_epilogue_times(torch, [step.layer[l] for l in gl], step.B, step.gdn_ws, args.kernel_reps)
    log(f"GDN with the gated RMSNorm epilogue: fused {t_fused * 1e3:.2f} µs, unfused pair {t_pair * 1e3:.2f} µs")
    work = (f"decode-step state path: {len(gl)} GDN + {len(al)} paged-attention layers, batch {batch}, "
            f"{args.ctx} positions per user, block 64, HIP-graph replay with the position advance")  # fmt: skip
    # the PMC traffic entries were measured at these shapes (the GDN's bytes do not depend on the context)
    tkey = {("gdn_decode_fused", 8): "gdn_decode_fused", ("gdn_decode_fused", 1): "gdn_decode_fused_b1"}.get((dom, batch))
    if dom == "paged_gqa_decode" and (batch, args.ctx, pps) == (8, 4096, 8):
        tkey = "paged_gqa_decode"
    out = entry(work, nbytes, ms, stats, roofline(dom, kern[dom][1], kern[dom][0], tkey or False),
                dict(kernels={k: dict(us_per_launch=round(t * 1e3, 2), bytes_per_launch=b, gbs=round(b / t / 1e6, 1),
                                      launches_per_step=n) for k, (t, b, n) in kern.items()}))  # fmt: skip
    out.update(batch=batch, context=args.ctx, layers=args.layers, pages_per_split=pps)
    out["gdn_epilogue"] = dict(fused_us_per_layer=round(t_fused * 1e3, 2), unfused_pair_us_per_layer=round(t_pair * 1e3, 2),
                               note="GDN decode with the gated RMSNorm epilogue (not part of the state-path step): in "
                                    "the same launch vs a second launch")  # fmt: skip
    if not args.no_cpu:
        log("timing the CPU oracle on a sample of the step")
        out["cpu_baseline"] = cpu_step(torch, step)
    del step, g
    torch.cuda.empty_cache()
    return out


def bench_gdn_layer(args, torch, tel):
    """One GDN layer at batch 1; the graph walks 96 layers' distinct buffers (627 MB, more than twice the
    256 MB Infinity Cache) twice, so every launch reads its state from HBM; per launch = replay / 192."""
    from qwen36_state import ops, workloads as W
    from qwen36_state.decode import layer_bytes

    layers = [W.gdn_layer(1, "cuda:0", seed=i) for i in range(96)]
    outs = [torch.empty(1, 48, 128, dtype=torch.bfloat16, device="cuda:0") for _ in layers]
    ws = torch.zeros(ops.lib().qs_gdn_workspace_bytes(1, 16), dtype=torch.uint8, device="cuda:0")

    R = 2  # passes over the 96 layers per replay, so the graph's start-up is spread over 192 launches

    def fn():
        for _ in range(R):
            for d, o in zip(layers, outs):
                ops.gdn_decode_fused(d["x"], d["conv_state"], d["taps"], d["g"], d["beta"], d["state"], out=o, ws=ws)

    g = capture(torch, fn)
    msr, stats = timed(torch, args, g.replay, tel=tel, settle_ms=SETTLE_MS)
    ms = msr / (len(layers) * R)
    stats = {k: (v / (len(layers) * R) if k.endswith("_ms") else v) for k, v in stats.items()}
    nbytes = layer_bytes(1, 0)
    out = entry("one GDN layer decode, batch 1: conv1d update (10240 channels) + L2-norm + gated delta rule on fp32 "
                "[1, 48, 128, 128] (48 layers' buffers rotate)", nbytes, ms, stats,
                roofline("gdn_decode_fused", nbytes, ms, "gdn_decode_fused_b1"))  # fmt: skip
    t_fused, t_pair = gdn_epilogue_times(torch, layers, 1, ws, 2)
    out["gdn_epilogue"] = dict(fused_us_per_layer=round(t_fused * 1e3, 2), unfused_pair_us_per_layer=round(t_pair * 1e3, 2),
                               note="with the gated RMSNorm epilogue: in the same launch vs a second launch")  # fmt: skip
    if not args.no_cpu:
        O = _oracle()
        c = {k: v.cpu() for k, v in layers[0].items()}
        t = cpu_time(torch, lambda: O.gdn_decode(c["x"].float(), c["conv_state"].float(), c["taps"].float(), c["g"],
                                                 c["beta"], c["state"], 16, 48, 128, 128))  # fmt: skip
        out["cpu_baseline"] = cpu_entry(torch, nbytes, t, "one GDN layer at batch 1")
    return out


def bench_attn_layer(args, torch, tel):
    """One attention layer at 32768 positions, batch 1; 4 layers with their own pools rotate (each launch
    reads 134 MB of pages that no other launch in the loop touches), 10 times per replay; per launch =
    replay / 40."""
    from qwen36_state import ops, workloads as W
    from qwen36_state.decode import layer_bytes

    pps = args.pps_attn1
    layers = [W.attn_layer(1, 32768, "cuda:0", seed=i) for i in range(4)]
    outs = [torch.empty(1, 1, 24, 256, dtype=torch.bfloat16, device="cuda:0") for _ in layers]
    ws = ops.attention_workspace(1, 1, 24, 4, 512, pps, "cuda:0")

    R = 10  # passes over the 4 layers per replay, so the graph's start-up is spread over 40 launches

    def fn():
        for _ in range(R):
            for d, o in zip(layers, outs):
                ops.paged_gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"], d["scale"],
                                     k_new=d["k_new"], v_new=d["v_new"], pages_per_split=pps, out=o, ws=ws)  # fmt: skip

    g = capture(torch, fn)
    msr, stats = timed(torch, args, g.replay, tel=tel, settle_ms=SETTLE_MS)
    ms = msr / (4 * R)
    stats = {k: (v / (4 * R) if k.endswith("_ms") else v) for k, v in stats.items()}
    nbytes = layer_bytes(1, 32768, attn=True)
    out = entry(f"one attention layer decode, batch 1, 32768 positions: append + paged GQA (24/4 heads x 256, block "
                f"64, 512 random pages of 2048), {pps} pages per split", nbytes, ms, stats,
                roofline("paged_gqa_decode", nbytes, ms, "paged_gqa_decode_b1_32k"), dict(pages_per_split=pps))  # fmt: skip
    if not args.no_cpu:
        O = _oracle()
        c = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in layers[0].items()}

        def run():
            O.paged_append(c["k_cache"], c["v_cache"], c["k_new"], c["v_new"], c["block_table"], c["seq_lens"] - 1)
            O.gqa_decode(c["q"], c["k_cache"], c["v_cache"], c["block_table"], c["seq_lens"], c["scale"])

        out["cpu_baseline"] = cpu_entry(torch, nbytes, cpu_time(torch, run), "one attention layer at 32768 positions")
    return out


def bench_verify(args, torch, tel):
    """The MTP verify step with acceptance by slot selection; the lengths are set back to the rows cached
    before the step between replays (outside the timed events), so every replay verifies at 8192."""
    from qwen36_state.decode import VerifyStep

    vs = VerifyStep.synthetic(1, 8192, T=4, device="cuda:0", pages_per_split=args.pps_verify)
    vs.step()
    vs.rewind()
    vs.capture()
    ms, stats = timed(torch, args, vs.replay, between=vs.rewind, tel=tel, settle_ms=SETTLE_MS)
    nbytes = vs.bytes_per_step(8192)
    out = entry("MTP verify step, batch 1, 8192 positions, 1 + 3 draft tokens through 48 GDN + 16 attention layers, "
                "then acceptance of a seeded length by snapshot-slot selection", nbytes, ms, stats,
                roofline("verify_step", nbytes, ms),
                dict(rollback_copy_bytes=vs.rollback_bytes(), accept=vs.accept.tolist(), pages_per_split=vs.pps))  # fmt: skip
    if not args.no_cpu:
        O = _oracle()
        gl = next(d for d in vs.layer if not d["attn"])
        al = next(d for d in vs.layer if d["attn"])
        c = {k: v.cpu() for k, v in gl.items() if torch.is_tensor(v)}
        S0, cs0 = (t.cpu() for t in vs.state_of(gl["gi"], 0))
        a = {k: v.cpu() for k, v in al.items() if torch.is_tensor(v)}
        table, lens = vs.block_table.cpu(), vs.base.cpu() + 4

        def run_g():
            O.gdn_verify(c["x"].float(), cs0[None].float(), c["taps"].float(), c["g"], c["beta"], S0[None], 16, 48,
                         128, 128)  # fmt: skip

        def run_a():
            O.paged_append(a["k_cache"], a["v_cache"], a["k_new"], a["v_new"], table, lens - 4)
            O.gqa_decode(a["q"], a["k_cache"], a["v_cache"], table, lens, al["scale"])

        tg, ta = cpu_time(torch, run_g), cpu_time(torch, run_a)
        out["cpu_baseline"] = cpu_entry(torch, nbytes, {n: 48 * tg[n] + 16 * ta[n] for n in tg},
                                        "1 GDN verify layer + 1 attention layer (T 4, 8192 positions), scaled to "
                                        "48 + 16 layers")  # fmt: skip
    del vs
    torch.cuda.empty_cache()
    return out


PREFILL_BYTES = 344982016
PREFILL_FLOPS = 71.94e9


def bench_prefill(args, torch, tel):
    """The chunked rule over one 8192-token prompt plus its paged K/V fill; two prompts rotate (each ~300 MB
    of inputs, outputs and pages besides the workspace), so each call reads them from HBM; per call =
    replay / 2."""
    from qwen36_state import ops, workloads as W

    prompts = [W.prefill(8192, "cuda:0", seed=i) for i in range(2)]
    kc = torch.zeros(2048, 4, 64, 256, dtype=torch.bfloat16, device="cuda:0")
    vc = torch.zeros_like(kc)
    nbytes_ws = ops.lib().qs_gdn_chunk_prefill_workspace_bytes(8192, 16, 48, 128, 128, 64)
    ws = torch.zeros(nbytes_ws, dtype=torch.uint8, device="cuda:0")
    finals = [torch.empty_like(d["S0"]) for d in prompts]

    def fn():
        for d, S in zip(prompts, finals):
            ops.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["S0"], ws=ws,
                                       final_state=S)  # fmt: skip
            ops.paged_kv_fill(d["kv_k"], d["kv_v"], kc, vc, d["page_table"])

    g = capture(torch, fn)
    a2 = argparse.Namespace(**{**vars(args), "steps": max(10, args.steps // 5)})
    msr, stats = timed(torch, a2, g.replay, tel=tel, settle_ms=SETTLE_MS)
    n = len(prompts)
    ms = msr / n
    stats = {k: (v / n if k.endswith("_ms") else v) for k, v in stats.items()}
    d = prompts[0]
    out = entry("chunked-prefill gated delta rule, 8192 tokens, chunk 64, 16/48 heads x 128 (WY form, bf16 MFMA, fp32 "
                "state) + paged fill of 8192 tokens of K/V (4 x 256) into 128 random pages", PREFILL_BYTES, ms, stats,
                roofline("gdn_chunk_prefill", PREFILL_BYTES, ms, flops=PREFILL_FLOPS),
                dict(flops=PREFILL_FLOPS, tflops=round(PREFILL_FLOPS / ms / 1e9, 1)))  # fmt: skip
    if not args.no_cpu:
        O = _oracle()
        n = 1024
        c = {k: v[:n].cpu() for k, v in d.items() if k in ("q", "k", "v", "g", "beta")}
        S0 = d["S0"].cpu()
        t = cpu_time(torch, lambda: O.gdn_chunk_prefill_wy(c["q"], c["k"], c["v"], c["g"], c["beta"], S0, 64))
        out["cpu_baseline"] = cpu_entry(torch, PREFILL_BYTES, {k: v * 8192 / n for k, v in t.items()},
                                        f"the chunked form on the first {n} of 8192 tokens, scaled by 8 (K/V fill not "
                                        "timed)")  # fmt: skip
    return out


def bench_conv_prefill(args, torch, tel):
    """The prompt conv with its carry over 8192 tokens of the 10240 q | k | v channels, read from a
    projection output with 128 further columns; two prompts rotate (1.3 GB per loop) so each launch reads
    and writes HBM rather than the Infinity Cache, 5 times per replay; per launch = replay / 10."""
    from qwen36_state import ops, workloads as W

    T, C, ldx = 8192, W.C_QKV, W.C_QKV + 128
    CQ, CV = ops.NK * ops.DK, ops.NV * ops.DV
    bufs = []
    for i in range(2):
        gen = W._gen("cuda:0", i)
        bufs.append(dict(x=W._randn((T, ldx), gen, "cuda:0", torch.bfloat16),
                         taps=W._randn((C, 4), gen, "cuda:0", torch.bfloat16, std=0.5),
                         cs=W._randn((C, 3), gen, "cuda:0", torch.bfloat16),
                         q=torch.empty(T, CQ, dtype=torch.bfloat16, device="cuda:0"),
                         k=torch.empty(T, CQ, dtype=torch.bfloat16, device="cuda:0"),
                         v=torch.empty(T, CV, dtype=torch.bfloat16, device="cuda:0"),
                         out=torch.empty(C, 3, dtype=torch.bfloat16, device="cuda:0")))  # fmt: skip
    R = 5  # passes over the two prompts per replay

    def calls(st):
        return [("qs_conv1d_prefill", (_p(b["x"]), ldx, _p(b["cs"]), _p(b["taps"]), _p(b["q"]), _p(b["k"]),
                                       _p(b["v"]), _p(b["out"]), T, CQ, CV, 4, st)) for b in bufs] * R  # fmt: skip

    g = capture_calls(torch, calls)
    msr, stats = timed(torch, args, g.replay, tel=tel, settle_ms=SETTLE_MS)
    ms = msr / (2 * R)
    stats = {k: (v / (2 * R) if k.endswith("_ms") else v) for k, v in stats.items()}
    nbytes = 2 * T * C * 2 + C * 4 * 2 + 2 * C * 3 * 2  # x in, q | k | v out, taps, carry in and out
    out = entry("prompt conv1d + SiLU with carry, 8192 tokens x 10240 channels (q | k | v of a 10368-column "
                "projection), conv state handed to the decode", nbytes, ms, stats,
                roofline("conv1d_prefill", nbytes, ms))  # fmt: skip
    if not args.no_cpu:
        O = _oracle()
        x = bufs[0]["x"][:1024, :C].cpu()
        taps, cs = bufs[0]["taps"].cpu(), bufs[0]["cs"].cpu()
        t = cpu_time(torch, lambda: O.conv1d_prefill(x.float(), cs.float(), taps.float()))
        out["cpu_baseline"] = cpu_entry(torch, nbytes, {k: v * 8 for k, v in t.items()},
                                        "the first 1024 of 8192 tokens, scaled by 8")  # fmt: skip
    return out


def mlp_bytes(B, H, I):
    """Algorithmic HBM bytes of one MLP half: the packed gate | up (MXFP4) and down (MXINT8: the same bytes as
    MXFP8) weights, x in, x_out (the norm weight is folded into gate | up, as the reference loads them)."""
    from qwen36_state._lib import lib

    L = lib()
    return 2 * L.qs_mx_packed_bytes(H, I, 4) + L.qs_mx_packed_bytes(I, H, 9) + 2 * B * H * 4


def bench_mlp_layer(args, torch, tel):
    """The MLP half of one decoder layer at one row (the reference's 1-chip MLP bench: x [1, 5120], gate | up
    [5120, 17408] 4-bit, down [17408, 5120] 8-bit, us per layer and weight GB/s): three layers' weights
    (560 MB, beyond the 256 MB Infinity Cache) rotate, twice per replay; per layer = replay / 6. The rmsnorm
    weight is folded into the rows of gate | up, as the reference's loader does (weights.py:107-112), so the
    call passes no gamma (the synthetic weights stand for folded ones)."""
    from qwen36_state import ops, workloads as W

    B, H, I = 1, ops.HIDDEN, ops.INTER
    layers = [W.mlp_layer(B, "cuda:0", seed=i, keep_fp32=(i == 0 and not args.no_cpu)) for i in range(3)]
    for d in layers:
        d["out"] = torch.empty_like(d["x"])
    ws = torch.empty(ops.lib().qs_mlp_decode_workspace_bytes(B, H, I), dtype=torch.uint8, device="cuda:0")
    R = 2

    def calls(st):
        return [("qs_mlp_decode", (_p(d["x"]), None, _p(d["gate"].packed), _p(d["up"].packed),
                                   _p(d["down"].packed), d["down"].fmt, _p(d["out"]), _p(ws), B, H, I,
                                   ctypes.c_float(ops.EPS), st)) for d in layers] * R  # fmt: skip

    g = capture_calls(torch, calls)
    msr, stats = timed(torch, args, g.replay, tel=tel, settle_ms=SETTLE_MS)
    n = len(layers) * R
    ms = msr / n
    stats = {k: (v / n if k.endswith("_ms") else v) for k, v in stats.items()}
    nbytes = mlp_bytes(B, H, I)
    out = entry("MLP half of one decoder layer, 1 row: rmsnorm (weight folded into gate | up) + gate | up 5120 x "
                "17408 MXFP4 with silu, down 17408 x 5120 MXINT8 in 4 K splits + residual (2 launches)", nbytes, ms,
                stats,
                roofline("mlp_decode", nbytes, ms))  # fmt: skip
    out["us_per_layer"] = out["us_per_step"]
    if not args.no_cpu:
        _oracle()
        from oracle import weight_stream as WS

        d = layers[0]
        x = d["x"].cpu()
        G, U, D = d["gate32"], d["up32"], d["down32"]
        t = cpu_time(torch, lambda: WS.mlp_half(x, None, G, U, D))
        out["cpu_baseline"] = cpu_entry(torch, nbytes, t, "the oracle's MLP half (fp32 weights, dequantization not "
                                        "timed) at the full shape, 1 row")  # fmt: skip
    return out


def ceilings(torch, reps=4):
    """The bare access patterns of the kernel families, timed like the kernels (back-to-back launches in a HIP
    graph, the buffers rotating over more than twice the 256 MB Infinity Cache), in GB/s of bytes moved:
    a nontemporal streaming read (134 MB per launch: the batch-8 attention working set; and 1 GiB), a 1:1
    nontemporal copy (25.2 MB -> 25.2 MB, in place like the GDN state's update and to a second buffer; and
    512 MB), and the paged attention's
    block-table gather of the batch-8, 4096-position working set with its load schedule and no compute."""
    from qwen36_state import workloads as W
    from qwen36_state._lib import lib

    L = lib()
    dev = "cuda:0"
    out = {}

    def run(name, nbytes, bufs, make):
        sink = torch.zeros(max(L.qs_probe_sink_words(nbytes), 4096), dtype=torch.int32, device=dev)
        ms = kernel_time(torch, lambda st: [make(b, sink, st) for b in bufs], reps)
        out[name] = dict(us=round(ms * 1e3, 2), gbs=round(nbytes / (ms * 1e-3) / 1e9, 1),
                         frac_of_peak=round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4))  # fmt: skip

    for nb, n in ((134217728, 4), (1 << 30, 1)):
        bufs = [torch.ones(nb // 4, dtype=torch.float32, device=dev) for _ in range(n)]
        run(f"read_{nb >> 20}MiB", nb, bufs, lambda b, sink, st: ("qs_probe_read", (_p(b), ctypes.c_size_t(b.numel() * 4),
                                                                                   _p(sink), st)))  # fmt: skip
        del bufs
    for nb, n, inplace in ((25165824, 24, True), (25165824, 24, False), (536870912, 1, False)):
        bufs = [(torch.ones(nb // 4, device=dev), None if inplace else torch.empty(nb // 4, device=dev)) for _ in range(n)]
        run(f"copy_{nb >> 20}MiB" + ("_in_place" if inplace else ""), 2 * nb, bufs,
            lambda b, sink, st: ("qs_probe_copy", (_p(b[0]), _p(b[0] if b[1] is None else b[1]), ctypes.c_size_t(nb),
                                                   st)))  # fmt: skip
        del bufs
    torch.cuda.empty_cache()
    B, ctx, pps = 8, 4096, 8
    d = W.attn_layer(B, ctx, dev, seed=3, num_blocks=2048)
    # four tables over disjoint quarters of the 2048-page pools, each a seeded permutation of its pages
    gen = torch.Generator().manual_seed(10)
    tabs = [(512 * i + torch.randperm(512, generator=gen)).to(torch.int32).reshape(B, ctx // 64).to(dev) for i in range(4)]
    gbytes = B * 4 * ctx * 256 * 2 * 2
    sink = torch.zeros(L.qs_probe_gather_sink_words(B, 4, ctx // 64, pps), dtype=torch.int32, device=dev)
    ms = kernel_time(torch, lambda st: [("qs_probe_gather", (_p(d["k_cache"]), _p(d["v_cache"]), _p(t), B, 4, ctx // 64,
                                                             ctx // 64, 2048, pps, _p(sink), st)) for t in tabs], reps)  # fmt: skip
    out["gather_attn_b8_4k"] = dict(us=round(ms * 1e3, 2), gbs=round(gbytes / (ms * 1e-3) / 1e9, 1),
                                    frac_of_peak=round(gbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4))  # fmt: skip
    del d, tabs
    torch.cuda.empty_cache()
    return out


def copy_ceiling(torch):
    """Device-to-device copy of 1 GiB (torch's copy kernel): GB/s counting the read and the write."""
    src = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    g = capture(torch, lambda: dst.copy_(src))
    ts, _ = replay_times(torch, g.replay, 20)
    ms = statistics.median(ts)
    del src, dst, g
    torch.cuda.empty_cache()
    return dict(kernel="torch copy_ of 1 GiB", gbs=round(2 * (1 << 30) / (ms * 1e-3) / 1e9, 1),
                frac_of_peak=round(2 * (1 << 30) / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4))  # fmt: skip


WORKLOADS = {
    "step": bench_step,
    "step-b1": lambda args, torch, tel: bench_step(args, torch, tel, batch=1, pps=args.pps_b1),
    "gdn-layer": bench_gdn_layer,
    "attn-layer": bench_attn_layer,
    "verify-step": bench_verify,
    "prefill": bench_prefill,
    "conv-prefill": bench_conv_prefill,
    "mlp-layer": bench_mlp_layer,
}
CONFIG_OF = {"gdn-layer": 0, "attn-layer": 1, "step": 2, "step-b1": "2 at batch 1", "verify-step": 3, "prefill": 4,
             "conv-prefill": "f2", "mlp-layer": "f4"}


# ------------------------------------------------------------------------------------------------ profiling


def profile_family(args, torch):
    """One kernel family back to back over distinct per-layer buffers (so the dispatches read HBM, not the
    Infinity Cache), for rocprofv3 counter runs; prints the algorithmic bytes of one dispatch."""
    from qwen36_state import ops, workloads as W
    from qwen36_state.decode import layer_bytes

    dev = "cuda:0"
    fam = args.profile_family
    if fam == "copy":
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.reps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy: {src.numel() * 4} bytes read and written per dispatch")
    elif fam == "conv":
        C = W.C_QKV
        bufs = [(W._randn((8192, C + 128), W._gen(dev, i), dev, torch.bfloat16),
                 W._randn((C, 4), W._gen(dev, 10 + i), dev, torch.bfloat16),
                 W._randn((C, 3), W._gen(dev, 20 + i), dev, torch.bfloat16)) for i in range(2)]  # fmt: skip
        for _ in range(args.reps):
            for x, taps, cs in bufs:
                ops.causal_conv1d_prefill(x[:, :C], taps, cs)
        torch.cuda.synchronize()
        print(f"conv1d_prefill: {2 * 8192 * C * 2 + C * 8 + C * 12} algorithmic bytes per dispatch")
    elif fam == "gdn":
        layers = [W.gdn_layer(8, dev, seed=i) for i in range(48)]
        for _ in range(args.reps):
            for d in layers:
                ops.gdn_decode_fused(d["x"], d["conv_state"], d["taps"], d["g"], d["beta"], d["state"])
        torch.cuda.synchronize()
        print(f"gdn_decode_fused: {layer_bytes(8, 4096)} algorithmic bytes per dispatch")
    elif fam == "attn":
        layers = [W.attn_layer(8, 4096, dev, seed=i) for i in range(16)]
        for _ in range(args.reps):
            for d in layers:
                ops.paged_gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"], d["scale"],
                                     k_new=d["k_new"], v_new=d["v_new"], pages_per_split=args.pps)  # fmt: skip
        torch.cuda.synchronize()
        print(f"paged_gqa_decode: {layer_bytes(8, 4096, attn=True)} algorithmic bytes per dispatch")
    elif fam == "prefill":
        d = W.prefill(8192, dev, seed=0)
        kc = torch.zeros(2048, 4, 64, 256, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        for _ in range(args.reps):
            ops.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["S0"])
            ops.paged_kv_fill(d["kv_k"], d["kv_v"], kc, vc, d["page_table"])
        torch.cuda.synchronize()
        print(f"chunk prefill: {PREFILL_BYTES} algorithmic bytes (with the K/V fill) per prefill")
    elif fam == "gdn1":
        layers = [W.gdn_layer(1, dev, seed=i) for i in range(96)]
        for _ in range(args.reps):
            for d in layers:
                ops.gdn_decode_fused(d["x"], d["conv_state"], d["taps"], d["g"], d["beta"], d["state"])
        torch.cuda.synchronize()
        print(f"gdn_decode_fused: {layer_bytes(1, 0)} algorithmic bytes per dispatch")
    elif fam == "attn1":
        layers = [W.attn_layer(1, 32768, dev, seed=i) for i in range(4)]
        for _ in range(args.reps):
            for d in layers:
                ops.paged_gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"], d["scale"],
                                     k_new=d["k_new"], v_new=d["v_new"], pages_per_split=args.pps_attn1)  # fmt: skip
        torch.cuda.synchronize()
        print(f"paged_gqa_decode: {layer_bytes(1, 32768, attn=True)} algorithmic bytes per call (main + merge)")
    elif fam == "verify":
        from qwen36_state.decode import VerifyStep

        vs = VerifyStep.synthetic(1, 8192, T=4, device=dev, pages_per_split=args.pps_verify)
        for _ in range(args.reps):
            vs.step()
            vs.rewind()
        torch.cuda.synchronize()
        print(f"verify step: {vs.bytes_per_step(8192)} algorithmic bytes per step")
    elif fam == "mlp":
        layers = [W.mlp_layer(1, dev, seed=i) for i in range(3)]
        for _ in range(args.reps):
            for d in layers:
                ops.mlp_decode(d["x"], None, d["gate"], d["up"], d["down"])
        torch.cuda.synchronize()
        print(f"mlp_decode: {mlp_bytes(1, ops.HIDDEN, ops.INTER)} algorithmic bytes per layer")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=["all"] + sorted(WORKLOADS), default="all")
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--pps", type=int, default=8, help="pages per split-K workgroup (step workload)")
    ap.add_argument("--pps-attn1", type=int, default=8, help="pages per split (attn-layer workload)")
    ap.add_argument("--pps-b1", type=int, default=1, help="pages per split (step-b1 workload)")
    ap.add_argument("--pps-verify", type=int, default=2, help="pages per split (verify-step workload)")
    ap.add_argument("--kernel-reps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baselines")
    ap.add_argument("--profile-family", choices=["gdn", "gdn1", "attn", "attn1", "verify", "conv", "copy", "prefill", "mlp"],
                    default=None)
    ap.add_argument("--reps", type=int, default=3, help="repetitions of --profile-family")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    torch.set_num_threads(cpu_threads())
    if args.profile_family:
        profile_family(args, torch)
        return
    tel = Telemetry()
    main_wl = "step" if args.workload == "all" else args.workload
    head = WORKLOADS[main_wl](args, torch, tel)
    head_tel = tel.summary()
    configs = {}
    if args.workload == "all":
        for wl in ("step-b1", "gdn-layer", "attn-layer", "verify-step", "prefill", "conv-prefill", "mlp-layer"):
            log(f"workload {wl}")
            configs[wl] = WORKLOADS[wl](args, torch, tel)
            configs[wl]["config"] = CONFIG_OF[wl]
            configs[wl]["telemetry"] = tel.summary()
            log(f"{wl}: {configs[wl]['us_per_step']} µs, {configs[wl]['value']} GB/s")
    ceiling = copy_ceiling(torch)
    probes = ceilings(torch)
    log("ceilings: " + ", ".join(f"{k} {v['gbs']} GB/s" for k, v in probes.items()))
    ms = head["us_per_step"] / 1e3
    out = dict(
        metric=METRIC, value=head["value"], unit="GB/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(ms, 4), us_per_step=head["us_per_step"], frac_of_peak=head["frac_of_peak"],
        higher_is_better=True, scaling="weak", vs_baseline=None, dtype="fp32-state/bf16-kv", data="synthetic",
        config=dict(workload=head["workload"], config_index=CONFIG_OF[main_wl], bytes_per_step=head["bytes_per_step"],
                    **{k: head[k] for k in ("batch", "context", "layers", "pages_per_split") if k in head}),
        roofline=head["roofline"],
        stats=dict(median_us=head["median_us"], p10_us=head["p10_us"], p90_us=head["p90_us"], replays=head["replays"]),
        telemetry=head_tel, copy_ceiling=ceiling, ceilings=probes,
    )  # fmt: skip
    for k in ("kernels", "gdn_epilogue", "cpu_baseline"):
        if k in head:
            out[k] = head[k]
    if configs:
        out["configs"] = configs
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
