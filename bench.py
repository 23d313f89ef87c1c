#!/usr/bin/env python
"""Decode-step state path of the 64-layer hybrid engine on one MI355X: µs per step and achieved HBM GB/s.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5]

Workload (default): the batch-8 decode step at 4096 positions per user — 48 Gated-DeltaNet layers (conv1d
update + L2-norm + gated delta rule on fp32 [8, 48, 128, 128] states, in place) and 16 attention layers
(append of one token's K/V into block-64 pages + paged GQA decode, 24 q heads / 4 KV heads x 256, over a
shared 2048-page pool through per-user random block tables), replayed as one HIP graph. Inputs are seeded
synthetic tensors already resident in HBM; the step moves 4,631,478,272 algorithmic bytes.

One JSON line: value = algorithmic bytes / step time (GB/s); ms_per_step; roofline of the dominant kernel
(per-launch algorithmic bytes / average launch time from HIP events over back-to-back launches on the
stream they run on); cpu_baseline = the CPU oracle timed on a bounded sample of the same step.
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "tt-qwen-resident_amd"))

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
METRIC = "decode-step state-path µs and achieved HBM GB/s (% of peak) at batch 1/8"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def launch_args(step, l, stream):
    """Pre-built C-ABI argument tuple of layer l (the timed loop calls the library with no Python checks)."""
    from qwen36_state.ops import CONV_K, DK, DV, HD, NK, NKV, NQ, NV

    d = step.layer[l]
    if d["attn"]:
        return "qs_paged_gqa_decode", (
            _p(d["q"]), _p(d["k_new"]), _p(d["v_new"]), _p(d["k_cache"]), _p(d["v_cache"]), _p(d["block_table"]),
            _p(d["seq_lens"]), _p(d["o"]), _p(step.attn_ws), step.B, 1, NQ, NKV, HD, 64,
            d["block_table"].shape[1], d["k_cache"].shape[0], step.pps, ctypes.c_float(d["scale"]), stream,
        )  # fmt: skip
    return "qs_gdn_decode_fused", (
        _p(d["x"]), _p(d["conv_state"]), _p(d["taps"]), _p(d["g"]), _p(d["beta"]), _p(d["state"]), _p(d["o"]),
        ctypes.c_void_p(0), _p(step.gdn_ws), step.B, NK, NV, DK, DV, CONV_K, ctypes.c_float(DK**-0.5),
        ctypes.c_float(1e-6), stream,
    )  # fmt: skip


def time_kernel(step, layers, reps, torch):
    """Average duration (ms) of one launch of the kernel the layers use: HIP events around reps x len(layers)
    back-to-back launches over the layers' distinct buffers, on the stream they are launched on."""
    from qwen36_state._lib import lib

    L = lib()
    stream = torch.cuda.current_stream()
    calls = [launch_args(step, l, ctypes.c_void_p(stream.cuda_stream)) for l in layers]
    fns = [getattr(L, name) for name, _ in calls]
    for f, (_, a) in zip(fns, calls):  # warm
        assert f(*a) == 0, L.qs_last_error()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        for f, (_, a) in zip(fns, calls):
            f(*a)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * len(layers))


def cpu_baseline(step, torch, n_gdn=2, n_attn=1, reps=3):
    """The CPU oracle on a bounded sample of the same step (n_gdn GDN + n_attn attention layers at the real
    shapes), scaled to the full step by layer count; median of reps after one warm-up."""
    sys.path.insert(0, REPO)
    from oracle import state_path as O
    from qwen36_state.ops import DK, DV, NK, NV

    gl, al = step.gdn_layers(), step.attn_layers()
    gdn = [{k: v.cpu() for k, v in step.layer[l].items() if torch.is_tensor(v)} for l in gl[:n_gdn]]
    att = [{k: v.cpu() for k, v in step.layer[l].items() if torch.is_tensor(v)} for l in al[:n_attn]]
    scale = step.layer[al[0]]["scale"]

    def run_gdn(d):
        O.gdn_decode(d["x"].float(), d["conv_state"].float(), d["taps"].float(), d["g"], d["beta"], d["state"],
                     NK, NV, DK, DV)  # fmt: skip

    def run_attn(d):
        kc, vc = d["k_cache"], d["v_cache"]
        pos = d["seq_lens"] - 1
        O.paged_append(kc, vc, d["k_new"], d["v_new"], d["block_table"], pos)
        O.gqa_decode(d["q"], kc, vc, d["block_table"], d["seq_lens"], scale)

    def timed(fn, ds):
        fn(ds[0])
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            for d in ds:
                fn(d)
            ts.append((time.perf_counter() - t0) / len(ds))
        return statistics.median(ts)

    tg, ta = timed(run_gdn, gdn), timed(run_attn, att)
    t_step = len(gl) * tg + len(al) * ta
    return dict(
        value=round(step.bytes_per_step() / t_step / 1e9, 3),
        unit="GB/s",
        cores=torch.get_num_threads(),
        kind="port",
        sample=f"{n_gdn} GDN + {n_attn} attention layers of the batch-{step.B} step at {step.ctx} positions "
        f"(median of {reps}), scaled to {len(gl)} + {len(al)} layers: {t_step * 1e3:.1f} ms per step "
        f"(GDN layer {tg * 1e3:.1f} ms, attention layer {ta * 1e3:.1f} ms)",
    )


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--pps", type=int, default=8, help="pages per split-K workgroup")
    ap.add_argument("--kernel-reps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--only-kernel", choices=["gdn", "attn"], help="only the per-kernel loop (for counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch

    from qwen36_state.decode import StatePathStep, layer_bytes

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    log(f"building the {args.layers}-layer step: batch {args.batch}, {args.ctx} positions")
    step = StatePathStep(args.batch, args.ctx, args.layers, device="cuda:0", pages_per_split=args.pps)
    gl, al = step.gdn_layers(), step.attn_layers()

    if args.only_kernel:
        layers = gl if args.only_kernel == "gdn" else al
        ms = time_kernel(step, layers, args.kernel_reps, torch)
        log(f"{args.only_kernel}: {ms * 1e3:.2f} µs per launch")
        return

    step.step()
    torch.cuda.synchronize()
    step.capture()
    log("graph captured; warm-up")
    for _ in range(args.warmup):
        step.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = step.bytes_per_step()
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"step: {ms * 1e3:.1f} µs, {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}% of peak)")

    # per-kernel launch times (back-to-back over the layers' own buffers)
    t_gdn = time_kernel(step, gl, args.kernel_reps, torch)
    t_att = time_kernel(step, al, args.kernel_reps, torch)
    b_gdn = layer_bytes(args.batch, args.ctx, attn=False)
    b_att = layer_bytes(args.batch, args.ctx, attn=True)
    kern = {
        "gdn_decode_fused": dict(ms=t_gdn, bytes=b_gdn, launches=len(gl)),
        "paged_gqa_decode": dict(ms=t_att, bytes=b_att, launches=len(al)),
    }
    for k, v in kern.items():
        log(f"{k}: {v['ms'] * 1e3:.2f} µs per launch, {v['bytes'] / v['ms'] / 1e6:.0f} GB/s")
    dom = max(kern, key=lambda k: kern[k]["ms"] * kern[k]["launches"])
    dk = kern[dom]
    achieved = dk["bytes"] / (dk["ms"] * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(REPO, "profiles", "pmc_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            traffic = json.load(f).get(dom, {}).get("hbm_bytes_per_launch")

    out = dict(
        metric=METRIC,
        value=round(gbs, 1),
        unit="GB/s",
        n_gpus=1,
        steps=args.steps,
        warmup=args.warmup,
        ms_per_step=round(ms, 4),
        us_per_step=round(ms * 1e3, 1),
        frac_of_peak=round(gbs / PEAK_HBM_GBS, 4),
        higher_is_better=True,
        scaling="weak",
        vs_baseline=None,
        dtype="fp32-state/bf16-kv",
        data="synthetic",
        config=dict(
            workload=f"decode-step state path: {len(gl)} GDN + {len(al)} paged-attention layers, batch "
            f"{args.batch}, {args.ctx} positions per user, block 64, HIP-graph replay",
            batch=args.batch,
            context=args.ctx,
            layers=args.layers,
            bytes_per_step=nbytes,
            pages_per_split=args.pps,
        ),
        kernels={k: dict(us_per_launch=round(v["ms"] * 1e3, 2), bytes_per_launch=v["bytes"],
                         gbs=round(v["bytes"] / v["ms"] / 1e6, 1), launches_per_step=v["launches"])
                 for k, v in kern.items()},  # fmt: skip
        roofline=dict(
            kernel=dom,
            bound="hbm",
            achieved=round(achieved, 1),
            peak=PEAK_HBM_GBS,
            unit="GB/s",
            frac=round(achieved / PEAK_HBM_GBS, 4),
            traffic=traffic,
        ),
    )
    if not args.no_cpu:
        log("timing the CPU oracle on a sample of the step")
        out["cpu_baseline"] = cpu_baseline(step, torch)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
