#!/usr/bin/env python
"""Decode-time state path of the hybrid Gated-DeltaNet / attention Qwen3.6-27B engine on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--workload step]

Default workload (the headline): the batch-8 decode step at 4096 positions per user — 48 Gated-DeltaNet
layers (conv1d update + L2-norm + gated delta rule on fp32 [8, 48, 128, 128] states, in place) and 16
attention layers (append of one token's K/V into block-64 pages + paged GQA decode, 24 q heads / 4 KV heads
x 256, over a shared 2048-page pool through per-user random block tables), replayed as one HIP graph.
Inputs are seeded synthetic tensors already resident in HBM; the step moves 4,631,478,272 algorithmic bytes.

Other workloads (one JSON line each): gdn-layer (one GDN layer, batch 1), attn-layer (one attention layer
at 32768 positions, batch 1), verify-step (MTP verify at batch 1, 8192 positions, 4 tokens, 64 layers +
rollback), prefill (chunked gated delta rule over 8192 tokens + the paged K/V fill), conv-prefill (the
prompt conv with its carry over 8192 tokens).

value = algorithmic bytes / time (GB/s); roofline = the dominant kernel's per-launch algorithmic bytes /
its average launch time (HIP events over back-to-back launches on the stream they run on); cpu_baseline =
the CPU oracle timed on a bounded sample of the same workload (step workload only).
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


def graph_time(torch, fn, steps, warmup):
    """ms per call of fn, replayed as a HIP graph: W untimed replays, then HIP events around K replays."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, g


def kernel_time(torch, make_calls, reps):
    """Average ms of one launch: reps x len(calls) back-to-back C-ABI launches (pre-built argument tuples)
    captured into a HIP graph on a side stream, replayed once untimed and once between HIP events, so no
    host work sits between the launches. make_calls(stream) returns the (entry point, args) list."""
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
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * len(fns))


def gdn_call(d, B, ws, stream, out):
    from qwen36_state.ops import CONV_K, DK, DV, NK, NV

    return "qs_gdn_decode_fused", (
        _p(d["x"]), _p(d["conv_state"]), _p(d["taps"]), _p(d["g"]), _p(d["beta"]), _p(d["state"]), _p(out),
        ctypes.c_void_p(0), _p(ws), B, NK, NV, DK, DV, CONV_K, ctypes.c_float(DK**-0.5), ctypes.c_float(1e-6),
        stream,
    )  # fmt: skip


def attn_call(d, B, T, pps, ws, stream, out):
    from qwen36_state.ops import HD, NKV, NQ

    return "qs_paged_gqa_decode", (
        _p(d["q"]), _p(d["k_new"]), _p(d["v_new"]), _p(d["k_cache"]), _p(d["v_cache"]), _p(d["block_table"]),
        _p(d["seq_lens"]), _p(out), _p(ws), B, T, NQ, NKV, HD, 64, d["block_table"].shape[1],
        d["k_cache"].shape[0], pps, ctypes.c_float(d["scale"]), stream,
    )  # fmt: skip


def roofline(name, nbytes, ms):
    achieved = nbytes / (ms * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(REPO, "profiles", "pmc_traffic.json")
    if os.path.exists(tf):
        with open(tf) as f:
            traffic = json.load(f).get(name, {}).get("hbm_bytes_per_launch")
    return dict(kernel=name, bound="hbm", achieved=round(achieved, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                frac=round(achieved / PEAK_HBM_GBS, 4), traffic=traffic, bytes_per_launch=nbytes,
                us_per_launch=round(ms * 1e3, 2))  # fmt: skip


def line(args, workload, nbytes, ms, dom, extra=None):
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = dict(
        metric=METRIC, value=round(gbs, 1), unit="GB/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(ms, 4), us_per_step=round(ms * 1e3, 1), frac_of_peak=round(gbs / PEAK_HBM_GBS, 4),
        higher_is_better=True, scaling="weak", vs_baseline=None, dtype="fp32-state/bf16-kv", data="synthetic",
        config=dict(workload=workload, bytes_per_step=nbytes), roofline=dom,
    )  # fmt: skip
    if extra:
        out.update(extra)
    return out


# ------------------------------------------------------------------------------------------------ workloads


def bench_step(args, torch):
    from qwen36_state.decode import StatePathStep, layer_bytes

    log(f"building the {args.layers}-layer step: batch {args.batch}, {args.ctx} positions")
    step = StatePathStep(args.batch, args.ctx, args.layers, device="cuda:0", pages_per_split=args.pps)
    gl, al = step.gdn_layers(), step.attn_layers()
    ms, _ = graph_time(torch, step.step, args.steps, args.warmup)
    nbytes = step.bytes_per_step()
    log(f"step: {ms * 1e3:.1f} µs, {nbytes / ms / 1e6:.0f} GB/s")
    t_gdn = kernel_time(torch, lambda st: [gdn_call(step.layer[l], step.B, step.gdn_ws, st, step.layer[l]["o"])
                                           for l in gl], args.kernel_reps)  # fmt: skip
    t_att = kernel_time(torch, lambda st: [attn_call(step.layer[l], step.B, 1, step.pps, step.attn_ws, st,
                                                     step.layer[l]["o"]) for l in al], args.kernel_reps)  # fmt: skip
    b_gdn, b_att = layer_bytes(args.batch, args.ctx), layer_bytes(args.batch, args.ctx, attn=True)
    kern = {"gdn_decode_fused": (t_gdn, b_gdn, len(gl)), "paged_gqa_decode": (t_att, b_att, len(al))}
    for k, (t, b, n) in kern.items():
        log(f"{k}: {t * 1e3:.2f} µs per launch, {b / t / 1e6:.0f} GB/s, {n} launches per step")
    dom = max(kern, key=lambda k: kern[k][0] * kern[k][2])
    out = line(args, f"decode-step state path: {len(gl)} GDN + {len(al)} paged-attention layers, batch "
               f"{args.batch}, {args.ctx} positions per user, block 64, HIP-graph replay", nbytes, ms,
               roofline(dom, kern[dom][1], kern[dom][0]),
               dict(kernels={k: dict(us_per_launch=round(t * 1e3, 2), bytes_per_launch=b,
                                     gbs=round(b / t / 1e6, 1), launches_per_step=n) for k, (t, b, n) in kern.items()}))  # fmt: skip
    out["config"].update(batch=args.batch, context=args.ctx, layers=args.layers, pages_per_split=args.pps)
    if not args.no_cpu:
        log("timing the CPU oracle on a sample of the step")
        out["cpu_baseline"] = cpu_baseline(step, torch)
    return out


def bench_gdn_layer(args, torch):
    """One GDN layer at batch 1; the timed loop walks 48 layers' distinct buffers (313 MB, more than the
    256 MB Infinity Cache) so every launch reads its state from HBM."""
    from qwen36_state import ops, workloads as W
    from qwen36_state.decode import layer_bytes

    layers = [W.gdn_layer(1, "cuda:0", seed=i) for i in range(48)]
    outs = [torch.empty(1, 48, 128, dtype=torch.bfloat16, device="cuda:0") for _ in layers]
    ws = ops.workspace("bench-gdn", ops.lib().qs_gdn_workspace_bytes(1, 16), "cuda:0")
    ms = kernel_time(torch, lambda st: [gdn_call(d, 1, ws, st, o) for d, o in zip(layers, outs)], args.kernel_reps)
    nbytes = layer_bytes(1, 0)
    return line(args, "one GDN layer decode, batch 1: conv1d update (10240 channels) + L2-norm + gated delta "
                "rule on fp32 [1, 48, 128, 128]", nbytes, ms, roofline("gdn_decode_fused", nbytes, ms))


def bench_attn_layer(args, torch):
    """One attention layer at 32768 positions, batch 1; 4 layers with their own pools rotate (each launch
    reads 134 MB of pages that no other launch in the loop touches)."""
    from qwen36_state import ops, workloads as W
    from qwen36_state.decode import layer_bytes

    pps = args.pps_attn1
    layers = [W.attn_layer(1, 32768, "cuda:0", seed=i) for i in range(4)]
    outs = [torch.empty(1, 1, 24, 256, dtype=torch.bfloat16, device="cuda:0") for _ in layers]
    ws = ops.attention_workspace(1, 1, 24, 4, 512, pps, "cuda:0")
    ms = kernel_time(torch, lambda st: [attn_call(d, 1, 1, pps, ws, st, o) for d, o in zip(layers, outs)],
                     args.kernel_reps)  # fmt: skip
    nbytes = layer_bytes(1, 32768, attn=True)
    return line(args, f"one attention layer decode, batch 1, 32768 positions: append + paged GQA (24/4 heads x "
                f"256, block 64, 512 random pages of 2048), split {pps} pages + merge", nbytes, ms,
                roofline("paged_gqa_decode", nbytes, ms), dict(pages_per_split=pps))  # fmt: skip


def bench_verify(args, torch):
    """The MTP verify step with acceptance by slot selection: the graph holds two consecutive steps (the
    two snapshot sets alternate), each with its KV lengths restored for the replay; time per step = half."""
    from qwen36_state.decode import VerifyStep

    vs = VerifyStep(1, 8192, T=4, device="cuda:0", pages_per_split=args.pps_verify)

    def fn():
        for _ in range(2):
            vs.verify()
            vs.rollback()
            vs.reset_lengths()

    ms2, _ = graph_time(torch, fn, args.steps, args.warmup)
    ms = ms2 / 2
    nbytes = vs.bytes_per_step()
    return line(args, "MTP verify step, batch 1, 8192 positions, 1 + 3 draft tokens through 48 GDN + 16 attention "
                "layers, then acceptance of a seeded length by snapshot-slot selection", nbytes, ms,
                roofline("verify_step", nbytes, ms),
                dict(rollback_copy_bytes=vs.rollback_bytes(), accept=vs.accept.tolist(), pages_per_split=vs.pps))  # fmt: skip


def bench_prefill(args, torch):
    from qwen36_state import ops, workloads as W

    d = W.prefill(8192, "cuda:0", seed=0)
    kc = torch.zeros(2048, 4, 64, 256, dtype=torch.bfloat16, device="cuda:0")
    vc = torch.zeros_like(kc)
    nbytes_ws = ops.lib().qs_gdn_chunk_prefill_workspace_bytes(8192, 16, 48, 128, 128, 64)
    ws = ops.workspace(("bench-prefill", 64), nbytes_ws, "cuda:0")

    def fn():
        ops.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["S0"], ws=ws)
        ops.paged_kv_fill(d["kv_k"], d["kv_v"], kc, vc, d["page_table"])

    ms, _ = graph_time(torch, fn, max(3, args.steps // 10), 1)
    nbytes = 344982016
    return line(args, "chunked-prefill gated delta rule, 8192 tokens, chunk 64, 16/48 heads x 128 (WY form, bf16 "
                "MFMA, fp32 state) + paged fill of 8192 tokens of K/V (4 x 256) into 128 random pages", nbytes, ms,
                roofline("gdn_chunk_prefill", nbytes, ms), dict(flops=71.94e9, tflops=round(71.94e9 / ms / 1e9, 1)))


def bench_conv_prefill(args, torch):
    """The prompt conv with its carry over 8192 tokens of the 10240 q | k | v channels, read from a
    projection output with 128 further columns; two prompts rotate (1.3 GB per loop) so each launch reads
    and writes HBM rather than the Infinity Cache."""
    from qwen36_state import ops, workloads as W

    T, C, ldx = 8192, W.C_QKV, W.C_QKV + 128
    CQ, CV = ops.NK * ops.DK, ops.NV * ops.DV
    bufs = []
    for i in range(2):
        gen = W._gen("cuda:0", i)
        bufs.append(dict(
            x=W._randn((T, ldx), gen, "cuda:0", torch.bfloat16),
            taps=W._randn((C, 4), gen, "cuda:0", torch.bfloat16, std=0.5),
            cs=W._randn((C, 3), gen, "cuda:0", torch.bfloat16),
            q=torch.empty(T, CQ, dtype=torch.bfloat16, device="cuda:0"),
            k=torch.empty(T, CQ, dtype=torch.bfloat16, device="cuda:0"),
            v=torch.empty(T, CV, dtype=torch.bfloat16, device="cuda:0"),
            out=torch.empty(C, 3, dtype=torch.bfloat16, device="cuda:0"),
        ))  # fmt: skip

    def calls(st):
        return [("qs_conv1d_prefill", (_p(b["x"]), ldx, _p(b["cs"]), _p(b["taps"]), _p(b["q"]), _p(b["k"]),
                                       _p(b["v"]), _p(b["out"]), T, CQ, CV, 4, st)) for b in bufs]  # fmt: skip

    ms = kernel_time(torch, calls, args.kernel_reps)
    nbytes = 2 * T * C * 2 + C * 4 * 2 + 2 * C * 3 * 2  # x in, q | k | v out, taps, carry in and out
    return line(args, "prompt conv1d + SiLU with carry, 8192 tokens x 10240 channels (q | k | v of a 10368-column "
                "projection), conv state handed to the decode", nbytes, ms, roofline("conv1d_prefill", nbytes, ms))


def cpu_baseline(step, torch, n_gdn=2, n_attn=1, reps=3):
    """The CPU oracle on a bounded sample of the step (n_gdn GDN + n_attn attention layers at the real
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
        O.paged_append(kc, vc, d["k_new"], d["v_new"], d["block_table"], d["seq_lens"] - 1)
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


WORKLOADS = {
    "step": bench_step,
    "gdn-layer": bench_gdn_layer,
    "attn-layer": bench_attn_layer,
    "verify-step": bench_verify,
    "prefill": bench_prefill,
    "conv-prefill": bench_conv_prefill,
}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="step")
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--pps", type=int, default=4, help="pages per split-K workgroup (step workload)")
    ap.add_argument("--pps-attn1", type=int, default=4, help="pages per split (attn-layer workload)")
    ap.add_argument("--pps-verify", type=int, default=2, help="pages per split (verify-step workload)")
    ap.add_argument("--kernel-reps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    out = WORKLOADS[args.workload](args, torch)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
