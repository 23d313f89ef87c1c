"""Launch one kernel family of the state path back to back, for rocprofv3 counter runs.

    python tt-qwen-resident_amd/qwen36_state/profile_kernels.py gdn    # fused GDN decode, batch 8, 48 layers
    python tt-qwen-resident_amd/qwen36_state/profile_kernels.py attn   # paged GQA decode, batch 8, 4096 pos, 16 layers
    python tt-qwen-resident_amd/qwen36_state/profile_kernels.py conv   # prompt conv with carry, 8192 tokens
    python tt-qwen-resident_amd/qwen36_state/profile_kernels.py copy   # 1 GiB device copy (counter calibration)

Each mode runs its launches `--reps` times over distinct per-layer buffers (so the dispatches read HBM, not
the Infinity Cache) and prints the algorithmic bytes of one dispatch.
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["gdn", "attn", "conv", "copy"])
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--pps", type=int, default=4)
    args = ap.parse_args()

    import torch

    from qwen36_state import ops, workloads as W
    from qwen36_state.decode import layer_bytes

    dev = "cuda:0"
    if args.mode == "copy":
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(args.reps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy: {src.numel() * 4} bytes read and written per dispatch")
        return
    if args.mode == "conv":
        T, C = 8192, W.C_QKV
        bufs = []
        for i in range(2):
            gen = W._gen(dev, i)
            bufs.append((W._randn((T, C + 128), gen, dev, torch.bfloat16), W._randn((C, 4), gen, dev, torch.bfloat16),
                         W._randn((C, 3), gen, dev, torch.bfloat16)))  # fmt: skip
        for _ in range(args.reps):
            for x, taps, cs in bufs:
                ops.causal_conv1d_prefill(x[:, :C], taps, cs)
        torch.cuda.synchronize()
        print(f"conv1d_prefill: {2 * T * C * 2 + C * 8 + C * 12} algorithmic bytes per dispatch")
        return
    if args.mode == "gdn":
        layers = [W.gdn_layer(8, dev, seed=i) for i in range(48)]
        for _ in range(args.reps):
            for d in layers:
                ops.gdn_decode_fused(d["x"], d["conv_state"], d["taps"], d["g"], d["beta"], d["state"])
        torch.cuda.synchronize()
        print(f"gdn_decode_fused: {layer_bytes(8, 4096)} algorithmic bytes per dispatch")
        return
    layers = [W.attn_layer(8, 4096, dev, seed=i) for i in range(16)]
    for _ in range(args.reps):
        for d in layers:
            ops.paged_gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"], d["scale"],
                                 k_new=d["k_new"], v_new=d["v_new"], pages_per_split=args.pps)  # fmt: skip
    torch.cuda.synchronize()
    print(f"paged_gqa_decode: {layer_bytes(8, 4096, attn=True)} algorithmic bytes per dispatch (+ merge)")


if __name__ == "__main__":
    main()
