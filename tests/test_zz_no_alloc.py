"""The allocation-free fused GDN decode (qs_gdn_decode_fused_noalloc, counters in the library's static device
array) against the workspace entry point qs_gdn_decode_fused, both called through the C ABI: captured into a
HIP graph on its first call and replayed on fresh inputs; two eager calls in a row, the second with a smaller
batch; each bit-identical to the workspace entry point on a copy of the same inputs (the same kernels run;
only where the counters live differs); an oversized batch is rejected."""
import ctypes

import pytest
import torch

from qwen36_state import ops, workloads as W

pytestmark = pytest.mark.gpu
NK, NV, DK, DV = 16, 48, 128, 128


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def run(entry, d, B, ws=None):
    L = ops.lib()
    o = torch.empty(B, NV, DV, dtype=torch.bfloat16, device=d["x"].device)
    y = torch.empty_like(d["x"])
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [_p(d["x"]), _p(d["conv_state"]), _p(d["taps"]), _p(d["g"]), _p(d["beta"]), _p(d["state"]), _p(o), _p(y)]
    if ws is not None:  # the workspace entry: no gated-norm epilogue (z, ldz, norm_w), then the workspace
        args += [ctypes.c_void_p(0), 0, ctypes.c_void_p(0), _p(ws)]
    args.append(ctypes.c_void_p(0))  # lens: every user active
    rc = getattr(L, entry)(*args, B, NK, NV, DK, DV, 4, ctypes.c_float(DK**-0.5), ctypes.c_float(1e-6), st)
    assert rc == 0, L.qs_last_error().decode()
    return o, y


def test_noalloc_captured_in_a_graph(dev):
    """The allocation-free entry captured into a HIP graph on its first call in the process (the one-time
    address lookup and the array's clear happen during the capture), then replayed twice on fresh inputs,
    with eager work between the replays: each replay equals the workspace entry point on a copy of the same
    inputs bit for bit, and the static counter array reads zero afterwards (the counters re-arm themselves)."""
    L = ops.lib()
    B = 8
    buf = W.gdn_layer(B, dev, seed=90)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            o, y = run("qs_gdn_decode_fused_noalloc", buf, B)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(2):
        fresh = W.gdn_layer(B, dev, seed=91 + rep)
        for k in ("x", "g", "beta", "state", "conv_state", "taps"):
            buf[k].copy_(fresh[k])
        ref = {k: v.clone() for k, v in fresh.items()}
        ws = torch.zeros(L.qs_gdn_workspace_bytes(B, NK), dtype=torch.uint8, device=dev)
        o_ref, y_ref = run("qs_gdn_decode_fused", ref, B, ws)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(y, y_ref), rep
        assert torch.equal(buf["state"], ref["state"]) and torch.equal(buf["conv_state"], ref["conv_state"]), rep
        _ = torch.randn(4096, device=dev).sum().item()  # eager work between the replays
    cnt = torch.full((16384,), -1, dtype=torch.int32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.qs_gdn_noalloc_scratch_read(_p(cnt), 16384, st) == 0, L.qs_last_error().decode()
    torch.cuda.synchronize()
    assert int(cnt.abs().sum()) == 0


@pytest.mark.parametrize("batches", [(8, 3)])
def test_noalloc_equals_workspace_entry(dev, batches):
    L = ops.lib()
    for i, B in enumerate(batches):
        d = W.gdn_layer(B, dev, seed=70 + i)
        a = {k: v.clone() for k, v in d.items()}
        ws = torch.zeros(L.qs_gdn_workspace_bytes(B, NK), dtype=torch.uint8, device=dev)
        o1, y1 = run("qs_gdn_decode_fused", a, B, ws)
        o2, y2 = run("qs_gdn_decode_fused_noalloc", d, B)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(y1, y2), B
        assert torch.equal(a["state"], d["state"]) and torch.equal(a["conv_state"], d["conv_state"]), B


def test_noalloc_rejects_oversized_batch(dev):
    L = ops.lib()
    f = ctypes.c_void_p(0x1000)
    rc = L.qs_gdn_decode_fused_noalloc(f, f, f, f, f, f, f, ctypes.c_void_p(0), ctypes.c_void_p(0), 1024, 16, 48, 128, 128, 4,
                                       ctypes.c_float(0.1), ctypes.c_float(1e-6), ctypes.c_void_p(0))  # fmt: skip
    assert rc == -1 and "exceeds" in L.qs_last_error().decode()
