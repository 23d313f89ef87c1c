"""Chunked-prefill gated delta rule on the GPU (WY form, chunk 64, MFMA) against the fp64 oracle: the
sequential recurrence for short sequences, its chunked WY restatement (pinned against the recurrence on the
CPU) for 8192 tokens. Final fp32 state rtol 1e-4; bf16 per-token output rtol 2e-2."""
import pytest
import torch
from conftest import assert_bf16_output, assert_prefill_state

from oracle import state_path as O
from qwen36_state import ops, workloads as W

pytestmark = pytest.mark.gpu


def run(dev, d, T):
    g = {k: v.to(dev) for k, v in d.items()}
    o, S = ops.chunk_gated_delta_rule(g["q"][:T], g["k"][:T], g["v"][:T], g["g"][:T], g["beta"][:T],
                                      initial_state=g["S0"], chunk_size=64)  # fmt: skip
    return o, S


def ref(d, T, wy=False):
    args = [d[n][:T].double() for n in ("q", "k", "v", "g", "beta")] + [d["S0"].double()]
    if wy:
        return O.gdn_chunk_prefill_wy(*args, chunk=64)
    return O.gdn_chunk_prefill(*args)


@pytest.mark.parametrize("T", [1, 64, 200])
def test_prefill_matches_recurrence(dev, T):
    d = W.prefill(T, "cpu", seed=T)
    o, S = run(dev, d, T)
    o_ref, S_ref = ref(d, T)
    assert_prefill_state(S, S_ref.float())
    assert_bf16_output(o, O.bf16(o_ref.float()))


@pytest.mark.parametrize("nk,nv", [(4, 4), (4, 8), (2, 8)])
def test_prefill_head_ratios(dev, nk, nv):
    """1, 2 and 4 value heads per key head (the prep forms K K^T and Q K^T once per key head and takes the
    value heads in turn); 130 tokens, a partial last chunk."""
    T = 130
    d = W.prefill(T, "cpu", seed=7)
    d = {"q": d["q"][:, :nk], "k": d["k"][:, :nk], "v": d["v"][:, :nv], "g": d["g"][:, :nv],
         "beta": d["beta"][:, :nv], "S0": d["S0"][:nv]}  # fmt: skip
    d = {n: t.contiguous() for n, t in d.items()}
    o, S = run(dev, d, T)
    o_ref, S_ref = ref(d, T)
    assert_prefill_state(S, S_ref.float())
    assert_bf16_output(o, O.bf16(o_ref.float()))


def test_prefill_rejects_more_than_four_value_heads_per_key_head(dev):
    d = W.prefill(64, "cpu", seed=8)
    with pytest.raises((RuntimeError, ValueError)):
        run(dev, {"q": d["q"][:, :1].contiguous(), "k": d["k"][:, :1].contiguous(), "v": d["v"][:, :8].contiguous(),
                  "g": d["g"][:, :8].contiguous(), "beta": d["beta"][:, :8].contiguous(), "S0": d["S0"][:8].contiguous()}, 64)  # fmt: skip


def test_prefill_8192_tokens(dev):
    """The prefill workload: one GDN layer over 8192 tokens (128 chunks), 16 key / 48 value heads."""
    d = W.prefill(8192, "cpu", seed=4)
    o, S = run(dev, d, 8192)
    o_ref, S_ref = ref(d, 8192, wy=True)
    assert_prefill_state(S, S_ref.float())
    assert_bf16_output(o, O.bf16(o_ref.float()))


def test_prefill_masked_rows_are_identity(dev):
    """g = 0, beta = 0 on every row (the prefill's masked rows) leaves the state unchanged."""
    d = W.prefill(100, "cpu", seed=5)
    d["g"].zero_()
    d["beta"].zero_()
    _, S = run(dev, d, 100)
    torch.testing.assert_close(S.cpu(), d["S0"], rtol=0, atol=1e-6)


def test_prefill_then_decode_continues(dev):
    """Prefill of T tokens then one decode step equals prefill of T + 1 tokens (the prefill-to-decode
    handoff: the final state is the decode state)."""
    d = W.prefill(130, "cpu", seed=6)
    g = {k: v.to(dev) for k, v in d.items()}
    _, S = ops.chunk_gated_delta_rule(g["q"][:129], g["k"][:129], g["v"][:129], g["g"][:129], g["beta"][:129],
                                      initial_state=g["S0"])  # fmt: skip
    state = S[None].contiguous()
    o1 = ops.gdn_decode_step(g["q"][129:130].contiguous(), g["k"][129:130].contiguous(), g["v"][129:130].contiguous(),
                             g["g"][129:130].contiguous(), g["beta"][129:130].contiguous(), state)  # fmt: skip
    o2, S2 = run(dev, d, 130)
    assert_prefill_state(state[0], S2.cpu())
    assert_bf16_output(o1[0], o2[129])


def test_prefill_repeatable(dev):
    d = W.prefill(300, "cpu", seed=7)
    a = run(dev, d, 300)
    b = run(dev, d, 300)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_prefill_4485_tokens(dev):
    """4485 tokens = 71 chunks, the last one of 5 tokens, against the WY oracle."""
    d = W.prefill(4485, "cpu", seed=8)
    o, S = run(dev, d, 4485)
    o_ref, S_ref = ref(d, 4485, wy=True)
    assert_prefill_state(S, S_ref.float())
    assert_bf16_output(o, O.bf16(o_ref.float()))


def test_prefill_graph_replays(dev):
    """The prefill captured into a HIP graph, replayed three times with eager work in between: every replay
    equals the eager result bit for bit."""
    d = W.prefill(4485, "cpu", seed=9)
    g = {k: v.to(dev) for k, v in d.items()}
    ws = ops.workspace(("prefill-graph", 64), ops.lib().qs_gdn_chunk_prefill_workspace_bytes(4485, 16, 48, 128, 128, 64),
                       dev)  # fmt: skip
    eager = ops.chunk_gated_delta_rule(g["q"], g["k"], g["v"], g["g"], g["beta"], initial_state=g["S0"], ws=ws)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            out = ops.chunk_gated_delta_rule(g["q"], g["k"], g["v"], g["g"], g["beta"], initial_state=g["S0"], ws=ws)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0], eager[0]) and torch.equal(out[1], eager[1])
        g["q"].add_(0)  # eager work between the replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("batched", [False, True])
def test_prefill_reference_call(dev, batched):
    """The reference prefill's call as written (prefill/pp_prefill.py:791-807): token-major q, k [T, 2048],
    v [T, 6144], scale DK^-1/2, output_final_state, chunk_size 32, output_head_major, and the ttnn-only
    memory_config / eye / tril / ones / masks (accepted and ignored), with and without the per-device
    leading batch dimension of 1. 200 tokens against the fp64 recurrence: S_T rtol 1e-4, head-major o
    rtol 2e-2."""
    T = 200
    d = W.prefill(T, "cpu", seed=11)
    g = {k: v.to(dev) for k, v in d.items()}
    q, k, v = g["q"].reshape(T, -1), g["k"].reshape(T, -1), g["v"].reshape(T, -1)
    gg, bb, S0 = g["g"], g["beta"], g["S0"]
    if batched:
        q, k, v, gg, bb, S0 = q[None], k[None], v[None], gg[None], bb[None], S0[None]
    eye, tril, ones = torch.eye(32), torch.tril(torch.ones(32, 32)), torch.ones(32, 32)
    o, S = ops.chunk_gated_delta_rule(
        q, k, v, gg, bb,
        scale=128**-0.5,
        initial_state=S0,
        output_final_state=True,
        chunk_size=32,
        output_head_major=True,
        memory_config="DRAM",
        eye=eye,
        tril=tril,
        ones=ones,
        masks=torch.zeros(32, 96),
    )  # fmt: skip
    if batched:
        assert o.shape == (1, 48, T, 128) and S.shape == (1, 48, 128, 128)
        o, S = o[0], S[0]
    assert o.shape == (48, T, 128) and S.shape == (48, 128, 128)
    o_ref, S_ref = ref(d, T)
    assert_prefill_state(S, S_ref.float())
    assert_bf16_output(o.transpose(0, 1), O.bf16(o_ref.float()))
    with pytest.raises(ValueError, match="chunk_size"):
        ops.chunk_gated_delta_rule(q, k, v, gg, bb, initial_state=S0, chunk_size=16)
