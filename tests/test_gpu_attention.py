"""Paged GQA decode attention on the GPU against the oracle (gather + fp32 softmax over the pages):
bf16 output rtol 2e-2; the fused append leaves the pools bit-identical to the oracle's append."""
import pytest
import torch
from conftest import assert_attn_output

from oracle import state_path as O
from qwen36_state import ops, workloads as W

pytestmark = pytest.mark.gpu

CNT_BYTES = 65536  # the fixed counter block at the head of an attention workspace


def run_case(dev, d, pps, fused=True):
    """Attention (+ append) on the GPU and the same step through the oracle; returns (o_gpu, o_ref,
    pools equal)."""
    g = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}
    B, T = d["q"].shape[:2]
    pos = d["seq_lens"] - T
    if fused:
        o = ops.paged_gqa_decode(g["q"], g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"], d["scale"],
                                 k_new=g["k_new"], v_new=g["v_new"], pages_per_split=pps)  # fmt: skip
    else:
        ops.paged_kv_append(g["k_new"], g["v_new"], g["k_cache"], g["v_cache"], g["block_table"], pos.to(dev))
        o = ops.paged_gqa_decode(g["q"], g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"], d["scale"],
                                 pages_per_split=pps)  # fmt: skip
    kc, vc = d["k_cache"].clone(), d["v_cache"].clone()
    O.paged_append(kc, vc, d["k_new"], d["v_new"], d["block_table"], pos)
    o_ref = O.gqa_decode(d["q"], kc, vc, d["block_table"], d["seq_lens"], d["scale"])
    same = torch.equal(g["k_cache"].cpu(), kc) and torch.equal(g["v_cache"].cpu(), vc)
    return o, O.bf16(o_ref), same


@pytest.mark.parametrize(
    "B,ctx,T,pps",
    [
        (1, 32768, 1, 8),  # the 32k layer as benchmarked: 512 pages, 64 splits through the merge launch
        (8, 4096, 1, 8),  # the batch-8 step's layer as benchmarked: 8 splits merged inside the launch
        (8, 4096, 1, 4),  # 16 splits merged inside the launch (the limit)
        (1, 8192, 4, 8),  # verify: 4 new rows, causal among them (24 query rows per KV head)
        (1, 32768, 1, 1),  # 512 splits (2048 workgroups) through the merge launch
        (2, 4096, 1, 64),  # one split: no merge
        (2, 3000, 6, 4),  # 36 query rows per KV head: the VALU kernel (two tokens per pass over the pages)
        (1, 700, 7, 64),  # VALU kernel, odd token count, one split
        (3, 900, 2, 4),  # 12 query rows per KV head: two tokens on the one-tile MFMA kernel
    ],
)
def test_attention(dev, B, ctx, T, pps):
    d = W.attn_layer(B, ctx, "cpu", seed=B + ctx + T + pps, T=T)
    o, o_ref, same = run_case(dev, d, pps)
    assert same
    assert_attn_output(o, o_ref)


def test_attention_ragged_users(dev):
    """Users at different lengths (1 position, exactly one page, one past a page, mid-page) in one launch."""
    d = W.attn_layer(4, 11 * 64, "cpu", seed=77, T=1, num_blocks=64)
    d["seq_lens"] = torch.tensor([1, 64, 65, 700], dtype=torch.int32)
    o, o_ref, same = run_case(dev, d, pps=2)
    assert same
    assert_attn_output(o, o_ref)
    # a user with a single position attends only to its new row: o = v_new exactly (up to bf16 rounding)
    torch.testing.assert_close(o[0, 0].cpu().float(), d["v_new"][0, 0].float().repeat_interleave(6, 0), rtol=0, atol=0)


def test_attention_unfused_equals_fused(dev):
    d = W.attn_layer(2, 1000, "cpu", seed=5, T=2, num_blocks=64)
    o1, ref, _ = run_case(dev, d, pps=4, fused=True)
    o2, _, same = run_case(dev, d, pps=4, fused=False)
    assert same
    assert torch.equal(o1.cpu(), o2.cpu())
    assert_attn_output(o1, ref)


@pytest.mark.parametrize(
    "G,T,lens,pps",
    [
        (6, 4, [8194], 2),  # the verify shape; new rows at 62..65 of a page pair that two splits share
        (6, 4, [8194], 1),  # each of those pages its own split
        (6, 5, [700, 337, 4099], 4),  # ragged users: new rows inside one slice, across slices, across pages
        (6, 3, [337], 64),  # one split (no merge); rows 14..16 span two waves' slices
        (4, 8, [1000, 9 * 64 + 4], 2),  # 8 new rows, the most held in registers; the second user's span pages
        (8, 4, [130, 64], 1),  # 32 query rows; the second user's new rows end its only page
        (2, 9, [777], 2),  # 9 new rows: more than the registers hold, through the pool instead
        (2, 16, [2000], 4),  # the most new rows a call takes (16)
    ],
)
def test_verify_append_from_registers(dev, G, T, lens, pps):
    """The MFMA kernel (17 to 32 query rows per KV head) with up to 8 new rows appends from registers (the new
    K rows in the score operand, the new V rows as the page is staged, the pool written after the page loop);
    more rows go through the pool first. Either way: output bit-equal to the unfused append followed by
    attention, pools equal to the oracle's append, output within the oracle's tolerance."""
    d = W.attn_layer(len(lens), max(lens), "cpu", seed=G * 100 + T + pps, T=T, num_blocks=512)
    d["seq_lens"] = torch.tensor(lens, dtype=torch.int32)
    nkv = d["k_cache"].shape[1]
    q = d["q"] if G * nkv <= d["q"].shape[2] else torch.cat([d["q"], d["q"]], dim=2)
    d["q"] = q[:, :, : G * nkv].contiguous()
    assert 16 < T * G <= 32  # the MFMA kernel's range
    o1, ref, same1 = run_case(dev, d, pps, fused=True)
    o2, _, same2 = run_case(dev, d, pps, fused=False)
    assert same1 and same2
    assert torch.equal(o1.cpu(), o2.cpu())
    assert_attn_output(o1, ref)


def test_attention_repeatable(dev):
    d = W.attn_layer(1, 32768, "cpu", seed=9)
    g = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}
    outs = [
        ops.paged_gqa_decode(g["q"], g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"], d["scale"],
                             k_new=g["k_new"], v_new=g["v_new"], pages_per_split=8).cpu()  # fmt: skip
        for _ in range(3)
    ]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


@pytest.mark.parametrize("B,ctx,T,pps", [(2, 1000, 1, 4), (1, 2048, 3, 2), (3, 700, 2, 64), (1, 900, 6, 4)])
def test_attn_mixer(dev, B, ctx, T, pps):
    """q/k RMSNorm + partial RoPE and the sigmoid gate around the paged attention (model.py:237-246), one
    token and three verify rows (MFMA kernel), one split (no merge), six rows (VALU kernel): the appended K rows within
    one bf16 ulp of the oracle's (rsqrt and the rotation differ in the last fp32 bits between libraries), V
    rows bit-exact, the output rtol 2e-2."""
    from conftest import bf16_ulp_mismatch

    d = W.attn_layer(B, ctx, "cpu", seed=ctx + T, T=T, num_blocks=64)
    gen = torch.Generator().manual_seed(ctx)
    gate = torch.randn(d["q"].shape, generator=gen).bfloat16()
    wq = (1 + 0.1 * torch.randn(256, generator=gen)) / 16.0
    wk = 1 + 0.1 * torch.randn(256, generator=gen)
    pos = (d["seq_lens"] - T)[:, None] + torch.arange(T)[None]
    cos, sin = O.rope_tables(pos + 5000)
    g = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}
    o = ops.attn_mixer_decode(g["q"], g["k_new"], g["v_new"], gate.to(dev), wq.to(dev), wk.to(dev), cos.to(dev),
                              sin.to(dev), g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"],
                              pages_per_split=pps)  # fmt: skip
    kc, vc = d["k_cache"].clone(), d["v_cache"].clone()
    o_ref = O.attn_mixer(d["q"], d["k_new"], d["v_new"], gate, wq, wk, cos, sin, kc, vc, d["block_table"],
                         d["seq_lens"])  # fmt: skip
    assert torch.equal(g["v_cache"].cpu(), vc)
    ulps, frac = bf16_ulp_mismatch(g["k_cache"].cpu(), kc)
    assert ulps <= 1 and frac < 1e-3, (ulps, frac)
    assert_attn_output(o, o_ref)
    # the rope tables of the wrapper equal the oracle's
    c2, s2 = ops.rope_tables(pos.to(dev) + 5000)
    assert torch.equal(c2.cpu(), cos) and torch.equal(s2.cpu(), sin)


def test_in_launch_merge_counters_rearm(dev):
    """Up to 16 splits are merged inside the attention launch by the last workgroup to arrive. The arrival
    counters at the workspace head read zero after every call, so one workspace serves repeated calls and
    calls of other shapes (here batch 8 one token, then batch 3 four verify rows, twice each): outputs repeat
    bit-exactly and match the oracle."""
    L = ops.lib()
    ws = torch.zeros(L.qs_paged_attention_workspace_bytes(8, 4, 24, 4, 256, 64, 4), dtype=torch.uint8, device=dev)
    cases = [(8, 4096, 1), (3, 2000, 4)]
    data = [W.attn_layer(B, ctx, "cpu", seed=B + T, T=T, num_blocks=1024) for B, ctx, T in cases]
    outs = []
    for rep in range(2):
        for d in data:
            g = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}
            o = ops.paged_gqa_decode(g["q"], g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"], d["scale"],
                                     pages_per_split=4, ws=ws)  # fmt: skip
            torch.cuda.synchronize()
            assert int(ws[:CNT_BYTES].view(torch.int32).abs().sum()) == 0, "counters not re-armed"
            outs.append(o.cpu())
    assert torch.equal(outs[0], outs[2]) and torch.equal(outs[1], outs[3])
    for d, o in zip(data, outs):
        ref = O.gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"], d["scale"])
        assert_attn_output(o, O.bf16(ref))


# More than 16 splits go through the separate merge launch (one workgroup per output row, the partials merged in
# split order): 18, 64, 512 and 1024 splits, verify rows on the MFMA kernel at 64, 32 and 18 splits, batch 3 with
# an idle user at 32 and 18 splits. Three calls give the same bits, match the oracle, leave the in-launch counters
# at zero and report nothing.
@pytest.mark.parametrize("B,ctx,T,pps", [(2, 1100, 1, 1), (1, 32768, 1, 8), (1, 32768, 1, 1), (1, 65536, 1, 1),
                                         (1, 8192, 4, 2), (3, 2000, 4, 1), (3, 1100, 4, 1)])  # fmt: skip
def test_many_splits_repeatable(dev, B, ctx, T, pps):
    d = W.attn_layer(B, ctx, "cpu", seed=3 * B + T + pps, T=T, num_blocks=B * (ctx // 64 + 1) + 64)
    if B == 3:
        d["seq_lens"][1] = 0  # idle: no workgroup of the user arrives at its counters
    g = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}
    mb = d["block_table"].shape[1]
    ws = torch.zeros(ops.lib().qs_paged_attention_workspace_bytes(B, T, 24, 4, 256, mb, pps), dtype=torch.uint8,
                     device=dev)  # fmt: skip
    st = ops.Status(dev)
    outs = []
    for _ in range(3):
        o = ops.paged_gqa_decode(g["q"], g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"], d["scale"],
                                 pages_per_split=pps, ws=ws, status=st.word)  # fmt: skip
        torch.cuda.synchronize()
        assert int(ws[:CNT_BYTES].view(torch.int32).abs().sum()) == 0, "counters not re-armed"
        outs.append(o.cpu())
    assert st.peek() == 0
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    ref = O.gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"], d["scale"])
    assert_attn_output(outs[0], O.bf16(ref))


@pytest.mark.parametrize("T", [1, 4])
def test_merge_launch_ragged(dev, T):
    """The merge launch over users of very different lengths: one user's 19 splits hold a single page of T rows
    among 18 empty splits (whose partials carry no weight), the other's all 19 pages."""
    d = W.attn_layer(2, 19 * 64, "cpu", seed=40 + T, T=T, num_blocks=64)
    d["seq_lens"] = torch.tensor([T, 19 * 64 - 5], dtype=torch.int32)
    o, o_ref, same = run_case(dev, d, pps=1)
    assert same
    assert_attn_output(o, o_ref)


@pytest.mark.parametrize("ctx,pps", [(131072, 64), (131072, 2), (262144, 4)])
def test_attention_long_context(dev, ctx, pps):
    """128k and 256k positions at batch 1 (the reference's published long-context decode points reach 256k):
    32 splits of the widest split (64 pages), exactly the 1024-split limit, and 1024 splits at 256k."""
    d = W.attn_layer(1, ctx, "cpu", seed=ctx // 1024 + pps, num_blocks=ctx // 64 + 64)
    o, o_ref, same = run_case(dev, d, pps)
    assert same
    assert_attn_output(o, o_ref)


def test_attention_split_limits(dev):
    """More than 1024 splits or more than 64 pages per split are rejected before any launch."""
    d = W.attn_layer(1, 131072, dev, seed=1, num_blocks=2048 + 64)
    for pps in (1, 65):
        with pytest.raises(ValueError, match="splits|pages_per_split"):
            ops.paged_gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"], d["scale"],
                                 pages_per_split=pps)  # fmt: skip


def test_attention_negative_control(dev):
    """The check fails when the oracle drops the appended row (a missed append dependency)."""
    d = W.attn_layer(2, 40, "cpu", seed=12, num_blocks=64)  # 40 positions: the new row carries ~1/40 of the weight
    o, ref, _ = run_case(dev, d, 4)
    assert_attn_output(o, ref)
    wrong = O.bf16(O.gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"] - 1, d["scale"]))
    with pytest.raises(AssertionError):
        assert_attn_output(o, wrong)
