"""GDN decode path on the GPU against the CPU oracle (conv1d update, gates, delta rule decode, fused
conv + delta rule, T-token verify, rollback). Tolerances: conv state, snapshots and rollback bit-exact;
conv outputs within one bf16 ulp (SiLU's exp differs in the last fp32 bit between libraries); fp32 state
rtol 1e-4; bf16 o rtol 2e-2. The delta-rule checks feed the oracle the kernel's own conv output so a
rare 1-ulp conv difference cannot masquerade as a state error."""
import pytest
import torch
from conftest import assert_bf16_output, assert_state, bf16_ulp_mismatch

from oracle import state_path as O
from qwen36_state import ops, workloads as W

pytestmark = pytest.mark.gpu
NK, NV, DK, DV = 16, 48, 128, 128


def inputs(B, seed=0, T=None):
    return W.gdn_layer(B, "cpu", seed=seed, T=T)


def to(d, dev):
    return {k: v.to(dev) for k, v in d.items()}


def check_conv(y_gpu, y_ref):
    ulps, frac = bf16_ulp_mismatch(y_gpu, y_ref)
    assert ulps <= 1 and frac < 1e-3, (ulps, frac)


@pytest.mark.parametrize("B", [1, 8])
def test_conv1d_update(dev, B):
    d = inputs(B, seed=B)
    g = to(d, dev)
    y = ops.causal_conv1d_update(g["x"], g["conv_state"], g["taps"])
    y_ref, cs_ref = O.conv1d_update(d["x"], d["conv_state"], d["taps"])
    assert torch.equal(g["conv_state"].cpu().float(), cs_ref)
    check_conv(y, y_ref)


def test_gates(dev):
    gen = torch.Generator().manual_seed(3)
    a, b = torch.randn(8, NV, generator=gen).bfloat16(), torch.randn(8, NV, generator=gen).bfloat16()
    dt, neg_a = 0.5 * torch.randn(NV, generator=gen), -torch.exp(torch.rand(NV, generator=gen) * 2 - 1)
    a[0, :4] = torch.tensor([25.0, 19.5, -30.0, 0.0]).bfloat16()  # around the softplus threshold
    g, beta = ops.gdn_gates(a.to(dev), b.to(dev), dt.to(dev), neg_a.to(dev))
    g_ref, b_ref = O.gdn_gates(a.float(), b.float(), dt, neg_a)
    torch.testing.assert_close(g.cpu(), g_ref, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(beta.cpu(), b_ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("B", [1, 8])
def test_gdn_decode_step(dev, B):
    """The unfused step (post-conv q, k, v) at the single-layer shapes: 16 key / 48 value heads, 128 x 128."""
    d = inputs(B, seed=10 + B)
    g = to(d, dev)
    o = ops.gdn_decode_step(g["q"], g["k"], g["v"], g["g"], g["beta"], g["state"])
    o_ref, S_ref = O.gdn_step(d["q"].float(), d["k"].float(), d["v"].float(), d["g"], d["beta"], d["state"])
    assert_state(g["state"], S_ref)
    assert_bf16_output(o, O.bf16(o_ref))


@pytest.mark.parametrize("B", [1, 8])
def test_gdn_decode_fused(dev, B):
    """Conv + L2-norm + delta rule in one launch, called twice in a row (the second call proves the
    per-key-head counters re-armed themselves)."""
    d = inputs(B, seed=20 + B)
    g = to(d, dev)
    S, cs = d["state"], d["conv_state"].float()
    for call in range(2):
        x = W._randn((B, W.C_QKV), torch.Generator().manual_seed(100 + call), "cpu", torch.bfloat16)
        y = torch.empty(B, W.C_QKV, dtype=torch.bfloat16, device=dev)
        o = ops.gdn_decode_fused(x.to(dev), g["conv_state"], g["taps"], g["g"], g["beta"], g["state"], y_out=y)
        y_ref, cs = O.conv1d_update(x, cs, d["taps"])
        check_conv(y, y_ref)
        assert torch.equal(g["conv_state"].cpu().float(), cs)
        q, k, v = O.split_qkv(y.cpu().float(), NK, NV, DK, DV)
        o_ref, S = O.gdn_step(q, k, v, d["g"], d["beta"], S)
        assert_state(g["state"], S)
        assert_bf16_output(o, O.bf16(o_ref))
        S = g["state"].cpu()  # continue from the kernel's state (no drift between the two references)


def test_gdn_masked_rows_leave_state(dev):
    """g = 0, beta = 0 is the identity on the state, bit-exact (the prefill's masking rule)."""
    d = inputs(2, seed=5)
    g = to(d, dev)
    before = g["state"].clone()
    ops.gdn_decode_step(g["q"], g["k"], g["v"], torch.zeros_like(g["g"]), torch.zeros_like(g["beta"]), g["state"])
    assert torch.equal(g["state"], before)


def test_gdn_repeatable(dev):
    d = inputs(8, seed=6)
    outs = []
    for _ in range(2):
        g = to(d, dev)
        o = ops.gdn_decode_fused(g["x"], g["conv_state"], g["taps"], g["g"], g["beta"], g["state"])
        outs.append((o.cpu(), g["state"].cpu(), g["conv_state"].cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,T", [(1, 4), (3, 2)])
def test_gdn_verify_and_rollback(dev, B, T):
    d = inputs(B, seed=30 + T, T=T)
    g = to(d, dev)
    o, states, convs, y = ops.gdn_verify_step(g["x"], g["conv_state"], g["taps"], g["g"], g["beta"], g["state"],
                                              return_y=True)  # fmt: skip
    # inputs untouched
    assert torch.equal(g["state"].cpu(), d["state"]) and torch.equal(g["conv_state"].cpu(), d["conv_state"])
    S, cs = d["state"], d["conv_state"].float()
    for t in range(T):
        y_ref, cs = O.conv1d_update(d["x"][:, t], cs, d["taps"])
        check_conv(y[:, t], y_ref)
        assert torch.equal(convs[t].cpu().float(), cs)
        q, k, v = O.split_qkv(y[:, t].cpu().float(), NK, NV, DK, DV)
        o_ref, S = O.gdn_step(q, k, v, d["g"][:, t], d["beta"][:, t], S)
        assert_state(states[t], S)
        assert_bf16_output(o[:, t], O.bf16(o_ref))
        S = states[t].cpu()
    # rollback to a seeded accepted length per user, with the KV truncation
    acc = torch.randint(1, T + 1, (B,), generator=torch.Generator().manual_seed(T), dtype=torch.int32)
    base = torch.full((B,), 8188, dtype=torch.int32)
    seq = torch.zeros(B, dtype=torch.int32, device=dev)
    ops.gdn_rollback(states, convs, acc.to(dev), g["state"], g["conv_state"], seq, base.to(dev))
    ref_s, ref_c = O.gdn_rollback(states.cpu(), convs.cpu(), acc)
    assert torch.equal(g["state"].cpu(), ref_s) and torch.equal(g["conv_state"].cpu(), ref_c)
    assert torch.equal(seq.cpu(), base + acc)


def test_rollback_layers_equals_per_layer(dev):
    """The one-launch rollback of L layers restores exactly what L single-layer rollbacks do."""
    L, T, B, C = 3, 3, 2, 10240
    gen = torch.Generator(device="cpu").manual_seed(77)
    states = torch.randn(L, T, B, NV, DK, DV, generator=gen).to(dev)
    convs = torch.randn(L, T, B, C, 3, generator=gen).to(torch.bfloat16).to(dev)
    acc = torch.tensor([2, 3], dtype=torch.int32, device=dev)
    base = torch.tensor([100, 200], dtype=torch.int32, device=dev)
    st1 = torch.zeros(L, B, NV, DK, DV, device=dev)
    cv1 = torch.zeros(L, B, C, 3, dtype=torch.bfloat16, device=dev)
    st2, cv2 = st1.clone(), cv1.clone()
    seq1 = torch.zeros(B, dtype=torch.int32, device=dev)
    seq2 = seq1.clone()
    ops.gdn_rollback_layers(states, convs, acc, st1, cv1, seq1, base)
    for l in range(L):
        ops.gdn_rollback(states[l], convs[l], acc, st2[l], cv2[l], seq2 if l == 0 else None, base if l == 0 else None)
    assert torch.equal(st1, st2) and torch.equal(cv1, cv2) and torch.equal(seq1, seq2)
    for l in range(L):
        for b in range(B):
            assert torch.equal(st1[l, b], states[l, int(acc[b]) - 1, b])


def test_verify_one_token_equals_decode(dev):
    d = inputs(2, seed=40)
    g1, g2 = to(d, dev), to(d, dev)
    o1 = ops.gdn_decode_fused(g1["x"], g1["conv_state"], g1["taps"], g1["g"], g1["beta"], g1["state"])
    o2, st, cv = ops.gdn_verify_step(g2["x"][:, None], g2["conv_state"], g2["taps"], g2["g"][:, None],
                                     g2["beta"][:, None], g2["state"])  # fmt: skip
    assert torch.equal(o1, o2[:, 0]) and torch.equal(g1["state"], st[0]) and torch.equal(g1["conv_state"], cv[0])


@pytest.mark.parametrize("B,T,accepted", [
    (3, 3, [2, 3, 1]),                  # 4 waves per slab, slots among the first four
    (2, 8, [8, 5]),                     # slots 7 and 4: past the four whose histories are read ahead
    (8, 6, [1, 2, 3, 4, 5, 6, 6, 1]),   # one wave per slab (batch 8), every slot
])  # fmt: skip
def test_verify_slots_equals_copy_rollback(dev, B, T, accepted):
    """Slot selection (the next verify reads snapshot a - 1 of the previous step in place) reproduces the
    copy rollback bit for bit: same outputs, snapshots and conv histories for the next verify step."""
    d = inputs(B, seed=51, T=T)
    g = to(d, dev)
    o1, states, convs = ops.gdn_verify_step(g["x"], g["conv_state"], g["taps"], g["g"], g["beta"], g["state"])
    acc = torch.tensor(accepted, dtype=torch.int32, device=dev)
    base = torch.arange(10, 10 * B + 1, 10, dtype=torch.int32, device=dev)
    # copy path: restore, then verify from the restored state
    st, cv = g["state"].clone(), g["conv_state"].clone()
    seq_c = torch.zeros(B, dtype=torch.int32, device=dev)
    ops.gdn_rollback(states, convs, acc, st, cv, seq_c, base)
    d2 = inputs(B, seed=52, T=T)
    g2 = to(d2, dev)
    ref = ops.gdn_verify_step(g2["x"], cv, g2["taps"], g2["g"], g2["beta"], st)
    # slot path: accept, then verify reading the snapshots in place
    slot = torch.full((B,), 7, dtype=torch.int32, device=dev)
    seq_s = torch.zeros(B, dtype=torch.int32, device=dev)
    ops.verify_accept(acc, T, slot, seq_s, base)
    assert torch.equal(slot.cpu(), acc.cpu() - 1) and torch.equal(seq_s, seq_c)
    out = (torch.empty_like(ref[0]), torch.empty_like(ref[1]), torch.empty_like(ref[2]))
    ops.gdn_verify_step_slots(g2["x"], convs, g2["taps"], g2["g"], g2["beta"], states, slot, out=out)
    for a, b in zip(out, ref):
        assert torch.equal(a, b)
    if B != 3:
        return
    # an out-of-range accept length leaves the slot and the length untouched
    bad = torch.tensor([0, 5, 2], dtype=torch.int32, device=dev)
    ops.verify_accept(bad, T, slot, seq_s, base)
    assert slot.cpu().tolist() == [1, 2, 1] and seq_s.cpu().tolist() == [12, 23, 32]


def test_gdn_gated_norm(dev):
    """The GDN mixer's gated RMSNorm epilogue (model.py:274-275) for a batch-8 decode and a T = 4 verify
    output: within one bf16 ulp of the oracle (rsqrt and exp differ in the last fp32 bits)."""
    gen = torch.Generator().manual_seed(61)
    for shape in ((8, NV, DV), (1, 4, NV, DV)):
        o = torch.randn(shape, generator=gen).bfloat16()
        z = (2 * torch.randn(shape, generator=gen)).bfloat16()
        w = 1 + 0.1 * torch.randn(DV, generator=gen)
        y = ops.gdn_gated_norm(o.to(dev), z.to(dev), w.to(dev))
        ulps, frac = bf16_ulp_mismatch(y, O.gdn_gated_norm(o, z, w))
        assert ulps <= 1 and frac < 1e-2, (ulps, frac)


@pytest.mark.parametrize("B", [1, 3, 8])
def test_gdn_decode_fused_gated_norm(dev, B):
    """The fused decode with the mixer's gated RMSNorm epilogue in the same launch (z, norm_w; model.py:
    274-275, kernels/gdn_head_compute.cpp:320-346): o = bf16(rmsnorm(o) norm_w silu(z)) per value head, from
    the fp32 o as the reference normalises it, against the oracle's gdn_gated_norm(gdn_step(...)) at rtol 2e-2
    (the oracle fed the kernel's own conv output); z is read as a strided slice of a wider projection row.
    Batch 1 and 3 (a head's 4 slabs on 4 waves each, 16 waves per workgroup) and 8 (one wave per slab). The
    state and conv state are bit-identical to the plain fused launch, whose o rounded to bf16 and then put
    through the separate epilogue lands within two bf16 ulps of the fused result."""
    d = inputs(B, seed=40 + B)
    gen = torch.Generator().manual_seed(41 + B)
    proj = (2 * torch.randn(B, NV * DV + 96, generator=gen)).bfloat16()  # z slice + the columns after it
    z = proj[:, : NV * DV]
    w = 1 + 0.1 * torch.randn(DV, generator=gen)
    g, g2 = to(d, dev), to(d, dev)
    y = torch.empty(B, W.C_QKV, dtype=torch.bfloat16, device=dev)
    zd = proj.to(dev)[:, : NV * DV]
    o = ops.gdn_decode_fused(g["x"], g["conv_state"], g["taps"], g["g"], g["beta"], g["state"], y_out=y, z=zd,
                             norm_w=w.to(dev))  # fmt: skip
    o_plain = ops.gdn_decode_fused(g2["x"], g2["conv_state"], g2["taps"], g2["g"], g2["beta"], g2["state"])
    assert torch.equal(g["state"], g2["state"]) and torch.equal(g["conv_state"], g2["conv_state"])
    q, k, v = O.split_qkv(y.cpu().float(), NK, NV, DK, DV)
    o_ref, S = O.gdn_step(q, k, v, d["g"], d["beta"], d["state"])
    assert_state(g["state"], S)
    ref = O.gdn_gated_norm(o_ref, z.float().view(B, NV, DV), w)
    assert_bf16_output(o, ref)
    two = ops.gdn_gated_norm(o_plain, zd.contiguous().view(B, NV, DV), w.to(dev))
    ulps, frac = bf16_ulp_mismatch(o, two)
    assert ulps <= 2, (ulps, frac)
    with pytest.raises(ValueError, match="both"):
        ops.gdn_decode_fused(g["x"], g["conv_state"], g["taps"], g["g"], g["beta"], g["state"], z=zd)
