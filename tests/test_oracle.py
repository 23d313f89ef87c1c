"""Pins the CPU oracle: golden fixtures (scalar fp64 loops), closed forms, invariants and special cases
chosen so a plausible mistake (a swapped tap order, a wrong key-head index, a dropped decay, a transposed
state, an off-by-one page index, a missing causal mask) fails at least one check. No GPU needed."""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import state_path as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "state_path_small.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k]) for k in z.files}


def bfr(*shape, gen, std=1.0):
    return O.bf16(std * torch.randn(*shape, generator=gen))


# ------------------------------------------------------------------------------------------- golden vectors


def test_golden_conv(gold):
    y, ns = O.conv1d_update(gold["conv_x"], gold["conv_state"], gold["conv_taps"])
    assert torch.equal(ns, gold["conv_new_state"])
    # bf16 outputs: at most one bf16 ulp from the fp64-silu fixture
    assert torch.allclose(y, gold["conv_y"], rtol=2**-8, atol=0)


def test_golden_gdn_step(gold):
    o, S2 = O.gdn_step(gold["gdn_q"], gold["gdn_k"], gold["gdn_v"], gold["gdn_g"], gold["gdn_beta"], gold["gdn_S"])
    torch.testing.assert_close(o, gold["gdn_o"], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(S2, gold["gdn_S2"], rtol=1e-12, atol=1e-12)


def test_golden_attention(gold):
    o = O.gqa_decode(gold["att_q"], gold["att_k"], gold["att_v"], gold["att_table"], gold["att_seq"],
                     scale=1 / math.sqrt(8), dtype=torch.float64)  # fmt: skip
    torch.testing.assert_close(o, gold["att_o"], rtol=1e-12, atol=1e-12)


def test_golden_prefill(gold):
    args = [gold[f"pre_{n}"] for n in ("q", "k", "v", "g", "beta", "S0")]
    o, S = O.gdn_chunk_prefill(*args)
    torch.testing.assert_close(o, gold["pre_o"], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(S, gold["pre_ST"], rtol=1e-12, atol=1e-12)
    o2, S2 = O.gdn_chunk_prefill_wy(*args, chunk=4)  # 9 tokens: chunks of 4, 4, 1
    torch.testing.assert_close(o2, gold["pre_o"], rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(S2, gold["pre_ST"], rtol=1e-10, atol=1e-12)


# ------------------------------------------------------------------------------------------- a1 conv


def test_conv_matches_loops():
    g = torch.Generator().manual_seed(0)
    x, cs, taps = bfr(3, 17, gen=g), bfr(3, 17, 3, gen=g), bfr(17, 4, gen=g, std=0.5)
    y, ns = O.conv1d_update(x, cs, taps)
    y2, ns2 = O.conv1d_update_loops(x, cs, taps)
    assert torch.equal(ns, ns2)
    assert torch.allclose(y, y2, rtol=2**-8, atol=0)


def test_conv_tap_order_and_impulse():
    """Tap 0 multiplies the oldest input (weights.py:58): state [a, 0, 0], x = 0 gives silu(w0 a); an
    impulse in x with a zero state gives silu(w3)."""
    taps = torch.tensor([[0.5, -0.25, 2.0, 1.5]])
    a = torch.tensor([[[3.0, 0.0, 0.0]]])
    y, ns = O.conv1d_update(torch.zeros(1, 1), a, taps)
    assert float(y) == float(O.bf16(torch.nn.functional.silu(torch.tensor(1.5))))
    assert ns.tolist() == [[[0.0, 0.0, 0.0]]]
    y, _ = O.conv1d_update(torch.ones(1, 1), torch.zeros(1, 1, 3), taps)
    assert float(y) == float(O.bf16(torch.nn.functional.silu(torch.tensor(1.5))))
    y, _ = O.conv1d_update(torch.zeros(1, 1), torch.tensor([[[0.0, 0.0, 1.0]]]), taps)
    assert float(y) == float(O.bf16(torch.nn.functional.silu(torch.tensor(2.0))))


def test_conv_shift_invariant():
    """After K-1 new inputs the state is exactly those inputs (oldest first)."""
    g = torch.Generator().manual_seed(1)
    cs, taps = bfr(2, 5, 3, gen=g), bfr(5, 4, gen=g)
    xs = [bfr(2, 5, gen=g) for _ in range(3)]
    for x in xs:
        _, cs = O.conv1d_update(x, cs, taps)
    assert torch.equal(cs, torch.stack(xs, -1))


@pytest.mark.parametrize("T", [0, 1, 2, 3, 7, 40])
def test_conv_prefill_equals_decode_steps(T):
    """The prompt conv equals T decode conv steps from the same carry: every output bit for bit, and the
    carry it leaves is the decode conv state (the reference's carry check, tests/test_pp_kernels.py:137-142,
    for full, partial and 1-row chunks)."""
    g = torch.Generator().manual_seed(10 + T)
    C = 24
    x, cs, taps = bfr(T, C, gen=g), bfr(C, 3, gen=g), bfr(C, 4, gen=g, std=0.5)
    y, ns = O.conv1d_prefill(x, cs, taps)
    st = cs[None].clone()
    for t in range(T):
        yt, st = O.conv1d_update(x[t][None], st, taps)
        assert torch.equal(y[t], yt[0])
    assert torch.equal(ns, st[0])
    assert y.shape == (T, C)


def test_conv_prefill_impulse_carry_and_split():
    """An impulse at token s with a zero carry gives silu(tap 3 - j) at token s + j (tap 0 on the oldest);
    no carry means a zero carry; prefill of a prompt in two pieces, the second from the first's carry,
    equals the prefill of the whole prompt."""
    taps = torch.tensor([[0.5, -0.25, 2.0, 1.5]])
    x = torch.zeros(9, 1)
    x[3, 0] = 1.0
    y, ns = O.conv1d_prefill(x, None, taps)
    silu = lambda v: float(O.bf16(F.silu(torch.tensor(v))))
    assert [float(v) for v in y[:, 0]] == [0.0, 0.0, 0.0, silu(1.5), silu(2.0), silu(-0.25), silu(0.5), 0.0, 0.0]
    assert ns.tolist() == [[0.0, 0.0, 0.0]]
    g = torch.Generator().manual_seed(3)
    x, taps = bfr(50, 16, gen=g), bfr(16, 4, gen=g)
    y, ns = O.conv1d_prefill(x, None, taps)
    y0, ns0 = O.conv1d_prefill(x, torch.zeros(16, 3), taps)
    assert torch.equal(y, y0) and torch.equal(ns, ns0)
    for cut in (1, 2, 17):
        ya, ca = O.conv1d_prefill(x[:cut], None, taps)
        yb, cb = O.conv1d_prefill(x[cut:], ca, taps)
        assert torch.equal(torch.cat([ya, yb]), y) and torch.equal(cb, ns)
    assert torch.equal(ns, x[-3:].t())


# ------------------------------------------------------------------------------------------- a2 / a3


def test_l2norm_unit_and_scale_invariant():
    g = torch.Generator().manual_seed(2)
    k = torch.randn(4, 128, generator=g, dtype=torch.float64)
    n = O.l2norm(k, eps=0.0)
    torch.testing.assert_close(n.norm(dim=-1), torch.ones(4, dtype=torch.float64))
    torch.testing.assert_close(O.l2norm(7.5 * k, eps=0.0), n)
    # eps enters under the square root: |k̂|^2 = s / (s + eps)
    s = k.pow(2).sum(-1)
    torch.testing.assert_close(O.l2norm(k, eps=1e-2).pow(2).sum(-1), s / (s + 1e-2))


def test_gates_scalar():
    a = torch.tensor([-3.0, 0.2, 19.0, 25.0])
    dt = torch.tensor([0.5, -0.1, 0.5, 0.0])
    neg_a = torch.tensor([-0.7, -1.3, -0.2, -0.9])
    b = torch.tensor([-2.0, 0.0, 1.0, 30.0])
    g, beta = O.gdn_gates(a, b, dt, neg_a)
    for i in range(4):
        z = float(a[i] + dt[i])
        sp = z if z > 20 else math.log1p(math.exp(z))
        assert abs(float(g[i]) - float(neg_a[i]) * sp) < 1e-5 * max(1.0, abs(sp))
        assert abs(float(beta[i]) - 1 / (1 + math.exp(-float(b[i])))) < 1e-6
    assert float(g[3]) == float(neg_a[3] * 25.0)  # above the threshold softplus is the identity


# ------------------------------------------------------------------------------------------- a4 delta rule


def _gdn_inputs(B=2, NK=2, NV=6, DK=8, DV=8, seed=3, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q, k = torch.randn(B, NK, DK, generator=g), torch.randn(B, NK, DK, generator=g)
    v = torch.randn(B, NV, DV, generator=g)
    gg = -torch.nn.functional.softplus(torch.randn(B, NV, generator=g))
    beta = torch.sigmoid(torch.randn(B, NV, generator=g))
    S = 0.1 * torch.randn(B, NV, DK, DV, generator=g)
    return [t.to(dtype) for t in (q, k, v, gg, beta, S)]


def test_gdn_step_matches_loops():
    q, k, v, g, beta, S = _gdn_inputs()
    o, S2 = O.gdn_step(q, k, v, g, beta, S)
    o2, S3 = O.gdn_step_loops(q, k, v, g, beta, S)
    torch.testing.assert_close(o, o2, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(S2, S3, rtol=1e-12, atol=1e-12)


def test_gdn_identity_when_masked():
    """g = 0, beta = 0 (the prefill's masked rows, prefill/pp_prefill.py:14-17) leaves the state bit-exact."""
    q, k, v, g, beta, S = _gdn_inputs(dtype=torch.float32)
    _, S2 = O.gdn_step(q, k, v, torch.zeros_like(g), torch.zeros_like(beta), S)
    assert torch.equal(S2, S)


def test_gdn_rank1_from_zero_state():
    q, k, v, g, beta, S = _gdn_inputs()
    o, S2 = O.gdn_step(q, k, v, g, beta, torch.zeros_like(S))
    kn = O.l2norm(k.repeat_interleave(3, 1))
    qn = O.l2norm(q.repeat_interleave(3, 1)) * 8**-0.5
    ref = beta[..., None, None] * kn[..., :, None] * v[..., None, :]
    torch.testing.assert_close(S2, ref)
    torch.testing.assert_close(o, (qn * kn).sum(-1, keepdim=True) * beta[..., None] * v)


def test_gdn_writes_value_at_key():
    """decay = 1, beta = 1: k̂^T S' = v up to the L2-norm eps (the delta rule's defining property)."""
    q, k, v, g, beta, S = _gdn_inputs()
    _, S2 = O.gdn_step(q, k, v, torch.zeros_like(g), torch.ones_like(beta), S, eps=0.0)
    kn = O.l2norm(k.repeat_interleave(3, 1), eps=0.0)
    torch.testing.assert_close((kn[..., None, :] @ S2).squeeze(-2), v, rtol=1e-10, atol=1e-10)


def test_gdn_key_head_grouping_and_columns():
    """Value head h reads key head h // (NV / NK); value columns are independent."""
    q, k, v, g, beta, S = _gdn_inputs()
    o, S2 = O.gdn_step(q, k, v, g, beta, S)
    for h in range(6):
        kh = h // 3
        oh, Sh = O.gdn_step(q[:, kh : kh + 1], k[:, kh : kh + 1], v[:, h : h + 1], g[:, h : h + 1],
                            beta[:, h : h + 1], S[:, h : h + 1])  # fmt: skip
        torch.testing.assert_close(oh[:, 0], o[:, h], rtol=0, atol=0)
        torch.testing.assert_close(Sh[:, 0], S2[:, h], rtol=0, atol=0)
    oc, Sc = O.gdn_step(q, k, v[..., 2:5], g, beta, S[..., 2:5].contiguous())
    torch.testing.assert_close(oc, o[..., 2:5], rtol=1e-14, atol=1e-14)
    torch.testing.assert_close(Sc, S2[..., 2:5], rtol=1e-14, atol=1e-14)


# ------------------------------------------------------------------------------------------- a7 verify


def test_verify_equals_sequential_and_rollback():
    g = torch.Generator().manual_seed(4)
    NK, NV, DK, DV, B, T = 1, 3, 4, 4, 2, 3
    C = 2 * NK * DK + NV * DV
    x, cs, taps = bfr(B, T, C, gen=g), bfr(B, C, 3, gen=g), bfr(C, 4, gen=g, std=0.5)
    gg = -torch.rand(B, T, NV, generator=g)
    beta = torch.rand(B, T, NV, generator=g)
    S = 0.1 * torch.randn(B, NV, DK, DV, generator=g)
    o, states, convs, ys = O.gdn_verify(x, cs, taps, gg, beta, S, NK, NV, DK, DV)
    St, cst = S, cs
    for t in range(T):
        ot, St, cst, yt = O.gdn_decode(x[:, t], cst, taps, gg[:, t], beta[:, t], St, NK, NV, DK, DV)
        assert torch.equal(ot, o[:, t]) and torch.equal(St, states[t]) and torch.equal(cst, convs[t])
    o1, s1, c1, _ = O.gdn_verify(x[:, :1], cs, taps, gg[:, :1], beta[:, :1], S, NK, NV, DK, DV)
    od, Sd, cd, _ = O.gdn_decode(x[:, 0], cs, taps, gg[:, 0], beta[:, 0], S, NK, NV, DK, DV)
    assert torch.equal(o1[:, 0], od) and torch.equal(s1[0], Sd) and torch.equal(c1[0], cd)
    st, cv = O.gdn_rollback(states, convs, [2, 3])
    assert torch.equal(st[0], states[1, 0]) and torch.equal(st[1], states[2, 1])
    assert torch.equal(cv[0], convs[1, 0]) and torch.equal(cv[1], convs[2, 1])


# ------------------------------------------------------------------------------------------- a5 / a9 paged


def test_paged_append_matches_loops_and_gather():
    g = torch.Generator().manual_seed(5)
    nb, nkv, block, hd, B, T = 9, 2, 4, 8, 3, 3
    k1 = bfr(nb, nkv, block, hd, gen=g)
    v1 = bfr(nb, nkv, block, hd, gen=g)
    k2, v2 = k1.clone(), v1.clone()
    table = torch.randperm(nb, generator=g)[:9].view(3, 3).int()
    pos = torch.tensor([0, 3, 7], dtype=torch.int32)  # crosses page boundaries
    kn, vn = bfr(B, T, nkv, hd, gen=g), bfr(B, T, nkv, hd, gen=g)
    O.paged_append(k1, v1, kn, vn, table, pos)
    O.paged_append_loops(k2, v2, kn, vn, table, pos)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    for b in range(B):
        gk = O.paged_gather(k1, table[b], int(pos[b]) + T)
        assert torch.equal(gk[:, int(pos[b]) :].permute(1, 0, 2), kn[b])


def test_paged_fill_roundtrip():
    g = torch.Generator().manual_seed(6)
    cache = torch.zeros(12, 2, 4, 8)
    x = bfr(2, 10, 8, gen=g)
    pt = torch.tensor([7, 2, 11], dtype=torch.int32)
    O.paged_fill(cache, x, pt)
    assert torch.equal(O.paged_gather(cache, pt, 10), x)
    assert torch.equal(cache[2, :, 1], x[:, 5])  # token 5 -> page pt[1] = 2, row 1
    untouched = [i for i in range(12) if i not in (7, 2, 11)]
    assert cache[untouched].abs().sum() == 0


# ------------------------------------------------------------------------------------------- a6 attention


def test_attention_one_position_and_shift_invariance():
    g = torch.Generator().manual_seed(7)
    kc, vc = torch.randn(4, 2, 4, 8, generator=g), torch.randn(4, 2, 4, 8, generator=g)
    table = torch.tensor([[3, 1]], dtype=torch.int32)
    q = torch.randn(1, 1, 4, 8, generator=g)
    o = O.gqa_decode(q, kc, vc, table, torch.tensor([1]), scale=0.3)
    for h in range(4):
        torch.testing.assert_close(o[0, 0, h], vc[3, h // 2, 0])
    # adding a constant score offset (q along a direction all keys share) leaves o unchanged
    kc2 = kc + 0.0
    kc2[..., 0] = 1.0
    q2 = q.clone()
    base = O.gqa_decode(q2, kc2, vc, table, torch.tensor([6]), scale=0.3)
    q2[..., 0] += 5.0
    torch.testing.assert_close(O.gqa_decode(q2, kc2, vc, table, torch.tensor([6]), scale=0.3), base)


def test_attention_split_merge_equals_one_pass():
    g = torch.Generator().manual_seed(8)
    K, V, q = torch.randn(200, 16, generator=g), torch.randn(200, 16, generator=g), torch.randn(16, generator=g)
    full = torch.softmax((K @ q) * 0.25, -1) @ V
    parts = O.attention_partials(q, K, V, 0.25, [(0, 64), (64, 128), (128, 192), (192, 200)])
    torch.testing.assert_close(O.merge_partials(parts), full)


def test_attention_causal_among_new_tokens():
    """Query t of a T-token step equals a 1-token step over the sequence truncated after t."""
    g = torch.Generator().manual_seed(9)
    kc, vc = torch.randn(6, 2, 4, 8, generator=g), torch.randn(6, 2, 4, 8, generator=g)
    table = torch.tensor([[5, 0, 3]], dtype=torch.int32)
    q = torch.randn(1, 4, 4, 8, generator=g)
    o = O.gqa_decode(q, kc, vc, table, torch.tensor([11]), scale=0.35)
    for t in range(4):
        ot = O.gqa_decode(q[:, t : t + 1], kc, vc, table, torch.tensor([8 + t]), scale=0.35)
        torch.testing.assert_close(o[:, t], ot[:, 0])


# ------------------------------------------------------------------------------------------- a8 prefill


def test_prefill_chunked_equals_recurrence():
    g = torch.Generator().manual_seed(10)
    T, NK, NV, DK = 150, 2, 6, 16
    q, k = torch.randn(T, NK, DK, generator=g).double(), torch.randn(T, NK, DK, generator=g).double()
    v = torch.randn(T, NV, DK, generator=g).double()
    gg = (-torch.nn.functional.softplus(torch.randn(T, NV, generator=g)) * torch.exp(-3 * torch.rand(T, NV, generator=g))).double()
    beta = torch.sigmoid(torch.randn(T, NV, generator=g)).double()
    S0 = 0.02 * torch.randn(NV, DK, DK, generator=g).double()
    o, S = O.gdn_chunk_prefill(q, k, v, gg, beta, S0)
    for chunk in (16, 32, 64):  # chunk-size independence, incl. the reference prefill's 32
        o2, S2 = O.gdn_chunk_prefill_wy(q, k, v, gg, beta, S0, chunk=chunk)
        torch.testing.assert_close(o2, o, rtol=1e-10, atol=1e-12)
        torch.testing.assert_close(S2, S, rtol=1e-10, atol=1e-12)
    # masked rows (g = 0, beta = 0) leave the state unchanged
    _, Sm = O.gdn_chunk_prefill(q[:5], k[:5], v[:5], torch.zeros(5, NV).double(), torch.zeros(5, NV).double(), S0)
    assert torch.equal(Sm, S0)


# ------------------------------------------------------------------------- the attention mixer's edges


def test_rmsnorm_closed_form_and_scale_invariance():
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(5, 256, generator=gen, dtype=torch.float64)
    y = O.rmsnorm(x, eps=1e-6)
    ms = x.pow(2).mean(-1)
    # mean(y^2) = mean(x^2) / (mean(x^2) + eps) exactly, and scaling x does not change y beyond the eps
    torch.testing.assert_close(y.pow(2).mean(-1), ms / (ms + 1e-6), rtol=1e-12, atol=0)
    torch.testing.assert_close(O.rmsnorm(7.0 * x, eps=1e-6), y, rtol=1e-6, atol=1e-9)
    w = torch.randn(256, generator=gen, dtype=torch.float64)
    torch.testing.assert_close(O.rmsnorm(x, w, 1e-6), y * w, rtol=0, atol=0)


def test_rope_tables_values():
    c, s = O.rope_tables(0)
    assert torch.equal(c, torch.ones(32)) and torch.equal(s, torch.zeros(32))
    c, s = O.rope_tables(torch.tensor([1, 1000]))
    # frequency 0 is theta^0 = 1 rad per position; the last one theta^(-62/64)
    assert abs(float(c[0, 0]) - math.cos(1.0)) < 1e-7 and abs(float(s[1, 0]) - math.sin(1000.0)) < 1e-6
    f = 1e7 ** (-62 / 64)
    assert abs(float(s[1, 31]) - math.sin(1000 * f)) < 1e-7


def test_rope_is_a_rotation_of_dim_pairs():
    gen = torch.Generator().manual_seed(12)
    t = torch.randn(3, 256, generator=gen, dtype=torch.float64)
    # identity at angle 0; dims past rot untouched
    c0, s0 = torch.ones(32, dtype=torch.float64), torch.zeros(32, dtype=torch.float64)
    assert torch.equal(O.rope(t, c0, s0), t)
    ang_a = torch.rand(32, generator=gen, dtype=torch.float64) * 6
    ang_b = torch.rand(32, generator=gen, dtype=torch.float64) * 6
    ra = O.rope(t, torch.cos(ang_a), torch.sin(ang_a))
    assert torch.equal(ra[:, 64:], t[:, 64:])
    # each pair (d, d + 32) keeps its norm, and rotations compose by adding angles
    torch.testing.assert_close(ra[:, :32] ** 2 + ra[:, 32:64] ** 2, t[:, :32] ** 2 + t[:, 32:64] ** 2)
    rab = O.rope(ra, torch.cos(ang_b), torch.sin(ang_b))
    torch.testing.assert_close(rab, O.rope(t, torch.cos(ang_a + ang_b), torch.sin(ang_a + ang_b)))
    # the pair (a, b) turns like the complex number a + i b multiplied by e^{i angle}
    z = torch.complex(t[:, :32], t[:, 32:64]) * torch.exp(1j * ang_a)
    torch.testing.assert_close(ra[:, :32], z.real)
    torch.testing.assert_close(ra[:, 32:64], z.imag)


def test_attn_mixer_reduces_to_attention():
    """With unit norm weights, no rotation and a gate at +30 (sigmoid = 1 in fp32) the mixer is plain
    attention over rmsnorm(q) (scale folded into wq) with rmsnorm(k) appended; a gate of 0 halves it."""
    d = __import__("qwen36_state.workloads", fromlist=["x"]).attn_layer(2, 300, "cpu", seed=4, T=2, num_blocks=16)
    B, T = 2, 2
    wq = torch.full((256,), 1 / 16.0)
    wk = torch.ones(256)
    cos, sin = O.rope_tables(torch.zeros(B, T, dtype=torch.long))
    kc, vc = d["k_cache"].clone(), d["v_cache"].clone()
    gate = torch.full(d["q"].shape, 30.0).bfloat16()
    o = O.attn_mixer(d["q"], d["k_new"], d["v_new"], gate, wq, wk, cos, sin, kc, vc, d["block_table"],
                     d["seq_lens"])  # fmt: skip
    kn = O.bf16(O.rmsnorm(d["k_new"].float()))
    kc2, vc2 = d["k_cache"].clone(), d["v_cache"].clone()
    O.paged_append(kc2, vc2, kn.bfloat16(), d["v_new"], d["block_table"], d["seq_lens"] - T)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    ref = O.gqa_decode(O.rmsnorm(d["q"].float()), kc2, vc2, d["block_table"], d["seq_lens"], 1 / 16.0)
    torch.testing.assert_close(o, O.bf16(ref), rtol=0, atol=0)
    o0 = O.attn_mixer(d["q"], d["k_new"], d["v_new"], torch.zeros_like(gate), wq, wk, cos, sin, kc, vc,
                      d["block_table"], d["seq_lens"])  # fmt: skip
    torch.testing.assert_close(o0, O.bf16(ref * 0.5), rtol=0, atol=0)


def test_gdn_gated_norm_special_cases():
    """The reference's own prefill check (test_pp_kernels.py:181-194 pattern, w = 1): on = o rsqrt(mean o^2
    + eps), out = on silu(z); silu(0) = 0 zeroes the output, and a constant row normalises to +-1."""
    gen = torch.Generator().manual_seed(13)
    o = torch.randn(4, 128, generator=gen)
    z = torch.randn(4, 128, generator=gen).bfloat16()
    w = torch.ones(128)
    ref = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + 1e-6) * F.silu(z.float())
    torch.testing.assert_close(O.gdn_gated_norm(o, z, w), O.bf16(ref), rtol=0, atol=0)
    assert torch.equal(O.gdn_gated_norm(o, torch.zeros_like(z), w), torch.zeros(4, 128))
    c = torch.full((1, 128), -3.0)
    big = torch.full((1, 128), 30.0).bfloat16()  # silu(30) = 30 in fp32
    torch.testing.assert_close(O.gdn_gated_norm(c, big, w), O.bf16(torch.full((1, 128), -30.0 / math.sqrt(1 + 1e-6 / 9))))
