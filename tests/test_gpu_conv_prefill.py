"""The prompt conv with its carry (causal conv1d + SiLU over T tokens, the decode conv state handed over)
on the GPU. Bit-exact against T successive decode conv launches (same tap-sum order), carry bit-exact,
outputs within one bf16 ulp of the oracle (SiLU's exp differs in the last fp32 bit between libraries);
the end-to-end prompt -> decode handoff holds the fp32 state to rtol 1e-4 and o to the bf16 rtol 2e-2."""
import pytest
import torch
from conftest import assert_bf16_output, assert_prefill_state, bf16_ulp_mismatch

from oracle import state_path as O
from qwen36_state import ops, workloads as W

pytestmark = pytest.mark.gpu
NK, NV, DK, DV = 16, 48, 128, 128
C = W.C_QKV
EXTRA = 64  # projection columns after the conv channels (x is read with a row stride of C + EXTRA)


def prompt(T, seed):
    gen = torch.Generator().manual_seed(seed)
    xp = W._randn((T, C + EXTRA), gen, "cpu", torch.bfloat16)
    cs = W._randn((C, 3), gen, "cpu", torch.bfloat16)
    taps = W._randn((C, 4), gen, "cpu", torch.bfloat16, std=0.5)
    return xp, cs, taps


def qkv_cat(q, k, v):
    T = q.shape[0]
    return torch.cat([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], dim=1)


@pytest.mark.parametrize("T", [0, 1, 2, 3, 17, 100])
def test_conv_prefill_equals_decode_steps(dev, T):
    """y of the prompt conv = y of T decode conv launches from the same carry, bit for bit; the carry it
    leaves is the decode conv state those launches leave (the reference checks new carry == the 3 inputs
    ending at the last valid row, tests/test_pp_kernels.py:137-142)."""
    xp, cs, taps = prompt(T, seed=T)
    xg, csg, tg = xp.to(dev), cs.to(dev), taps.to(dev)
    q, k, v, cs_out = ops.causal_conv1d_prefill(xg[:, :C] if T else xg, tg, csg)
    st = csg[None].clone()
    ys = [ops.causal_conv1d_update(xg[t : t + 1, :C].contiguous(), st, tg) for t in range(T)]
    torch.cuda.synchronize()
    assert torch.equal(cs_out.cpu(), st[0].cpu())
    if T:
        assert torch.equal(qkv_cat(q, k, v).cpu(), torch.cat(ys).cpu())
    y_ref, cs_ref = O.conv1d_prefill(xp[:, :C].float(), cs.float(), taps.float())
    assert torch.equal(cs_out.cpu().float(), cs_ref)
    if T:
        ulps, frac = bf16_ulp_mismatch(qkv_cat(q, k, v), y_ref)
        assert ulps <= 1 and frac < 1e-3, (ulps, frac)


def test_conv_prefill_fresh_in_place_and_split(dev):
    """No carry is a zero carry; the carry may be updated in place; a prompt conv in three pieces, each from
    the previous piece's carry, equals the conv of the whole prompt."""
    xp, cs, taps = prompt(77, seed=5)
    xg, tg = xp.to(dev)[:, :C], taps.to(dev)
    q, k, v, whole = ops.causal_conv1d_prefill(xg, tg)
    q0, k0, v0, whole0 = ops.causal_conv1d_prefill(xg, tg, torch.zeros(C, 3, dtype=torch.bfloat16, device=dev))
    assert torch.equal(qkv_cat(q, k, v), qkv_cat(q0, k0, v0)) and torch.equal(whole, whole0)
    carry = torch.zeros(C, 3, dtype=torch.bfloat16, device=dev)
    parts = []
    for lo, hi in ((0, 2), (2, 35), (35, 77)):
        pq, pk, pv, out = ops.causal_conv1d_prefill(xg[lo:hi], tg, carry, conv_state_out=carry)
        assert out is carry
        parts.append(qkv_cat(pq, pk, pv))
    assert torch.equal(torch.cat(parts), qkv_cat(q, k, v))
    assert torch.equal(carry, whole)
    assert torch.equal(whole, xg[-3:].t())


def test_conv_prefill_8192_tokens(dev):
    """The prompt length of the prefill workload: 8192 tokens of the 10240 q | k | v channels."""
    T = 8192
    xp, cs, taps = prompt(T, seed=11)
    q, k, v, cs_out = ops.causal_conv1d_prefill(xp.to(dev)[:, :C], taps.to(dev), cs.to(dev))
    y_ref, cs_ref = O.conv1d_prefill(xp[:, :C].float(), cs.float(), taps.float())
    assert torch.equal(cs_out.cpu().float(), cs_ref)
    ulps, frac = bf16_ulp_mismatch(qkv_cat(q, k, v), y_ref)
    assert ulps <= 1 and frac < 1e-3, (ulps, frac)


def test_prompt_then_decode_equals_token_by_token(dev):
    """The prefill -> decode handoff end to end: prompt conv + chunked delta rule over T tokens, then one
    fused decode step from the handed-over conv state and GDN state, equals T + 1 fused decode steps from
    the start (conv state bit-exact, fp32 state and o to their tolerances)."""
    T = 150
    gen = torch.Generator().manual_seed(21)
    xp = W._randn((T + 1, C), gen, "cpu", torch.bfloat16).to(dev)
    taps = W._randn((C, 4), gen, "cpu", torch.bfloat16, std=0.5).to(dev)
    g, beta = W.gates(T + 1, gen, "cpu")
    g, beta = g.to(dev), beta.to(dev)
    S0 = W._randn((NV, DK, DV), gen, "cpu", std=0.02).to(dev)

    q, k, v, carry = ops.causal_conv1d_prefill(xp[:T], taps)
    _, S = ops.chunk_gated_delta_rule(q, k, v, g[:T], beta[:T], initial_state=S0)
    conv_state, state = carry[None].clone(), S[None].clone()
    o = ops.gdn_decode_fused(xp[T : T + 1].contiguous(), conv_state, taps, g[T : T + 1].contiguous(),
                             beta[T : T + 1].contiguous(), state)  # fmt: skip

    conv_ref = torch.zeros(1, C, 3, dtype=torch.bfloat16, device=dev)
    state_ref = S0[None].clone()
    for t in range(T + 1):
        o_ref = ops.gdn_decode_fused(xp[t : t + 1].contiguous(), conv_ref, taps, g[t : t + 1].contiguous(),
                                     beta[t : t + 1].contiguous(), state_ref)  # fmt: skip
        if t == T - 1:
            assert torch.equal(conv_ref[0], carry)
    torch.cuda.synchronize()
    assert torch.equal(conv_state, conv_ref)
    assert_prefill_state(state, state_ref.cpu())
    assert_bf16_output(o, o_ref.cpu())


def test_conv_prefill_other_head_counts(dev):
    """2 key / 6 value heads (q, k 256 channels each, v 768): the q | k | v split follows the head counts;
    outputs and carry equal 33 decode conv launches bit for bit."""
    nk, nv, T = 2, 6, 33
    Cs = 2 * nk * DK + nv * DV
    gen = torch.Generator().manual_seed(77)
    xp = W._randn((T, Cs + 16), gen, "cpu", torch.bfloat16).to(dev)
    cs = W._randn((Cs, 3), gen, "cpu", torch.bfloat16).to(dev)
    taps = W._randn((Cs, 4), gen, "cpu", torch.bfloat16, std=0.5).to(dev)
    q, k, v, out = ops.causal_conv1d_prefill(xp[:, :Cs], taps, cs, nk=nk, nv=nv)
    assert q.shape == (T, nk, DK) and v.shape == (T, nv, DV)
    st = cs[None].clone()
    ys = torch.cat([ops.causal_conv1d_update(xp[t : t + 1, :Cs].contiguous(), st, taps) for t in range(T)])
    assert torch.equal(qkv_cat(q, k, v), ys) and torch.equal(out, st[0])
