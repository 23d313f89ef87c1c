"""Prefill -> decode handoff on the GPU, in the pattern of the reference's handoff test
(tests/test_pp_kernels.py:197-236: GDN states, conv histories and KV caches moved into the decode's layouts,
bit-exact). Here the decode reads the prefill's paged pools directly and the prompt's GDN state and conv
carry are written straight into the user's slot of the batched decode state, so the handoff moves nothing;
the paged <-> row conversion (fill and its inverse, the gather) is bit-exact both ways. Tolerances: pools,
rows, conv states and other users' results bit-exact; the prompt user's fp32 state rtol 1e-4 and o rtol 2e-2
against token-by-token decode."""
import pytest
import torch
from conftest import assert_bf16_output, assert_prefill_state

from oracle import state_path as O
from qwen36_state import ops, workloads as W

pytestmark = pytest.mark.gpu
NK, NV, DK, DV = 16, 48, 128, 128
NKV, NQ, HD, BLOCK = 4, 24, 256, 64
C = W.C_QKV


def pools(nb, dev, seed):
    gen = torch.Generator().manual_seed(seed)
    kc = W._randn((nb, NKV, BLOCK, HD), gen, "cpu", torch.bfloat16).to(dev)
    return kc, W._randn((nb, NKV, BLOCK, HD), gen, "cpu", torch.bfloat16).to(dev)


@pytest.mark.parametrize("T,start", [(1000, 0), (77, 37), (1, 63)])
def test_gather_inverts_fill(dev, T, start):
    """Rows filled into a sequence's pages come back unchanged through the gather; the gather of positions
    0 .. n-1 equals the oracle's export gather (prefill/pp_prefill.py:1241-1249)."""
    kc, vc = pools(64, dev, seed=T)
    gen = torch.Generator().manual_seed(T + 1)
    table = torch.randperm(64, generator=gen)[: (start + T + BLOCK - 1) // BLOCK].int().to(dev)
    k = W._randn((NKV, T, HD), gen, "cpu", torch.bfloat16).to(dev)
    v = W._randn((NKV, T, HD), gen, "cpu", torch.bfloat16).to(dev)
    ops.paged_kv_fill(k, v, kc, vc, table, start=start)
    k2, v2 = ops.paged_kv_gather(kc, vc, table, T, start=start)
    assert torch.equal(k2, k) and torch.equal(v2, v)
    n = start + T
    k3, v3 = ops.paged_kv_gather(kc, vc, table, n)
    assert torch.equal(k3.cpu(), O.paged_gather(kc.cpu(), table.cpu(), n))
    assert torch.equal(v3.cpu(), O.paged_gather(vc.cpu(), table.cpu(), n))


def test_gather_out_of_range_page_reads_zeros(dev):
    kc, vc = pools(16, dev, seed=3)
    table = torch.tensor([5, -1, 99, 2], dtype=torch.int32, device=dev)
    k, v = ops.paged_kv_gather(kc, vc, table, 4 * BLOCK)
    assert torch.equal(k[:, :BLOCK], kc[5]) and torch.equal(v[:, 3 * BLOCK :], vc[2])
    assert not k[:, BLOCK : 3 * BLOCK].any() and not v[:, BLOCK : 3 * BLOCK].any()


def test_prompt_handoff_into_a_batch_slot(dev):
    """User 1 of a batch of 3 takes a 100-token prompt: the prompt conv writes its carry into conv_state[1],
    the chunked delta rule its final state into state[1], the paged fill its K/V into its pages. One batched
    decode step then runs every user. User 1 matches 101 token-by-token decode steps; users 0 and 2 match the
    same decode step without the prompt, bit for bit; the pools equal those of 100 decode appends."""
    B, u, T = 3, 1, 100
    gen = torch.Generator().manual_seed(40)
    rnd = lambda shape, dt=torch.bfloat16, std=1.0: W._randn(shape, gen, "cpu", dt, std).to(dev)
    taps = rnd((C, 4), std=0.5)
    state, conv_state = rnd((B, NV, DK, DV), torch.float32, 0.02), rnd((B, C, 3))
    S0 = rnd((NV, DK, DV), torch.float32, 0.02)
    xp = rnd((T + 1, C))
    g, beta = (t.to(dev) for t in W.gates(T + 1, gen, "cpu"))
    x_dec = rnd((B, C))
    x_dec[u] = xp[T]
    g_dec, beta_dec = (t.to(dev) for t in W.gates(B, gen, "cpu"))
    g_dec[u], beta_dec[u] = g[T], beta[T]

    # attention layer: users 0 and 2 hold 200 and 300 positions, user 1 gets the prompt's K/V
    kc, vc = pools(32, dev, seed=41)
    table = torch.randperm(32, generator=gen)[: B * 8].reshape(B, 8).int().to(dev)
    kp, vp = rnd((NKV, T, HD)), rnd((NKV, T, HD))
    q, k_new, v_new = rnd((B, 1, NQ, HD)), rnd((B, 1, NKV, HD)), rnd((B, 1, NKV, HD))
    seq_lens = torch.tensor([201, T + 1, 301], dtype=torch.int32, device=dev)

    # the same step without the prompt (users 0 and 2), and user 1 token by token
    st_ref, cs_ref = state.clone(), conv_state.clone()
    o_ref = ops.gdn_decode_fused(x_dec, cs_ref, taps, g_dec, beta_dec, st_ref)
    s1, c1 = S0[None].clone(), torch.zeros(1, C, 3, dtype=torch.bfloat16, device=dev)
    for t in range(T + 1):
        o1 = ops.gdn_decode_fused(xp[t : t + 1].contiguous(), c1, taps, g[t : t + 1].contiguous(),
                                  beta[t : t + 1].contiguous(), s1)  # fmt: skip
    kc_ref, vc_ref = kc.clone(), vc.clone()
    for t in range(T):
        ops.paged_kv_append(kp[:, t][None, None].contiguous(), vp[:, t][None, None].contiguous(), kc_ref, vc_ref,
                            table[u : u + 1].contiguous(), torch.tensor([t], dtype=torch.int32, device=dev))  # fmt: skip

    # the handoff: prompt results land in user 1's slots, then one batched decode step
    qq, kk, vv, _ = ops.causal_conv1d_prefill(xp[:T], taps, None, conv_state_out=conv_state[u])
    ops.chunk_gated_delta_rule(qq, kk, vv, g[:T], beta[:T], initial_state=S0, final_state=state[u])
    ops.paged_kv_fill(kp, vp, kc, vc, table[u].contiguous())
    assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref)
    o = ops.gdn_decode_fused(x_dec, conv_state, taps, g_dec, beta_dec, state)
    ao = ops.paged_gqa_decode(q, kc, vc, table, seq_lens, 1 / 16, k_new=k_new, v_new=v_new, pages_per_split=2)
    ao_ref = ops.paged_gqa_decode(q, kc_ref, vc_ref, table, seq_lens, 1 / 16, k_new=k_new, v_new=v_new,
                                  pages_per_split=2)  # fmt: skip
    torch.cuda.synchronize()

    for b in (0, 2):
        assert torch.equal(state[b], st_ref[b]) and torch.equal(conv_state[b], cs_ref[b])
        assert torch.equal(o[b], o_ref[b])
    assert torch.equal(conv_state[u], c1[0])
    assert_prefill_state(state[u], s1[0].cpu())
    assert_bf16_output(o[u], o1[0].cpu())
    assert torch.equal(ao, ao_ref) and torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref)
    krow, vrow = ops.paged_kv_gather(kc, vc, table[u].contiguous(), T + 1)
    assert torch.equal(krow[:, :T], kp) and torch.equal(krow[:, T], k_new[u, 0])
    assert torch.equal(vrow[:, :T], vp) and torch.equal(vrow[:, T], v_new[u, 0])
