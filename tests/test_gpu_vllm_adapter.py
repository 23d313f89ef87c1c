"""The vLLM-facing adapter of the state path against the oracle, with random vLLM-style page tables (each user a
random set of blocks of a shared pool): two prompts prefilled into decode slots 0 and 2 (slot 1 idle), then
three decode steps of the batch. Checked at every call: the pools on every page bit-exact against the index
oracle's fill and appends; the prompt's conv carry bit-exact against the oracle's prompt conv; the prompt's
GDN state against the sequential recurrence (prefill tolerance) from the kernel's own conv outputs; the decode
steps against the oracle's decode from the raw projection slice (in the two stages of the fused GDN tests: the
conv output within one ulp, then every state against the oracle's delta rule driven by the kernel's conv
output); the idle slot untouched bit for bit; a position past max_seq_len rejected."""
import pytest
import torch
from conftest import (
    assert_attn_output,
    assert_bf16_output,
    assert_prefill_state,
    assert_state,
    conv_mismatch_heads,
    perturbed_ok,
)

from oracle import state_path as O
from qwen36_state import ops
from qwen36_state.vllm_adapter import StatePathAdapter
from qwen36_state.workloads import C_QKV

pytestmark = pytest.mark.gpu
NK, NV, DK, DV, NKV, HD, NQ = 16, 48, 128, 128, 4, 256, 24
LAYERS, B, MAX_LEN, NUM_BLOCKS = 4, 3, 512, 40  # layers 0-2 GDN, 3 attention; 8 blocks per user


def prompt_inputs(T, gen):
    out = []
    for l in range(LAYERS):
        if (l + 1) % 4 == 0:
            out.append(dict(k=torch.randn(NKV, T, HD, generator=gen).bfloat16(),
                            v=torch.randn(NKV, T, HD, generator=gen).bfloat16()))  # fmt: skip
        else:
            g = -torch.nn.functional.softplus(torch.randn(T, NV, generator=gen)) * torch.exp(-3 * torch.rand(T, NV, generator=gen))
            out.append(dict(x=torch.randn(T, C_QKV + 64, generator=gen).bfloat16(), g=g,
                            beta=torch.sigmoid(torch.randn(T, NV, generator=gen))))  # fmt: skip
    return out


def decode_inputs(gen):
    out = []
    for l in range(LAYERS):
        if (l + 1) % 4 == 0:
            out.append(dict(q=torch.randn(B, 1, NQ, HD, generator=gen).bfloat16(),
                            k_new=torch.randn(B, 1, NKV, HD, generator=gen).bfloat16(),
                            v_new=torch.randn(B, 1, NKV, HD, generator=gen).bfloat16()))  # fmt: skip
        else:
            g = -torch.nn.functional.softplus(torch.randn(B, NV, generator=gen)) * torch.exp(-3 * torch.rand(B, NV, generator=gen))
            out.append(dict(x=torch.randn(B, C_QKV, generator=gen).bfloat16(), g=g,
                            beta=torch.sigmoid(torch.randn(B, NV, generator=gen))))  # fmt: skip
    return out


def to(xs, dev):
    return [{k: v.to(dev) for k, v in x.items()} for x in xs]


class Ref:
    """The oracle's copy of the adapter's state: the whole pools, per GDN layer the slots' states and conv
    histories, the slots' lengths."""

    def __init__(self, ad):
        z = lambda: torch.zeros(NUM_BLOCKS, NKV, 64, HD, dtype=torch.bfloat16)  # noqa: E731
        self.kc, self.vc = z(), z()
        self.S = {l: torch.zeros(B, NV, DK, DV) for l in range(3)}
        self.cs = {l: torch.zeros(B, C_QKV, 3) for l in range(3)}
        self.lens = [-1] * B
        self.taps = [t.cpu() for t in ad.taps]


def prefill_two(dev, ad, kv, gen, tables):
    """Prompts of 100 and 37 tokens into slots 0 and 2 (slot 1 idle), checked against the oracle."""
    ref = Ref(ad)
    for slot, T in ((0, 100), (2, 37)):
        inp = prompt_inputs(T, gen)
        outs = ad.prefill_forward(to(inp, dev), tables[slot : slot + 1], kv, torch.tensor([T]), slot=slot)
        O.paged_fill(ref.kc, inp[3]["k"], tables[slot])
        O.paged_fill(ref.vc, inp[3]["v"], tables[slot])
        for l in range(3):
            x = inp[l]
            y_ref, carry = O.conv1d_prefill(x["x"][:, :C_QKV].float(), None, ref.taps[l].float())
            assert torch.equal(ad.conv_state[l, slot].cpu().float(), carry), (slot, l)
            ref.cs[l][slot] = carry
            # the state from the kernel's own conv outputs (their parity with the oracle is the conv tests')
            q, k, v, _ = ops.causal_conv1d_prefill(x["x"].to(dev), ad.taps[l])
            o_ref, S_ref = O.gdn_chunk_prefill(q.cpu().float(), k.cpu().float(), v.cpu().float(), x["g"], x["beta"],
                                               torch.zeros(NV, DK, DV))  # fmt: skip
            assert_prefill_state(ad.gdn_state[l, slot], S_ref)
            assert_bf16_output(outs[l], O.bf16(o_ref))
            ref.S[l][slot] = ad.gdn_state[l, slot].cpu()  # continue from the kernel's prompt state
        ref.lens[slot] = T
    assert torch.equal(kv[0][0].cpu(), ref.kc) and torch.equal(kv[0][1].cpu(), ref.vc)
    return ref


def check_decode(dev, ad, kv, ref, inp, outs, tables, gdn=None, conv=None):
    """One decode step's outputs (and, given, the GDN states / conv histories after it) against the oracle
    stepped from ``ref`` with the inputs ``inp``; advances ``ref``."""
    gdn = ad.gdn_state.cpu() if gdn is None else gdn
    conv = ad.conv_state.cpu() if conv is None else conv
    active = [b for b in range(B) if ref.lens[b] >= 0]
    for l in range(3):
        x = inp[l]
        o_ref, S2, cs2, y_ref = O.gdn_decode(x["x"][active].float(), ref.cs[l][active], ref.taps[l].float(),
                                             x["g"][active], x["beta"][active], ref.S[l][active], NK, NV, DK, DV)  # fmt: skip
        assert torch.equal(conv[l][active].float(), cs2), l
        y_k = ops.causal_conv1d_update(x["x"][active].to(dev), ref.cs[l][active].bfloat16().to(dev), ad.taps[l]).cpu()
        pert = conv_mismatch_heads(y_k, y_ref, NK, NV)
        assert perturbed_ok(pert)
        q, k, v = O.split_qkv(y_k.float(), NK, NV, DK, DV)
        o_y, S_y = O.gdn_step(q, k, v, x["g"][active], x["beta"][active], ref.S[l][active])
        assert torch.equal(S_y[~pert], S2[~pert]), l
        assert_state(gdn[l][active], S_y)
        assert_bf16_output(outs[l][active], O.bf16(o_y))
        ref.S[l][active], ref.cs[l][active] = S_y, cs2
    a = inp[3]
    pos_a = torch.tensor([ref.lens[b] for b in active], dtype=torch.int32)
    O.paged_append(ref.kc, ref.vc, a["k_new"][active], a["v_new"][active], tables[active], pos_a)
    o_ref = O.gqa_decode(a["q"][active], ref.kc, ref.vc, tables[active], pos_a + 1, HD**-0.5)
    assert_attn_output(outs[3][active], O.bf16(o_ref))
    assert torch.count_nonzero(outs[3][1]) == 0  # the idle slot's attention output is zero
    ref.lens = [p + 1 if p >= 0 else p for p in ref.lens]


def test_vllm_adapter_prefill_then_decode(dev):
    gen = torch.Generator().manual_seed(2024)
    ad = StatePathAdapter(B, MAX_LEN, layers=LAYERS, device=dev)
    kv = ad.allocate_kv_cache((NUM_BLOCKS, NKV, 64, HD), torch.bfloat16, 1)
    perm = torch.randperm(NUM_BLOCKS, generator=gen).to(torch.int32)
    tables = perm[: B * 8].view(B, 8)  # vLLM-style: each slot a random set of blocks
    ref = prefill_two(dev, ad, kv, gen, tables)
    idle_state = (ad.gdn_state[:, 1].clone(), ad.conv_state[:, 1].clone())
    for step in range(3):
        inp = decode_inputs(gen)
        pos = torch.tensor(ref.lens, dtype=torch.int32)
        outs = ad.decode_forward(to(inp, dev), pos, tables, reload_page_table=True, read_from_device=True)
        check_decode(dev, ad, kv, ref, inp, outs, tables)
        assert torch.equal(kv[0][0].cpu(), ref.kc) and torch.equal(kv[0][1].cpu(), ref.vc), step
        assert torch.equal(ad.gdn_state[:, 1], idle_state[0]) and torch.equal(ad.conv_state[:, 1], idle_state[1])
        assert ad.lens.cpu().tolist() == ref.lens

    with pytest.raises(ValueError, match="max_seq_len"):
        ad.decode_forward(to(decode_inputs(gen), dev), torch.tensor([MAX_LEN, -1, 40], dtype=torch.int32))


def test_vllm_adapter_async_decode(dev):
    """Three decode_forward calls queued with no host synchronisation between them (torch's sync debug mode
    raises on any), as the reference's asynchronous steps with late reads (generator_vllm.py:117-160): the
    first reloads positions and the page table from the host, the second copies its inputs in, the third
    takes inputs the caller wrote into the step's own buffers (reload_inputs=False) and the positions the
    device advanced to.
    Each step's outputs, states and conv histories (device copies made in stream order) match the oracle."""
    gen = torch.Generator().manual_seed(77)
    ad = StatePathAdapter(B, MAX_LEN, layers=LAYERS, device=dev)
    kv = ad.allocate_kv_cache((NUM_BLOCKS, NKV, 64, HD), torch.bfloat16, 1)
    tables = torch.randperm(NUM_BLOCKS, generator=gen).to(torch.int32)[: B * 6].view(B, 6)
    ref = prefill_two(dev, ad, kv, gen, tables)
    inps = [decode_inputs(gen) for _ in range(3)]
    dev_inps = [to(x, dev) for x in inps]
    pos = torch.tensor(ref.lens, dtype=torch.int32).pin_memory()
    torch.cuda.synchronize()
    snaps = []
    torch.cuda.set_sync_debug_mode("error")
    try:
        for k in range(3):
            if k == 0:
                outs = ad.decode_forward(dev_inps[0], pos, tables.pin_memory(), reload_page_table=True)
            elif k == 1:
                pos1 = torch.tensor([p + 1 if p >= 0 else p for p in ref.lens], dtype=torch.int32)
                outs = ad.decode_forward(dev_inps[1], pos1)
            else:
                for dst, src in zip(ad.step_inputs(), dev_inps[2]):
                    for key, t in dst.items():
                        t.copy_(src[key], non_blocking=True)
                outs = ad.decode_forward(None, None, reload_inputs=False)
            snaps.append(([o.clone() for o in outs], ad.gdn_state.clone(), ad.conv_state.clone()))
    finally:
        torch.cuda.set_sync_debug_mode("default")
    ad.read_decode_output()
    for k in range(3):
        outs, gdn, conv = snaps[k]
        check_decode(dev, ad, kv, ref, inps[k], [o.cpu() for o in outs], tables, gdn.cpu(), conv.cpu())
    assert ad.lens.cpu().tolist() == ref.lens
    assert torch.equal(kv[0][0].cpu(), ref.kc) and torch.equal(kv[0][1].cpu(), ref.vc)


def test_vllm_adapter_rejects_bad_calls(dev):
    ad = StatePathAdapter(2, 256, layers=4, device=dev)
    with pytest.raises(ValueError, match="allocate_kv_cache"):
        ad.decode_forward([], torch.tensor([0, 0]))
    with pytest.raises(ValueError, match="kv_cache_shape"):
        ad.allocate_kv_cache((16, 4, 32, 256), torch.bfloat16, 1)
    with pytest.raises(ValueError, match="attention layers"):
        ad.allocate_kv_cache((16, 4, 64, 256), torch.bfloat16, 2)
    kv = ad.allocate_kv_cache((16, 4, 64, 256), torch.bfloat16, 1)
    with pytest.raises(ValueError, match="one user"):
        ad.prefill_forward([], torch.zeros(2, 4, dtype=torch.int32), kv, torch.tensor([10]))
    with pytest.raises(ValueError, match="blocks"):
        ad.prefill_forward([], torch.zeros(1, 1, dtype=torch.int32), kv, torch.tensor([100]))
    # a page table one block short of the new token's position: the entry past it is -1, so the row is neither
    # written nor attended and the step reports it
    gen = torch.Generator().manual_seed(5)
    ad.prefill_forward(to(prompt_inputs(64, gen), dev), torch.tensor([[3]], dtype=torch.int32), kv, torch.tensor([64]))
    before = (kv[0][0].clone(), kv[0][1].clone())
    inp = [{k: v[:2] for k, v in x.items()} for x in decode_inputs(gen)]
    with pytest.raises(ValueError, match="outside the KV pool"):
        ad.decode_forward(to(inp, dev), torch.tensor([64, -1], dtype=torch.int32), torch.tensor([[3], [5]], dtype=torch.int32),
                          reload_page_table=True, read_from_device=True)  # fmt: skip
    assert torch.equal(kv[0][0], before[0]) and torch.equal(kv[0][1], before[1])
