"""The batched 64-layer decode step (48 GDN + 16 attention layers, batch 8, 4096 positions): spot layers
against their own oracle calls, and HIP-graph replays bit-identical to the eager step (replayed several
times from a restored state, with eager work and synchronisation in between)."""
import pytest
import torch
from conftest import assert_bf16_output, assert_state

from oracle import state_path as O
from qwen36_state import ops
from qwen36_state.decode import StatePathStep

pytestmark = pytest.mark.gpu
NK, NV, DK, DV = 16, 48, 128, 128


@pytest.fixture(scope="module")
def step(dev):
    s = StatePathStep(8, 4096, 64, device=dev)
    yield s
    del s
    torch.cuda.empty_cache()


def test_step_layers_match_oracle(step, dev):
    gdn = {l: {k: v.clone() for k, v in step.layer[l].items() if torch.is_tensor(v)} for l in (0, 62)}
    cpu_in = {l: {k: v.cpu() for k, v in d.items()} for l, d in gdn.items()}
    att3 = {k: v.cpu() for k, v in step.layer[3].items() if torch.is_tensor(v)}
    step.step()
    torch.cuda.synchronize()
    for l, d in gdn.items():
        # the same launch on a copy, with the conv output exposed, reproduces the step's layer bit-exactly
        y = torch.empty_like(d["x"])
        o = ops.gdn_decode_fused(d["x"], d["conv_state"], d["taps"], d["g"], d["beta"], d["state"], y_out=y)
        L, c = step.layer[l], cpu_in[l]
        assert torch.equal(o, L["o"]) and torch.equal(d["state"], L["state"])
        assert torch.equal(d["conv_state"], L["conv_state"])
        _, cs = O.conv1d_update(c["x"], c["conv_state"], c["taps"])
        assert torch.equal(L["conv_state"].cpu().float(), cs)
        q, k, v = O.split_qkv(y.cpu().float(), NK, NV, DK, DV)
        o_ref, S_ref = O.gdn_step(q, k, v, c["g"], c["beta"], c["state"])
        assert_state(L["state"], S_ref)
        assert_bf16_output(L["o"], O.bf16(o_ref))
    # attention layer 3: append + attention over the shared block table
    kc, vc = att3["k_cache"], att3["v_cache"]
    O.paged_append(kc, vc, att3["k_new"], att3["v_new"], att3["block_table"], att3["seq_lens"] - 1)
    o_ref = O.gqa_decode(att3["q"], kc, vc, att3["block_table"], att3["seq_lens"], step.layer[3]["scale"])
    assert_bf16_output(step.layer[3]["o"], O.bf16(o_ref))
    rows = O.paged_gather(step.layer[3]["k_cache"].cpu(), att3["block_table"][5], 4096)[:, -1]
    assert torch.equal(rows, att3["k_new"][5, 0])


def test_graph_replay_equals_eager(step, dev):
    snap = step.snapshot()
    step.step()
    torch.cuda.synchronize()
    ref = [(d["o"].clone(), d["state"].clone() if not d["attn"] else None) for d in step.layer]
    step.capture()
    for rep in range(3):
        step.restore(snap)
        torch.cuda.synchronize()
        step.replay()
        torch.cuda.synchronize()
        for l, d in enumerate(step.layer):
            assert torch.equal(d["o"], ref[l][0]), (rep, l)
            if not d["attn"]:
                assert torch.equal(d["state"], ref[l][1]), (rep, l)
        _ = torch.randn(1024, device=dev).sum().item()  # eager work between replays


def test_verify_step_slots_equals_copy(dev):
    """Two consecutive MTP verify steps (8 layers, batch 2, T = 3): acceptance by slot selection gives the
    same outputs and accepted states as acceptance by copies."""
    from qwen36_state.decode import VerifyStep

    steps = {m: VerifyStep(2, 1024, T=3, layers=8, device=dev, rollback=m) for m in ("slots", "copy")}
    for k in range(2):
        for vs in steps.values():
            vs.verify()
            vs.rollback()
            vs.reset_lengths()
        torch.cuda.synchronize()
        a, c = steps["slots"], steps["copy"]
        for la, lc in zip(a.layer, c.layer):
            assert torch.equal(la["o"], lc["o"]), (k, "o")
        for gi in range(6):
            for b in range(2):
                sa, ca = a.state_of(gi, b)
                sc, cc = c.state_of(gi, b)
                assert torch.equal(sa, sc) and torch.equal(ca, cc), (k, gi, b)
