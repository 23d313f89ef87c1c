"""Whole steps of the 64-layer state path as they are benchmarked, every layer against its own oracle call:

- the decode step at batch 8, 4096 positions, 8 pages per split (the in-launch merge of 8 splits);
- three consecutive graph replays of a decode step whose positions cross a page boundary (4095, 4096,
  4097): each replay advances the positions on the device, and the oracle carries its own state, conv
  history and pools from step to step;
- the MTP verify step at batch 1, 8192 positions, T = 4, 2 pages per split, two steps in a row with the
  seeded acceptance (the pattern of tests/test_resident_verify.py:42-72);
- HIP-graph replays bit-identical to the eager step, and acceptance by slot selection equal to the copy
  rollback."""
import pytest
import torch
from stepcheck import OracleState, check_decode_step, check_verify_step, inputs_of

from qwen36_state.decode import StatePathStep, VerifyStep

pytestmark = pytest.mark.gpu


def test_decode_step_as_benched(dev):
    """StatePathStep(8, 4096, pps 8): all 48 GDN and 16 attention layers of one graph replay."""
    step = StatePathStep.synthetic(8, 4096, device=dev, pages_per_split=8, check=True)
    ref, inp = OracleState(step), inputs_of(step)
    step.capture()
    step.replay()
    torch.cuda.synchronize()
    step.status.check()
    check_decode_step(step, ref, inp)


def test_decode_steps_cross_a_page(dev):
    """Three graph replays from 4095 cached rows: the new rows land at positions 4095 (last row of page 63),
    4096 and 4097 (page 64); new inputs are written into the step's buffers between replays."""
    step = StatePathStep.synthetic(8, 4096, layers=8, device=dev, pages_per_split=4, max_blocks=68,
                                   num_blocks=640, check=True)  # fmt: skip
    step.capture()
    ref = OracleState(step)
    gen = torch.Generator().manual_seed(99)
    for k in range(3):
        assert int(step.lens[0]) == 4095 + k
        if k:
            for d in step.layer:
                for key in (("q", "k_new", "v_new") if d["attn"] else ("x",)):
                    d[key].copy_(torch.randn(d[key].shape, generator=gen).to(d[key].dtype))
        inp = inputs_of(step)
        step.replay()
        torch.cuda.synchronize()
        step.status.check()
        check_decode_step(step, ref, inp)


@pytest.mark.parametrize("steps,max_blocks", [(1, None), (2, 130)])
def test_verify_steps_as_benched(dev, steps, max_blocks):
    """VerifyStep(1, 8192, T 4, pps 2): all 64 layers of graph replays with the seeded acceptance. One step
    with the benchmark's 128-page table (64 splits); two steps in a row with a 130-page table (the second
    step's rows pass position 8191)."""
    vs = VerifyStep.synthetic(1, 8192, T=4, device=dev, pages_per_split=2, max_blocks=max_blocks, check=True)

    def cur(l):
        gi = vs.layer[l]["gi"]
        S, c = zip(*(vs.state_of(gi, b) for b in range(vs.B)))
        return torch.stack(S), torch.stack(c)

    ref = OracleState(vs, gdn_state_of=cur)
    vs.capture()
    for k in range(steps):
        inp = inputs_of(vs)
        vs.replay()
        torch.cuda.synchronize()
        vs.status.check()
        check_verify_step(vs, ref, inp, vs.accept.cpu())


def test_graph_replay_equals_eager(dev):
    step = StatePathStep.synthetic(8, 4096, layers=16, device=dev, pages_per_split=4)
    snap = step.snapshot()
    step.step()
    torch.cuda.synchronize()
    ref = [(d["o"].clone(), d["state"].clone() if not d["attn"] else None) for d in step.layer]
    lens_after = step.lens.clone()
    step.capture()
    for rep in range(3):
        step.restore(snap)
        torch.cuda.synchronize()
        step.replay()
        torch.cuda.synchronize()
        assert torch.equal(step.lens, lens_after)
        for l, d in enumerate(step.layer):
            assert torch.equal(d["o"], ref[l][0]), (rep, l)
            if not d["attn"]:
                assert torch.equal(d["state"], ref[l][1]), (rep, l)
        _ = torch.randn(1024, device=dev).sum().item()  # eager work between replays


def test_verify_step_slots_equals_copy(dev):
    """Two consecutive MTP verify steps (8 layers, batch 2, T = 3): acceptance by slot selection gives the
    same outputs, accepted states and lengths as acceptance by copies."""
    steps = {m: VerifyStep.synthetic(2, 1024, T=3, layers=8, device=dev, rollback=m, max_blocks=20, num_blocks=64)
             for m in ("slots", "copy")}  # fmt: skip
    for k in range(2):
        for vs in steps.values():
            vs.step()
        torch.cuda.synchronize()
        a, c = steps["slots"], steps["copy"]
        assert torch.equal(a.lens, c.lens)
        for la, lc in zip(a.layer, c.layer):
            assert torch.equal(la["o"], lc["o"]), (k, "o")
        for gi in range(6):
            for b in range(2):
                sa, ca = a.state_of(gi, b)
                sc, cc = c.state_of(gi, b)
                assert torch.equal(sa, sc) and torch.equal(ca, cc), (k, gi, b)


@pytest.mark.parametrize("B", [3, 8])
@pytest.mark.parametrize("mode", ["slots", "copy"])
def test_verify_step_idle_user(dev, mode, B):
    """Two verify steps (8 layers, T = 3; batch 3: a slab's rows over 4 waves, batch 8: one wave per slab) with
    user 1 an idle slot (lens -1): its length, its current state and conv history and its pages stay as they
    were whatever its accept length, and users 0 and 2 get bit for bit what they get in the same step with
    every user active."""
    mk = lambda: VerifyStep.synthetic(B, 1024, T=3, layers=8, device=dev, rollback=mode, max_blocks=20,  # noqa: E731
                                      num_blocks=20 * B, check=True)  # fmt: skip
    act, idle = mk(), mk()
    idle.lens[1] = -1
    n_gdn = sum(not d["attn"] for d in idle.layer)
    before = [tuple(t.clone() for t in idle.state_of(gi, 1)) for gi in range(n_gdn)]
    pages = idle.block_table[1].long()
    pools = [(d["k_cache"][pages].clone(), d["v_cache"][pages].clone()) for d in idle.layer if d["attn"]]
    for k in range(2):
        act.step()
        idle.step()
        torch.cuda.synchronize()
        idle.status.check()
        assert int(idle.lens[1]) == -1, k
        assert torch.equal(idle.lens[[0, 2]], act.lens[[0, 2]]), k
        for la, li in zip(act.layer, idle.layer):
            assert torch.equal(la["o"][[0, 2]], li["o"][[0, 2]]), (k, "o")
        for gi in range(n_gdn):
            for b in (0, 2):
                sa, ca = act.state_of(gi, b)
                si, ci = idle.state_of(gi, b)
                assert torch.equal(sa, si) and torch.equal(ca, ci), (k, gi, b)
            S1, c1 = idle.state_of(gi, 1)
            assert torch.equal(S1, before[gi][0]) and torch.equal(c1, before[gi][1]), (k, gi, "idle state")
        for (kc, vc), d in zip(pools, (d for d in idle.layer if d["attn"])):
            assert torch.equal(d["k_cache"][pages], kc) and torch.equal(d["v_cache"][pages], vc), (k, "idle pages")
