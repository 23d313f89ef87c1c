"""Invalid lengths, positions, block-table entries and accept lengths are reported in the caller's status word
instead of being masked, and the kernels handle them in their documented, bounded way (every kernel exits
normally): an idle slot (length below the step's rows) appends nothing and returns zeros; a length past the
block table is reported and treated like an idle slot; a table entry outside the pool is reported and not
attended; the length advance reports a length that runs past the table."""
import pytest
import torch
from conftest import assert_attn_output

from oracle import state_path as O
from qwen36_state import ops, workloads as W

pytestmark = pytest.mark.gpu


def to(d, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}


@pytest.mark.parametrize("T,pps", [(1, 2), (1, 1), (3, 4)])  # 10 splits merged in launch, 20 by the merge launch, verify rows
def test_idle_and_overlong_users(dev, T, pps):
    d = W.attn_layer(4, 20 * 64, "cpu", seed=3 + T, T=T, num_blocks=128)  # 20 pages per user
    d["seq_lens"] = torch.tensor([0, 700, 20 * 64 + 1, 300], dtype=torch.int32)  # idle, ok, past the table, ok
    g = to(d, dev)
    st = ops.Status(dev)
    o = ops.paged_gqa_decode(g["q"], g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"], d["scale"],
                             k_new=g["k_new"], v_new=g["v_new"], pages_per_split=pps, status=st.word)  # fmt: skip
    assert st.peek() == ops.STATUS_LENGTH
    with pytest.raises(ValueError, match="past its block table"):
        st.check()
    assert st.peek() == 0
    assert torch.count_nonzero(o[0]) == 0 and torch.count_nonzero(o[2]) == 0
    # the valid users match the oracle; only their rows were appended
    kc, vc = d["k_cache"].clone(), d["v_cache"].clone()
    ok = [1, 3]
    O.paged_append(kc, vc, d["k_new"][ok], d["v_new"][ok], d["block_table"][ok], d["seq_lens"][ok] - T)
    assert torch.equal(g["k_cache"].cpu(), kc) and torch.equal(g["v_cache"].cpu(), vc)
    ref = O.gqa_decode(d["q"][ok], kc, vc, d["block_table"][ok], d["seq_lens"][ok], d["scale"])
    assert_attn_output(o[ok], O.bf16(ref))


def test_bad_table_entry_reported(dev):
    d = W.attn_layer(2, 10 * 64, "cpu", seed=8, num_blocks=64)
    d["block_table"][1, 4] = 64  # one past the pool
    g = to(d, dev)
    st = ops.Status(dev)
    ops.paged_gqa_decode(g["q"], g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"], d["scale"],
                         k_new=g["k_new"], v_new=g["v_new"], pages_per_split=4, status=st.word)  # fmt: skip
    assert st.peek() == ops.STATUS_PAGE
    # the append alone reports it too when the new row's page is the bad one
    st.word.zero_()
    d["block_table"][0, 9] = -5
    g = to(d, dev)
    ops.paged_kv_append(g["k_new"], g["v_new"], g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"] - 1,
                        status=st.word)  # fmt: skip
    assert st.peek() == ops.STATUS_PAGE


@pytest.mark.parametrize("T", [1, 4])  # the one-token kernel and the verify kernel, both appending in the launch
def test_bad_entry_on_the_new_rows_page(dev, T):
    """A table entry outside the pool on the page that holds a user's new rows: reported, neither attended
    nor written (the user's new rows that land in valid pages still reach the pool, and no other page
    changes); the other user is untouched by it and matches the oracle."""
    d = W.attn_layer(2, 10 * 64 + 2, "cpu", seed=11 + T, T=T, num_blocks=64)  # 11 pages per user
    last = (int(d["seq_lens"][1]) - 1) // 64  # the page of user 1's last new row
    d["block_table"][1, last] = 64  # one past the pool
    g = to(d, dev)
    st = ops.Status(dev)
    o = ops.paged_gqa_decode(g["q"], g["k_cache"], g["v_cache"], g["block_table"], g["seq_lens"], d["scale"],
                             k_new=g["k_new"], v_new=g["v_new"], pages_per_split=2, status=st.word)  # fmt: skip
    assert st.peek() == ops.STATUS_PAGE
    kc, vc = d["k_cache"].clone(), d["v_cache"].clone()
    O.paged_append(kc, vc, d["k_new"][:1], d["v_new"][:1], d["block_table"][:1], d["seq_lens"][:1] - T)
    for t in range(T):  # user 1: only the rows whose page is in the pool
        pos = int(d["seq_lens"][1]) - T + t
        page = int(d["block_table"][1, pos // 64])
        if page < 64:
            kc[page, :, pos % 64] = d["k_new"][1, t]
            vc[page, :, pos % 64] = d["v_new"][1, t]
    assert torch.equal(g["k_cache"].cpu(), kc) and torch.equal(g["v_cache"].cpu(), vc)
    ref = O.gqa_decode(d["q"][:1], kc, vc, d["block_table"][:1], d["seq_lens"][:1], d["scale"])
    assert_attn_output(o[:1], O.bf16(ref))


def test_advance_lengths(dev):
    lens = torch.tensor([0, 4095, -1, 8191, 8190], dtype=torch.int32, device=dev)
    base = torch.empty_like(lens)
    st = ops.Status(dev)
    ops.advance_lengths(lens, 1, 8192, base_out=base, status=st.word)
    assert base.cpu().tolist() == [0, 4095, -1, 8191, 8190]
    assert lens.cpu().tolist() == [1, 4096, -1, 8192, 8191]
    assert st.peek() == 0
    ops.advance_lengths(lens, 2, 8192, status=st.word)  # 8192 + 2 and 8191 + 2 pass the table
    assert lens.cpu().tolist() == [3, 4098, -1, 8194, 8193]
    assert st.peek() == ops.STATUS_LENGTH


def test_accept_out_of_range_reported(dev):
    acc = torch.tensor([2, 0, 5], dtype=torch.int32, device=dev)
    slot = torch.full((3,), 9, dtype=torch.int32, device=dev)
    lens = torch.zeros(3, dtype=torch.int32, device=dev)
    base = torch.tensor([10, 20, 30], dtype=torch.int32, device=dev)
    st = ops.Status(dev)
    ops.verify_accept(acc, 4, slot, lens, base, status=st.word)
    assert slot.cpu().tolist() == [1, 9, 9] and lens.cpu().tolist() == [12, 0, 0]
    assert st.peek() == ops.STATUS_ACCEPT


def test_step_reports_running_past_the_table(dev):
    """A decode step whose users reach the end of their block table: the step after the last valid one
    reports QS_STATUS_LENGTH and leaves the pools' valid rows untouched."""
    from qwen36_state.decode import StatePathStep

    step = StatePathStep.synthetic(2, 128, layers=4, device=dev, num_blocks=64, check=True)  # 2 pages per user
    step.step()  # appends at 127: the last row of the table
    step.status.check()
    att = step.layer[3]
    pages = step.block_table.flatten().long()
    before = att["k_cache"][pages].clone()
    step.step()  # would append at 128
    assert step.status.peek() == ops.STATUS_LENGTH
    assert torch.equal(att["k_cache"][pages], before)
    assert torch.count_nonzero(att["o"]) == 0
