"""The fused GDN decode and verify from the raw projection slice x, checked end to end against the oracle run
from the same x (conv update, split, L2 norms, gates as given, delta rule): nothing of the kernel's own
output is fed back into the reference.

The conv outputs y (bf16) agree with the oracle's bit for bit except where SiLU's fp32 value sits within an
ulp of a bf16 rounding boundary; there the exponential's last bit decides, and it differs between libraries.
So the check has two stages: y against the oracle's (at most one ulp apart, and the value heads whose q, k or
v channels differ at most 6, or 2% of the heads), then every head's state against the oracle's delta rule
(L2 norms, gates as given) driven by the kernel's y, at the fp32 state tolerance (rtol 1e-4), and o at rtol
2e-2. For every head whose inputs agree that reference equals the oracle's own from x bit for bit, which the
tests assert. A negative control (the reference's own, tests/test_resident_verify.py:47-51) shows the state
check fails when a token's dependency on the previous token is dropped."""
import pytest
import torch
from conftest import assert_bf16_output, assert_state, bf16_ulp_mismatch, conv_mismatch_heads, perturbed_ok

from oracle import state_path as O
from qwen36_state import ops, workloads as W

pytestmark = pytest.mark.gpu
DK = DV = 128


def layer(B, nk, nv, seed, T=None):
    """Seeded GDN inputs for nk key / nv value heads (the distributions of the workloads module)."""
    gen = torch.Generator().manual_seed(seed)
    C = 2 * nk * DK + nv * DV
    xs = (B, C) if T is None else (B, T, C)
    gs = (B, nv) if T is None else (B, T, nv)
    g = -torch.nn.functional.softplus(torch.randn(gs, generator=gen)) * torch.exp(-3 * torch.rand(gs, generator=gen))
    return dict(
        state=0.02 * torch.randn(B, nv, DK, DV, generator=gen),
        conv_state=torch.randn(B, C, 3, generator=gen).bfloat16(),
        taps=(0.5 * torch.randn(C, 4, generator=gen)).bfloat16(),
        x=torch.randn(xs, generator=gen).bfloat16(),
        g=g,
        beta=torch.sigmoid(torch.randn(gs, generator=gen)),
    )


def from_y(y, g, beta, S, nk, nv):
    """The oracle's delta rule driven by the kernel's conv output y [B, C]: (o, S')."""
    q, k, v = O.split_qkv(y.cpu().float(), nk, nv, DK, DV)
    return O.gdn_step(q, k, v, g, beta, S)


def check_state(got, S_y, S_x, pert):
    """Every head against the oracle from the kernel's y; the heads whose inputs agree also equal the oracle's
    own from x bit for bit. got, S_y, S_x [B, nv, DK, DV]; pert [B, nv] bool."""
    assert perturbed_ok(pert), int(pert.sum())
    assert torch.equal(S_y[~pert], S_x[~pert])
    assert_state(got, S_y)


@pytest.mark.parametrize(
    "B,nk,nv,seed",
    [
        (1, 16, 48, 0),  # one GDN layer at batch 1 (4 waves per slab)
        (8, 16, 48, 1),  # a layer of the batch-8 step (6 slab waves per workgroup)
        (12, 16, 32, 2),  # 2 value heads per key head, 1536 slab units (4 slab waves per workgroup)
        (2, 16, 32, 3),  # 2 value heads per key head, small batch (4 waves per slab)
    ],
)
def test_gdn_decode_from_x(dev, B, nk, nv, seed):
    d = layer(B, nk, nv, seed)
    g = {k: v.to(dev) for k, v in d.items()}
    ws = torch.zeros(ops.lib().qs_gdn_workspace_bytes(B, nk), dtype=torch.uint8, device=dev)
    y = torch.empty_like(g["x"])
    o = ops.gdn_decode_fused(g["x"], g["conv_state"], g["taps"], g["g"], g["beta"], g["state"], nk=nk, y_out=y,
                             ws=ws)  # fmt: skip
    o_ref, S_ref, cs_ref, y_ref = O.gdn_decode(d["x"].float(), d["conv_state"].float(), d["taps"].float(), d["g"],
                                               d["beta"], d["state"], nk, nv, DK, DV)  # fmt: skip
    torch.cuda.synchronize()
    assert int(ws.view(torch.int32).abs().sum()) == 0, "conv counters not re-armed"
    assert torch.equal(g["conv_state"].cpu().float(), cs_ref)
    ulps, _ = bf16_ulp_mismatch(y, y_ref)
    assert ulps <= 1
    o_y, S_y = from_y(y, d["g"], d["beta"], d["state"], nk, nv)
    check_state(g["state"].cpu(), S_y, S_ref, conv_mismatch_heads(y, y_ref, nk, nv))
    assert_bf16_output(o, O.bf16(o_y))


@pytest.mark.parametrize("B,T,nk,nv,seed", [(1, 4, 16, 48, 10), (2, 3, 16, 48, 11), (12, 2, 16, 32, 12)])
def test_gdn_verify_from_x(dev, B, T, nk, nv, seed):
    """T tokens from x through the verify kernel against T sequential oracle decode steps from the same x."""
    d = layer(B, nk, nv, seed, T=T)
    g = {k: v.to(dev) for k, v in d.items()}
    o, states, convs, y = ops.gdn_verify_step(g["x"], g["conv_state"], g["taps"], g["g"], g["beta"], g["state"],
                                              nk=nk, return_y=True)  # fmt: skip
    o_ref, s_ref, c_ref, y_ref = O.gdn_verify(d["x"].float(), d["conv_state"].float(), d["taps"].float(), d["g"],
                                              d["beta"], d["state"], nk, nv, DK, DV)  # fmt: skip
    assert torch.equal(convs.cpu().float(), c_ref)
    assert bf16_ulp_mismatch(y, y_ref)[0] <= 1
    pert = conv_mismatch_heads(y, y_ref, nk, nv)  # [B, T, nv], cumulative over tokens
    S_y = d["state"]
    for t in range(T):
        o_y, S_y = from_y(y[:, t], d["g"][:, t], d["beta"][:, t], S_y, nk, nv)
        check_state(states[t].cpu(), S_y, s_ref[t], pert[:, t])
        assert_bf16_output(o[:, t], O.bf16(o_y))
    # negative control: token 1 computed from the input state instead of token 0's state (a dropped
    # dependency) must fail the state check
    q, k, v = O.split_qkv(y_ref[:, 1], nk, nv, DK, DV)
    _, wrong = O.gdn_step(q, k, v, d["g"][:, 1], d["beta"][:, 1], d["state"])
    with pytest.raises(AssertionError):
        assert_state(states[1].cpu(), wrong)


def test_gdn_decode_two_steps_from_x(dev):
    """Two decode steps in a row from x, the oracle carrying its own state and conv history (no reset to the
    kernel's values between the steps): the second step's state is the composition."""
    B, nk, nv = 8, 16, 48
    d = layer(B, nk, nv, 20, T=2)
    g = {k: v.to(dev) for k, v in d.items()}
    S, cs, S_y = d["state"], d["conv_state"].float(), d["state"]
    ys, yr = [], []
    for t in range(2):
        y = torch.empty(B, 2 * nk * DK + nv * DV, dtype=torch.bfloat16, device=dev)
        o = ops.gdn_decode_fused(g["x"][:, t].contiguous(), g["conv_state"], g["taps"], g["g"][:, t].contiguous(),
                                 g["beta"][:, t].contiguous(), g["state"], y_out=y)  # fmt: skip
        o_ref, S, cs, y_ref = O.gdn_decode(d["x"][:, t].float(), cs, d["taps"].float(), d["g"][:, t], d["beta"][:, t],
                                           S, nk, nv, DK, DV)  # fmt: skip
        o_y, S_y = from_y(y, d["g"][:, t], d["beta"][:, t], S_y, nk, nv)
        ys.append(y)
        yr.append(y_ref)
        assert_bf16_output(o, O.bf16(o_y))
    assert torch.equal(g["conv_state"].cpu().float(), cs)
    pert = conv_mismatch_heads(torch.stack(ys, 1), torch.stack(yr, 1), nk, nv)[:, -1]
    check_state(g["state"].cpu(), S_y, S, pert)
    # negative control: the second step applied to the initial state instead of the first step's
    _, wrong, _, _ = O.gdn_decode(d["x"][:, 1].float(), d["conv_state"].float(), d["taps"].float(), d["g"][:, 1],
                                  d["beta"][:, 1], d["state"], nk, nv, DK, DV)  # fmt: skip
    with pytest.raises(AssertionError):
        assert_state(g["state"].cpu(), wrong)
