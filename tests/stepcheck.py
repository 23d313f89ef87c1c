"""Oracle checks of whole decode / verify steps (test helpers): every layer of a StatePathStep or VerifyStep
against its own oracle call from the same inputs, the oracle carrying its own state from step to step.

GDN layers are checked in two stages: the conv output (one bf16 ulp at most, and few heads touched) against
the oracle's, and every state against the oracle's delta rule driven by the kernel's conv output, at the fp32
state tolerance; that state is what the oracle carries on.

The KV pools are compared on the pages the block table names: those pages are gathered into a compact pool
(page i of the compact pool = table entry i in row-major order), so the oracle works on a table arange(B mb)
and the step's pools are compared on the same pages after the step, bit for bit."""
import torch
from conftest import assert_attn_output, assert_bf16_output, assert_state, conv_mismatch_heads, perturbed_ok

from oracle import state_path as O
from qwen36_state.ops import DK, DV, NK, NV

def _cpu(t):
    return t.detach().cpu().clone()


class OracleState:
    """CPU copy of a step's resident state: GDN states and conv histories, the pages in use, lengths."""

    def __init__(self, step, gdn_state_of=None):
        self.table = _cpu(step.block_table)
        self.pages = self.table.flatten().long()
        B, mb = self.table.shape
        self.ctable = torch.arange(B * mb, dtype=torch.int32).view(B, mb)
        self.lens = _cpu(step.lens)
        self.gdn, self.kv = {}, {}
        for l, d in enumerate(step.layer):
            if d["attn"]:
                self.kv[l] = (_cpu(d["k_cache"][self.pages.to(d["k_cache"].device)]),
                              _cpu(d["v_cache"][self.pages.to(d["v_cache"].device)]))  # fmt: skip
            else:
                S, cs = gdn_state_of(l) if gdn_state_of else (d["state"], d["conv_state"])
                self.gdn[l] = [_cpu(S), _cpu(cs).float()]


def inputs_of(step):
    """CPU copies of every layer's step inputs."""
    out = {}
    for l, d in enumerate(step.layer):
        keys = ("q", "k_new", "v_new") if d["attn"] else ("x", "g", "beta")
        out[l] = {k: _cpu(d[k]) for k in keys}
    return out


def check_decode_step(step, ref, inp):
    """One decode step of ``step`` (already run) against the oracle applied to ``ref`` (advanced in place)
    with the inputs ``inp`` captured before the step."""
    pos = ref.lens.clone()  # rows cached before the step = the new row's position
    ref.lens = ref.lens + 1
    assert torch.equal(step.lens.cpu(), ref.lens), "positions advanced by one"
    for l, d in enumerate(step.layer):
        x = inp[l]
        if d["attn"]:
            kc, vc = ref.kv[l]
            O.paged_append(kc, vc, x["k_new"], x["v_new"], ref.ctable, pos)
            o_ref = O.gqa_decode(x["q"], kc, vc, ref.ctable, ref.lens, d["scale"])
            assert_attn_output(d["o"], O.bf16(o_ref))
            dev_pages = ref.pages.to(d["k_cache"].device)
            assert torch.equal(d["k_cache"][dev_pages].cpu(), kc), f"layer {l}: K pages"
            assert torch.equal(d["v_cache"][dev_pages].cpu(), vc), f"layer {l}: V pages"
        else:
            S, cs = ref.gdn[l]
            o_ref, S2, cs2, y_ref = O.gdn_decode(x["x"].float(), cs, d["taps"].cpu().float(), x["g"], x["beta"], S,
                                                 NK, NV, DK, DV)  # fmt: skip
            assert torch.equal(d["conv_state"].cpu().float(), cs2), f"layer {l}: conv state"
            # the kernel's conv output, recomputed from the same bits the kernel read (y is not exported by the
            # step)
            y_k = _kernel_conv(x["x"], cs, d["taps"].cpu())
            o_y, S_y = _from_y(y_k, x["g"], x["beta"], S)
            _check_state(d["state"].cpu(), S_y, S2, conv_mismatch_heads(y_k, y_ref, NK, NV), l)
            assert_bf16_output(d["o"], O.bf16(o_y))
            ref.gdn[l] = [S_y, cs2]


def _kernel_conv(x, cs, taps):
    """The conv output y the fused kernel computes, taken from the kernel itself: one qs_conv1d_update launch
    (the same tap order and SiLU as the fused kernel) on copies of the inputs."""
    from qwen36_state import ops

    dev = torch.device("cuda:0")
    st = cs.to(torch.bfloat16).to(dev)
    return ops.causal_conv1d_update(x.to(dev), st, taps.to(dev)).cpu()


def _from_y(y, g, beta, S):
    """The oracle's delta rule driven by the conv output y [B, C]: (o, S')."""
    q, k, v = O.split_qkv(y.float(), NK, NV, DK, DV)
    return O.gdn_step(q, k, v, g, beta, S)


def _check_state(got, S_y, S_x, pert, l):
    """Every head against the oracle driven by the kernel's conv output (S_y); where the head's conv inputs
    agree with the oracle's, S_y is the oracle's own state from x (S_x) bit for bit."""
    assert perturbed_ok(pert), f"layer {l}: conv inputs of {int(pert.sum())} of {pert.numel()} heads differ"
    assert torch.equal(S_y[~pert], S_x[~pert]), f"layer {l}"
    assert_state(got, S_y)


def check_verify_step(vs, ref, inp, accept):
    """One verify step of ``vs`` (already run, acceptance included) against T sequential oracle decode
    steps per layer, then the oracle's own acceptance: the state after the step is snapshot a - 1."""
    T = vs.T
    B = ref.lens.shape[0]
    base = ref.lens.clone()
    ref.lens = base + T  # lengths the verify layers see
    for l, d in enumerate(vs.layer):
        x = inp[l]
        if d["attn"]:
            kc, vc = ref.kv[l]
            O.paged_append(kc, vc, x["k_new"], x["v_new"], ref.ctable, base)
            o_ref = O.gqa_decode(x["q"], kc, vc, ref.ctable, ref.lens, d["scale"])
            assert_attn_output(d["o"], O.bf16(o_ref))
            dev_pages = ref.pages.to(d["k_cache"].device)
            assert torch.equal(d["k_cache"][dev_pages].cpu(), kc), f"layer {l}: K pages"
            assert torch.equal(d["v_cache"][dev_pages].cpu(), vc), f"layer {l}: V pages"
        else:
            S, cs = ref.gdn[l]
            o_ref, s_ref, c_ref, y_ref = O.gdn_verify(x["x"].float(), cs, d["taps"].cpu().float(), x["g"], x["beta"],
                                                      S, NK, NV, DK, DV)  # fmt: skip
            gi = d["gi"]
            # the snapshot set this step wrote (the accepted state lives in it)
            sset = 1 - vs.parity if vs.mode == "slots" else 0
            snaps, convs = vs.g_states[sset, gi].cpu(), vs.g_convs[sset, gi].cpu()
            assert torch.equal(convs.float(), c_ref), f"layer {l}: conv snapshots"
            y_k = torch.stack([_kernel_conv(x["x"][:, t].contiguous(), (c_ref[t - 1] if t else cs), d["taps"].cpu())
                               for t in range(T)], 1)  # fmt: skip
            pert = conv_mismatch_heads(y_k, y_ref, NK, NV)  # cumulative over the tokens
            s_y, S_y = [], S
            for t in range(T):
                o_y, S_y = _from_y(y_k[:, t], x["g"][:, t], x["beta"][:, t], S_y)
                s_y.append(S_y)
                _check_state(snaps[t], S_y, s_ref[t], pert[:, t], l)
                assert_bf16_output(d["o"][:, t], O.bf16(o_y))
            # acceptance: the oracle's state is its snapshot a - 1; the kernel's current state is the kernel's
            # snapshot a - 1, bit for bit
            idx = accept.long() - 1
            ar = torch.arange(B)
            ref.gdn[l] = [torch.stack(s_y)[idx, ar].clone(), c_ref[idx, ar].clone()]
            for b in range(B):
                S_cur, c_cur = vs.state_of(gi, b)
                assert torch.equal(S_cur.cpu(), snaps[idx[b], b]) and torch.equal(c_cur.cpu(), convs[idx[b], b])
    ref.lens = base + accept
    assert torch.equal(vs.lens.cpu(), ref.lens), "lengths after acceptance"
