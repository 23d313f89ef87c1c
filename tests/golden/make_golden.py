"""Writes tests/golden/state_path_small.npz: tiny hand-checkable cases of every state-path function,
computed with scalar fp64 loops written from the reference's math (not with the vectorised oracle), so the
oracle can be pinned against them. The reference ships no golden vectors of its own (its accuracy data is
a tt-metal .refpt file that is not in the tree), so these are the fixtures.

    python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import state_path as O  # noqa: E402


def bf(t):
    return t.to(torch.bfloat16).to(torch.float32)


def attention_loops(q, k_cache, v_cache, table, seq_lens):
    """softmax(q . k * scale) v over each user's pages, scalar fp64 loops (model.py:239-244)."""
    B, T, nq, hd = q.shape
    nkv, block = k_cache.shape[1], k_cache.shape[2]
    G = nq // nkv
    scale = 1.0 / math.sqrt(hd)
    out = np.zeros((B, T, nq, hd))
    for b in range(B):
        n = int(seq_lens[b])
        for t in range(T):
            valid = n - T + t + 1
            for h in range(nq):
                s = []
                for p in range(valid):
                    page, row = int(table[b, p // block]), p % block
                    s.append(scale * sum(float(q[b, t, h, d]) * float(k_cache[page, h // G, row, d]) for d in range(hd)))
                m = max(s)
                e = [math.exp(x - m) for x in s]
                L = sum(e)
                for d in range(hd):
                    acc = 0.0
                    for p in range(valid):
                        page, row = int(table[b, p // block]), p % block
                        acc += e[p] * float(v_cache[page, h // G, row, d])
                    out[b, t, h, d] = acc / L
    return out


def main():
    g = torch.Generator().manual_seed(1234)
    rn = lambda *s: torch.randn(*s, generator=g)
    f = {}
    # conv1d update: B=2, C=6, K=4
    x, cs, taps = bf(rn(2, 6)), bf(rn(2, 6, 3)), bf(0.5 * rn(6, 4))
    y, ns = O.conv1d_update_loops(x, cs, taps)
    f.update(conv_x=x, conv_state=cs, conv_taps=taps, conv_y=y, conv_new_state=ns)
    # gated delta rule step: B=2, NK=1, NV=3, DK=DV=4 (fp64 scalar loops)
    q, k, v = rn(2, 1, 4).double(), rn(2, 1, 4).double(), rn(2, 3, 4).double()
    gg = (-torch.nn.functional.softplus(rn(2, 3)) * torch.exp(-3 * torch.rand(2, 3, generator=g))).double()
    beta = torch.sigmoid(rn(2, 3)).double()
    S = (0.5 * rn(2, 3, 4, 4)).double()
    o, S2 = O.gdn_step_loops(q, k, v, gg, beta, S)
    f.update(gdn_q=q, gdn_k=k, gdn_v=v, gdn_g=gg, gdn_beta=beta, gdn_S=S, gdn_o=o, gdn_S2=S2)
    # paged attention: B=2, T=2, NQ=4, NKV=2, HD=8, block 4, 6 pages, seq_lens 7 and 3
    kc, vc = rn(6, 2, 4, 8).double(), rn(6, 2, 4, 8).double()
    table = torch.tensor([[4, 1], [2, 5]], dtype=torch.int32)
    seq = torch.tensor([7, 3], dtype=torch.int32)
    qa = rn(2, 2, 4, 8).double()
    f.update(att_q=qa, att_k=kc, att_v=vc, att_table=table, att_seq=seq,
             att_o=torch.from_numpy(attention_loops(qa, kc, vc, table, seq)))  # fmt: skip
    # prefill: T=9 tokens, NK=1, NV=2, DK=DV=4, sequential scalar steps
    T = 9
    pq, pk, pv = rn(T, 1, 4).double(), rn(T, 1, 4).double(), rn(T, 2, 4).double()
    pg = (-torch.nn.functional.softplus(rn(T, 2)) * torch.exp(-3 * torch.rand(T, 2, generator=g))).double()
    pb = torch.sigmoid(rn(T, 2)).double()
    S = (0.3 * rn(2, 4, 4)).double()
    os_ = []
    St = S[None]
    for t in range(T):
        o, St = O.gdn_step_loops(pq[t : t + 1], pk[t : t + 1], pv[t : t + 1], pg[t : t + 1], pb[t : t + 1], St)
        os_.append(o[0])
    f.update(pre_q=pq, pre_k=pk, pre_v=pv, pre_g=pg, pre_beta=pb, pre_S0=S, pre_o=torch.stack(os_), pre_ST=St[0])
    np.savez(os.path.join(HERE, "state_path_small.npz"), **{k: v.numpy() for k, v in f.items()})
    print(f"wrote {len(f)} arrays")


if __name__ == "__main__":
    main()
