"""Paged KV append and fill on the GPU: bit-exact against the oracle's index arithmetic, with random
block tables, page-boundary crossings and untouched pages checked unchanged."""
import pytest
import torch

from oracle import state_path as O
from qwen36_state import ops, workloads as W

pytestmark = pytest.mark.gpu


def pools(nb, seed, nkv=4, hd=256):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(nb, nkv, 64, hd, generator=g).bfloat16(), torch.randn(nb, nkv, 64, hd, generator=g).bfloat16())


@pytest.mark.parametrize("B,T", [(1, 1), (3, 4), (8, 1)])
def test_append(dev, B, T):
    nb = 96
    kc, vc = pools(nb, seed=B * 10 + T)
    g = torch.Generator().manual_seed(T)
    table = torch.randperm(nb, generator=g)[: B * 10].view(B, 10).int()
    pos = torch.tensor([61, 0, 127, 5, 300, 63, 64, 2][:B], dtype=torch.int32)  # 61 + 4 crosses a page
    k, v = torch.randn(B, T, 4, 256, generator=g).bfloat16(), torch.randn(B, T, 4, 256, generator=g).bfloat16()
    gk, gv = kc.to(dev), vc.to(dev)
    ops.paged_kv_append(k.to(dev), v.to(dev), gk, gv, table.to(dev), pos.to(dev))
    O.paged_append(kc, vc, k, v, table, pos)
    assert torch.equal(gk.cpu(), kc) and torch.equal(gv.cpu(), vc)


def test_fill_prefill_kv(dev):
    """8192 tokens of 4 KV heads into 128 pages of a 2048-page pool through a random table."""
    d = W.prefill(8192, "cpu", seed=3)
    nb = 2048
    kc = torch.zeros(nb, 4, 64, 256, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    pt = d["page_table"]
    ops.paged_kv_fill(d["kv_k"].to(dev), d["kv_v"].to(dev), kc, vc, pt.to(dev))
    kcc, vcc = kc.cpu(), vc.cpu()
    assert torch.equal(O.paged_gather(kcc, pt, 8192), d["kv_k"])
    assert torch.equal(O.paged_gather(vcc, pt, 8192), d["kv_v"])
    mask = torch.ones(nb, dtype=torch.bool)
    mask[pt.long()] = False
    assert kcc[mask].abs().sum() == 0 and vcc[mask].abs().sum() == 0


def test_paged_fill_cache_signature(dev):
    """ttnn's paged_fill_cache(cache, x, page_table, batch_idx): row batch_idx of a [B, n] table."""
    g = torch.Generator().manual_seed(4)
    cache = torch.randn(40, 4, 64, 256, generator=g).bfloat16()
    x = torch.randn(1, 4, 150, 256, generator=g).bfloat16()
    table = torch.randperm(40, generator=g)[:12].view(3, 4).int()
    gc = cache.to(dev)
    ops.paged_fill_cache(gc, x.to(dev), table.to(dev), batch_idx=2)
    O.paged_fill(cache, x[0], table[2])
    assert torch.equal(gc.cpu(), cache)
