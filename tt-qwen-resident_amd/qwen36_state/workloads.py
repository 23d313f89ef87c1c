"""Seeded synthetic inputs of the state-path workloads (generated on the target device).

Distributions: GDN state ~ N(0, 0.02^2) fp32; q, k, v, conv inputs and conv state ~ N(0, 1) in bf16;
conv taps = bf16(0.5 N(0, 1)) (model.py:189); log decay g = -softplus(N(0, 1)) * exp(U(-3, 0)); beta =
sigmoid(N(0, 1)); K/V pools ~ N(0, 1) bf16; block tables are slices of one seeded permutation of the pool.
"""
import torch

from .ops import BLOCK, CONV_K, DK, DV, HD, HIDDEN, INTER, MXFP4, MXINT8, NK, NKV, NQ, NV, MxWeight

C_QKV = 2 * NK * DK + NV * DV  # 10240 conv channels q | k | v


def _gen(device, seed):
    return torch.Generator(device=device).manual_seed(seed)


def _randn(shape, gen, device, dtype=torch.float32, std=1.0):
    t = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    return t.to(dtype)


def gates(B, gen, device, T=None):
    shape = (B, NV) if T is None else (B, T, NV)
    n = torch.randn(shape, generator=gen, device=device)
    u = torch.rand(shape, generator=gen, device=device) * -3.0
    g = -torch.nn.functional.softplus(n) * torch.exp(u)
    beta = torch.sigmoid(torch.randn(shape, generator=gen, device=device))
    return g.contiguous(), beta.contiguous()


def gdn_layer(B, device, seed=0, T=None):
    """One GDN layer's decode inputs: state, conv state, taps, x (q|k|v projection slice), g, beta, and
    the post-conv q, k, v of the same distributions for the unfused step. T adds a token axis (verify)."""
    gen = _gen(device, seed)
    d = dict(
        state=_randn((B, NV, DK, DV), gen, device, std=0.02),
        conv_state=_randn((B, C_QKV, CONV_K - 1), gen, device, torch.bfloat16),
        taps=_randn((C_QKV, CONV_K), gen, device, torch.bfloat16, std=0.5),
    )
    xs = (B, C_QKV) if T is None else (B, T, C_QKV)
    d["x"] = _randn(xs, gen, device, torch.bfloat16)
    d["g"], d["beta"] = gates(B, gen, device, T)
    if T is None:
        d["q"] = _randn((B, NK, DK), gen, device, torch.bfloat16)
        d["k"] = _randn((B, NK, DK), gen, device, torch.bfloat16)
        d["v"] = _randn((B, NV, DV), gen, device, torch.bfloat16)
    return d


def block_tables(B, pages_per_user, num_blocks, device, seed=0):
    """Per-user tables = disjoint slices of one seeded permutation of the pool [B, pages_per_user] int32."""
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(num_blocks, generator=gen)[: B * pages_per_user]
    return perm.view(B, pages_per_user).to(torch.int32).to(device)


def attn_layer(B, ctx, device, seed=0, T=1, num_blocks=2048, pools=True):
    """One attention layer's decode inputs at context ``ctx`` positions after appending T tokens:
    pools [num_blocks, NKV, 64, HD], block table [B, ceil(ctx / 64)], seq_lens = ctx, q [B, T, NQ, HD],
    new K/V rows [B, T, NKV, HD]."""
    gen = _gen(device, seed)
    pages = (ctx + BLOCK - 1) // BLOCK
    d = dict(
        q=_randn((B, T, NQ, HD), gen, device, torch.bfloat16),
        k_new=_randn((B, T, NKV, HD), gen, device, torch.bfloat16),
        v_new=_randn((B, T, NKV, HD), gen, device, torch.bfloat16),
        block_table=block_tables(B, pages, num_blocks, device, seed),
        seq_lens=torch.full((B,), ctx, dtype=torch.int32, device=device),
        scale=1.0 / 16.0,
    )
    if pools:
        d["k_cache"] = _randn((num_blocks, NKV, BLOCK, HD), gen, device, torch.bfloat16)
        d["v_cache"] = _randn((num_blocks, NKV, BLOCK, HD), gen, device, torch.bfloat16)
    return d


def prefill(T, device, seed=0):
    """Chunked-prefill inputs of one GDN layer: q, k [T, NK, DK], v [T, NV, DV], g, beta [T, NV], S0, and
    the layer's K/V [NKV, T, HD] with a random page table for the paged fill."""
    gen = _gen(device, seed)
    g, beta = gates(T, gen, device)
    return dict(
        q=_randn((T, NK, DK), gen, device, torch.bfloat16),
        k=_randn((T, NK, DK), gen, device, torch.bfloat16),
        v=_randn((T, NV, DV), gen, device, torch.bfloat16),
        g=g,
        beta=beta,
        S0=_randn((NV, DK, DV), gen, device, std=0.02),
        kv_k=_randn((NKV, T, HD), gen, device, torch.bfloat16),
        kv_v=_randn((NKV, T, HD), gen, device, torch.bfloat16),
        page_table=block_tables(1, (T + BLOCK - 1) // BLOCK, 2048, device, seed)[0].contiguous(),
    )


def mlp_layer(B, device, seed=0, H=None, I=None, keep_fp32=False, down_fmt=MXINT8):
    """One decoder layer's MLP half: x [B, H] fp32, gamma [H], the gate | up weights [H, I] as MXFP4 and the
    down weight [I, H] as MXINT8 (the reference's 8-bit precision; down_fmt MXFP8 for E4M3) (random normal
    scaled by 1 / sqrt(fan-in), quantized on the device, one weight in fp32 at a time). keep_fp32 also
    returns the fp32 weights on the host as gate32, up32, down32."""
    H = HIDDEN if H is None else H
    I = INTER if I is None else I
    gen = _gen(device, seed)
    d = dict(x=_randn((B, H), gen, device), gamma=1 + _randn((H,), gen, device, std=0.1))
    for name, shape, fmt, std in (("gate", (H, I), MXFP4, H**-0.5), ("up", (H, I), MXFP4, H**-0.5),
                                  ("down", (I, H), down_fmt, 0.5 * I**-0.5)):  # fmt: skip
        w = _randn(shape, gen, device, std=std)
        d[name] = MxWeight.quantize(w, fmt)
        if keep_fp32:
            d[name + "32"] = w.cpu()
        del w
    return d
