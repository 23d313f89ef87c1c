"""CPU restatement of the decode-time state path (TEST INFRASTRUCTURE ONLY — see the package docstring).

Reference citations are ``path:line`` into sott0n/tt-qwen-resident. All arithmetic runs in the dtype of the
state argument (fp32 by default, fp64 when a test asks for a high-precision reference); values that the
reference rounds to bf16 are rounded here at the same points with round-to-nearest-even.

Layouts (caller-facing, shared with the HIP library):
  conv state      [B, C, K-1]  oldest input first (tap 0 multiplies the oldest input, weights.py:58)
  conv taps       [C, K]
  GDN state       [B, NV, DK, DV] fp32, indexed S[k][v] (model.py:161, :270-273)
  paged K/V pool  [num_blocks, NKV, block, HD] (prefill/pp_prefill.py:207-211)
  block table     [B, max_blocks] int32; position p of user b lives in page table[b, p // block], row p % block
"""
import math

import torch
import torch.nn.functional as F

EPS = 1e-6  # L2-norm eps, model.py:264-267 (also RMSNorm eps, common.py:15)
SOFTPLUS_THRESHOLD = 20.0  # kernels/gdn_head_compute.cpp:188

__all__ = [
    "EPS",
    "bf16",
    "conv1d_update",
    "conv1d_update_loops",
    "conv1d_prefill",
    "l2norm",
    "gdn_gates",
    "gdn_step",
    "gdn_step_loops",
    "split_qkv",
    "gdn_decode",
    "gdn_verify",
    "gdn_rollback",
    "paged_slot",
    "paged_append",
    "paged_append_loops",
    "paged_fill",
    "paged_gather",
    "gqa_decode",
    "attention_partials",
    "merge_partials",
    "rmsnorm",
    "gdn_gated_norm",
    "rope_tables",
    "rope",
    "attn_mixer",
    "gdn_chunk_prefill",
    "gdn_chunk_prefill_wy",
]


def bf16(t):
    """Round to bf16 (round-to-nearest-even) and back to fp32 — model.py:84-85."""
    return t.to(torch.bfloat16).to(torch.float32)


# --------------------------------------------------------------------------------------------- a1: conv1d


def conv1d_update(x, conv_state, taps):
    """One decode step of the causal depthwise conv1d + SiLU over the q|k|v mixer channels.

    Restates ``torch_step`` model.py:255-259: ``window = cat([hist, x])`` oldest first, the output is
    ``bf16(silu(sum_j taps[:, j] * window[j]))`` and the history becomes ``window[1:]``. The tap sum runs in
    a fixed order (tap 0 first); each product of two bf16 values is exact in fp32, so the only rounding is
    in the three additions.

    x [B, C], conv_state [B, C, K-1], taps [C, K] (all bf16-valued float tensors)
    returns y [B, C] (bf16-valued fp32), new conv state [B, C, K-1]
    """
    K = taps.shape[1]
    assert conv_state.shape[-1] == K - 1
    win = torch.cat([conv_state.float(), x.float()[..., None]], dim=-1)  # [B, C, K] oldest first
    t = taps.float()
    acc = win[..., 0] * t[:, 0]
    for j in range(1, K):
        acc = acc + win[..., j] * t[:, j]
    y = bf16(F.silu(acc))
    return y, win[..., 1:].clone()


def conv1d_prefill(x, conv_state, taps):
    """Causal depthwise conv1d + SiLU over the T prompt tokens of one sequence, with the carry.

    Restates the prefill conv (prefill/kernels/conv_compute.cpp:4-10, its statement in the reference test
    tests/test_pp_kernels.py:135-140): ``win = cat([carry, x])`` oldest first, ``y_t = bf16(silu(sum_j
    win[t + j] taps[:, j]))`` with the tap sum in the decode order (tap 0 first), and the new carry is
    ``win[T : T + K - 1]``, the last K - 1 inputs (bits unchanged).

    x [T, C]; conv_state [C, K-1] or None (zeros); taps [C, K] (bf16-valued float tensors)
    returns y [T, C] (bf16-valued fp32), new conv state [C, K-1]
    """
    T, C = x.shape
    K = taps.shape[1]
    carry = torch.zeros(C, K - 1) if conv_state is None else conv_state.float()
    win = torch.cat([carry.t(), x.float()], dim=0)  # [T + K - 1, C]
    t = taps.float()
    acc = win[0:T] * t[:, 0]
    for j in range(1, K):
        acc = acc + win[j : j + T] * t[:, j]
    y = bf16(F.silu(acc))
    return y, win[T : T + K - 1].t().contiguous()


def conv1d_update_loops(x, conv_state, taps):
    """Per-channel scalar restatement of :func:`conv1d_update` (brute force, for small C only)."""
    B, C = x.shape
    K = taps.shape[1]
    y = torch.zeros(B, C)
    new = torch.zeros(B, C, K - 1)
    for b in range(B):
        for c in range(C):
            win = [float(conv_state[b, c, j]) for j in range(K - 1)] + [float(x[b, c])]
            acc = torch.tensor(win[0], dtype=torch.float32) * torch.tensor(float(taps[c, 0]), dtype=torch.float32)
            for j in range(1, K):
                acc = acc + torch.tensor(win[j], dtype=torch.float32) * torch.tensor(float(taps[c, j]))
            s = float(acc) / (1.0 + math.exp(-float(acc)))
            y[b, c] = bf16(torch.tensor(s, dtype=torch.float32))
            for j in range(K - 1):
                new[b, c, j] = win[j + 1]
    return y, new


# --------------------------------------------------------------------------------------------- a2/a3


def l2norm(x, eps=EPS, scale=1.0):
    """``x * rsqrt(sum(x^2) + eps) * scale`` over the last dim — model.py:264-267 (q: scale = DK^-1/2)."""
    return x * torch.rsqrt(x.pow(2).sum(-1, keepdim=True) + eps) * scale


def gdn_gates(a, b, dt_bias, neg_a):
    """Per value head: ``g = neg_a * softplus(a + dt_bias)`` (log decay), ``beta = sigmoid(b)``.

    Restates model.py:268-269 (decay = exp(g)) with the softplus threshold 20 of
    kernels/gdn_head_compute.cpp:188; ``neg_a = -exp(A_log)`` per weights.py:60.
    """
    g = neg_a * F.softplus(a + dt_bias, beta=1.0, threshold=SOFTPLUS_THRESHOLD)
    return g, torch.sigmoid(b)


# --------------------------------------------------------------------------------------------- a4: delta rule


def gdn_step(q, k, v, g, beta, S, scale=None, eps=EPS):
    """One gated delta rule decode step for all (user, value head) pairs.

    Restates ``torch_step`` model.py:262-273 vectorised over heads:
        qn = l2norm(q[kh]) * DK^-1/2, kn = l2norm(k[kh]) with kh = h // (NV // NK)   (model.py:263-267)
        decay = exp(g), delta = beta * (v - (decay * kn) @ S)                         (model.py:268-271)
        S' = decay * S + outer(kn, delta), o = qn @ S'                                (model.py:272-274)
    q, k [B, NK, DK]; v [B, NV, DV]; g, beta [B, NV]; S [B, NV, DK, DV] (S[k][v]).
    Returns o [B, NV, DV] (unrounded, in S's dtype) and the new state S'.
    """
    dt = S.dtype
    B, NV, DK, DV = S.shape
    NK = q.shape[1]
    rep = NV // NK
    if scale is None:
        scale = DK**-0.5
    qh = q.to(dt).repeat_interleave(rep, dim=1)  # [B, NV, DK]
    kh = k.to(dt).repeat_interleave(rep, dim=1)
    qn = l2norm(qh, eps) * scale
    kn = l2norm(kh, eps)
    decay = torch.exp(g.to(dt))[..., None]  # [B, NV, 1]
    kS = ((decay * kn)[..., None, :] @ S).squeeze(-2)  # [B, NV, DV]
    delta = beta.to(dt)[..., None] * (v.to(dt) - kS)
    S2 = decay[..., None] * S + kn[..., :, None] * delta[..., None, :]
    o = (qn[..., None, :] @ S2).squeeze(-2)
    return o, S2


def gdn_step_loops(q, k, v, g, beta, S, scale=None, eps=EPS):
    """fp64 scalar-loop restatement of :func:`gdn_step` (brute force, tiny shapes only)."""
    B, NV, DK, DV = S.shape
    NK = q.shape[1]
    rep = NV // NK
    scale = DK**-0.5 if scale is None else scale
    o = torch.zeros(B, NV, DV, dtype=torch.float64)
    S2 = torch.zeros(B, NV, DK, DV, dtype=torch.float64)
    for b in range(B):
        for h in range(NV):
            kh = h // rep
            qq = [float(q[b, kh, i]) for i in range(DK)]
            kk = [float(k[b, kh, i]) for i in range(DK)]
            rq = 1.0 / math.sqrt(sum(x * x for x in qq) + eps)
            rk = 1.0 / math.sqrt(sum(x * x for x in kk) + eps)
            qn = [x * rq * scale for x in qq]
            kn = [x * rk for x in kk]
            dec = math.exp(float(g[b, h]))
            bt = float(beta[b, h])
            for j in range(DV):
                ks = sum(dec * kn[i] * float(S[b, h, i, j]) for i in range(DK))
                delta = bt * (float(v[b, h, j]) - ks)
                col = [dec * float(S[b, h, i, j]) + kn[i] * delta for i in range(DK)]
                for i in range(DK):
                    S2[b, h, i, j] = col[i]
                o[b, h, j] = sum(qn[i] * col[i] for i in range(DK))
    return o, S2


def split_qkv(y, NK, NV, DK, DV):
    """Split the conv output's channels ``q (NK*DK) | k (NK*DK) | v (NV*DV)`` — model.py:260, weights.py:51-73."""
    B = y.shape[0]
    qd = NK * DK
    return (
        y[:, :qd].reshape(B, NK, DK),
        y[:, qd : 2 * qd].reshape(B, NK, DK),
        y[:, 2 * qd : 2 * qd + NV * DV].reshape(B, NV, DV),
    )


def gdn_decode(x, conv_state, taps, g, beta, S, NK, NV, DK, DV, scale=None, eps=EPS):
    """GDN mixer state path of one decode step: conv1d update, split, L2-norm, delta rule (model.py:255-273).

    Returns (o [B, NV, DV] unrounded, S', new conv state, conv output y [B, C])."""
    y, cs = conv1d_update(x, conv_state, taps)
    q, k, v = split_qkv(y, NK, NV, DK, DV)
    o, S2 = gdn_step(q, k, v, g, beta, S, scale, eps)
    return o, S2, cs, y


# --------------------------------------------------------------------------------------------- a7: verify


def gdn_verify(x, conv_state, taps, g, beta, S, NK, NV, DK, DV, scale=None, eps=EPS):
    """T tokens through :func:`gdn_decode` in sequence, keeping every intermediate state.

    The reference verify step runs row 1 from row 0's new state and writes it to the other slot
    (kernels/gdn_head_reader.cpp:149-187, gdn_head_writer.cpp:60-66, :109); its test replays the rows as
    consecutive batch-1 steps (tests/test_resident_verify.py:42-72). Here T is general.
    x [B, T, C]; g, beta [B, T, NV]. Returns o [B, T, NV, DV], states [T, B, NV, DK, DV],
    conv states [T, B, C, K-1], conv outputs y [B, T, C].
    """
    T = x.shape[1]
    os_, ss, cs_, ys = [], [], [], []
    cs = conv_state
    for t in range(T):
        o, S, cs, y = gdn_decode(x[:, t], cs, taps, g[:, t], beta[:, t], S, NK, NV, DK, DV, scale, eps)
        os_.append(o)
        ss.append(S)
        cs_.append(cs)
        ys.append(y)
    return torch.stack(os_, 1), torch.stack(ss, 0), torch.stack(cs_, 0), torch.stack(ys, 1)


def gdn_rollback(states, conv_states, accept):
    """State and conv history after accepting ``accept[b]`` in [1, T] tokens: snapshot ``accept[b] - 1``.

    The reference selects the slot instead of copying (model.py:1314-1318, README.md:413-421; the hub sets
    ``slot ^= accept``, kernels/mlp_hub.cpp:48-58); the resulting state is the same bytes."""
    B = states.shape[1]
    idx = torch.as_tensor(accept, dtype=torch.long) - 1
    ar = torch.arange(B)
    return states[idx, ar].clone(), conv_states[idx, ar].clone()


# --------------------------------------------------------------------------------------------- a5/a9: paged


def paged_slot(block_table, b, pos, block):
    """(page, row) of position ``pos`` of user ``b`` — the vLLM block-table contract (block 64,
    tt-model.yaml:41) as the prefill's page tables use it (prefill/pp_prefill.py:873-886)."""
    return int(block_table[b, pos // block]), pos % block


def paged_append(k_cache, v_cache, k_new, v_new, block_table, positions):
    """Write T new K/V rows per user at positions ``positions[b] + t`` (in place, bit-exact copy).

    k_new, v_new [B, T, NKV, HD]; caches [num_blocks, NKV, block, HD]. The reference decode splices the new
    row into its cache tile (kernels/attn_compute_common.hpp:281-322, torch model.py:245-246); here the row
    goes to the page the block table names."""
    B, T = k_new.shape[:2]
    block = k_cache.shape[2]
    pos = torch.as_tensor(positions, dtype=torch.long)[:, None] + torch.arange(T)[None]  # [B, T]
    bt = torch.as_tensor(block_table, dtype=torch.long)
    pages = torch.gather(bt, 1, pos // block)  # [B, T]
    rows = pos % block
    k_cache[pages, :, rows, :] = k_new.to(k_cache.dtype)
    v_cache[pages, :, rows, :] = v_new.to(v_cache.dtype)


def paged_append_loops(k_cache, v_cache, k_new, v_new, block_table, positions):
    """Pure-Python loop restatement of :func:`paged_append`."""
    B, T = k_new.shape[:2]
    block = k_cache.shape[2]
    for b in range(B):
        for t in range(T):
            page, row = paged_slot(block_table, b, int(positions[b]) + t, block)
            k_cache[page, :, row, :] = k_new[b, t]
            v_cache[page, :, row, :] = v_new[b, t]


def paged_fill(cache, x, page_table, start=0):
    """``paged_fill_cache(cache, x, page_table, batch_idx)``: token i of x [NKV, T, HD] goes to page
    ``page_table[(start + i) // block]``, row ``(start + i) % block`` (prefill/pp_prefill.py:826-827, fill
    tables :882; gather restatement :1243-1244)."""
    NKV, T, HD = x.shape
    block = cache.shape[2]
    pos = start + torch.arange(T)
    pt = torch.as_tensor(page_table, dtype=torch.long)
    pages = pt[pos // block]
    cache[pages, :, pos % block, :] = x.permute(1, 0, 2).to(cache.dtype)


def paged_gather(cache, table_row, n):
    """Positions 0..n-1 of one user as [NKV, n, HD] — the export_state gather, prefill/pp_prefill.py:1243-1244."""
    block = cache.shape[2]
    nb = (n + block - 1) // block
    pages = torch.as_tensor(table_row[:nb], dtype=torch.long)
    c = cache[pages]  # [nb, NKV, block, HD]
    return c.permute(1, 0, 2, 3).reshape(cache.shape[1], nb * block, cache.shape[3])[:, :n]


# --------------------------------------------------------------------------------------------- a6: attention


def gqa_decode(q, k_cache, v_cache, block_table, seq_lens, scale, dtype=torch.float32):
    """Paged GQA decode attention, T query tokens per user, causal among the T new tokens.

    Restates model.py:239-244 (``softmax(qn @ K.T) @ V`` over the cache rows 0..pos, scale folded into the
    q norm weight at model.py:237) over the gathered pages: query token t of user b sees positions
    ``0 .. seq_lens[b] - T + t``; query head h reads KV head ``h // (NQ // NKV)`` (weights.py:5-6).
    q [B, T, NQ, HD] → o [B, T, NQ, HD] in ``dtype`` (unrounded)."""
    B, T, NQ, HD = q.shape
    NKV = k_cache.shape[1]
    G = NQ // NKV
    out = torch.zeros(B, T, NQ, HD, dtype=dtype)
    for b in range(B):
        n = int(seq_lens[b])
        K = paged_gather(k_cache, block_table[b], n).to(dtype)  # [NKV, n, HD]
        V = paged_gather(v_cache, block_table[b], n).to(dtype)
        for t in range(T):
            valid = n - T + t + 1
            for h in range(NQ):
                s = (K[h // G, :valid] @ q[b, t, h].to(dtype)) * scale
                p = torch.softmax(s, dim=-1)
                out[b, t, h] = p @ V[h // G, :valid]
    return out


def attention_partials(q, K, V, scale, bounds):
    """Split-K partials of one query row over position ranges ``bounds`` = [(lo, hi), ...]: per range the
    running max m, the sum l of exp(s - m) and the unnormalised o (the worker side of the reference's
    online softmax, kernels/attn_worker_compute.cpp:77-208)."""
    parts = []
    for lo, hi in bounds:
        s = (K[lo:hi] @ q) * scale
        m = s.max()
        p = torch.exp(s - m)
        parts.append((m, p.sum(), p @ V[lo:hi]))
    return parts


def merge_partials(parts):
    """Merge split-K partials in order: global max, rescale, sum, normalise (the leader side,
    kernels/attn_leader_writer.cpp:86-106 and kernels/attn_leader_compute.cpp:42-79)."""
    M = max(float(m) for m, _, _ in parts)
    L = sum(float(l) * math.exp(float(m) - M) for m, l, _ in parts)
    o = sum(o * math.exp(float(m) - M) for m, _, o in parts)
    return o / L


# ------------------------------------------------------------------------- the attention mixer's edges


def rmsnorm(x, w=None, eps=EPS):
    """x * rsqrt(mean(x^2) + eps) over the last dim, times w — model.py:86-89 (EPS common.py:15)."""
    y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return y if w is None else y * w


def gdn_gated_norm(o, z, norm_w, eps=EPS):
    """The GDN mixer's epilogue per value head — model.py:274-275: bf16(rmsnorm(o, norm_w) * silu(z))."""
    return bf16(rmsnorm(o.float(), norm_w, eps) * F.silu(z.float()))


def rope_tables(pos, rot=64, theta=1e7):
    """cos, sin of position(s) ``pos`` for the first ``rot`` dims: inverse frequencies theta^(-2i/rot),
    computed in float64 and rounded to float32 — model.py:128-132 (ROPE_THETA, ROT model.py:51-52).
    pos: int or integer tensor of any shape -> cos, sin [..., rot // 2]."""
    inv = 1.0 / theta ** (torch.arange(0, rot, 2, dtype=torch.float64) / rot)
    ang = torch.as_tensor(pos, dtype=torch.float64)[..., None] * inv
    return torch.cos(ang).float(), torch.sin(ang).float()


def rope(t, cos, sin, rot=64):
    """Rotary embedding of the first ``rot`` dims with the halves paired — model.py:135-140:
    t[:h] = a cos - b sin, t[h:rot] = b cos + a sin (a = t[:h], b = t[h:rot], h = rot / 2); cos, sin
    broadcast over the leading dims of t except the last."""
    h = rot // 2
    t = t.clone()
    a, b = t[..., :h].clone(), t[..., h:rot].clone()
    t[..., :h] = a * cos - b * sin
    t[..., h:rot] = b * cos + a * sin
    return t


def attn_mixer(q, k_new, v_new, gate, wq, wk, cos, sin, k_cache, v_cache, block_table, seq_lens, rot=64, eps=EPS):
    """The attention mixer around the paged cache for T tokens per user — model.py:237-246:
    qn = rope(rmsnorm(q, wq)) (fp32; wq carries the softmax scale, model.py:237), kn = bf16(rope(rmsnorm(k,
    wk))), kn and v appended at positions seq_lens - T + t (the caches are updated in place), and
    o = bf16(softmax(qn K^T) V * sigmoid(gate)), causal among the T new rows.
    q, gate [B, T, NQ, HD]; k_new, v_new [B, T, NKV, HD]; cos, sin [B, T, rot / 2] -> o [B, T, NQ, HD]."""
    cq, sq = cos[:, :, None], sin[:, :, None]
    qn = rope(rmsnorm(q.float(), wq, eps), cq, sq, rot)
    kn = bf16(rope(rmsnorm(k_new.float(), wk, eps), cq, sq, rot))
    T = q.shape[1]
    paged_append(k_cache, v_cache, kn.to(k_cache.dtype), v_new, block_table, seq_lens - T)
    o = gqa_decode(qn, k_cache, v_cache, block_table, seq_lens, 1.0)
    return bf16(o * torch.sigmoid(gate.float()))


# --------------------------------------------------------------------------------------------- a8: prefill


def gdn_chunk_prefill(q, k, v, g, beta, S0, scale=None, eps=EPS):
    """Prefill of one sequence through the gated delta rule, restated as the sequential recurrence.

    The reference calls tt-metal's ``chunk_gated_delta_rule(q, k, v, g, beta, scale=DK^-1/2, initial_state,
    output_final_state=True, chunk_size=32)`` (prefill/pp_prefill.py:783-813), which L2-normalises q and k
    per head itself; mathematically it is T applications of the decode step (the equivalence the reference's
    test_pp_prefill_matches_decode relies on, tests/test_pp_prefill.py:26-103).
    q, k [T, NK, DK]; v [T, NV, DV]; g, beta [T, NV]; S0 [NV, DK, DV] → o [T, NV, DV], S_T."""
    T = q.shape[0]
    S = S0[None]
    os_ = []
    for t in range(T):
        o, S = gdn_step(q[t : t + 1], k[t : t + 1], v[t : t + 1], g[t : t + 1], beta[t : t + 1], S, scale, eps)
        os_.append(o[0])
    return torch.stack(os_, 0), S[0]


def gdn_chunk_prefill_wy(q, k, v, g, beta, S0, chunk=64, scale=None, eps=EPS):
    """The chunked (WY / UT-transform) form of :func:`gdn_chunk_prefill`, a second restatement.

    Per chunk with start state S0, cumulative log decay G_i = sum_{j<=i} g_j and gamma_i = exp(G_i):
        A_ij = beta_i (k_i . k_j) gamma_i / gamma_j  (i > j),  Tm = (I + A)^-1
        W = Tm diag(beta gamma) K,  U = Tm diag(beta) V,  delta = U - W S0
        O = diag(gamma) Q S0 + ((Q K^T) o M) delta with M_ij = gamma_i / gamma_j (i >= j)
        S_C = gamma_C S0 + (diag(gamma_C / gamma) K)^T delta
    (the chunked gated delta rule of Yang et al., "Gated Delta Networks", as FLA's
    ``chunk_gated_delta_rule`` computes it). Runs in S0's dtype."""
    dt = S0.dtype
    T, NK, DK = q.shape
    NV, _, DV = S0.shape
    rep = NV // NK
    scale = DK**-0.5 if scale is None else scale
    qn = l2norm(q.to(dt).repeat_interleave(rep, 1), eps) * scale  # [T, NV, DK]
    kn = l2norm(k.to(dt).repeat_interleave(rep, 1), eps)
    vv = v.to(dt)
    S = S0.clone()
    out = torch.zeros(T, NV, DV, dtype=dt)
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        C = c1 - c0
        Q = qn[c0:c1].transpose(0, 1)  # [NV, C, DK]
        Kc = kn[c0:c1].transpose(0, 1)
        Vc = vv[c0:c1].transpose(0, 1)  # [NV, C, DV]
        gc = g[c0:c1].to(dt).transpose(0, 1)  # [NV, C]
        bc = beta[c0:c1].to(dt).transpose(0, 1)
        G = torch.cumsum(gc, -1)
        ratio = torch.exp(G[:, :, None] - G[:, None, :])  # gamma_i / gamma_j
        strict = torch.tril(torch.ones(C, C, dtype=torch.bool), -1)
        causal = torch.tril(torch.ones(C, C, dtype=torch.bool))
        A = (bc[:, :, None] * (Kc @ Kc.transpose(1, 2)) * ratio) * strict
        Tm = torch.linalg.inv(torch.eye(C, dtype=dt) + A)
        gam = torch.exp(G)
        W = Tm @ ((bc * gam)[..., None] * Kc)
        U = Tm @ (bc[..., None] * Vc)
        delta = U - W @ S
        P = (Q @ Kc.transpose(1, 2)) * ratio * causal
        O = gam[..., None] * (Q @ S) + P @ delta
        out[c0:c1] = O.transpose(0, 1)
        last = gam[:, -1]
        S = last[:, None, None] * S + (((last[:, None] / gam)[..., None] * Kc).transpose(1, 2) @ delta)
    return out, S
