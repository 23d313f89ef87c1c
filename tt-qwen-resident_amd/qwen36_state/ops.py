"""Operator-level Python API of the MI355X state path, over the C ABI of libqwen_state.so.

Each op keeps the signature and argument meaning of the reference call it replaces (cited per op), checks
shapes, dtypes, devices and contiguity (ValueError on a mismatch, like the reference's asserts), and
enqueues HIP kernels on the current torch stream. Tensors are caller-owned; state arguments are updated in
place as in the reference. Nothing here computes on the CPU.
"""
import ctypes

import torch

from ._lib import call, lib

NK, NV, DK, DV, CONV_K = 16, 48, 128, 128, 4  # model.py:48
NQ, NKV, HD = 24, 4, 256  # model.py:50
ROT, ROPE_THETA = 64, 1e7  # model.py:51-52
BLOCK = 64  # vLLM block size, tt-model.yaml:41
EPS = 1e-6  # model.py:264-267


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _chk(t, name, dtype, shape=None, dev=None):
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a GPU (got {t.device})")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)} (got {tuple(t.shape)})")
    if dev is not None and t.device != dev:
        raise ValueError(f"{name} is on {t.device}, expected {dev}")
    return t


# ------------------------------------------------------------------------------------------- workspaces

_WS = {}


def workspace(kind, nbytes, device):
    """A zeroed device workspace of at least ``nbytes`` for ``kind`` on ``device`` and the current stream.

    The kernels leave their counters zeroed again, so the buffer is reused by every later call on the
    same stream. It must exist before a HIP graph capture starts (warm the op up once first)."""
    device = torch.device(device)
    key = (kind, device, torch.cuda.current_stream(device).cuda_stream)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise ValueError(f"{kind} workspace must be allocated before graph capture: run the op once first")
        ws = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


# ------------------------------------------------------------------------------------------- status word

STATUS_LENGTH, STATUS_PAGE, STATUS_ACCEPT = 1, 2, 4  # QS_STATUS_* of include/qwen_state.h
_STATUS_TEXT = {
    STATUS_LENGTH: "a sequence length ran past its block table",
    STATUS_PAGE: "a block-table entry needed by a valid position lies outside the KV pool",
    STATUS_ACCEPT: "an accept length lies outside [1, T]",
}


class Status:
    """The device status word the kernels report invalid lengths, table entries and accept lengths into
    (an int32 the caller owns; kernels only OR bits into it). ``check()`` synchronises the device, raises
    ValueError naming every reported condition (the reference's asserts, generator_vllm.py:94, :130) and
    clears the word; ``peek()`` reads it without raising."""

    def __init__(self, device):
        self.word = torch.zeros(1, dtype=torch.int32, device=device)

    def peek(self):
        return int(self.word.item())

    def check(self):
        v = self.peek()
        if v:
            self.word.zero_()
            raise ValueError("; ".join(t for bit, t in _STATUS_TEXT.items() if v & bit) + f" (status {v:#x})")


def advance_lengths(lens, T, max_len, base_out=None, status=None):
    """The step's position advance (model.py:1314-1351, :1499-1508): base_out <- lens, lens <- lens + T for
    every user with lens >= 0 (negative = idle slot). lens [B] int32 on the device; a length past max_len is
    reported in ``status``."""
    dev = lens.device
    _chk(lens, "lens", torch.int32)
    B = lens.shape[0]
    if base_out is not None:
        _chk(base_out, "base_out", torch.int32, (B,), dev)
    call("qs_advance_lengths", _p(lens), _p(base_out), B, int(T), int(max_len), _p(status), _stream(dev))


# ------------------------------------------------------------------------------------------- a1, a3


def causal_conv1d_update(x, conv_state, taps):
    """y = silu(causal conv1d over [state, x]) with the state shifted in place (model.py:255-259).

    x [B, C] bf16, conv_state [B, C, K-1] bf16, taps [C, K] bf16 -> y [B, C] bf16."""
    dev = x.device
    B, C = x.shape
    _chk(x, "x", torch.bfloat16)
    _chk(taps, "taps", torch.bfloat16, (C, CONV_K), dev)
    _chk(conv_state, "conv_state", torch.bfloat16, (B, C, CONV_K - 1), dev)
    y = torch.empty_like(x)
    call("qs_conv1d_update", _p(x), _p(conv_state), _p(taps), _p(y), B, C, CONV_K, _stream(dev))
    return y


def gdn_gates(a, b, dt_bias, neg_a):
    """g = neg_a * softplus(a + dt_bias), beta = sigmoid(b) (model.py:268-269). a, b [B, NV] bf16."""
    dev = a.device
    B, nv = a.shape
    _chk(a, "a", torch.bfloat16)
    _chk(b, "b", torch.bfloat16, (B, nv), dev)
    _chk(dt_bias, "dt_bias", torch.float32, (nv,), dev)
    _chk(neg_a, "neg_a", torch.float32, (nv,), dev)
    g = torch.empty(B, nv, dtype=torch.float32, device=dev)
    beta = torch.empty_like(g)
    call("qs_gdn_gates", _p(a), _p(b), _p(dt_bias), _p(neg_a), _p(g), _p(beta), B, nv, _stream(dev))
    return g, beta


# ------------------------------------------------------------------------------------------- a2 + a4


def gdn_decode_step(q, k, v, g, beta, state, scale=None, eps=EPS, out=None):
    """One gated delta rule decode step (model.py:262-273), state [B, NV, DK, DV] fp32 updated in place.

    q, k [B, NK, DK] bf16 (before the L2-norm); v [B, NV, DV] bf16; g (log decay), beta [B, NV] fp32.
    Returns o = qn^T S' [B, NV, DV] bf16."""
    dev = state.device
    _chk(state, "state", torch.float32)
    B, nv, dk, dv = state.shape
    nk = q.shape[1]
    _chk(q, "q", torch.bfloat16, (B, nk, dk), dev)
    _chk(k, "k", torch.bfloat16, (B, nk, dk), dev)
    _chk(v, "v", torch.bfloat16, (B, nv, dv), dev)
    _chk(g, "g", torch.float32, (B, nv), dev)
    _chk(beta, "beta", torch.float32, (B, nv), dev)
    scale = dk**-0.5 if scale is None else scale
    o = out if out is not None else torch.empty(B, nv, dv, dtype=torch.bfloat16, device=dev)
    _chk(o, "out", torch.bfloat16, (B, nv, dv), dev)
    call("qs_gdn_decode_step", _p(q), _p(k), _p(v), _p(g), _p(beta), _p(state), _p(o),
         B, nk, nv, dk, dv, float(scale), float(eps), _stream(dev))  # fmt: skip
    return o


def gdn_decode_fused(x, conv_state, taps, g, beta, state, nk=NK, scale=None, eps=EPS, out=None, y_out=None,
                     ws=None, lens=None, z=None, norm_w=None):  # fmt: skip
    """Conv1d update + L2-norm + delta rule of one decode step in one launch (model.py:255-273).

    x [B, C] bf16 is the projection's q|k|v slice (C = 2 nk DK + NV DV); conv_state [B, C, 3] and state
    [B, NV, DK, DV] are updated in place. Returns o [B, NV, DV] bf16 (y_out, if given, receives the conv
    output [B, C]). lens [B] int32 (optional, the step's lengths): users with lens < 0 are idle slots, left
    untouched. With z [B, NV DV] (or [B, NV, DV]; rows may be strided, e.g. a slice of the projection output)
    and norm_w [DV] fp32 the mixer's gated RMSNorm epilogue runs in the same launch (model.py:274-275): o is
    bf16(rmsnorm(o) norm_w silu(z)) per value head, normalised from the fp32 o."""
    dev = state.device
    _chk(state, "state", torch.float32)
    B, nv, dk, dv = state.shape
    C = 2 * nk * dk + nv * dv
    _chk(x, "x", torch.bfloat16, (B, C), dev)
    _chk(conv_state, "conv_state", torch.bfloat16, (B, C, CONV_K - 1), dev)
    _chk(taps, "taps", torch.bfloat16, (C, CONV_K), dev)
    _chk(g, "g", torch.float32, (B, nv), dev)
    _chk(beta, "beta", torch.float32, (B, nv), dev)
    if y_out is not None:
        _chk(y_out, "y_out", torch.bfloat16, (B, C), dev)
    scale = dk**-0.5 if scale is None else scale
    o = out if out is not None else torch.empty(B, nv, dv, dtype=torch.bfloat16, device=dev)
    _chk(o, "out", torch.bfloat16, (B, nv, dv), dev)
    if ws is None:
        ws = workspace("gdn", lib().qs_gdn_workspace_bytes(B, nk), dev)
    if lens is not None:
        _chk(lens, "lens", torch.int32, (B,), dev)
    ldz = 0
    if (z is None) != (norm_w is None):
        raise ValueError("give both z and norm_w or neither")
    if z is not None:
        if not isinstance(z, torch.Tensor) or not z.is_cuda or z.dtype != torch.bfloat16 or z.device != dev:
            raise ValueError(f"z must be a bf16 tensor on {dev}")
        z = z.reshape(B, nv * dv) if z.dim() == 3 and z.is_contiguous() else z
        if z.dim() != 2 or tuple(z.shape) != (B, nv * dv) or z.stride(1) != 1:
            raise ValueError(f"z must be [B, NV DV] = [{B}, {nv * dv}] with unit column stride")
        ldz = z.stride(0) if B > 1 else nv * dv
        _chk(norm_w, "norm_w", torch.float32, (dv,), dev)
    call("qs_gdn_decode_fused", _p(x), _p(conv_state), _p(taps), _p(g), _p(beta), _p(state), _p(o), _p(y_out),
         _p(z), ldz, _p(norm_w), _p(ws), _p(lens), B, nk, nv, dk, dv, CONV_K, float(scale), float(eps),
         _stream(dev))  # fmt: skip
    return o


# ------------------------------------------------------------------------------------------- a7


def gdn_gated_norm(o, z, norm_w, eps=EPS, out=None):
    """The GDN mixer's gated RMSNorm epilogue (model.py:274-275): bf16(rmsnorm(o) * norm_w * silu(z)) per head.
    o, z [..., DV] bf16 (same shape); norm_w [DV] fp32."""
    dev = o.device
    _chk(o, "o", torch.bfloat16)
    _chk(z, "z", torch.bfloat16, tuple(o.shape), dev)
    dv = o.shape[-1]
    _chk(norm_w, "norm_w", torch.float32, (dv,), dev)
    y = torch.empty_like(o) if out is None else out
    _chk(y, "out", torch.bfloat16, tuple(o.shape), dev)
    call("qs_gdn_gated_norm", _p(o), _p(z), _p(norm_w), _p(y), o.numel() // dv, dv, float(eps), _stream(dev))
    return y


def gdn_verify_step(x, conv_state, taps, g, beta, state, nk=NK, scale=None, eps=EPS, return_y=False, out=None,
                    lens=None):  # fmt: skip
    """T tokens per user through conv + delta rule, keeping every intermediate (the verify rows of the
    reference GDN head cores, kernels/gdn_head_reader.cpp:149-187, gdn_head_writer.cpp:60-66).

    x [B, T, C]; g, beta [B, T, NV]; conv_state [B, C, 3] and state [B, NV, DK, DV] are read only.
    Returns o [B, T, NV, DV] bf16, states [T, B, NV, DK, DV] fp32, conv_states [T, B, C, 3] bf16
    (and the conv outputs y [B, T, C] with return_y). ``out`` = (o, states, conv_states) preallocated.
    lens [B] int32 (optional, the step's lengths): a user with lens < 0 is an idle slot; nothing is computed
    or written for it."""
    dev = state.device
    _chk(state, "state", torch.float32)
    B, nv, dk, dv = state.shape
    T = x.shape[1]
    C = 2 * nk * dk + nv * dv
    _chk(x, "x", torch.bfloat16, (B, T, C), dev)
    _chk(conv_state, "conv_state", torch.bfloat16, (B, C, CONV_K - 1), dev)
    _chk(taps, "taps", torch.bfloat16, (C, CONV_K), dev)
    _chk(g, "g", torch.float32, (B, T, nv), dev)
    _chk(beta, "beta", torch.float32, (B, T, nv), dev)
    scale = dk**-0.5 if scale is None else scale
    if out is None:
        o = torch.empty(B, T, nv, dv, dtype=torch.bfloat16, device=dev)
        states = torch.empty(T, B, nv, dk, dv, dtype=torch.float32, device=dev)
        convs = torch.empty(T, B, C, CONV_K - 1, dtype=torch.bfloat16, device=dev)
    else:
        o, states, convs = out
        _chk(o, "out o", torch.bfloat16, (B, T, nv, dv), dev)
        _chk(states, "out states", torch.float32, (T, B, nv, dk, dv), dev)
        _chk(convs, "out conv_states", torch.bfloat16, (T, B, C, CONV_K - 1), dev)
    y = torch.empty(B, T, C, dtype=torch.bfloat16, device=dev) if return_y else None
    if lens is not None:
        _chk(lens, "lens", torch.int32, (B,), dev)
    call("qs_gdn_verify_step", _p(x), _p(conv_state), _p(convs), _p(taps), _p(g), _p(beta), _p(state),
         _p(states), _p(o), _p(y), _p(lens), B, T, nk, nv, dk, dv, CONV_K, float(scale), float(eps),
         _stream(dev))  # fmt: skip
    return (o, states, convs, y) if return_y else (o, states, convs)


def gdn_verify_step_slots(x, conv_states_in, taps, g, beta, states_in, in_slot, out, nk=NK, scale=None, eps=EPS,
                          lens=None):  # fmt: skip
    """gdn_verify_step whose per-user input is a slot of the previous verify step's snapshots (the reference's
    slot select, kernels/gdn_head_reader.cpp:17-20): user b reads states_in[in_slot[b], b] and
    conv_states_in[in_slot[b], b]. states_in [S, B, NV, DK, DV], conv_states_in [S, B, C, 3], in_slot [B]
    int32 on the device; out = (o, states, conv_states) must not alias the inputs. lens [B] int32 (optional,
    the step's lengths): a user with lens < 0 is an idle slot, whose input slot is carried unchanged into
    the same slot of ``out`` (no token verified, no o written)."""
    dev = states_in.device
    _chk(states_in, "states_in", torch.float32)
    S, B, nv, dk, dv = states_in.shape
    T = x.shape[1]
    C = 2 * nk * dk + nv * dv
    _chk(x, "x", torch.bfloat16, (B, T, C), dev)
    _chk(conv_states_in, "conv_states_in", torch.bfloat16, (S, B, C, CONV_K - 1), dev)
    _chk(taps, "taps", torch.bfloat16, (C, CONV_K), dev)
    _chk(g, "g", torch.float32, (B, T, nv), dev)
    _chk(beta, "beta", torch.float32, (B, T, nv), dev)
    _chk(in_slot, "in_slot", torch.int32, (B,), dev)
    o, states, convs = out
    _chk(o, "out o", torch.bfloat16, (B, T, nv, dv), dev)
    _chk(states, "out states", torch.float32, (T, B, nv, dk, dv), dev)
    _chk(convs, "out conv_states", torch.bfloat16, (T, B, C, CONV_K - 1), dev)
    scale = dk**-0.5 if scale is None else scale
    if lens is not None:
        _chk(lens, "lens", torch.int32, (B,), dev)
    call("qs_gdn_verify_step_slots", _p(x), _p(conv_states_in), _p(convs), _p(taps), _p(g), _p(beta), _p(states_in),
         _p(states), _p(in_slot), S, _p(o), None, _p(lens), B, T, nk, nv, dk, dv, CONV_K, float(scale), float(eps),
         _stream(dev))  # fmt: skip
    return o, states, convs


def verify_accept(accept_len, T, slot, seq_lens=None, base_lens=None, status=None):
    """Acceptance by slot selection: slot <- accept_len - 1 (the snapshot the next verify step reads) and
    seq_lens <- base_lens + accept_len when given; no state moves (kernels/mlp_hub.cpp:48-58). An accept
    length outside [1, T] leaves the user untouched and sets QS_STATUS_ACCEPT in ``status``; an idle slot
    (base_lens < 0) keeps its slot and length."""
    dev = slot.device
    B = slot.shape[0]
    _chk(accept_len, "accept_len", torch.int32, (B,), dev)
    _chk(slot, "slot", torch.int32, (B,), dev)
    if seq_lens is not None:
        _chk(seq_lens, "seq_lens", torch.int32, (B,), dev)
        _chk(base_lens, "base_lens", torch.int32, (B,), dev)
    call("qs_verify_accept", _p(accept_len), _p(slot), _p(seq_lens), _p(base_lens), B, T, _p(status), _stream(dev))


def gdn_rollback(states, conv_states, accept_len, state, conv_state, seq_lens=None, base_lens=None):
    """Restore state <- states[accept_len - 1], conv_state <- conv_states[accept_len - 1] per user (bit-exact),
    and seq_lens <- base_lens + accept_len when given (the KV truncation). accept_len [B] int32 on device,
    each in [1, T] (the reference's slot/ring advance, kernels/mlp_hub.cpp:48-58); an idle slot (base_lens
    < 0) is left untouched."""
    dev = state.device
    T, B, nv, dk, dv = states.shape
    C = conv_states.shape[2]
    _chk(states, "states", torch.float32, None, dev)
    _chk(conv_states, "conv_states", torch.bfloat16, (T, B, C, CONV_K - 1), dev)
    _chk(state, "state", torch.float32, (B, nv, dk, dv), dev)
    _chk(conv_state, "conv_state", torch.bfloat16, (B, C, CONV_K - 1), dev)
    _chk(accept_len, "accept_len", torch.int32, (B,), dev)
    if seq_lens is not None:
        _chk(seq_lens, "seq_lens", torch.int32, (B,), dev)
        _chk(base_lens, "base_lens", torch.int32, (B,), dev)
    call("qs_gdn_rollback", _p(states), _p(state), _p(conv_states), _p(conv_state), _p(accept_len), _p(seq_lens),
         _p(base_lens), B, T, nv, dk, dv, C, CONV_K, _stream(dev))  # fmt: skip


def gdn_rollback_layers(states, conv_states, accept_len, state, conv_state, seq_lens=None, base_lens=None):
    """gdn_rollback for L layers in one launch: states [L, T, B, NV, DK, DV], conv_states [L, T, B, C, K-1],
    state [L, B, NV, DK, DV], conv_state [L, B, C, K-1] (each layer's slice contiguous; the layer stride
    is read from the tensor), seq_lens set once (the hub's all-layer slot switch, kernels/mlp_hub.cpp:48-58)."""
    dev = state.device
    L, T, B, nv, dk, dv = states.shape
    C = conv_states.shape[3]
    for name, t, dt, shp in (("states", states, torch.float32, (L, T, B, nv, dk, dv)),
                             ("conv_states", conv_states, torch.bfloat16, (L, T, B, C, CONV_K - 1)),
                             ("state", state, torch.float32, (L, B, nv, dk, dv)),
                             ("conv_state", conv_state, torch.bfloat16, (L, B, C, CONV_K - 1))):  # fmt: skip
        if t.dtype != dt or tuple(t.shape) != shp or t.device != dev:
            raise ValueError(f"{name}: expected {dt} {shp} on {dev}, got {t.dtype} {tuple(t.shape)} on {t.device}")
        if not t[0].is_contiguous():
            raise ValueError(f"{name}: each layer's slice must be contiguous")
    _chk(accept_len, "accept_len", torch.int32, (B,), dev)
    if seq_lens is not None:
        _chk(seq_lens, "seq_lens", torch.int32, (B,), dev)
        _chk(base_lens, "base_lens", torch.int32, (B,), dev)
    call("qs_gdn_rollback_layers", _p(states), states.stride(0), _p(state), state.stride(0), _p(conv_states),
         conv_states.stride(0), _p(conv_state), conv_state.stride(0), _p(accept_len), _p(seq_lens), _p(base_lens),
         L, B, T, nv, dk, dv, C, CONV_K, _stream(dev))  # fmt: skip


# ------------------------------------------------------------------------------------------- a5, a9


def _pool_dims(k_cache, v_cache, dev):
    _chk(k_cache, "k_cache", torch.bfloat16, None, dev)
    _chk(v_cache, "v_cache", torch.bfloat16, tuple(k_cache.shape), dev)
    if k_cache.dim() != 4:
        raise ValueError("KV pools must be [num_blocks, NKV, block, HD]")
    return k_cache.shape


def paged_kv_append(k, v, k_cache, v_cache, block_table, positions, status=None):
    """Write T new rows per user at positions[b] + t through the block table (bit-exact copies).

    k, v [B, T, NKV, HD] bf16; pools [num_blocks, NKV, block, HD]; block_table [B, max_blocks] int32;
    positions [B] int32 (first new position; negative = idle slot). Rows past the table or on an entry
    outside the pool are skipped and reported in ``status``."""
    dev = k_cache.device
    nb, nkv, block, hd = _pool_dims(k_cache, v_cache, dev)
    B, T = k.shape[:2]
    _chk(k, "k", torch.bfloat16, (B, T, nkv, hd), dev)
    _chk(v, "v", torch.bfloat16, (B, T, nkv, hd), dev)
    _chk(block_table, "block_table", torch.int32, None, dev)
    if block_table.dim() != 2 or block_table.shape[0] != B:
        raise ValueError(f"block_table must be [B={B}, max_blocks]")
    _chk(positions, "positions", torch.int32, (B,), dev)
    call("qs_paged_kv_append", _p(k), _p(v), _p(k_cache), _p(v_cache), _p(block_table), _p(positions),
         B, T, nkv, hd, block, block_table.shape[1], nb, _p(status), _stream(dev))  # fmt: skip


def paged_kv_fill(k, v, k_cache, v_cache, page_table, start=0):
    """Fill one sequence's K and V [NKV, T, HD] into the pools through its page table [n] (int32)."""
    dev = k_cache.device
    nb, nkv, block, hd = _pool_dims(k_cache, v_cache, dev)
    T = k.shape[1]
    _chk(k, "k", torch.bfloat16, (nkv, T, hd), dev)
    _chk(v, "v", torch.bfloat16, (nkv, T, hd), dev)
    _chk(page_table, "page_table", torch.int32, None, dev)
    if page_table.dim() != 1:
        raise ValueError("page_table must be one sequence's [n] table")
    call("qs_paged_kv_fill", _p(k), _p(v), _p(k_cache), _p(v_cache), _p(page_table), T, int(start), nkv, hd,
         block, page_table.shape[0], nb, _stream(dev))  # fmt: skip


def paged_kv_gather(k_cache, v_cache, page_table, n, start=0):
    """Positions start .. start+n-1 of one sequence out of the pools into contiguous K, V [NKV, n, HD]: the
    inverse of paged_kv_fill (the KV export of prefill/pp_prefill.py:1241-1249). page_table [m] int32."""
    dev = k_cache.device
    nb, nkv, block, hd = _pool_dims(k_cache, v_cache, dev)
    _chk(page_table, "page_table", torch.int32, None, dev)
    if page_table.dim() != 1:
        raise ValueError("page_table must be one sequence's [n] table")
    k = torch.empty(nkv, n, hd, dtype=torch.bfloat16, device=dev)
    v = torch.empty_like(k)
    call("qs_paged_kv_gather", _p(k_cache), _p(v_cache), _p(page_table), _p(k), _p(v), int(n), int(start), nkv, hd,
         block, page_table.shape[0], nb, _stream(dev))  # fmt: skip
    return k, v


def paged_fill_cache(cache, x, page_table, batch_idx=0):
    """``ttnn.experimental.paged_fill_cache(cache, x, page_table, batch_idx)`` (prefill/pp_prefill.py:826-827).

    cache [num_blocks, NKV, block, HD] bf16; x [1, NKV, T, HD] bf16; page_table [B, n] int32: token i goes
    to page page_table[batch_idx, i // block], row i % block."""
    dev = cache.device
    _chk(cache, "cache", torch.bfloat16, None, dev)
    nb, nkv, block, hd = cache.shape
    if x.dim() != 4 or x.shape[0] != 1:
        raise ValueError("x must be [1, NKV, T, HD]")
    T = x.shape[2]
    _chk(x, "x", torch.bfloat16, (1, nkv, T, hd), dev)
    _chk(page_table, "page_table", torch.int32, None, dev)
    row = page_table[batch_idx]
    call("qs_paged_kv_fill", _p(x), None, _p(cache), None, ctypes.c_void_p(row.data_ptr()), T, 0, nkv, hd, block,
         row.shape[0], nb, _stream(dev))  # fmt: skip


# ------------------------------------------------------------------------------------------- a6


def attention_workspace(B, T, nq, nkv, max_blocks, pages_per_split, device):
    nbytes = lib().qs_paged_attention_workspace_bytes(B, T, nq, nkv, HD, max_blocks, pages_per_split)
    return workspace(("attn", pages_per_split), nbytes, device)


def paged_gqa_decode(q, k_cache, v_cache, block_table, seq_lens, scale, k_new=None, v_new=None,
                     pages_per_split=8, out=None, ws=None, status=None):  # fmt: skip
    """Paged GQA decode attention ``softmax(q K^T scale) V`` over each user's pages (model.py:239-244).

    q [B, T, NQ, HD] bf16; seq_lens [B] int32 = valid positions after this step; query t of user b sees
    positions 0 .. seq_lens[b] - T + t. With k_new, v_new [B, T, NKV, HD] the new rows are appended in the
    same launch. A user with seq_lens[b] < T is an idle slot (zero output, nothing appended); lengths past
    the block table and table entries outside the pool are reported in ``status`` (an int32 device word,
    ``Status``). Returns o [B, T, NQ, HD] bf16."""
    dev = k_cache.device
    nb, nkv, block, hd = _pool_dims(k_cache, v_cache, dev)
    B, T, nq = q.shape[:3]
    _chk(q, "q", torch.bfloat16, (B, T, nq, hd), dev)
    if (k_new is None) != (v_new is None):
        raise ValueError("give both k_new and v_new or neither")
    if k_new is not None:
        _chk(k_new, "k_new", torch.bfloat16, (B, T, nkv, hd), dev)
        _chk(v_new, "v_new", torch.bfloat16, (B, T, nkv, hd), dev)
    _chk(block_table, "block_table", torch.int32, None, dev)
    if block_table.dim() != 2 or block_table.shape[0] != B:
        raise ValueError(f"block_table must be [B={B}, max_blocks]")
    _chk(seq_lens, "seq_lens", torch.int32, (B,), dev)
    mb = block_table.shape[1]
    o = out if out is not None else torch.empty(B, T, nq, hd, dtype=torch.bfloat16, device=dev)
    _chk(o, "out", torch.bfloat16, (B, T, nq, hd), dev)
    if ws is None and (mb + pages_per_split - 1) // pages_per_split > 1:
        ws = attention_workspace(B, T, nq, nkv, mb, pages_per_split, dev)
    call("qs_paged_gqa_decode", _p(q), _p(k_new), _p(v_new), _p(k_cache), _p(v_cache), _p(block_table),
         _p(seq_lens), _p(o), _p(ws), B, T, nq, nkv, hd, block, mb, nb, int(pages_per_split), float(scale),
         _p(status), _stream(dev))  # fmt: skip
    return o


# ------------------------------------------------------------------------------------------- a8


def causal_conv1d_prefill(x, taps, conv_state=None, conv_state_out=None, nk=NK, nv=NV):
    """silu(causal conv1d) of a prompt's q | k | v columns into q, k, v with the carry
    (prefill/pp_prefill.py:384-445; the conv history handed to the decode, prefill/pp_prefill.py:1128-1175).

    x [T, >= C] bf16 with unit column stride (the projection output; its first C = 2 nk DK + nv DV columns
    are the conv channels), taps [C, K] bf16, conv_state [C, K-1] bf16 or None (a fresh prompt: zeros).
    conv_state_out [C, K-1] receives the last K-1 inputs (the decode conv state; it may be conv_state
    itself, a new tensor when None). Returns (q [T, nk, DK], k [T, nk, DK], v [T, nv, DV], conv_state_out)."""
    dev = x.device
    CQ, CV = nk * DK, nv * DV
    C = 2 * CQ + CV
    if not isinstance(x, torch.Tensor) or x.dim() != 2 or not x.is_cuda or x.dtype != torch.bfloat16:
        raise ValueError("x must be a 2-D bf16 tensor on a GPU")
    T = x.shape[0]
    if x.shape[1] < C or (T > 0 and x.stride(1) != 1):
        raise ValueError(f"x must hold the {C} conv channels in unit-stride columns (got {tuple(x.shape)})")
    ldx = x.stride(0) if T > 1 else C
    _chk(taps, "taps", torch.bfloat16, (C, CONV_K), dev)
    if conv_state is not None:
        _chk(conv_state, "conv_state", torch.bfloat16, (C, CONV_K - 1), dev)
    if conv_state_out is None:
        conv_state_out = torch.empty(C, CONV_K - 1, dtype=torch.bfloat16, device=dev)
    _chk(conv_state_out, "conv_state_out", torch.bfloat16, (C, CONV_K - 1), dev)
    q = torch.empty(T, nk, DK, dtype=torch.bfloat16, device=dev)
    k = torch.empty(T, nk, DK, dtype=torch.bfloat16, device=dev)
    v = torch.empty(T, nv, DV, dtype=torch.bfloat16, device=dev)
    call("qs_conv1d_prefill", _p(x), ldx, _p(conv_state), _p(taps), _p(q), _p(k), _p(v), _p(conv_state_out), T, CQ,
         CV, CONV_K, _stream(dev))  # fmt: skip
    return q, k, v, conv_state_out


def chunk_gated_delta_rule(q, k, v, g, beta, *, scale=None, initial_state=None, output_final_state=True,
                           chunk_size=64, output_head_major=False, memory_config=None, eye=None, tril=None,
                           ones=None, masks=None, eps=EPS, ws=None, final_state=None):  # fmt: skip
    """``chunk_gated_delta_rule(q, k, v, g, beta, *, scale, initial_state, output_final_state, chunk_size,
    output_head_major, memory_config, eye, tril, ones, masks)`` exactly as the reference prefill calls it
    (prefill/pp_prefill.py:791-807).

    q, k [T, NK*DK] or [T, NK, DK] bf16 token-major (L2-normalised inside, q times scale), v [T, NV*DV] or
    [T, NV, DV] bf16, g, beta [T, NV] fp32, initial_state [NV, DK, DV] fp32. The reference's per-device
    tensors carry a leading batch dimension of 1 (q [1, T, NK*DK], g [1, T, NV], initial_state
    [1, NV, DK, DV]); that form is accepted too and keeps the dimension on the outputs.
    Returns (o, final_state): o [T, NV, DV] bf16 ([NV, T, DV] with output_head_major), final_state
    [NV, DK, DV] fp32 (None unless output_final_state). final_state, when given, is written in place (it may
    be initial_state, or one user's slot of the decode state [B, NV, DK, DV], which hands the prompt's state
    to the decode without a copy).

    chunk_size: 32 (the reference's) or 64. The chunked form equals the recurrence for any chunk size, so
    both run the kernels' 64-token chunks. memory_config, eye, tril, ones and masks are the ttnn
    implementation's memory placement and its precomputed constant tiles; the HIP kernels need none of
    them, so they are accepted and ignored."""
    del memory_config, eye, tril, ones, masks
    if chunk_size not in (32, 64):
        raise ValueError(f"chunk_size must be 32 or 64 (got {chunk_size})")
    batched = isinstance(g, torch.Tensor) and g.dim() == 3
    if batched:
        if g.shape[0] != 1:
            raise ValueError(f"one sequence per call: the leading batch dimension must be 1 (g {tuple(g.shape)})")
        for name, t in (("q", q), ("k", k), ("v", v), ("beta", beta)):
            if not isinstance(t, torch.Tensor) or t.dim() < 2 or t.shape[0] != 1:
                raise ValueError(f"{name} must carry the leading batch dimension 1 like g")
        q, k, v, g, beta = q[0], k[0], v[0], g[0], beta[0]
        if initial_state is not None:
            if initial_state.dim() != 4 or initial_state.shape[0] != 1:
                raise ValueError("initial_state must be [1, NV, DK, DV] in the batched form")
            initial_state = initial_state[0]
        if final_state is not None:
            final_state = final_state[0] if final_state.dim() == 4 else final_state
    dev = q.device
    T = q.shape[0]
    nv = g.shape[1]
    q3 = q.reshape(T, -1, DK)
    nk = q3.shape[1]
    _chk(q3, "q", torch.bfloat16, (T, nk, DK), dev)
    _chk(k.reshape(T, -1, DK), "k", torch.bfloat16, (T, nk, DK), dev)
    _chk(v.reshape(T, -1, DV), "v", torch.bfloat16, (T, nv, DV), dev)
    _chk(g, "g", torch.float32, (T, nv), dev)
    _chk(beta, "beta", torch.float32, (T, nv), dev)
    if initial_state is None:
        initial_state = torch.zeros(nv, DK, DV, dtype=torch.float32, device=dev)
    _chk(initial_state, "initial_state", torch.float32, (nv, DK, DV), dev)
    scale = DK**-0.5 if scale is None else scale
    o = torch.empty(T, nv, DV, dtype=torch.bfloat16, device=dev)
    S = torch.empty(nv, DK, DV, dtype=torch.float32, device=dev) if final_state is None else final_state
    _chk(S, "final_state", torch.float32, (nv, DK, DV), dev)
    if ws is None:
        nbytes = lib().qs_gdn_chunk_prefill_workspace_bytes(T, nk, nv, DK, DV, int(chunk_size))
        ws = workspace("prefill", nbytes, dev)
    call("qs_gdn_chunk_prefill", _p(q), _p(k), _p(v), _p(g), _p(beta), _p(initial_state), _p(o), _p(S), _p(ws),
         T, nk, nv, DK, DV, int(chunk_size), float(scale), float(eps), _stream(dev))  # fmt: skip
    if output_head_major:
        o = o.transpose(0, 1).contiguous()
    S = S if output_final_state else None
    if batched:
        return o[None], (S[None] if S is not None else None)
    return o, S


# ------------------------------------------------------------------------------ the attention mixer's edges


def rope_tables(positions, rot=ROT, theta=ROPE_THETA):
    """cos, sin [..., rot / 2] fp32 of integer positions (any shape, on the positions' device), computed in
    float64 as model.py:128-132 does."""
    inv = 1.0 / theta ** (torch.arange(0, rot, 2, dtype=torch.float64, device=positions.device) / rot)
    ang = positions.to(torch.float64)[..., None] * inv
    return torch.cos(ang).float().contiguous(), torch.sin(ang).float().contiguous()


def attn_mixer_decode(q, k_new, v_new, gate, wq, wk, cos, sin, k_cache, v_cache, block_table, seq_lens,
                      pages_per_split=8, eps=EPS, rot=ROT, out=None, ws=None, status=None):  # fmt: skip
    """The attention mixer of a decode (T = 1) or verify (T > 1) step around the paged cache (model.py:237-246):
    qn = rope(rmsnorm(q) * wq), kn = bf16(rope(rmsnorm(k_new) * wk)) appended with v_new at positions
    seq_lens - T + t, o = bf16(softmax(qn K^T) V * sigmoid(gate)).

    q, gate [B, T, NQ, HD] bf16; k_new, v_new [B, T, NKV, HD] bf16; wq, wk [HD] fp32 (wq carries the softmax
    scale, model.py:237); cos, sin [B, T, rot / 2] fp32 (``rope_tables``); the rest as ``paged_gqa_decode``."""
    dev = k_cache.device
    nb, nkv, block, hd = _pool_dims(k_cache, v_cache, dev)
    B, T, nq, _ = q.shape
    _chk(q, "q", torch.bfloat16, (B, T, nq, hd), dev)
    _chk(gate, "gate", torch.bfloat16, (B, T, nq, hd), dev)
    _chk(k_new, "k_new", torch.bfloat16, (B, T, nkv, hd), dev)
    _chk(v_new, "v_new", torch.bfloat16, (B, T, nkv, hd), dev)
    _chk(wq, "wq", torch.float32, (hd,), dev)
    _chk(wk, "wk", torch.float32, (hd,), dev)
    if rot:
        _chk(cos, "cos", torch.float32, (B, T, rot // 2), dev)
        _chk(sin, "sin", torch.float32, (B, T, rot // 2), dev)
    _chk(block_table, "block_table", torch.int32, None, dev)
    _chk(seq_lens, "seq_lens", torch.int32, (B,), dev)
    mb = block_table.shape[1]
    o = torch.empty(B, T, nq, hd, dtype=torch.bfloat16, device=dev) if out is None else out
    if ws is None:
        ws = attention_workspace(B, T, nq, nkv, mb, pages_per_split, dev)
    call("qs_attn_mixer_decode", _p(q), _p(k_new), _p(v_new), _p(gate), _p(wq), _p(wk),
         _p(cos if rot else None), _p(sin if rot else None), rot, _p(k_cache), _p(v_cache), _p(block_table),
         _p(seq_lens), _p(o), _p(ws), B, T, nq, nkv, hd, block, mb, nb, pages_per_split, float(eps), _p(status),
         _stream(dev))  # fmt: skip
    return o


# ----------------------------------------------------------- weight-streaming projections and the MLP half

HIDDEN, INTER = 5120, 17408  # common.py:13-14
MXFP4, MXFP8, MXINT8 = 4, 8, 9  # fmt codes of include/qwen_state.h


class MxWeight:
    """A weight W [K, N] (y = h W) quantized on the device to OCP MXFP4, MXINT8 or MXFP8 and laid out in the
    kernels' fragment order (the reference quantizes to 4- / 8-bit block floating point on the host and lays
    the tiles out per DRAM bank: common.py:115-116, tests/bench_resident_mlp.py:51-96). MXINT8 keeps a sign
    and 7 magnitude bits per value, the precision of the reference's bfloat8_b (model.py:53-58)."""

    def __init__(self, packed, K, N, fmt):
        self.packed, self.K, self.N, self.fmt = packed, K, N, fmt

    @classmethod
    def quantize(cls, w, fmt):
        """Quantize an fp32 [K, N] weight on its device (32 values along K per E8M0 scale)."""
        dev = w.device
        K, N = w.shape
        _chk(w, "w", torch.float32, (K, N), dev)
        nbytes = lib().qs_mx_packed_bytes(K, N, fmt)
        if nbytes == 0:
            raise ValueError(f"fmt {fmt} (4, 8 or 9) needs N % 16 == 0 and K % {128 if fmt == MXFP4 else 64} == 0 "
                             f"(got K {K}, N {N})")  # fmt: skip
        packed = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        call("qs_mx_quantize", _p(w), _p(packed), K, N, int(fmt), _stream(dev))
        return cls(packed, K, N, fmt)


def mx_linear(h, weight, out=None, ws=None):
    """y = h W for 1..16 rows h [B, K] bf16 and a streamed MxWeight: the reference's M = 1 projections of
    rmsnorm'd rows through the weight ring (kernels/streamer_compute.cpp:371-449). Returns y [B, N] fp32."""
    dev = h.device
    B = h.shape[0]
    _chk(h, "h", torch.bfloat16, (B, weight.K), dev)
    if not 1 <= B <= 16:
        raise ValueError(f"1 to 16 rows (got {B})")
    y = torch.empty(B, weight.N, dtype=torch.float32, device=dev) if out is None else out
    _chk(y, "out", torch.float32, (B, weight.N), dev)
    if ws is None:
        ws = workspace(("mx_gemv", weight.fmt), lib().qs_mx_gemv_workspace_bytes(B, weight.K, weight.N, weight.fmt), dev)
    call("qs_mx_gemv", _p(h), _p(weight.packed), _p(y), _p(ws), B, weight.K, weight.N, int(weight.fmt), _stream(dev))
    return y


def mlp_decode(x, gamma, gate, up, down, eps=EPS, out=None, ws=None):
    """The MLP half of a decoder layer for 1..16 rows (tests/bench_resident_mlp.py:98-105):
    x + (silu(h G) * (h U)) D with h = bf16(x * rsqrt(mean(x^2) + eps) * gamma), z = silu(h G) * (h U) kept
    in bf16. x [B, H] fp32, gamma [H] fp32 or None when the norm weight is folded into the rows of gate and up
    (weights.py:107-112); gate, up MxWeight MXFP4 [H, I]; down MxWeight MXINT8 (the reference's 8-bit
    precision) or MXFP8 [I, H]. Returns x_out [B, H] fp32 (``out`` may be ``x``)."""
    dev = x.device
    B, H = x.shape
    _chk(x, "x", torch.float32, (B, H), dev)
    if gamma is not None:
        _chk(gamma, "gamma", torch.float32, (H,), dev)
    I = gate.N
    for w, name, shape, fmts in ((gate, "gate", (H, I), (MXFP4,)), (up, "up", (H, I), (MXFP4,)),
                                 (down, "down", (I, H), (MXINT8, MXFP8))):  # fmt: skip
        if (w.K, w.N) != shape or w.fmt not in fmts:
            raise ValueError(f"{name} must be a {shape} weight in format {' or '.join(map(str, fmts))} "
                             f"(got {(w.K, w.N)} format {w.fmt})")  # fmt: skip
    nbytes = lib().qs_mlp_decode_workspace_bytes(B, H, I)
    if nbytes == 0:
        raise ValueError(f"1 to 16 rows, H % 128 == 0, I % 64 == 0 (got B {B}, H {H}, I {I})")
    y = torch.empty_like(x) if out is None else out
    _chk(y, "out", torch.float32, (B, H), dev)
    if ws is None:
        ws = workspace("mlp", nbytes, dev)
    call("qs_mlp_decode", _p(x), _p(gamma), _p(gate.packed), _p(up.packed), _p(down.packed), int(down.fmt), _p(y),
         _p(ws), B, H, I, float(eps), _stream(dev))  # fmt: skip
    return y
