"""The decode-step and verify-step state path of the 64-layer hybrid engine, over caller-owned buffers.

``StatePathStep`` is ``ResidentModel.step`` (model.py:1499-1508) restricted to the state path: every step
first advances each user's position by one (the position advance of ``token_state``, model.py:1314-1351),
then runs the 64 layers in order (attention iff (l + 1) % interval == 0, model.py:93-94): a GDN layer runs
the fused conv1d update + L2-norm + delta rule with its fp32 state and conv history updated in place; an
attention layer appends the step's K/V row into its paged pools at the user's position and runs paged GQA
decode over positions 0 .. that position. In the engine each layer's inputs come from the previous layer's
projections (outside this path), so the step is a chain of dependent launches; ``capture()`` records it as
one HIP graph (the resident engine's trace replay, model.py:1485-1508), and each replay advances the
positions by itself on the device.

``VerifyStep`` is the MTP verify step (model.py:426-456, the reference's 2-row form generalised to T rows):
positions advance by T, every GDN layer keeps its T intermediate states and conv histories, every attention
layer appends T rows and attends causally among them, and the acceptance of a per-user length a (device
memory) selects snapshot a - 1 and sets the length to the rows cached before the step plus a
(kernels/mlp_hub.cpp:48-58).

The caller owns every buffer; a step allocates nothing. ``synthetic()`` builds seeded buffers of the
benchmark shapes (each layer independently seeded, so each layer can be checked against its own oracle
call).
"""
import torch

from . import ops
from . import workloads as W
from .ops import BLOCK, CONV_K, DK, DV, HD, NK, NKV, NQ, NV


def is_attn(l, interval):
    """model.py:93-94"""
    return interval > 0 and (l + 1) % interval == 0


def layer_bytes(B, ctx, T=1, attn=False, snapshots=False):
    """Algorithmic HBM bytes of one layer of the step (each tensor the path must read or write, once).

    GDN: state read + write (T snapshot writes in verify), conv state read + write (T snapshots), taps,
    the projection slice x, g and beta, the output o. Attention: K and V of all ctx positions per KV head,
    the T new rows (read from the inputs + written to the pages), q, o, the user's block-table row."""
    if not attn:
        st = B * NV * DK * DV * 4
        conv = B * W.C_QKV * (CONV_K - 1) * 2
        writes = T if snapshots else 1
        return (st + writes * st) + (conv + writes * conv) + W.C_QKV * CONV_K * 2 + B * T * (
            W.C_QKV * 2 + NV * 8 + NV * DV * 2
        )
    row = NKV * HD * 2
    pages = (ctx + BLOCK - 1) // BLOCK
    return B * (2 * ctx * row + 2 * 2 * T * row + T * NQ * HD * 2 * 2 + pages * 4)


def step_bytes(B, ctx, layers=64, interval=4, T=1):
    n_attn = sum(is_attn(l, interval) for l in range(layers))
    return (layers - n_attn) * layer_bytes(B, ctx, T, False, T > 1) + n_attn * layer_bytes(B, ctx, T, True)


def _check_table(block_table, lens, B, device):
    ops._chk(block_table, "block_table", torch.int32, None, device)
    if block_table.dim() != 2 or block_table.shape[0] != B:
        raise ValueError(f"block_table must be [B={B}, max_blocks]")
    ops._chk(lens, "lens", torch.int32, (B,), device)


def _synthetic_layers(B, ctx, layers, interval, device, seed, num_blocks, T, table):
    """Seeded per-layer inputs and resident buffers; attention layers share ``table``."""
    out = []
    for l in range(layers):
        if is_attn(l, interval):
            d = W.attn_layer(B, ctx, device, seed=seed + 1000 + l, T=T, num_blocks=num_blocks)
            del d["block_table"], d["seq_lens"]
            d["o"] = torch.empty(B, T, NQ, HD, dtype=torch.bfloat16, device=device)
            d["attn"] = True
        else:
            d = W.gdn_layer(B, device, seed=seed + l, T=None if T == 1 else T)
            for k in ("q", "k", "v"):
                d.pop(k, None)
            d["o"] = torch.empty((B, NV, DV) if T == 1 else (B, T, NV, DV), dtype=torch.bfloat16, device=device)
            d["attn"] = False
        out.append(d)
    return out


def _synthetic_table(B, ctx, device, seed, num_blocks, max_blocks):
    pages = (ctx + BLOCK - 1) // BLOCK
    max_blocks = pages if max_blocks is None else max_blocks
    if max_blocks < pages:
        raise ValueError(f"max_blocks {max_blocks} cannot hold {ctx} positions")
    if B * max_blocks > num_blocks:
        raise ValueError(f"{B} users x {max_blocks} pages do not fit a {num_blocks}-page pool")
    return W.block_tables(B, max_blocks, num_blocks, device, seed)


class StatePathStep:
    """One decode step (one token per user) of the state path over caller-owned buffers.

    layers: one dict per layer, caller-owned (``synthetic`` shows the shapes):
      GDN        x [B, C] bf16, g, beta [B, NV] fp32 (this step's inputs); state [B, NV, DK, DV] fp32,
                 conv_state [B, C, 3] bf16 (resident, updated in place); taps [C, 4] bf16; o [B, NV, DV] bf16
      attention  q [B, 1, NQ, HD], k_new, v_new [B, 1, NKV, HD] bf16 (inputs); k_cache, v_cache
                 [num_blocks, NKV, 64, HD] bf16 (resident); scale; o [B, 1, NQ, HD] bf16
    block_table [B, max_blocks] int32 (shared by the attention layers, vLLM's contract); lens [B] int32 on the
    device: the rows cached per user before the next step (negative = idle slot), advanced by every step.
    status: an ``ops.Status`` the kernels report invalid lengths and table entries into, or None."""

    def __init__(self, layers, block_table, lens, interval=4, pages_per_split=8, status=None):
        self.layer = layers
        self.layers, self.interval = len(layers), interval
        self.block_table, self.lens = block_table, lens
        self.device = lens.device
        self.B = lens.shape[0]
        _check_table(block_table, lens, self.B, self.device)
        for l, d in enumerate(layers):
            if bool(d["attn"]) != is_attn(l, interval):
                raise ValueError(f"layer {l}: the layer pattern is attention iff (l + 1) % {interval} == 0")
        self.max_len = block_table.shape[1] * BLOCK
        self.pps = pages_per_split
        self.status = status
        self.gdn_ws = torch.zeros(max(ops.lib().qs_gdn_workspace_bytes(self.B, NK), 256), dtype=torch.uint8,
                                  device=self.device)  # fmt: skip
        nbytes = ops.lib().qs_paged_attention_workspace_bytes(self.B, 1, NQ, NKV, HD, block_table.shape[1],
                                                              pages_per_split)  # fmt: skip
        self.attn_ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)
        self.graph = None

    @classmethod
    def synthetic(cls, B, ctx, layers=64, interval=4, device="cuda", seed=0, num_blocks=2048, pages_per_split=8,
                  max_blocks=None, check=False):  # fmt: skip
        """Seeded buffers of the decode step at ``ctx`` positions: the first step appends at position
        ctx - 1 (lens starts at ctx - 1) and attends ctx positions. Per-user tables are disjoint slices of
        one seeded permutation of the pool; max_blocks (default ceil(ctx / 64)) sets the table width."""
        device = torch.device(device)
        table = _synthetic_table(B, ctx, device, seed, num_blocks, max_blocks)
        lay = _synthetic_layers(B, ctx, layers, interval, device, seed, num_blocks, 1, table)
        lens = torch.full((B,), ctx - 1, dtype=torch.int32, device=device)
        status = ops.Status(device) if check else None
        return cls(lay, table, lens, interval, pages_per_split, status)

    @property
    def ctx(self):
        """Positions attended by the next step of user 0 (host read: tests and reports only)."""
        return int(self.lens[0]) + 1

    def run_layer(self, l):
        d = self.layer[l]
        st = self.status.word if self.status is not None else None
        if d["attn"]:
            ops.paged_gqa_decode(d["q"], d["k_cache"], d["v_cache"], self.block_table, self.lens, d["scale"],
                                 k_new=d["k_new"], v_new=d["v_new"], pages_per_split=self.pps, out=d["o"],
                                 ws=self.attn_ws, status=st)  # fmt: skip
        else:
            ops.gdn_decode_fused(d["x"], d["conv_state"], d["taps"], d["g"], d["beta"], d["state"], out=d["o"],
                                 ws=self.gdn_ws, lens=self.lens)  # fmt: skip

    def step(self):
        """One eager step on the current stream: the position advance, then every layer in order."""
        st = self.status.word if self.status is not None else None
        ops.advance_lengths(self.lens, 1, self.max_len, status=st)
        for l in range(self.layers):
            self.run_layer(l)

    def capture(self):
        """Record one step into a HIP graph (every buffer already exists, so nothing allocates)."""
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        g = torch.cuda.CUDAGraph()
        torch.cuda.synchronize(self.device)
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self.step()
        torch.cuda.current_stream(self.device).wait_stream(s)
        self.graph = g
        return g

    def replay(self):
        self.graph.replay()

    def rewind(self, n=1):
        """Move every active user's position back by n steps (benchmark replays at a fixed context; the KV
        rows already written stay in the pages and are overwritten by the next steps)."""
        self.lens.sub_(torch.where(self.lens >= n, n, 0).to(torch.int32))

    def bytes_per_step(self, ctx=None):
        return step_bytes(self.B, self.ctx if ctx is None else ctx, self.layers, self.interval)

    def gdn_layers(self):
        return [l for l in range(self.layers) if not self.layer[l]["attn"]]

    def attn_layers(self):
        return [l for l in range(self.layers) if self.layer[l]["attn"]]

    def snapshot(self):
        """Device copy of the recurrent state (GDN states, conv histories, lengths) for restore()."""
        return [(d["state"].clone(), d["conv_state"].clone()) for d in self.layer if not d["attn"]], self.lens.clone()

    def restore(self, snap):
        gdn, lens = snap
        for d, (s, c) in zip((d for d in self.layer if not d["attn"]), gdn):
            d["state"].copy_(s)
            d["conv_state"].copy_(c)
        self.lens.copy_(lens)


class VerifyStep:
    """The MTP verify step of the state path: T tokens per user (1 accepted + T - 1 drafts) through every
    layer, then the acceptance of ``accept`` [B] int32 (device memory, e.g. the draft check's output).

    A step: lens advances by T (base <- the rows cached before the step); GDN layers keep all T intermediate
    states and conv histories; attention layers append T rows at base .. base + T - 1 and attend causally
    among them; acceptance sets lens <- base + a and makes snapshot a - 1 the current state. An idle slot
    (lens < 0) is skipped by every launch: its length, its current state and conv history and the pools
    stay as they are.

    rollback="slots" (default, the reference's scheme: slot select, no copy, README.md:413-421): two snapshot
    sets alternate; step k writes set k % 2 and reads each user's input from slot a - 1 of the other set.
    rollback="copy": every GDN layer's state and conv history are restored from snapshot a - 1 by bit-exact
    copies in one launch, and the next step reads them in place."""

    def __init__(self, layers, block_table, lens, accept, T, g_states, g_convs, g_state=None, g_conv=None,
                 interval=4, pages_per_split=2, rollback="slots", status=None):  # fmt: skip
        if rollback not in ("slots", "copy"):
            raise ValueError("rollback must be 'slots' or 'copy'")
        self.layer, self.layers, self.interval, self.T = layers, len(layers), interval, T
        self.block_table, self.lens, self.accept = block_table, lens, accept
        self.device = lens.device
        self.B = lens.shape[0]
        _check_table(block_table, lens, self.B, self.device)
        ops._chk(accept, "accept", torch.int32, (self.B,), self.device)
        self.max_len = block_table.shape[1] * BLOCK
        self.pps = pages_per_split
        self.mode = rollback
        self.status = status
        self.g_states, self.g_convs, self.g_state, self.g_conv = g_states, g_convs, g_state, g_conv
        self.base = torch.zeros_like(lens)
        self.slot = torch.zeros(self.B, dtype=torch.int32, device=self.device)
        self.parity = 0  # snapshot set the next verify step writes (slots mode)
        nbytes = ops.lib().qs_paged_attention_workspace_bytes(self.B, T, NQ, NKV, HD, block_table.shape[1],
                                                              pages_per_split)  # fmt: skip
        self.attn_ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)
        self.graphs = None

    @classmethod
    def synthetic(cls, B, ctx, T=4, layers=64, interval=4, device="cuda", seed=0, num_blocks=2048,
                  pages_per_split=2, rollback="slots", max_blocks=None, check=False):  # fmt: skip
        """Seeded buffers of the verify step at ``ctx`` positions after its T rows (lens starts at ctx - T)
        and a seeded accept length in [1, T] per user. GDN tensors live layer-major in one tensor each:
        snapshots [sets, n_gdn, T, B, ...] (2 sets in slots mode, whose set 1 starts out holding the initial
        state in slot 0) and, in copy mode, the current states [n_gdn, B, ...]."""
        device = torch.device(device)
        table = _synthetic_table(B, ctx, device, seed, num_blocks, max_blocks)
        lay = _synthetic_layers(B, ctx, layers, interval, device, seed, num_blocks, T, table)
        lens = torch.full((B,), ctx - T, dtype=torch.int32, device=device)
        gen = torch.Generator().manual_seed(seed + 7)
        accept = torch.randint(1, T + 1, (B,), generator=gen, dtype=torch.int32).to(device)
        n_gdn = sum(not d["attn"] for d in lay)
        f32, bf = torch.float32, torch.bfloat16
        sets = 2 if rollback == "slots" else 1
        g_states = torch.empty(sets, n_gdn, T, B, NV, DK, DV, dtype=f32, device=device)
        g_convs = torch.empty(sets, n_gdn, T, B, W.C_QKV, CONV_K - 1, dtype=bf, device=device)
        g_state = g_conv = None
        if rollback == "copy":
            g_state = torch.empty(n_gdn, B, NV, DK, DV, dtype=f32, device=device)
            g_conv = torch.empty(n_gdn, B, W.C_QKV, CONV_K - 1, dtype=bf, device=device)
        gi = 0
        for d in lay:
            if d["attn"]:
                continue
            if rollback == "copy":
                g_state[gi].copy_(d["state"])
                g_conv[gi].copy_(d["conv_state"])
            else:
                g_states[1, gi, 0].copy_(d["state"])
                g_convs[1, gi, 0].copy_(d["conv_state"])
            del d["state"], d["conv_state"]
            d["gi"] = gi
            gi += 1
        status = ops.Status(device) if check else None
        return cls(lay, table, lens, accept, T, g_states, g_convs, g_state, g_conv, interval, pages_per_split,
                   rollback, status)  # fmt: skip

    def _st(self):
        return self.status.word if self.status is not None else None

    def verify(self):
        """The position advance and all layers of the verify step (no acceptance): the target model's forward."""
        ops.advance_lengths(self.lens, self.T, self.max_len, base_out=self.base, status=self._st())
        p = self.parity
        for d in self.layer:
            if d["attn"]:
                ops.paged_gqa_decode(d["q"], d["k_cache"], d["v_cache"], self.block_table, self.lens, d["scale"],
                                     k_new=d["k_new"], v_new=d["v_new"], pages_per_split=self.pps, out=d["o"],
                                     ws=self.attn_ws, status=self._st())  # fmt: skip
            elif self.mode == "slots":
                gi = d["gi"]
                ops.gdn_verify_step_slots(d["x"], self.g_convs[1 - p, gi], d["taps"], d["g"], d["beta"],
                                          self.g_states[1 - p, gi], self.slot,
                                          out=(d["o"], self.g_states[p, gi], self.g_convs[p, gi]),
                                          lens=self.lens)  # fmt: skip
            else:
                gi = d["gi"]
                ops.gdn_verify_step(d["x"], self.g_conv[gi], d["taps"], d["g"], d["beta"], self.g_state[gi],
                                    out=(d["o"], self.g_states[0, gi], self.g_convs[0, gi]), lens=self.lens)  # fmt: skip

    def rollback(self):
        """Accept: select the snapshot slots (slots mode) or restore every GDN layer from its snapshot in one
        launch (copy mode), and set lens = base + accept (the KV truncation)."""
        if self.mode == "slots":
            ops.verify_accept(self.accept, self.T, self.slot, self.lens, self.base, status=self._st())
            self.parity ^= 1
        else:
            ops.gdn_rollback_layers(self.g_states[0], self.g_convs[0], self.accept, self.g_state, self.g_conv,
                                    self.lens, self.base)  # fmt: skip

    def step(self):
        self.verify()
        self.rollback()

    def capture(self):
        """Record the step as HIP graphs: one per snapshot set in slots mode (replays alternate), one in copy
        mode."""
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        torch.cuda.synchronize(self.device)
        self._p0 = self.parity
        graphs = []
        for _ in range(2 if self.mode == "slots" else 1):  # each capture of step() flips the parity
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                with torch.cuda.graph(g, stream=s):
                    self.step()
            graphs.append(g)
        torch.cuda.current_stream(self.device).wait_stream(s)
        self.graphs = graphs
        return graphs

    def replay(self):
        """One step: the graph that writes the snapshot set the next step writes."""
        if self.mode == "slots":
            self.graphs[self.parity ^ self._p0].replay()
            self.parity ^= 1
        else:
            self.graphs[0].replay()

    def rewind(self):
        """Set every length back to the rows cached before the last step (benchmark replays at a fixed
        context)."""
        self.lens.copy_(self.base)

    def state_of(self, gi, b):
        """The accepted (current) fp32 state and conv history of user b in GDN layer gi."""
        if self.mode == "slots":
            s = int(self.slot[b])
            return self.g_states[1 - self.parity, gi, s, b], self.g_convs[1 - self.parity, gi, s, b]
        return self.g_state[gi, b], self.g_conv[gi, b]

    def bytes_per_step(self, ctx):
        """Algorithmic bytes of the verify step at ``ctx`` positions after its T rows (acceptance by slot
        selection moves none; the copy mode's restore is rollback_bytes())."""
        return step_bytes(self.B, ctx, self.layers, self.interval, self.T)

    def rollback_bytes(self):
        if self.mode == "slots":
            return 0
        n_gdn = sum(not d["attn"] for d in self.layer)
        return n_gdn * self.B * (2 * NV * DK * DV * 4 + 2 * W.C_QKV * (CONV_K - 1) * 2)
