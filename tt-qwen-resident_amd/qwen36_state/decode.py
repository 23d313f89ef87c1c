"""The batched decode-step state path of the 64-layer hybrid engine, replayed as one HIP graph.

Per step and layer l (attention iff (l + 1) % interval == 0, model.py:93-94): a GDN layer runs the fused
conv1d update + L2-norm + delta rule with its fp32 state and conv history updated in place; an attention
layer appends the step's K/V rows into its paged pools and runs paged GQA decode attention. All layers
run in order on one stream (in the engine each layer's inputs come from the previous layer's projections,
which are outside this path), so the step is 64 dependent launches; ``capture()`` records them into one
HIP graph so the step costs one host submission (the resident engine's trace replay, model.py:1485-1508).

The caller owns every buffer (all allocated here once, up front); a step allocates nothing. Every layer
has its own independently seeded inputs, so each layer can be checked against its own oracle call.
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


class StatePathStep:
    """``layers`` layers of state path for B users at ``ctx`` positions (after this step's append)."""

    def __init__(self, B, ctx, layers=64, interval=4, device="cuda", seed=0, num_blocks=2048, pages_per_split=8):
        self.B, self.ctx, self.layers, self.interval = B, ctx, layers, interval
        self.device = torch.device(device)
        self.pps = pages_per_split
        pages = (ctx + BLOCK - 1) // BLOCK
        if B * pages > num_blocks:
            raise ValueError(f"{B} users x {pages} pages do not fit a {num_blocks}-page pool")
        # one block table per user shared by every attention layer (vLLM's contract); each layer owns pools
        self.block_table = W.block_tables(B, pages, num_blocks, self.device, seed)
        self.seq_lens = torch.full((B,), ctx, dtype=torch.int32, device=self.device)
        self.layer = []
        for l in range(layers):
            if is_attn(l, interval):
                d = W.attn_layer(B, ctx, self.device, seed=seed + 1000 + l, T=1, num_blocks=num_blocks)
                d["block_table"], d["seq_lens"] = self.block_table, self.seq_lens
                d["o"] = torch.empty(B, 1, NQ, HD, dtype=torch.bfloat16, device=self.device)
                d["attn"] = True
            else:
                d = W.gdn_layer(B, self.device, seed=seed + l)
                for k in ("q", "k", "v"):
                    del d[k]
                d["o"] = torch.empty(B, NV, DV, dtype=torch.bfloat16, device=self.device)
                d["attn"] = False
            self.layer.append(d)
        self.gdn_ws = ops.workspace("gdn-step", ops.lib().qs_gdn_workspace_bytes(B, NK), self.device)
        mb = self.block_table.shape[1]
        self.attn_ws = ops.attention_workspace(B, 1, NQ, NKV, mb, pages_per_split, self.device)
        self.graph = None

    def run_layer(self, l):
        d = self.layer[l]
        if d["attn"]:
            ops.paged_gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"], d["scale"],
                                 k_new=d["k_new"], v_new=d["v_new"], pages_per_split=self.pps, out=d["o"],
                                 ws=self.attn_ws)  # fmt: skip
        else:
            ops.gdn_decode_fused(d["x"], d["conv_state"], d["taps"], d["g"], d["beta"], d["state"], out=d["o"],
                                 ws=self.gdn_ws)  # fmt: skip

    def step(self):
        """One eager step: every layer in order on the current stream."""
        for l in range(self.layers):
            self.run_layer(l)

    def capture(self):
        """Record one step into a HIP graph (buffers and workspaces already exist, so nothing allocates)."""
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            # the workspaces are per stream: make the capture stream's own before capturing
            self.gdn_ws = ops.workspace("gdn-step", self.gdn_ws.numel(), self.device)
            self.attn_ws = ops.workspace(("attn", self.pps), self.attn_ws.numel(), self.device)
            torch.cuda.synchronize(self.device)
            with torch.cuda.graph(g, stream=s):
                self.step()
        torch.cuda.current_stream(self.device).wait_stream(s)
        self.graph = g
        return g

    def replay(self):
        self.graph.replay()

    def bytes_per_step(self):
        return step_bytes(self.B, self.ctx, self.layers, self.interval)

    def gdn_layers(self):
        return [l for l in range(self.layers) if not self.layer[l]["attn"]]

    def attn_layers(self):
        return [l for l in range(self.layers) if self.layer[l]["attn"]]

    def snapshot(self):
        """Host-free copy of the recurrent state (GDN states and conv histories) for restore()."""
        return [(d["state"].clone(), d["conv_state"].clone()) for d in self.layer if not d["attn"]]

    def restore(self, snap):
        for d, (s, c) in zip((d for d in self.layer if not d["attn"]), snap):
            d["state"].copy_(s)
            d["conv_state"].copy_(c)


class VerifyStep:
    """The MTP verify step of the 64-layer state path: T tokens per user (1 accepted + T - 1 drafts) through
    every layer — GDN layers keep all T intermediate states and conv histories, attention layers append T
    rows and attend causally among them — then the acceptance of a seeded length a per user.

    rollback="slots" (default, the reference's scheme: slot select, no copy, README.md:413-421): two snapshot
    sets alternate; step k writes set k % 2 and reads each user's input from slot a - 1 of the other set,
    so accepting is slot[b] = a - 1 and seq_lens[b] = base + a. rollback="copy": every GDN layer's state and
    conv history are restored from snapshot a - 1 by bit-exact copies in one launch, and the next step
    reads them in place.

    The reference verify step is the 2-row form of the same protocol (model.py:426-456; acceptance
    kernels/mlp_hub.cpp:48-58)."""

    def __init__(self, B, ctx, T=4, layers=64, interval=4, device="cuda", seed=0, num_blocks=2048,
                 pages_per_split=2, rollback="slots"):  # fmt: skip
        if rollback not in ("slots", "copy"):
            raise ValueError("rollback must be 'slots' or 'copy'")
        self.B, self.ctx, self.T, self.layers, self.interval = B, ctx, T, layers, interval
        self.device = torch.device(device)
        self.pps = pages_per_split
        self.mode = rollback
        pages = (ctx + BLOCK - 1) // BLOCK
        self.block_table = W.block_tables(B, pages, num_blocks, self.device, seed)
        self.seq_lens = torch.full((B,), ctx, dtype=torch.int32, device=self.device)
        self.base_lens = self.seq_lens - T
        gen = torch.Generator().manual_seed(seed + 7)
        self.accept = torch.randint(1, T + 1, (B,), generator=gen, dtype=torch.int32).to(self.device)
        self.slot = torch.zeros(B, dtype=torch.int32, device=self.device)
        self.parity = 0  # snapshot set the next verify step writes (slots mode)
        # GDN tensors live layer-major in one tensor each: states / conv histories [n_gdn, B, ...] (copy mode)
        # and the T snapshots [sets, n_gdn, T, B, ...] (2 sets in slots mode, whose set 1 starts out holding
        # the initial state in slot 0)
        n_gdn = sum(not is_attn(l, interval) for l in range(layers))
        f32, bf = torch.float32, torch.bfloat16
        sets = 2 if rollback == "slots" else 1
        self.g_states = torch.empty(sets, n_gdn, T, B, NV, DK, DV, dtype=f32, device=self.device)
        self.g_convs = torch.empty(sets, n_gdn, T, B, W.C_QKV, CONV_K - 1, dtype=bf, device=self.device)
        if rollback == "copy":
            self.g_state = torch.empty(n_gdn, B, NV, DK, DV, dtype=f32, device=self.device)
            self.g_conv = torch.empty(n_gdn, B, W.C_QKV, CONV_K - 1, dtype=bf, device=self.device)
        self.layer = []
        gi = 0
        for l in range(layers):
            if is_attn(l, interval):
                d = W.attn_layer(B, ctx, self.device, seed=seed + 1000 + l, T=T, num_blocks=num_blocks)
                d["block_table"], d["seq_lens"] = self.block_table, self.seq_lens
                d["o"] = torch.empty(B, T, NQ, HD, dtype=torch.bfloat16, device=self.device)
                d["attn"] = True
            else:
                d = W.gdn_layer(B, self.device, seed=seed + l, T=T)
                if rollback == "copy":
                    self.g_state[gi].copy_(d["state"])
                    self.g_conv[gi].copy_(d["conv_state"])
                    d["state"], d["conv_state"] = self.g_state[gi], self.g_conv[gi]
                else:
                    self.g_states[1, gi, 0].copy_(d["state"])
                    self.g_convs[1, gi, 0].copy_(d["conv_state"])
                    del d["state"], d["conv_state"]
                d["o"] = torch.empty(B, T, NV, DV, dtype=torch.bfloat16, device=self.device)
                d["gi"] = gi
                d["attn"] = False
                gi += 1
            self.layer.append(d)
        mb = self.block_table.shape[1]
        self.attn_ws = ops.attention_workspace(B, T, NQ, NKV, mb, pages_per_split, self.device)
        self.graph = None

    def verify(self):
        """All layers of the verify step (no acceptance): what the target model's forward does."""
        p = self.parity
        for d in self.layer:
            if d["attn"]:
                ops.paged_gqa_decode(d["q"], d["k_cache"], d["v_cache"], d["block_table"], d["seq_lens"],
                                     d["scale"], k_new=d["k_new"], v_new=d["v_new"], pages_per_split=self.pps,
                                     out=d["o"], ws=self.attn_ws)  # fmt: skip
            elif self.mode == "slots":
                gi = d["gi"]
                ops.gdn_verify_step_slots(d["x"], self.g_convs[1 - p, gi], d["taps"], d["g"], d["beta"],
                                          self.g_states[1 - p, gi], self.slot,
                                          out=(d["o"], self.g_states[p, gi], self.g_convs[p, gi]))  # fmt: skip
            else:
                gi = d["gi"]
                ops.gdn_verify_step(d["x"], d["conv_state"], d["taps"], d["g"], d["beta"], d["state"],
                                    out=(d["o"], self.g_states[0, gi], self.g_convs[0, gi]))  # fmt: skip

    def rollback(self):
        """Accept seeded lengths: select the snapshot slots (slots mode) or restore every GDN layer from its
        snapshot in one launch (copy mode), and truncate the KV length."""
        if self.mode == "slots":
            ops.verify_accept(self.accept, self.T, self.slot, self.seq_lens, self.base_lens)
            self.parity ^= 1
        else:
            ops.gdn_rollback_layers(self.g_states[0], self.g_convs[0], self.accept, self.g_state, self.g_conv,
                                    self.seq_lens, self.base_lens)  # fmt: skip

    def step(self):
        self.verify()
        self.rollback()

    def state_of(self, gi, b):
        """The accepted (current) fp32 state and conv history of user b in GDN layer gi."""
        if self.mode == "slots":
            s = int(self.slot[b])
            return self.g_states[1 - self.parity, gi, s, b], self.g_convs[1 - self.parity, gi, s, b]
        return self.g_state[gi, b], self.g_conv[gi, b]

    def reset_lengths(self):
        """Undo the KV truncation so the same step can be replayed (benchmarking)."""
        self.seq_lens.copy_(self.base_lens + self.T)

    def bytes_per_step(self):
        """Algorithmic bytes of the verify step (acceptance by slot selection moves none; the copy mode's
        restore is rollback_bytes())."""
        return step_bytes(self.B, self.ctx, self.layers, self.interval, self.T)

    def rollback_bytes(self):
        if self.mode == "slots":
            return 0
        n_gdn = sum(not d["attn"] for d in self.layer)
        return n_gdn * self.B * (2 * NV * DK * DV * 4 + 2 * W.C_QKV * (CONV_K - 1) * 2)
