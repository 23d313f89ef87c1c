"""The state-path half of an MI355X vLLM model adapter for the hybrid GDN / attention Qwen3.6 engine.

The reference adapter (generator_vllm.py:34-160) serves one user, owns its caches and ignores vLLM's paged
KV cache: ``allocate_kv_cache`` returns [] (generator_vllm.py:84-85) and the page table handed to
``prefill_forward`` / ``decode_forward`` is never read. This adapter keeps the same three calls and honours
the block-table contract instead:

- ``allocate_kv_cache(kv_cache_shape, dtype, num_layers)`` returns real per-layer paged pools
  ``[num_blocks, NKV, 64, HD]`` bf16, one (K, V) pair per attention layer, and captures the decode step over
  them;
- ``prefill_forward(inputs, page_table, kv_cache, prompt_lens, slot)`` runs one user's prompt through the state
  path: the prompt conv with its carry (the carry lands in the user's decode conv slot), the chunked gated delta
  rule (its final state lands in the user's decode state slot) and the paged fill of the prompt's K / V through
  the user's page table;
- ``decode_forward(inputs, start_pos, page_table, reload_inputs, reload_page_table, read_from_device)`` runs
  one decode step of every active slot over the block table: positions advance on the device, K / V rows are
  appended at ``start_pos`` and attended through the pages; a slot with ``start_pos < 0`` is idle and left
  untouched. Like the reference's (generator_vllm.py:117-160, ``execute_trace(blocking=False)`` at
  model.py:1505) the call is asynchronous: it enqueues the step and returns its device output buffers
  without waiting; the device status word of each step is read back one step late (or at once with
  ``read_from_device=True``). With ``reload_inputs=False`` nothing is copied from the host: the caller has
  written the step's inputs into ``step_inputs()`` (its projections can write there directly) and the
  positions are the ones the previous step advanced to on the device.

The embedding, the projections, the MLP, the lm_head and sampling are outside the state path, so the calls take
the layers' projection outputs in place of token ids and return the layers' mixer outputs:

- GDN layer: ``x`` (the q | k | v slice of the projection), ``g`` (log decay), ``beta``;
- attention layer: ``q``, ``k``, ``v`` (prefill: ``k``, ``v`` [NKV, T, HD] for the fill; decode: ``q``
  [B, 1, NQ, HD], ``k_new``, ``v_new`` [B, 1, NKV, HD]).

The prompt's own attention (the reference's ``chunked_scaled_dot_product_attention``, prefill/pp_prefill.py:
828-837) is outside the path: ``prefill_forward`` returns None for attention layers.
"""
import torch

from . import ops
from .decode import StatePathStep, is_attn
from .ops import BLOCK, CONV_K, DK, DV, HD, NK, NKV, NQ, NV
from .workloads import C_QKV


class StatePathAdapter:
    """vLLM-facing adapter of the state path for ``max_batch_size`` decode slots of up to ``max_seq_len``
    positions. ``taps`` (optional): one [C, 4] bf16 conv weight per GDN layer (the model's conv1d weights,
    weights.py:58); seeded synthetic taps otherwise."""

    model_capabilities = {
        "supports_prefix_caching": False,
        "supports_async_decode": True,
        "supports_sample_on_device": False,
    }

    def __init__(self, max_batch_size, max_seq_len, layers=64, interval=4, device="cuda", taps=None,
                 pages_per_split=8, seed=0):  # fmt: skip
        self.device = torch.device(device)
        self.B, self.max_seq_len = int(max_batch_size), int(max_seq_len)
        self.layers, self.interval = layers, interval
        self.attn = [l for l in range(layers) if is_attn(l, interval)]
        self.gdn = [l for l in range(layers) if not is_attn(l, interval)]
        self.max_blocks = (self.max_seq_len + BLOCK - 1) // BLOCK
        self.pps = pages_per_split
        dev, B, ng = self.device, self.B, len(self.gdn)
        # unused entries are -1 (outside every pool): a position whose page the caller did not map is then
        # neither written nor attended, and the kernels report it (QS_STATUS_PAGE) instead of using page 0
        self.block_table = torch.full((B, self.max_blocks), -1, dtype=torch.int32, device=dev)
        self.lens = torch.full((B,), -1, dtype=torch.int32, device=dev)  # rows cached per slot; -1 = idle
        self.gdn_state = torch.zeros(ng, B, NV, DK, DV, dtype=torch.float32, device=dev)
        self.conv_state = torch.zeros(ng, B, C_QKV, CONV_K - 1, dtype=torch.bfloat16, device=dev)
        if taps is None:
            gen = torch.Generator().manual_seed(seed)
            taps = [(0.5 * torch.randn(C_QKV, CONV_K, generator=gen)).bfloat16().to(dev) for _ in self.gdn]
        if len(taps) != ng:
            raise ValueError(f"taps: expected one [C, 4] tensor per GDN layer ({ng}), got {len(taps)}")
        self.taps = [ops._chk(t, "taps", torch.bfloat16, (C_QKV, CONV_K), dev) for t in taps]
        self.status = ops.Status(dev)
        self.kv = None
        self.step = None
        # host staging for asynchronous steps: pinned rings for the positions and the block table (a slot is
        # rewritten only after the copy that read it has run) and for the status word read back per step
        self._ring = 4
        self._pos_host = [torch.empty(B, dtype=torch.int32).pin_memory() for _ in range(self._ring)]
        self._tab_host = [torch.empty(B, self.max_blocks, dtype=torch.int32).pin_memory() for _ in range(self._ring)]
        self._st_host = [torch.zeros(1, dtype=torch.int32).pin_memory() for _ in range(self._ring)]
        self._in_ev = [None] * self._ring
        self._st_ev = [None] * self._ring
        self._n = 0  # steps enqueued
        self._pending = []  # (step number, ring slot) of status words not checked yet

    # --------------------------------------------------------------------------------------------- vLLM calls

    def allocate_kv_cache(self, kv_cache_shape, dtype, num_layers):
        """Per-attention-layer paged pools: kv_cache_shape = (num_blocks, NKV, block, HD), dtype bf16,
        num_layers = the model's full-attention layers. Returns [(k_cache, v_cache), ...]."""
        nb, nkv, blk, hd = (int(s) for s in kv_cache_shape)
        if dtype != torch.bfloat16:
            raise ValueError(f"KV pools are bf16 (got {dtype})")
        if (nkv, blk, hd) != (NKV, BLOCK, HD):
            raise ValueError(f"kv_cache_shape must be (num_blocks, {NKV}, {BLOCK}, {HD}) (got {tuple(kv_cache_shape)})")
        if num_layers != len(self.attn):
            raise ValueError(f"num_layers must be the {len(self.attn)} attention layers (got {num_layers})")
        z = lambda: torch.zeros(nb, NKV, BLOCK, HD, dtype=torch.bfloat16, device=self.device)  # noqa: E731
        self.kv = [(z(), z()) for _ in range(num_layers)]
        self._build_step()
        return self.kv

    def prefill_forward(self, inputs, page_table, kv_cache, prompt_lens, slot=0):
        """One user's prompt through the state path into decode slot ``slot``.

        inputs: one dict per layer, GDN {x [T, >= C] bf16 (unit column stride), g, beta [T, NV] fp32},
        attention {k, v [NKV, T, HD] bf16}; page_table [1, n] int32 (the user's blocks, n <= max_blocks);
        kv_cache: the pools allocate_kv_cache returned; prompt_lens [1] (T). Returns the GDN layers' outputs
        o [T, NV, DV] bf16 (None for attention layers)."""
        if kv_cache is not self.kv:
            raise ValueError("kv_cache must be the pools allocate_kv_cache returned")
        page_table = torch.as_tensor(page_table)
        if page_table.dim() != 2 or page_table.shape[0] != 1:
            raise ValueError("one user per prefill: page_table must be [1, n]")
        T = int(torch.as_tensor(prompt_lens).reshape(-1)[0])
        if not 0 < T < self.max_seq_len:
            raise ValueError(f"prompt length {T} must be in [1, max_seq_len = {self.max_seq_len})")
        if not 0 <= slot < self.B:
            raise ValueError(f"slot {slot} outside [0, {self.B})")
        n = page_table.shape[1]
        if n > self.max_blocks or n * BLOCK < T:
            raise ValueError(f"page_table of {n} blocks for {T} tokens and at most {self.max_blocks} blocks")
        if len(inputs) != self.layers:
            raise ValueError(f"inputs: one dict per layer ({self.layers}), got {len(inputs)}")
        row = page_table[0].to(device=self.device, dtype=torch.int32).contiguous()
        outs = []
        for l, x in enumerate(inputs):
            if is_attn(l, self.interval):
                kc, vc = self.kv[self.attn.index(l)]
                ops.paged_kv_fill(x["k"][:, :T].contiguous(), x["v"][:, :T].contiguous(), kc, vc, row)
                outs.append(None)
                continue
            gi = self.gdn.index(l)
            # a fresh prompt: zero carry in; the carry out is the slot's decode conv state
            q, k, v, _ = ops.causal_conv1d_prefill(x["x"][:T], self.taps[gi], None, self.conv_state[gi, slot])
            o, _ = ops.chunk_gated_delta_rule(q, k, v, x["g"][:T].contiguous(), x["beta"][:T].contiguous(),
                                              final_state=self.gdn_state[gi, slot])  # fmt: skip
            outs.append(o)
        self.block_table[slot].fill_(-1)
        self.block_table[slot, :n] = row
        self.lens[slot] = T
        return outs

    def decode_forward(self, inputs, start_pos, page_table=None, *args, reload_inputs=True, reload_page_table=False,
                       read_from_device=False, **kwargs):  # fmt: skip
        """One decode step of every slot, enqueued without waiting (generator_vllm.py:117-160).

        inputs: one dict per layer, GDN {x [B, C], g, beta [B, NV]}, attention {q [B, 1, NQ, HD], k_new, v_new
        [B, 1, NKV, HD]}, copied into the step's buffers on the device (a tensor that already is the step's
        buffer is not copied; inputs=None copies nothing); start_pos [B] (host or device int32: each slot's
        new-token position = its cached rows; negative = idle slot). With reload_inputs=False neither is
        reloaded: the caller wrote the inputs into ``step_inputs()`` and the positions are where the previous
        step left them on the device. page_table [B, n] int32 (n <= max_blocks) is loaded when
        reload_page_table is set (entries past n become -1). Returns the step's output buffers (GDN o
        [B, NV, DV], attention o [B, 1, NQ, HD]), valid once the stream reaches the end of the step; they
        are rewritten by the next step.

        Errors: a host-side start_pos past max_seq_len raises ValueError at once (generator_vllm.py:94). The
        kernels' status word (a length past the table, a block-table entry outside the pool) is copied to the
        host after every step and checked at the next call, or at once with read_from_device=True (which
        waits for the step); a reported condition raises ValueError naming the step."""
        if self.step is None:
            raise ValueError("allocate_kv_cache must run before decode_forward")
        # every argument is checked before anything is enqueued
        pos = pt = None
        if reload_inputs:
            pos = torch.as_tensor(start_pos).reshape(-1)
            if pos.shape[0] != self.B:
                raise ValueError(f"start_pos must hold one position per slot ({self.B})")
            if not pos.is_cuda:
                pos = pos.to(torch.int32)
                if int(pos.max()) >= self.max_seq_len:
                    raise ValueError(f"position {int(pos.max())} is past max_seq_len {self.max_seq_len}")
            if inputs is not None and len(inputs) != self.layers:
                raise ValueError(f"inputs: one dict per layer ({self.layers}), got {len(inputs)}")
        if page_table is not None and reload_page_table:
            pt = torch.as_tensor(page_table)
            if pt.dim() != 2 or pt.shape[0] != self.B or pt.shape[1] > self.max_blocks:
                raise ValueError(f"page_table must be [{self.B}, <= {self.max_blocks}]")
        self._check_status(wait=False)
        r = self._n % self._ring
        if self._in_ev[r] is not None:
            self._in_ev[r].synchronize()  # the copies that read this ring slot four steps ago have run
        if pos is not None:
            if pos.is_cuda:
                self.lens.copy_(pos.to(torch.int32), non_blocking=True)
            else:
                self._pos_host[r].copy_(pos)
                self.lens.copy_(self._pos_host[r], non_blocking=True)
        if pt is not None:
            n = pt.shape[1]
            if pt.is_cuda:
                self.block_table[:, n:].fill_(-1)
                self.block_table[:, :n].copy_(pt.to(torch.int32), non_blocking=True)
            else:
                h = self._tab_host[r]
                h.fill_(-1)
                h[:, :n] = pt.to(torch.int32)
                self.block_table.copy_(h, non_blocking=True)
        if reload_inputs and inputs is not None:
            for d, x in zip(self.step.layer, inputs):
                for key in (("q", "k_new", "v_new") if d["attn"] else ("x", "g", "beta")):
                    if x[key] is not d[key]:
                        d[key].copy_(x[key], non_blocking=True)
        stream = torch.cuda.current_stream(self.device)
        ev = torch.cuda.Event()
        ev.record(stream)
        self._in_ev[r] = ev
        self.step.replay()
        # the step's status word to the host (read one step late), then cleared for the next step
        if self._st_ev[r] is not None:
            self._st_ev[r].synchronize()
        self._st_host[r].copy_(self.status.word, non_blocking=True)
        self.status.word.zero_()
        sev = torch.cuda.Event()
        sev.record(stream)
        self._st_ev[r] = sev
        self._pending.append((self._n, r))
        self._n += 1
        if read_from_device:
            self._check_status(wait=True)
        return [d["o"] for d in self.step.layer]

    def step_inputs(self):
        """The step's own input buffers, one dict per layer (GDN {x, g, beta}, attention {q, k_new, v_new}):
        a caller that writes its projections here calls decode_forward(None, ..., reload_inputs=False) or
        passes these same tensors, and no copy is made."""
        return [{k: d[k] for k in (("q", "k_new", "v_new") if d["attn"] else ("x", "g", "beta"))}
                for d in self.step.layer]  # fmt: skip

    def read_decode_output(self, outs=None):
        """Wait for the enqueued steps and check their status words (raises ValueError on a reported
        condition); returns ``outs`` (the buffers decode_forward returned)."""
        self._check_status(wait=True)
        return outs

    def _check_status(self, wait):
        """Check the status words of finished steps, oldest first: every enqueued step with wait=True, else the
        finished ones, and always the oldest while a full ring is pending (its host slot is needed next)."""
        while self._pending:
            n, r = self._pending[0]
            if wait or len(self._pending) >= self._ring:
                self._st_ev[r].synchronize()
            elif not self._st_ev[r].query():
                return
            self._pending.pop(0)
            v = int(self._st_host[r][0])
            if v:
                self._pending.clear()
                text = "; ".join(t for bit, t in ops._STATUS_TEXT.items() if v & bit)
                raise ValueError(f"decode step {n}: {text} (status {v:#x})")

    # --------------------------------------------------------------------------------------------- internals

    def _build_step(self):
        """The decode step over the adapter's buffers (state slots, pools, block table, lengths), captured."""
        dev, B = self.device, self.B
        layers = []
        for l in range(self.layers):
            if is_attn(l, self.interval):
                kc, vc = self.kv[self.attn.index(l)]
                layers.append(dict(attn=True, k_cache=kc, v_cache=vc, scale=HD**-0.5,
                                   q=torch.zeros(B, 1, NQ, HD, dtype=torch.bfloat16, device=dev),
                                   k_new=torch.zeros(B, 1, NKV, HD, dtype=torch.bfloat16, device=dev),
                                   v_new=torch.zeros(B, 1, NKV, HD, dtype=torch.bfloat16, device=dev),
                                   o=torch.zeros(B, 1, NQ, HD, dtype=torch.bfloat16, device=dev)))  # fmt: skip
            else:
                gi = self.gdn.index(l)
                layers.append(dict(attn=False, state=self.gdn_state[gi], conv_state=self.conv_state[gi],
                                   taps=self.taps[gi], x=torch.zeros(B, C_QKV, dtype=torch.bfloat16, device=dev),
                                   g=torch.zeros(B, NV, device=dev), beta=torch.zeros(B, NV, device=dev),
                                   o=torch.zeros(B, NV, DV, dtype=torch.bfloat16, device=dev)))  # fmt: skip
        self.step = StatePathStep(layers, self.block_table, self.lens, self.interval, self.pps, self.status)
        self.step.capture()
