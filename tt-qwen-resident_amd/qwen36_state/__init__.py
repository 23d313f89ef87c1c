"""qwen36_state — MI355X (gfx950) decode-time state path of the hybrid Gated-DeltaNet / attention
Qwen3.6-27B engine: HIP kernels behind the C ABI of libqwen_state.so (include/qwen_state.h), driven from
PyTorch-ROCm.

    ops        operator API mirroring the reference call sites (conv1d update, gates, delta rule decode /
               verify / rollback, paged KV append / fill, paged GQA decode, chunked prefill)
    decode     the batched 64-layer state-path step (48 GDN + 16 attention layers) with HIP-graph replay
    workloads  seeded synthetic inputs of the benchmark configurations
"""
from . import ops  # noqa: F401
from ._lib import LIB_PATH, QSError, lib  # noqa: F401
