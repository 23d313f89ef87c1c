"""The C ABI: the library loads, exports every entry point include/qwen_state.h declares, and rejects bad
arguments with QS_EINVAL before any launch (no GPU needed); the Python ops validate before calling."""
import ctypes
import os
import re

import pytest
import torch

import qwen36_state as Q
from qwen36_state import _lib, ops

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "qwen_state.h")
FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation first
NUL = ctypes.c_void_p(0)
S = ctypes.c_void_p(0)


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(qs_\w+)\s*\(", text)))


def test_exports_every_declared_symbol():
    L = Q.lib()
    names = declared()
    assert len(names) >= 14
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib.SIGNATURES, n
    assert set(_lib.SIGNATURES) == set(names)
    assert L.qs_abi_version() == 4


def test_rejects_bad_arguments():
    L = Q.lib()
    # null pointer
    assert L.qs_gdn_decode_step(NUL, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 16, 48, 128, 128, 0.1, 1e-6, S) == -1
    assert "null" in L.qs_last_error().decode()
    # unsupported head dims / grouping
    assert L.qs_gdn_decode_step(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 16, 48, 64, 128, 0.1, 1e-6, S) == -1
    assert L.qs_gdn_decode_step(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 16, 40, 128, 128, 0.1, 1e-6, S) == -1
    assert "multiple" in L.qs_last_error().decode()
    assert L.qs_conv1d_update(FAKE, FAKE, FAKE, FAKE, 1, 10240, 3, S) == -1
    assert L.qs_gdn_verify_step(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NUL, NUL,
                                1, 9, 16, 48, 128, 128, 4, 0.1, 1e-6, S) == -1  # fmt: skip
    assert L.qs_gdn_verify_step(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NUL, NUL,
                                1, 4, 16, 48, 128, 128, 4, 0.1, 1e-6, S) == -1  # fmt: skip  (states_out aliases)
    assert "alias" in L.qs_last_error().decode()
    # attention: head dim, block size, group size, missing workspace
    args = lambda hd, blk, nq, mb, pps, ws: (FAKE, NUL, NUL, FAKE, FAKE, FAKE, FAKE, FAKE, ws, 1, 1, nq, 4, hd, blk,
                                             mb, 2048, pps, 0.0625, NUL, S)  # fmt: skip
    assert L.qs_paged_gqa_decode(*args(128, 64, 24, 512, 8, FAKE)) == -1
    assert L.qs_paged_gqa_decode(*args(256, 32, 24, 512, 8, FAKE)) == -1
    assert L.qs_paged_gqa_decode(*args(256, 64, 20, 512, 8, FAKE)) == -1
    assert L.qs_paged_gqa_decode(*args(256, 64, 24, 512, 8, NUL)) == -1
    assert "workspace" in L.qs_last_error().decode()
    # fill: a table too short for the tokens
    assert L.qs_paged_kv_fill(FAKE, FAKE, FAKE, FAKE, FAKE, 200, 0, 4, 256, 64, 3, 2048, S) == -1
    assert L.qs_paged_kv_append(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 1, 4, 250, 64, 8, 8, NUL, S) == -1
    # the length advance: null lengths, aliasing base
    assert L.qs_advance_lengths(NUL, NUL, 4, 1, 4096, NUL, S) == -1
    assert L.qs_advance_lengths(FAKE, FAKE, 4, 1, 4096, NUL, S) == -1
    assert "alias" in L.qs_last_error().decode()
    # gather: a table too short for the positions, a pool without its output
    assert L.qs_paged_kv_gather(FAKE, FAKE, FAKE, FAKE, FAKE, 200, 0, 4, 256, 64, 3, 2048, S) == -1
    assert L.qs_paged_kv_gather(FAKE, FAKE, FAKE, NUL, FAKE, 100, 0, 4, 256, 64, 3, 2048, S) == -1
    # prompt conv: taps, ldx below C or not a multiple of 8, CQ not a multiple of 8, misalignment, null x
    conv = lambda x, ldx, T, cq, k: (x, ldx, NUL, FAKE, FAKE, FAKE, FAKE, FAKE, T, cq, 6144, k, S)
    assert L.qs_conv1d_prefill(*conv(FAKE, 10240, 5, 2048, 3)) == -1
    assert L.qs_conv1d_prefill(*conv(FAKE, 10000, 5, 2048, 4)) == -1
    assert L.qs_conv1d_prefill(*conv(FAKE, 10244, 5, 2048, 4)) == -1
    assert L.qs_conv1d_prefill(*conv(FAKE, 10240, 5, 2044, 4)) == -1
    assert L.qs_conv1d_prefill(*conv(ctypes.c_void_p(0x1008), 10240, 5, 2048, 4)) == -1
    assert "aligned" in L.qs_last_error().decode()
    assert L.qs_conv1d_prefill(*conv(NUL, 10240, 5, 2048, 4)) == -1
    assert "null" in L.qs_last_error().decode()


def test_workspace_sizes():
    L = Q.lib()
    assert L.qs_gdn_workspace_bytes(8, 16) == 8 * 16 * 2 * 4
    one = L.qs_paged_attention_workspace_bytes(1, 1, 24, 4, 256, 512, 8)
    assert one > 64 * 4 * 6 * 256 * 4  # at least the level-0 partials of 64 splits
    assert L.qs_paged_attention_workspace_bytes(1, 1, 24, 4, 128, 512, 8) == 0


def test_ops_validate_before_calling():
    cpu = torch.zeros(1, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        ops.gdn_decode_step(cpu, cpu, torch.zeros(1, 48, 128, dtype=torch.bfloat16), torch.zeros(1, 48),
                            torch.zeros(1, 48), torch.zeros(1, 48, 128, 128))  # fmt: skip
    with pytest.raises(ValueError):
        ops.paged_gqa_decode(torch.zeros(1, 1, 24, 256), torch.zeros(8, 4, 64, 256), torch.zeros(8, 4, 64, 256),
                             torch.zeros(1, 8, dtype=torch.int32), torch.zeros(1, dtype=torch.int32), 0.0625)  # fmt: skip
