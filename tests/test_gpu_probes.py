"""The bandwidth probes of csrc/probes.hip (measurement kernels behind bench.py's ceilings): the copy probe
moves every byte (to a second buffer and in place) over both of its grid shapes; the read and gather probes
touch only their sink, which a constant input leaves at zero; bad sizes and null pointers are rejected
before any launch."""
import ctypes

import pytest
import torch

from qwen36_state._lib import lib

pytestmark = pytest.mark.gpu
CHUNK = 16384


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


# 256 and 512 chunks: one workgroup per CU of 4 or 8 waves; 1, 300 and 8193: 4-wave workgroups, the last
# grid-strided past 8192 waves
@pytest.mark.parametrize("nchunks", [1, 256, 300, 512, 8193])
def test_copy_probe_moves_every_byte(dev, nchunks):
    L = lib()
    n = nchunks * CHUNK // 4
    g = torch.Generator(device=dev).manual_seed(nchunks)
    src = torch.randint(-(2**31), 2**31 - 1, (n,), generator=g, dtype=torch.int32, device=dev)
    dst = torch.zeros_like(src)
    assert L.qs_probe_copy(_p(src), _p(dst), ctypes.c_size_t(n * 4), None) == 0
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    ref = src.clone()
    assert L.qs_probe_copy(_p(src), _p(src), ctypes.c_size_t(n * 4), None) == 0  # in place
    torch.cuda.synchronize()
    assert torch.equal(src, ref)


@pytest.mark.parametrize("nchunks", [1, 256, 8193])
def test_read_probe_touches_only_its_sink(dev, nchunks):
    L = lib()
    nbytes = nchunks * CHUNK
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)  # every 16-byte piece folds to zero
    sink = torch.zeros(L.qs_probe_sink_words(nbytes), dtype=torch.int32, device=dev)
    assert L.qs_probe_read(_p(buf), ctypes.c_size_t(nbytes), _p(sink), None) == 0
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
    assert bool((buf == 1).all())


def test_gather_probe_over_a_block_table(dev):
    L = lib()
    B, NKV, mb, pps, nblocks = 2, 4, 24, 8, 64
    kc = torch.zeros(nblocks, NKV, 64, 256, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    table = torch.randperm(nblocks)[: B * mb].view(B, mb).to(torch.int32)
    table[1, 5] = -1  # an entry outside the pool reads zeros
    table = table.to(dev)
    sink = torch.zeros(L.qs_probe_gather_sink_words(B, NKV, mb, pps), dtype=torch.int32, device=dev)
    assert L.qs_probe_gather(_p(kc), _p(vc), _p(table), B, NKV, mb, mb, nblocks, pps, _p(sink), None) == 0
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0


def test_probes_reject_bad_arguments(dev):
    L = lib()
    buf = torch.zeros(2 * CHUNK // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    assert L.qs_probe_read(_p(buf), ctypes.c_size_t(CHUNK + 4), _p(sink), None) != 0
    assert b"multiple" in L.qs_last_error()
    assert L.qs_probe_copy(_p(buf), None, ctypes.c_size_t(CHUNK), None) != 0
    assert L.qs_probe_read(_p(buf), ctypes.c_size_t(0), _p(sink), None) != 0
    t = torch.zeros(1, 4, dtype=torch.int32, device=dev)
    assert L.qs_probe_gather(_p(buf), _p(buf), _p(t), 1, 4, 4, 5, 1, 2, _p(sink), None) != 0  # npages > max_blocks
