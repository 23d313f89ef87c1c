"""Pins of the weight-streaming oracle (oracle/weight_stream.py) on the CPU: hand-written golden vectors for the
E2M1 / E4M3 encodings (OCP Microscaling Formats v1.0, tables 5.2-5.3) and for block quantization (scale choice,
ties to even, saturation, zero blocks), a hand-indexed layout case, and the MLP half's closed forms."""
import math

import numpy as np

import torch

from oracle import weight_stream as WS


def test_e2m1_decode_closed_form():
    got = WS.e2m1_decode(torch.arange(16))
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        v = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)  # bias 1, one mantissa bit
        assert got[c].item() == (-v if s else v)
    assert WS.e2m1_decode(torch.tensor([7, 15])).tolist() == [6.0, -6.0]


def test_e4m3_decode_known_values():
    want = {0x00: 0.0, 0x01: 2.0**-9, 0x07: 7 * 2.0**-9, 0x08: 2.0**-6, 0x38: 1.0, 0x3C: 1.5, 0x77: 240.0,
            0x7E: 448.0, 0x80: -0.0, 0xB8: -1.0, 0xFE: -448.0}  # fmt: skip
    got = WS.e4m3_decode(torch.tensor(list(want)))
    assert got.tolist() == list(want.values())
    assert math.isnan(WS.e4m3_decode(torch.tensor([0x7F])).item())
    assert math.isnan(WS.e4m3_decode(torch.tensor([0xFF])).item())


def _block(vals):
    w = torch.zeros(32, 1, dtype=torch.float64)
    w[: len(vals), 0] = torch.tensor(vals, dtype=torch.float64)
    return w


def test_mxfp4_quantize_golden():
    # amax 6 -> floor(log2 6) - 2 = 0 -> scale 1; ties go to the even code, zero keeps no sign
    codes, e = WS.mx_quantize(_block([6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.3, 0.1, -0.1, -6.0, 0.5]), 4)
    assert e.tolist() == [[127]]
    assert codes[:13, 0].tolist() == [7, 0, 2, 2, 4, 4, 6, 6, 9, 0, 0, 15, 1]
    # amax 7.9: same scale, 7.9 saturates to 6; amax 8: scale 2, 8 -> 4 (code 6), 3 -> 1.5 (code 3)
    codes, e = WS.mx_quantize(_block([7.9, 1.0]), 4)
    assert e.tolist() == [[127]] and codes[:2, 0].tolist() == [7, 2]
    codes, e = WS.mx_quantize(_block([8.0, 3.0]), 4)
    assert e.tolist() == [[128]] and codes[:2, 0].tolist() == [6, 3]
    codes, e = WS.mx_quantize(torch.zeros(32, 1), 4)
    assert e.tolist() == [[127]] and codes.sum().item() == 0


def test_mxfp8_quantize_golden():
    # amax 480 -> floor(log2 480) - 8 = 0 -> scale 1; 480 saturates to 448 (0x7e)
    vals = [480.0, 448.0, 1.0, 1.0625, 1.1875, 2.0**-10, 3 * 2.0**-10, -1.0, 2.0**-6, 0.0]
    codes, e = WS.mx_quantize(_block(vals), 8)
    assert e.tolist() == [[127]]
    assert codes[: len(vals), 0].tolist() == [0x7E, 0x7E, 0x38, 0x38, 0x3A, 0x00, 0x02, 0xB8, 0x08, 0x00]
    # a small block: amax 0.01 -> floor(log2 0.01) = -7 -> e = 127 - 7 - 8 = 112; 0.01 2^15 = 327.68 -> 320
    codes, e = WS.mx_quantize(_block([0.01]), 8)
    assert e.tolist() == [[112]] and WS.e4m3_decode(codes[:1, 0]).item() == 320.0


def test_int8_decode_closed_form():
    # two's complement times 2^-6 (OCP MX v1.0 section 5.3): 0x7f = 127/64, 0x80 = -2, 0xff = -1/64
    got = WS.int8_decode(torch.tensor([0x00, 0x01, 0x40, 0x7F, 0x80, 0x81, 0xC0, 0xFF]))
    assert got.tolist() == [0.0, 1 / 64, 1.0, 127 / 64, -2.0, -127 / 64, -1.0, -1 / 64]


def test_mxint8_quantize_golden():
    # amax 1.984375 = 127/64 -> floor(log2) = 0, emax 0 -> e = 127, scale 1: code = round(64 v), ties to even,
    # saturating at +-127 (1.999 -> 127.94 -> 127), negative values as two's complement
    vals = [1.984375, 1.0, 0.5, -1.0, 1.999, -1.999, 2.0**-7, 3 * 2.0**-7, -3 * 2.0**-7, 0.3, 0.0]
    codes, e = WS.mx_quantize(_block(vals), 9)
    assert e.tolist() == [[127]]
    assert codes[: len(vals), 0].tolist() == [127, 64, 32, 192, 127, 129, 0, 2, 254, 19, 0]
    # amax 2 -> floor(log2) = 1 -> e = 128: codes are round(32 v); 3 -> 96
    codes, e = WS.mx_quantize(_block([2.0, 3.0, -0.046875]), 9)
    assert e.tolist() == [[128]] and codes[:3, 0].tolist() == [64, 96, 254]
    # a small block: amax 0.01 -> floor(log2 0.01) = -7 -> e = 120; 0.01 2^13 = 81.92 -> 82
    codes, e = WS.mx_quantize(_block([0.01, -0.005]), 9)
    assert e.tolist() == [[120]] and codes[:2, 0].tolist() == [82, 215]
    assert WS.mx_dequantize(codes, e, 9)[:2, 0].tolist() == [82 * 2.0**-13, -41 * 2.0**-13]
    codes, e = WS.mx_quantize(torch.zeros(32, 1), 9)
    assert e.tolist() == [[127]] and codes.sum().item() == 0


def test_mxint8_keeps_seven_magnitude_bits():
    """Per block, MXINT8's error is at most half a step of 2^(floor(log2 amax) - 6), one step where the value
    saturates at 127: over random normal blocks its worst relative error on the largest values is ~2^-7,
    against ~2^-4 for E4M3 (three mantissa bits)."""
    g = torch.Generator().manual_seed(4)
    w = torch.randn(4096, 8, generator=g, dtype=torch.float64) * 0.02
    for fmt in (8, 9):
        codes, e = WS.mx_quantize(w, fmt)
        err = (WS.mx_dequantize(codes, e, fmt) - w).abs()
        step = torch.pow(2.0, e.double() - 127 - (6 if fmt == 9 else 0)).repeat_interleave(32, 0)
        if fmt == 9:
            sat = WS.int8_decode(codes).abs() == 127 / 64
            assert torch.all(err[~sat] <= 0.5 * step[~sat] + 1e-18) and torch.all(err <= step + 1e-18)
        big = w.abs() > 0.5 * w.abs().reshape(-1, 32, 8).amax(1).repeat_interleave(32, 0)
        rel = (err[big] / w.abs()[big]).max().item()
        assert (rel < 2.0**-6) if fmt == 9 else (2.0**-6 < rel < 2.0**-3), (fmt, rel)


def test_quantize_is_nearest_representable():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(256, 8, generator=g, dtype=torch.float64) * 0.03
    for fmt, top in ((4, 6.0), (8, 448.0), (9, 127 / 64)):
        codes, e = WS.mx_quantize(w, fmt)
        deq = WS.mx_dequantize(codes, e, fmt)
        scale = torch.pow(2.0, e.double() - 127).repeat_interleave(32, 0)
        mags = {4: torch.tensor(WS.E2M1, dtype=torch.float64), 8: WS.e4m3_decode(torch.arange(0x7F)),
                9: torch.arange(128, dtype=torch.float64) / 64}[fmt]  # fmt: skip
        y = (w / scale).abs()
        best = (y.reshape(-1, 1) - mags[None, :]).abs().min(1).values.reshape(w.shape)
        assert torch.all((deq / scale).abs() - y <= best + 1e-12)
        assert torch.all((deq / scale).abs() <= top)


def test_pack_layout_by_hand():
    K, N = 256, 32
    codes = torch.tensor([[(3 * k + n) % 16 for n in range(N)] for k in range(K)], dtype=torch.uint8)
    scales = torch.tensor([[(k + 2 * n) % 200 + 20 for n in range(N)] for k in range(K // 32)], dtype=torch.uint8)
    p = WS.mx_pack(codes, scales, 4)
    assert p.size == (N // 16) * (K // 128) * 1088
    for t, q, g, r, s, j in ((0, 0, 0, 0, 0, 0), (1, 1, 3, 15, 3, 3), (0, 1, 2, 7, 1, 2), (1, 0, 1, 9, 2, 1)):
        blk = (t * (K // 128) + q) * 1088
        k0, n = 128 * q + 32 * s + 8 * g + 2 * j, 16 * t + r
        assert p[blk + 16 * (16 * g + r) + 4 * s + j] == codes[k0, n] | (codes[k0 + 1, n] << 4)
        assert p[blk + 1024 + 4 * r + s] == scales[(128 * q + 32 * s) // 32, n]
    c2, s2 = WS.mx_unpack(p, K, N, 4)
    assert torch.equal(c2, codes) and torch.equal(s2, scales)
    codes8 = torch.tensor([[(5 * k + 3 * n) % 256 for n in range(N)] for k in range(K)], dtype=torch.uint8)
    p8 = WS.mx_pack(codes8, scales, 8)
    for t, q, g, r, s, j in ((0, 0, 0, 0, 0, 0), (1, 3, 3, 15, 1, 7), (0, 2, 1, 4, 0, 5)):
        blk = (t * (K // 64) + q) * 1056
        assert p8[blk + 16 * (16 * g + r) + 8 * s + j] == codes8[64 * q + 32 * s + 8 * g + j, 16 * t + r]
        assert p8[blk + 1024 + 2 * r + s] == scales[(64 * q + 32 * s) // 32, 16 * t + r]
    c8, s8 = WS.mx_unpack(p8, K, N, 8)
    assert torch.equal(c8, codes8) and torch.equal(s8, scales)
    # MXINT8 shares the 8-bit layout byte for byte
    assert np.array_equal(WS.mx_pack(codes8, scales, 9), p8)


def _mlp_weights(H, I, seed=1):
    g = torch.Generator().manual_seed(seed)
    G = torch.randn(H, I, generator=g, dtype=torch.float64) / math.sqrt(H)
    U = torch.randn(H, I, generator=g, dtype=torch.float64) / math.sqrt(H)
    D = torch.randn(I, H, generator=g, dtype=torch.float64) * (0.5 / math.sqrt(I))
    gamma = 1 + 0.1 * torch.randn(H, generator=g, dtype=torch.float64)
    x = torch.randn(2, H, generator=g, dtype=torch.float64)
    return x, gamma, G, U, D


def test_mlp_half_closed_forms():
    x, gamma, G, U, D = _mlp_weights(64, 128)
    assert torch.equal(WS.mlp_half(x, gamma, G, U, torch.zeros_like(D)), x)
    d1 = WS.mlp_half(x, gamma, G, U, D) - x
    d2 = WS.mlp_half(x, gamma, G, U, 2 * D) - x
    torch.testing.assert_close(d2, 2 * d1, rtol=1e-12, atol=1e-14)
    # rmsnorm is scale invariant (eps = 0, a power-of-4 scale keeps every rounding of h and z the same)
    torch.testing.assert_close(WS.mlp_half(4 * x, gamma, G, U, D, eps=0.0) - 4 * x,
                               WS.mlp_half(x, gamma, G, U, D, eps=0.0) - x, rtol=1e-12, atol=1e-13)  # fmt: skip


def test_mlp_half_matches_loops():
    x, gamma, G, U, D = _mlp_weights(8, 16, seed=3)
    out = WS.mlp_half(x, gamma, G, U, D)
    for b in range(x.shape[0]):
        ms = sum(v * v for v in x[b].tolist()) / 8
        h = [float(torch.tensor(x[b, k].item() / math.sqrt(ms + 1e-6) * gamma[k].item()).to(torch.bfloat16)) for k in range(8)]
        z = []
        for i in range(16):
            gi = sum(h[k] * G[k, i].item() for k in range(8))
            ui = sum(h[k] * U[k, i].item() for k in range(8))
            z.append(float(torch.tensor(gi / (1 + math.exp(-gi)) * ui).to(torch.bfloat16)))
        for n in range(8):
            want = x[b, n].item() + sum(z[i] * D[i, n].item() for i in range(16))
            assert abs(out[b, n].item() - want) <= 1e-12 * (1 + abs(want))


def test_mlp_half_folded_gamma_is_unit_gamma():
    x, gamma, G, U, D = _mlp_weights(32, 64, seed=5)
    assert torch.equal(WS.mlp_half(x, None, G, U, D), WS.mlp_half(x, torch.ones(32, dtype=torch.float64), G, U, D))
    # folding gamma into the rows of G and U changes only where h is rounded to bf16
    folded = WS.mlp_half(x, None, gamma[:, None] * G, gamma[:, None] * U, D)
    torch.testing.assert_close(folded, WS.mlp_half(x, gamma, G, U, D), rtol=2e-2, atol=1e-2)
