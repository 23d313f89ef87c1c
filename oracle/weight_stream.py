"""CPU restatement of the weight-streaming projections and the MLP half (TEST INFRASTRUCTURE ONLY).

The reference streams its projection and MLP weights in Tenstorrent block floating point (bfp4 for gate | up,
bfp8 for down; `quantize` at common.py:115-116 goes through ttnn, absent here) and checks its MLP half against
a torch reference built from the dequantized weights (tests/bench_resident_mlp.py:98-105). This build stores
the same roles in the OCP microscaling formats: MXFP4 (E2M1 values) and MXFP8 (E4M3 values), which the MI355X
converts in hardware, and MXINT8 (two's-complement int8 values times 2^-6), 32 values along K per E8M0 scale
(OCP Microscaling Formats (MX) v1.0, sections 5.2-5.3 and 6). MXINT8 carries a sign and 7 magnitude bits per
value under a shared power-of-two scale, the precision of the reference's 8-bit block floating point
(bfloat8_b: sign + 7-bit mantissa per value, one exponent per 16 values, model.py:53-58); E4M3 keeps 3.
The checker therefore restates:

  e2m1_decode / e4m3_decode / int8_decode   the element encodings (closed forms of the spec);
  mx_quantize                 scale 2^(floor(log2 amax) - emax) per block (emax 2 / 8 / 0 for E2M1 / E4M3 /
                              INT8), nearest code with ties to the even code, saturation at the largest finite
                              value (brute force over all codes; INT8 saturates symmetrically at +-127);
  mx_pack / mx_unpack         the kernels' fragment-order layout of a packed weight (include/qwen_state.h);
  mlp_half                    x + bf16(silu(h G) (h U)) D, h = bf16(x rsqrt(mean(x^2) + eps) gamma), the
                              reference's torch_reference with the intermediate rounded to bf16 where the
                              kernels keep it (the reference's device path also holds it in 16-bit tiles).

Pinned by tests/test_oracle_weight_stream.py: hand-written golden vectors for the three encodings and for
quantization (ties, saturation, zero blocks, scale choice), the half-step error bound of MXINT8, a hand-indexed
layout case, and the MLP's closed forms (D = 0 is the identity, the delta is linear in D, rmsnorm's scale
invariance).
"""
import numpy as np
import torch
import torch.nn.functional as F

from .state_path import EPS, bf16

__all__ = ["E2M1", "MXFP4", "MXFP8", "MXINT8", "e2m1_decode", "e4m3_decode", "int8_decode", "mx_quantize",
           "mx_dequantize", "mx_pack", "mx_unpack", "mlp_half"]  # fmt: skip

MXFP4, MXFP8, MXINT8 = 4, 8, 9  # format codes of include/qwen_state.h
E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)  # codes 0..7 (OCP MX v1.0 table 5.2: exponent bias 1)
# largest power of two of an element: E2M1 6 = 1.5 2^2, E4M3 448 = 1.75 2^8, INT8 1.984375 = 127 2^-6 < 2^1
_EMAX = {4: 2, 8: 8, 9: 0}
_KG = {4: 128, 8: 64, 9: 64}  # K values per layout block
_STEPS = {4: 4, 8: 2, 9: 2}


def e2m1_decode(codes):
    """4-bit E2M1 codes (bit 3 = sign) -> float64."""
    c = torch.as_tensor(codes).long()
    mag = torch.tensor(E2M1, dtype=torch.float64)[c & 7]
    return torch.where((c & 8) != 0, -mag, mag)


def e4m3_decode(codes):
    """8-bit E4M3 codes (OCP: bias 7, subnormals, no infinities, S.1111.111 = NaN) -> float64."""
    c = torch.as_tensor(codes).long()
    e, m = (c >> 3) & 15, (c & 7).double()
    mag = torch.where(e == 0, m * 2.0**-9, (1 + m / 8) * torch.pow(2.0, (e - 7).double()))
    mag = torch.where((c & 0x7F) == 0x7F, torch.full_like(mag, float("nan")), mag)
    return torch.where((c & 0x80) != 0, -mag, mag)


def int8_decode(codes):
    """8-bit MXINT8 codes (two's complement) -> float64: the integer times 2^-6 (OCP MX v1.0 section 5.3)."""
    c = torch.as_tensor(codes).long() & 0xFF
    return torch.where(c >= 128, c - 256, c).double() * 2.0**-6


def _magnitudes(fmt):
    """Finite non-negative magnitudes by code (monotonic in the code), and the sign bit."""
    if fmt == 4:
        return torch.tensor(E2M1, dtype=torch.float64), 8
    if fmt == 9:
        return torch.arange(128, dtype=torch.float64) * 2.0**-6, None
    return e4m3_decode(torch.arange(0x7F)), 0x80


def mx_quantize(w, fmt):
    """w [K, N] -> (codes uint8 [K, N], scale exponents uint8 [K / 32, N]).

    Block (32 values of K in one column): e = floor(log2 amax) - emax + 127 clamped to [1, 254] (127 for an
    all-zero block); value code = the nearest finite magnitude of |w| 2^(127 - e), ties to the even code,
    sign bit set for negative nonzero codes (INT8: the two's complement of the signed magnitude)."""
    w = torch.as_tensor(w, dtype=torch.float64)
    K, N = w.shape
    blk = w.reshape(K // 32, 32, N)
    amax = blk.abs().amax(1)  # [K / 32, N]
    _, ex = torch.frexp(amax)
    e = torch.where(amax > 0, (ex - 1 - _EMAX[fmt] + 127).clamp(1, 254), torch.full_like(ex, 127))
    y = blk * torch.pow(2.0, (127 - e).double())[:, None, :]
    mags, sign = _magnitudes(fmt)
    a = y.abs().reshape(-1)
    dist = (a[:, None] - mags[None, :]).abs()
    tie = dist == dist.min(1, keepdim=True).values
    score = tie.long() * (2 - (torch.arange(len(mags)) & 1))[None, :]  # among the nearest, the even code
    code = score.argmax(1).reshape(y.shape)
    if sign is None:  # INT8: two's complement of the signed magnitude (-127 .. 127)
        code = torch.where(y < 0, (256 - code) & 0xFF, code)
    else:
        code = torch.where((y < 0) & (code > 0), code | sign, code)
    return code.reshape(K, N).to(torch.uint8), e.to(torch.uint8)


def mx_dequantize(codes, scales, fmt):
    """codes [K, N], scale exponents [K / 32, N] -> float64 [K, N]."""
    v = {4: e2m1_decode, 8: e4m3_decode, 9: int8_decode}[fmt](codes)
    s = torch.pow(2.0, torch.as_tensor(scales).double() - 127).repeat_interleave(32, 0)
    return v * s


def mx_pack(codes, scales, fmt):
    """The kernels' fragment-order bytes of a quantized W [K, N]: per 16-column tile t and K group q, 1024 value
    bytes (lane 16 g + r: column 16 t + r, values KG q + 32 s + 8 g .. + 7 of each step s; MXFP4 low nibble
    first) then the group's scales, column r's at 1024 + STEPS r + s."""
    c = np.asarray(codes, dtype=np.uint8)
    sc = np.asarray(scales, dtype=np.uint8)
    K, N = c.shape
    kg, st = _KG[fmt], _STEPS[fmt]
    nq, nt = K // kg, N // 16
    if fmt == 4:
        v = c.reshape(nq, st, 4, 8, nt, 16)  # q, s, g, j, t, r
        v = v[:, :, :, 0::2] | (v[:, :, :, 1::2] << 4)  # byte j / 2 of the step
    else:
        v = c.reshape(nq, st, 4, 8, nt, 16)
    v = v.transpose(4, 0, 2, 5, 1, 3).reshape(nt, nq, 1024)  # t, q, (g, r, s, byte)
    s = sc.reshape(nq, st, nt, 16).transpose(2, 0, 3, 1).reshape(nt, nq, 16 * st)  # t, q, (r, s)
    return np.concatenate([v, s], axis=2).reshape(-1)


def mx_unpack(packed, K, N, fmt):
    """Inverse of :func:`mx_pack`: packed bytes -> (codes [K, N], scale exponents [K / 32, N])."""
    p = np.asarray(packed, dtype=np.uint8)
    kg, st = _KG[fmt], _STEPS[fmt]
    nq, nt = K // kg, N // 16
    blk = p.reshape(nt, nq, 1024 + 16 * st)
    v = blk[:, :, :1024]
    if fmt == 4:
        b = v.reshape(nt, nq, 4, 16, st, 4)  # t, q, g, r, s, byte
        c = np.stack([b & 15, b >> 4], axis=-1).reshape(nt, nq, 4, 16, st, 8)
    else:
        c = v.reshape(nt, nq, 4, 16, st, 8)
    codes = c.transpose(1, 4, 2, 5, 0, 3).reshape(K, N)  # q, s, g, j, t, r
    s = blk[:, :, 1024:].reshape(nt, nq, 16, st).transpose(1, 3, 0, 2).reshape(K // 32, N)
    return torch.from_numpy(codes.copy()), torch.from_numpy(s.copy())


def mlp_half(x, gamma, G, U, D, eps=EPS):
    """x + bf16(silu(h G) (h U)) D with h = bf16(x rsqrt(mean(x^2) + eps) gamma) per row
    (tests/bench_resident_mlp.py:98-105; EPS common.py:15). x [B, H]; G, U [H, I]; D [I, H] (dequantized)."""
    dt = G.dtype
    x = x.to(dt)
    g = torch.ones(x.shape[-1], dtype=dt) if gamma is None else gamma.to(dt)  # None: folded into G and U
    h = bf16(x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * g).to(dt)
    z = bf16(F.silu(h @ G) * (h @ U)).to(dt)
    return x + z @ D
