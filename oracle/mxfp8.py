"""CPU oracle for MXFP8 weights (E4M3 elements, one E8M0 scale per 32 consecutive elements).

TEST INFRASTRUCTURE ONLY, like oracle/smollm2.py: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline may import it.

The reference has no MXFP8 decode path; its quantisation rule for MX tensors is the CPU
known-answer code of its rmsnorm kernel (prime_kernels/rmsnorm/test.cu:126-144), restated here:
  per block of 32:  amax = max |x|                      (fp32, NaN ignored like std::fmax)
                    s    = e8m0(amax * (1/448))         rounded toward +inf, saturating (:131-133)
                    inv  = bf16(2^(127 - s))            (e8m0_to_bf16raw(254 - s), :134)
                    q    = e4m3(bf16(x * inv))          round-to-nearest-even, saturate (:137-139)
  dequantised weight w = bf16(e4m3_value(q) * 2^(s - 127)): exact for any real weight scale (the
  product is a bf16 normal); below 2^-126 it rounds to a bf16 subnormal, and it overflows to
  +-inf only for scale codes >= 247, which no bf16 input produces.
OCP MX v1.0 defines the formats: E4M3 ("fn": bias 7, no infinities, 0x7f/0xff NaN, max 448)
and E8M0 (2^(c-127), c = 255 NaN).

Scales are stored [rows, scale_stride(cols)]: cols/32 codes per row, zero-padded to a multiple
of 16 bytes (the layout the kernel streams).

Pinned by tests/test_oracle_mxfp8.py: e4m3 rounding against a brute-force nearest search over
all 65,536 bf16 patterns and against torch's float8_e4m3fn cast; e8m0 rounding against the
smallest power of two >= f; the decode table against torch; dequantisation exhaustively.
"""

from __future__ import annotations

import numpy as np
import torch

BLOCK = 32
E4M3_MAX = 448.0


def scale_stride(cols: int) -> int:
    return ((cols // BLOCK + 15) // 16) * 16


def e4m3_values() -> np.ndarray:
    """float32 value of each of the 256 E4M3 codes (NaN for 0x7f / 0xff)."""
    c = np.arange(256)
    s = np.where(c >> 7, -1.0, 1.0)
    e = (c >> 3) & 15
    m = c & 7
    v = np.where(e == 0, np.ldexp(m.astype(np.float64), -9), np.ldexp(1.0 + m / 8.0, e - 7))
    v = s * v
    v[(e == 15) & (m == 7)] = np.nan
    return v.astype(np.float32)


def e8m0_ceil(f: np.ndarray) -> np.ndarray:
    """E8M0 code of the smallest power of two >= f (f >= 0 float32); 0 and values up to 2^-127 map
    to code 0 (2^-127), +inf saturates to 254, NaN to 255."""
    f = np.asarray(f, dtype=np.float32)
    u = f.view(np.uint32)
    e = (u >> 23) & 255
    m = u & 0x7FFFFF
    code = np.minimum(e + (m != 0), 254)
    code = np.where(e == 0, np.where(m > 0x400000, 1, 0), code)
    code = np.where(e == 255, 254, code)
    code = np.where(np.isnan(f), 255, code)
    return code.astype(np.uint8)


def e4m3_sat(v: np.ndarray) -> np.ndarray:
    """E4M3 code of float32 values (bf16-representable): round to nearest even, |x| >= 448 -> +-448,
    NaN -> 0x7f with the sign."""
    v = np.asarray(v, dtype=np.float32)
    sign = ((v.view(np.uint32) >> 31) << 7).astype(np.uint32)
    a = np.abs(v)
    with np.errstate(invalid="ignore", over="ignore"):
        sub = np.rint(a * np.float32(512.0)).astype(np.int64)  # subnormal steps of 2^-9 (a < 2^-6)
        e = ((a.view(np.uint32) >> 23) & 255).astype(np.int64) - 127
        mant = (a * np.ldexp(np.float32(1.0), -e).astype(np.float32)).astype(np.float32)
        m = np.rint((mant - np.float32(1.0)) * np.float32(8.0)).astype(np.int64)
    carry = m == 8
    m = np.where(carry, 0, m)
    e = np.where(carry, e + 1, e)
    normal = ((e + 7) << 3) | m
    code = np.where(a < np.float32(2.0 ** -6), sub, normal)
    code = np.where(a >= np.float32(E4M3_MAX), 0x7E, code)
    code = np.where(np.isnan(v), 0x7F, code)
    return (code.astype(np.uint32) | sign).astype(np.uint8)


def _bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def quantize(w: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """bf16 [rows, cols] -> (e4m3 codes uint8 [rows, cols], e8m0 codes uint8 [rows, scale_stride(cols)])."""
    rows, cols = w.shape
    if cols % BLOCK:
        raise ValueError("cols must be a multiple of 32")
    x = w.detach().to("cpu", torch.float32).numpy().reshape(rows, cols // BLOCK, BLOCK)
    amax = np.fmax.reduce(np.abs(x), axis=2)
    codes = e8m0_ceil((amax * np.float32(1.0 / 448.0)).astype(np.float32))
    inv = np.where(codes >= 254, np.float32(2.0 ** -127),
                   np.ldexp(np.float32(1.0), 127 - codes.astype(np.int64)).astype(np.float32)).astype(np.float32)
    scaled = _bf16_round(x * inv[..., None])
    q = e4m3_sat(scaled).reshape(rows, cols)
    s = np.zeros((rows, scale_stride(cols)), dtype=np.uint8)
    s[:, :cols // BLOCK] = codes
    return q, s


def dequantize(q: np.ndarray, s: np.ndarray) -> torch.Tensor:
    """(e4m3 codes [rows, cols], e8m0 codes [rows, >= cols/32]) -> bf16 [rows, cols], exact."""
    q = np.asarray(q, dtype=np.uint8)
    rows, cols = q.shape
    vals = e4m3_values()[q].astype(np.float64)
    sc = np.asarray(s, dtype=np.int64)[:, :cols // BLOCK]
    scale = np.where(sc == 255, np.nan, np.ldexp(1.0, sc - 127))
    w = vals * np.repeat(scale, BLOCK, axis=1)
    with np.errstate(over="ignore"):  # e4m3 * 2^(s-127) overflows bf16 for s >= 247: +-inf
        w32 = w.astype(np.float32)
    return torch.from_numpy(w32).to(torch.bfloat16)


def quantize_layer(layer) -> tuple:
    """bf16 layer (norm1, qkv, o, norm2, gate_up, down) -> 10-tuple of the MXFP8 layout with numpy
    arrays for the quantised matrices (norms unchanged)."""
    norm1, qkv, o, norm2, gate_up, down = layer
    out = [norm1]
    for m in (qkv, o):
        out += list(quantize(m))
    out.append(norm2)
    for m in (gate_up, down):
        out += list(quantize(m))
    return tuple(out)


def dequantize_layer(qlayer) -> tuple:
    """10-tuple MXFP8 layer -> the bf16 6-tuple the decode oracle takes (exact)."""
    norm1, qkv, qkv_s, o, o_s, norm2, gu, gu_s, down, down_s = qlayer
    return (norm1, dequantize(qkv, qkv_s), dequantize(o, o_s), norm2, dequantize(gu, gu_s),
            dequantize(down, down_s))
