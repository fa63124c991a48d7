"""Pin the MXFP8 oracle (oracle/mxfp8.py) against what the formats and the rounding rule fix:
brute-force nearest search, torch's own float8_e4m3fn cast, powers of two.  CPU only."""

import math

import numpy as np
import pytest
import torch

from oracle import mxfp8 as M


def _all_bf16_values() -> np.ndarray:
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    v = bits.view(np.float32)
    return v[np.isfinite(v)]


def _brute_e4m3(v: np.ndarray) -> np.ndarray:
    """Nearest finite E4M3 value (ties to the even code), saturating: an independent search."""
    vals = M.e4m3_values().astype(np.float64)
    finite = np.where(np.isfinite(vals))[0]
    pos = finite[(vals[finite] > 0) | ((vals[finite] == 0) & (finite < 128))]  # +0 and positives
    pv = vals[pos]
    a = np.abs(v.astype(np.float64))
    d = np.abs(a[:, None] - pv[None, :])
    best = d.min(axis=1, keepdims=True)
    cand = d == best
    # ties: the code with an even mantissa (lowest bit 0)
    even = cand & ((pos[None, :] & 1) == 0)
    pick = np.where(even.any(axis=1), np.argmax(even, axis=1), np.argmax(cand, axis=1))
    code = pos[pick]
    code = np.where(a >= 448.0, 0x7E, code)
    sign = (v.view(np.uint32) >> 31) << 7
    return (code | sign).astype(np.uint8)


def test_e4m3_rounding_matches_brute_force_on_every_bf16_value():
    v = _all_bf16_values()
    got = M.e4m3_sat(v)
    want = _brute_e4m3(v)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(v[i]), int(got[i]), int(want[i])) for i in bad[:5]]


def test_e4m3_rounding_matches_torch_float8_cast_in_range():
    """torch's float8_e4m3fn cast (round to nearest even) agrees wherever it does not overflow."""
    v = _all_bf16_values()
    v = v[np.abs(v) < 464.0]
    t = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(M.e4m3_sat(v), t)


def test_e4m3_decode_table_matches_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    t = codes.view(torch.float8_e4m3fn).float().numpy()
    ours = M.e4m3_values()
    nan = np.isnan(t)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], t[~nan])
    assert np.nanmax(ours) == 448.0 and np.nanmin(ours[ours > 0]) == 2.0 ** -9


def test_e8m0_is_smallest_power_of_two_not_below():
    rng = np.random.default_rng(1)
    f = np.concatenate([
        rng.uniform(0, 1, 2000).astype(np.float32) * np.float32(2.0) ** rng.integers(-140, 120, 2000),
        np.float32(2.0) ** np.arange(-126, 127, dtype=np.float32),
        np.nextafter(np.float32(2.0) ** np.arange(-120, 120, dtype=np.float32), np.float32(np.inf)),
        np.nextafter(np.float32(2.0) ** np.arange(-120, 120, dtype=np.float32), np.float32(0)),
    ]).astype(np.float32)
    codes = M.e8m0_ceil(f).astype(np.int64)
    for x, c in zip(f.tolist(), codes.tolist()):
        if x <= 2.0 ** -127:
            assert c == 0, x
            continue
        assert math.ldexp(1.0, c - 127) >= x and (c == 0 or math.ldexp(1.0, c - 128) < x), (x, c)
    assert M.e8m0_ceil(np.array([np.inf, np.nan, 0.0], np.float32)).tolist() == [254, 255, 0]
    assert M.e8m0_ceil(np.array([2.0 ** 200], np.float64).astype(np.float32)).tolist() == [254]


def test_dequantize_exhaustive_codes_and_scales():
    q = np.repeat(np.arange(256, dtype=np.uint8)[None, :], 255, axis=0)  # [255 scales, 256 codes]
    s = np.repeat(np.arange(255, dtype=np.uint8)[:, None], 256 // 32, axis=1)
    w = M.dequantize(q, s).float().numpy()
    vals = M.e4m3_values().astype(np.float64)
    for sc in range(255):
        want = vals * math.ldexp(1.0, sc - 127)  # exact in float64
        got = w[sc].astype(np.float64)
        fin = np.isfinite(want)
        big = fin & (np.abs(want) > 3.3895313892515355e38)  # beyond the largest finite bf16
        normal = fin & ~big & ((np.abs(want) >= 2.0 ** -126) | (want == 0))
        assert np.array_equal(got[normal], want[normal]), sc  # exactly representable in bf16
        # below 2^-126 bf16 is subnormal: the product is rounded to nearest even there
        small = fin & ~big & ~normal
        rounded = torch.from_numpy(want[small].astype(np.float32)).to(torch.bfloat16).double().numpy()
        assert np.array_equal(got[small], rounded), sc
        assert np.array_equal(got[big], np.sign(want[big]) * np.inf), sc  # overflow (scale codes >= 247)
        assert np.isnan(got[~fin]).all()


def test_quantize_block_rule_and_round_trip_bound():
    """Each block's scale is e8m0(amax/448) rounded up, so the largest magnitude lands in
    (224, 448]; dequantised values are within half an e4m3 step of the input."""
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(64, 960, generator=g) * 0.02).to(torch.bfloat16)
    w[0, :32] = 0  # an all-zero block
    w[1, 5] = 300.0  # a large outlier
    q, s = M.quantize(w)
    assert q.shape == (64, 960) and s.shape == (64, M.scale_stride(960)) and (s[:, 30:] == 0).all()
    assert s[0, 0] == 0 and (q[0, :32] == 0).all()
    x = w.float().numpy().reshape(64, 30, 32)
    amax = np.abs(x).max(axis=2)
    scale = np.ldexp(1.0, s[:, :30].astype(np.int64) - 127)
    nz = amax > 0
    assert ((amax[nz] / scale[nz]) <= 448.0).all() and ((amax[nz] / scale[nz]) > 224.0).all()
    d = M.dequantize(q, s).float().numpy().reshape(64, 30, 32).astype(np.float64)
    y = np.abs(x) / scale[..., None]  # the scaled magnitude that was rounded to e4m3
    step = np.ldexp(1.0, np.floor(np.log2(np.maximum(y, 2.0 ** -30))).astype(np.int64) - 3)
    step = np.maximum(step, 2.0 ** -9) * scale[..., None]  # e4m3 spacing (subnormals: 2^-9)
    assert (np.abs(d - x) <= step / 2).all()


def test_planted_mistake_is_caught():
    """Rounding the scale to nearest instead of up (a plausible slip) lets a block's amax exceed
    448 after scaling, which the block rule above rejects."""
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(8, 64, generator=g) * 0.02).to(torch.bfloat16)
    x = w.float().numpy().reshape(8, 2, 32)
    amax = np.abs(x).max(axis=2).astype(np.float32)
    f = (amax * np.float32(1.0 / 448.0)).astype(np.float32)
    nearest = np.rint(np.log2(f.astype(np.float64))).astype(np.int64) + 127
    assert (nearest != M.e8m0_ceil(f)).any()
    assert ((amax / np.ldexp(1.0, nearest - 127)) > 448.0).any()
