"""Pin the lossless gate/up codec oracle (oracle/lossless.py) on the CPU: the reference's own
known-answer vector, exhaustive round trips over every bf16 pattern, the escape rule against an
independent per-chunk loop, the capacity / row_offsets semantics, and a planted mistake."""

import numpy as np
import pytest

from oracle import lossless as LZ

# research/smollm2_360m_decode/experiments/lossless-gu-codec-survey-r1/survey.py:63-69: five
# chunks of crafted edge patterns (signed zeros, subnormals, an exponent spread of exactly 8,
# infinities and NaNs, consecutive exponents).
KNOWN_ANSWER = np.array([
    0x8000, 0x0000, 0x0001, 0x007F, 0x8001, 0x0002, 0x0003, 0x0004,
    0x0080, 0x0480, 0x0081, 0x0882, 0x0083, 0x0884, 0x0085, 0x0086,
    0x0100, 0x0180, 0x0200, 0x0280, 0x0300, 0x0380, 0x0400, 0x0480,
    0x7F80, 0xFF80, 0x7FC1, 0xFFC2, 0x7F81, 0xFF82, 0x7FFF, 0xFFFF,
    0x8180, 0x8200, 0x8280, 0x8300, 0x8380, 0x8400, 0x8480, 0x8500,
], dtype=np.uint16)


def _known_answer_checks(enc_fn=LZ.encode):
    src = KNOWN_ANSWER.reshape(1, 40)
    enc = enc_fn(src)
    h = enc["headers"].reshape(-1).astype(np.int64)
    esc = np.nonzero((h >> 24) == 255)[0].tolist()
    assert esc == [1, 3], esc                                     # survey.py:71-72
    assert (h[[1, 3]] & 0xFFFFFF).tolist() == [0, 1]              # survey.py:74-76
    assert np.array_equal(LZ.decode(enc["plane"], enc["headers"], enc["raw"]), src)  # :77-79
    perm = enc["headers"].copy().reshape(-1)                      # :80-85
    perm[1] = (perm[1] & 0xFF000000) | 1
    perm[3] = (perm[3] & 0xFF000000) | 0
    raw_flipped = enc["raw"].reshape(-1, 8)[::-1].reshape(-1)
    assert np.array_equal(LZ.decode(enc["plane"], perm.reshape(1, 5), raw_flipped), src)


def test_reference_known_answer_vector():
    _known_answer_checks()


def test_known_answer_layout_details():
    enc = LZ.encode(KNOWN_ANSWER.reshape(1, 40))
    h = enc["headers"].reshape(-1)
    # chunk 0: exponents {0,0,0,0,0,0,0,0} -> base 0, no deltas
    assert int(h[0]) == 0
    # chunk 2: exponents 2,3,4,5,6,7,8,9 -> base 2, deltas 0..7
    assert int(h[2]) == (2 << 24) | sum(i << (3 * i) for i in range(8))
    # chunk 4 (0x8180 .. 0x8500, negative): exponents 3..10 -> base 3, deltas 0..7
    assert int(h[4]) == (3 << 24) | sum(i << (3 * i) for i in range(8))
    assert enc["plane"][0, 32] == 0x80 and enc["plane"][0, 0] == 0x80 and enc["plane"][0, 3] == 0x7F
    assert enc["row_offsets"].tolist() == [0, 2] and enc["count"] == 2
    assert enc["prefix"].tolist() == [0, 1, 1, 2, 2] and enc["flags"].tolist() == [0, 1, 0, 1, 0]


@pytest.mark.parametrize("order", ["sequential", "shuffled"])
def test_round_trip_every_bf16_pattern(order):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    if order == "shuffled":
        bits = np.random.default_rng(0).permutation(bits)
    m = bits.reshape(512, 128)
    enc = LZ.encode(m)
    assert np.array_equal(LZ.decode(enc["plane"], enc["headers"], enc["raw"]), m)
    if order == "shuffled":
        assert enc["count"] > 0.5 * m.size / 8        # most shuffled chunks escape


def _escape_brute(chunk) -> bool:
    es = [(int(v) >> 7) & 255 for v in chunk]
    return min(es) == 255 or max(es) - min(es) > 7


def test_escape_rule_against_per_chunk_loop():
    rng = np.random.default_rng(1)
    # chunks built around chosen exponent spreads 0..12 plus all-255 and near-255 cases
    rows = []
    for spread in list(range(13)) * 40:
        base = int(rng.integers(0, 256 - spread))
        e = base + rng.integers(0, spread + 1, 8)
        e[0], e[1] = base, base + spread
        words = (rng.integers(0, 2, 8) << 15) | (e << 7) | rng.integers(0, 128, 8)
        rows.append(rng.permutation(words))
    rows.append([0x7F80 | int(x) for x in rng.integers(0, 128, 8)])      # all exponent 255
    rows.append([0x7F00] + [0x7F80] * 7)                                  # 254..255: not escaped
    m = np.array(rows, dtype=np.uint64).astype(np.uint16).reshape(-1, 8)
    enc = LZ.encode(m)
    want = np.array([_escape_brute(r) for r in m])
    got = (enc["headers"].reshape(-1) >> 24) == 255
    assert np.array_equal(got, want)
    assert np.array_equal(LZ.decode(enc["plane"], enc["headers"], enc["raw"]), m)


def test_capacity_row_offsets_and_enabled():
    rng = np.random.default_rng(2)
    m = (rng.standard_normal((64, 960)) * 0.02).astype(np.float32)
    bits = (m.view(np.uint32) >> 16).astype(np.uint16)
    bits[3, 0:8] = [0x7F80] * 8                     # exponent 255 chunk: escaped
    bits[10, 8:16] = [0x0001, 0x3F80] + [0] * 6     # spread 127: escaped
    full = LZ.encode(bits)
    n = full["count"]
    assert n > 2
    per_row = ((full["headers"] >> 24) == 255).sum(axis=1)
    assert np.array_equal(np.diff(full["row_offsets"].astype(np.int64)), per_row)
    assert full["row_offsets"][-1] == n and full["prefix"][-1] == n
    # capacity exactly the count: enabled, raw complete
    ok = LZ.encode(bits, capacity=n)
    assert ok["enabled"] == 1 and ok["raw"].size == 8 * n
    assert np.array_equal(LZ.decode(ok["plane"], ok["headers"], ok["raw"]), bits)
    # one short: disabled, raw keeps the first capacity escapes, headers unchanged
    short = LZ.encode(bits, capacity=n - 1)
    assert short["enabled"] == 0 and short["raw"].size == 8 * (n - 1)
    assert np.array_equal(short["headers"], full["headers"])
    assert np.array_equal(short["raw"], full["raw"][: 8 * (n - 1)])
    # escaped words come back through the raw table in chunk order
    esc_chunks = bits.reshape(-1, 8)[(full["headers"].reshape(-1) >> 24) == 255]
    assert np.array_equal(full["raw"].reshape(-1, 8), esc_chunks)


def test_planted_mistakes_are_caught(monkeypatch):
    """An escape threshold one too strict (spread 6) moves the reference vector's escapes off
    [1, 3]; one too loose (spread 8, more than 3 bits hold) breaks the per-chunk escape rule and
    the round trip of chunks built with a spread of exactly 8."""
    monkeypatch.setattr(LZ, "MAX_SPREAD", 6)
    with pytest.raises(AssertionError):
        _known_answer_checks()
    monkeypatch.setattr(LZ, "MAX_SPREAD", 8)
    with pytest.raises(AssertionError):
        test_escape_rule_against_per_chunk_loop()
