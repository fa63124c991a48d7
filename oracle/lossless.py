"""CPU oracle for the lossless bf16 gate/up codec (exponent-delta byte plane).

TEST INFRASTRUCTURE ONLY, like oracle/smollm2.py: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline may import it.

What it restates (reference files under Mantissagithub/prime-kernels):
  codec      prime_kernels/lossless_bf16/csrc/lossless_bf16.cu:16-103 (encode_chunks,
             scatter_escapes, publish_offsets, publish_mode, decode_chunks) and the CPU
             encode/decode research/smollm2_360m_decode/experiments/
             lossless-gu-codec-survey-r1/survey.py:22-59
  layout     prime_kernels/lossless_bf16/csrc/encoded_gu.h:6-13 (plane, headers, raw,
             row_offsets, enabled); host lifecycle prime_kernels/lossless_bf16/__init__.py:52-181

A matrix of bf16 words [rows, cols] is cut into chunks of 8 consecutive words of a row
(cols / 8 chunks per row, numbered row-major).  Per chunk, with e_i = (word_i >> 7) & 255:
  plane[i]  = (word_i >> 8 & 0x80) | (word_i & 0x7f)          sign and mantissa, one byte
  escape    = min(e) == 255 or max(e) - min(e) > 7
  header    = min(e) << 24 | sum_i (e_i - min(e)) << 3i           (not escaped)
            = 0xFF << 24 | ordinal                                (escaped; ordinal = number
                                                                   of escaped chunks before it)
  raw[8*ordinal + i] = word_i for escaped chunks with ordinal < capacity
  row_offsets[r] = escaped chunks in rows 0..r-1 (rows + 1 entries)
  enabled   = 1 if the number of escaped chunks <= capacity, else 0 (the decode step then
              reads the dense matrix)
Decoding a non-escaped chunk: word_i = (p_i & 0x80) << 8 | (base + delta_i) << 7 | (p_i & 0x7f).

Pinned by tests/test_oracle_lossless.py: the reference's own known-answer vector
(survey.py:63-88: escapes at chunks [1, 3], dense raw indices [0, 1], a header-indexed
permuted-table round trip), an exhaustive round trip over all 65,536 bf16 patterns, a
brute-force escape rule on random chunks, and a planted mistake.
"""

from __future__ import annotations

import numpy as np

CHUNK = 8
ESCAPE = 255
MAX_SPREAD = 7   # largest exponent spread a chunk's 3-bit deltas can carry


def _words(bits) -> np.ndarray:
    a = np.asarray(bits)
    if a.dtype != np.uint16:
        a = a.astype(np.uint16)
    return a


def encode(bits, capacity: int | None = None) -> dict:
    """bf16 bit patterns [rows, cols] (uint16) -> the codec's buffers.

    capacity None keeps every escape (the survey's CPU encoder); an integer keeps the first
    `capacity` escaped chunks in `raw` and sets `enabled` as the library does."""
    w = _words(bits)
    if w.ndim != 2 or w.shape[1] % CHUNK:
        raise ValueError("bits must be [rows, cols] with cols a multiple of 8")
    rows, cols = w.shape
    ch = w.reshape(rows, cols // CHUNK, CHUNK).astype(np.uint32)
    e = (ch >> 7) & 255
    base = e.min(axis=2)
    spread = e.max(axis=2) - base
    esc = (base == ESCAPE) | (spread > MAX_SPREAD)
    delta = np.where(esc[..., None], 0, e - base[..., None])
    packed = np.zeros(base.shape, dtype=np.uint32)
    for i in range(CHUNK):
        packed |= delta[..., i].astype(np.uint32) << (3 * i)
    flat_esc = esc.reshape(-1)
    ordinal = np.cumsum(flat_esc, dtype=np.int64) - 1           # inclusive prefix - 1
    headers = (base.astype(np.uint32) << 24) | packed
    headers = headers.reshape(-1)
    headers[flat_esc] = (np.uint32(0xFF) << 24) | ordinal[flat_esc].astype(np.uint32)
    plane = (((ch >> 8) & 0x80) | (ch & 0x7F)).astype(np.uint8).reshape(rows, cols)
    count = int(flat_esc.sum())
    keep = count if capacity is None else min(count, capacity)
    raw = ch.reshape(-1, CHUNK)[flat_esc][:keep].astype(np.uint16).reshape(-1)
    per_row = esc.sum(axis=1)
    row_offsets = np.concatenate([[0], np.cumsum(per_row)]).astype(np.uint32)
    prefix = np.cumsum(flat_esc, dtype=np.int64).astype(np.uint32)
    return {
        "plane": plane,
        "headers": headers.reshape(rows, cols // CHUNK),
        "raw": raw,
        "row_offsets": row_offsets,
        "count": count,
        "enabled": int(capacity is None or count <= capacity),
        "flags": flat_esc.astype(np.uint32),
        "prefix": prefix,
    }


def decode(plane, headers, raw) -> np.ndarray:
    """(plane [rows, cols] u8, headers [rows, cols/8] u32, raw u16) -> bf16 bits [rows, cols]."""
    p = np.asarray(plane, dtype=np.uint8)
    rows, cols = p.shape
    h = np.asarray(headers, dtype=np.uint32).reshape(rows, cols // CHUNK)
    base = (h >> 24)[..., None]
    shifts = (np.arange(CHUNK, dtype=np.uint32) * 3)[None, None, :]
    delta = ((h & 0xFFFFFF)[..., None] >> shifts) & 7
    pc = p.reshape(rows, cols // CHUNK, CHUNK).astype(np.uint32)
    words = ((pc & 0x80) << 8) | (((base + delta) & 0x1FF) << 7) | (pc & 0x7F)
    esc = (h >> 24) == ESCAPE
    if esc.any():
        table = np.asarray(raw, dtype=np.uint16).reshape(-1, CHUNK).astype(np.uint32)
        idx = (h[esc] & 0xFFFFFF).astype(np.int64)
        if idx.size and int(idx.max()) >= table.shape[0]:
            raise ValueError("an escape ordinal is past the raw table")
        words[esc] = table[idx]
    return (words & 0xFFFF).astype(np.uint16).reshape(rows, cols)


def encoded_bytes(enc: dict) -> int:
    """Bytes a decode step streams for one encoded matrix: plane, headers and its escapes."""
    return enc["plane"].size + enc["headers"].size * 4 + enc["count"] * CHUNK * 2
