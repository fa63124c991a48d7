"""Lossless cache of the 32 bf16 gate/up matrices of SmolLM2-360M for the batch-1 decode step.

Interface of prime_kernels.lossless_bf16 (reference __init__.py:52-181): `EncodedGUCache(weights)`
with `table`, `refresh(weights)`, `statistics()` and `decode_layer(i)`, and the buffer format of
include/prime_lossless.h (per layer: a byte plane [5120, 960], a u32 header per 8-weight chunk,
an escape table of whole chunks, row offsets, and an enabled flag that the encoder clears when the
layer's escapes do not fit its table).

Design.  All encoding, decoding and scanning runs in the library's HIP kernels on the cache's
device.  An encoder pass launches every layer back to back and copies each layer's escape count
to a device vector right behind its launch, so a pass costs one host synchronisation.  Preparation
is two passes: with empty tables (the encoder only counts, and disables every layer that has
escapes), then with tables sized at HEADROOM times the count.  `refresh` is one pass into the
existing tables; a layer that now has more escapes than its table holds stays disabled, and the
decode step reads its dense matrix.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from prime_kernels_amd import _native

LAYERS = 32
ROWS = 5120
COLS = 960
CHUNKS = ROWS * (COLS // 8)          # 8-weight chunks per matrix
HEADROOM = 1.25                      # escape-table capacity / escapes found at preparation
DESCRIPTOR_BYTES = 5 * ctypes.sizeof(ctypes.c_void_p)   # one descriptor per layer (prime_lossless.h)


@dataclass
class _LayerCode:
    """Device buffers of one encoded layer and its escape bookkeeping (in chunks)."""

    plane: torch.Tensor          # [ROWS, COLS] u8
    headers: torch.Tensor        # [ROWS, COLS / 8] u32
    raw: torch.Tensor            # [capacity * 8] u16, the escaped chunks verbatim
    row_offsets: torch.Tensor    # [ROWS + 1] u32, first escape ordinal of each row
    enabled: torch.Tensor        # [] u32, written by the encoder
    capacity: int = 0
    found: int = 0


def _raise_on(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"lossless gate/up cache: {what}: {_native.status_string(rc)}")


class EncodedGUCache:
    """The encoded gate/up matrices of all 32 layers, on the weights' device."""

    def __init__(self, weights):
        weights = tuple(weights)
        if len(weights) != LAYERS:
            raise ValueError(f"expected the gate_up matrices of {LAYERS} layers, got {len(weights)}")
        self.device = weights[0].device if isinstance(weights[0], torch.Tensor) else None
        self._check(weights)
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("prepare the lossless gate/up cache before graph capture")
        self._lib = _native.library()
        dev = self.device
        u32 = torch.uint32
        # scratch shared by the layers of a pass (the encoder's chunk flags and their inclusive scan)
        self._scan_bytes = self._lib.lossless_scan_workspace_bytes()
        self._scan = torch.empty((self._scan_bytes,), dtype=torch.uint8, device=dev)
        self._flags = torch.empty((CHUNKS,), dtype=u32, device=dev)
        self._prefix = torch.empty((CHUNKS,), dtype=u32, device=dev)
        self._counts = torch.empty((LAYERS,), dtype=u32, device=dev)
        self._layers = [
            _LayerCode(plane=torch.empty((ROWS, COLS), dtype=torch.uint8, device=dev),
                       headers=torch.empty((ROWS, COLS // 8), dtype=u32, device=dev),
                       raw=torch.empty((8,), dtype=torch.uint16, device=dev),
                       row_offsets=torch.empty((ROWS + 1,), dtype=u32, device=dev),
                       enabled=torch.empty((), dtype=u32, device=dev))
            for _ in range(LAYERS)]
        self.table = torch.empty((LAYERS * DESCRIPTOR_BYTES,), dtype=torch.uint8, device=dev)
        # pass 1 counts (no table has room), pass 2 encodes into tables with headroom
        counts = self._encode_pass(weights, [0] * LAYERS)
        for code, n in zip(self._layers, counts):
            code.capacity = max(1, math.ceil(n * HEADROOM))
            code.raw = torch.empty((code.capacity * 8,), dtype=torch.uint16, device=dev)
        counts = self._encode_pass(weights, [c.capacity for c in self._layers])
        for code, n in zip(self._layers, counts):
            code.found = n
        stream = torch.cuda.current_stream(dev)
        for i, code in enumerate(self._layers):
            _raise_on(self._lib.lossless_write_descriptor(
                self.table.data_ptr(), i, code.plane.data_ptr(), code.headers.data_ptr(), code.raw.data_ptr(),
                code.row_offsets.data_ptr(), code.enabled.data_ptr(), stream.cuda_stream), f"descriptor {i}")
        stream.synchronize()
        self._weights = weights
        self.generation = 1

    # -- the tensors the cache encodes ------------------------------------------------------------

    def _check(self, weights) -> None:
        for i, t in enumerate(weights):
            ok = (isinstance(t, torch.Tensor) and t.is_cuda and t.device == self.device and t.dtype == torch.bfloat16
                  and tuple(t.shape) == (ROWS, COLS) and t.is_contiguous() and t.data_ptr() % 16 == 0)
            if not ok:
                raise ValueError(f"gate_up matrix {i}: need a contiguous, 16-byte aligned bf16 [{ROWS}, {COLS}] "
                                 f"tensor on {self.device}")

    @property
    def weights(self) -> tuple:
        """The gate_up tensors the cache was last encoded from."""
        return self._weights

    # -- encoding ---------------------------------------------------------------------------------

    def _encode_pass(self, weights, capacities) -> list:
        """Encode every layer on the current stream; returns the escape chunks each layer has."""
        stream = torch.cuda.current_stream(self.device)
        for i, (t, code) in enumerate(zip(weights, self._layers)):
            _raise_on(self._lib.lossless_encode_layer(
                t.data_ptr(), code.plane.data_ptr(), code.headers.data_ptr(), code.raw.data_ptr(),
                code.row_offsets.data_ptr(), self._flags.data_ptr(), self._prefix.data_ptr(), self._scan.data_ptr(),
                self._scan_bytes, code.enabled.data_ptr(), capacities[i], stream.cuda_stream), f"encode layer {i}")
            # the scan total, copied before the next layer reuses the scan
            self._counts[i:i + 1].copy_(self._prefix[CHUNKS - 1:])
        stream.synchronize()
        return [int(n) for n in self._counts.view(torch.int32).cpu().tolist()]

    @torch.inference_mode()
    def refresh(self, weights) -> None:
        """Re-encode new values of the gate_up matrices into the existing tables (after a weight
        reload).  Synchronous; decode steps on the device must not be running."""
        weights = tuple(weights)
        if len(weights) != LAYERS:
            raise ValueError(f"expected the gate_up matrices of {LAYERS} layers, got {len(weights)}")
        self._check(weights)
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the lossless gate/up cache cannot be refreshed during graph capture")
        torch.cuda.synchronize(self.device)
        counts = self._encode_pass(weights, [c.capacity for c in self._layers])
        for code, n in zip(self._layers, counts):
            code.found = n
        self._weights = weights
        self.generation += 1

    # -- state ------------------------------------------------------------------------------------

    def enabled(self, index: int) -> bool:
        """Whether layer `index` is read from its encoding (False: its escapes overflowed)."""
        return bool(int(self._layers[index].enabled.view(torch.int32)))

    def buffers(self, index: int) -> dict:
        """Layer `index`'s device buffers in the format's names, and its enabled flag."""
        c = self._layers[index]
        return {"plane": c.plane, "headers": c.headers, "raw": c.raw, "row_offsets": c.row_offsets,
                "enabled": c.enabled}

    def _owned(self):
        yield from (self._scan, self._flags, self._prefix, self._counts, self.table)
        for c in self._layers:
            yield from (c.plane, c.headers, c.raw, c.row_offsets, c.enabled)

    def statistics(self) -> dict:
        flags = torch.stack([c.enabled.view(torch.int32) for c in self._layers]).cpu().tolist()
        return {
            "generation": self.generation,
            "active_layers": sum(1 for f in flags if f),
            "layers": LAYERS,
            "escape_chunks": [c.found for c in self._layers],
            "raw_capacities": [c.capacity for c in self._layers],
            "allocated_bytes": sum(t.numel() * t.element_size() for t in self._owned()),
        }

    def decode_layer(self, index: int) -> torch.Tensor:
        """Layer `index`'s gate_up matrix rebuilt from its encoding (a copy of the dense matrix for a
        disabled layer): bit-identical to the matrix it was encoded from."""
        if not 0 <= index < LAYERS:
            raise IndexError(f"layer {index} is not in 0..{LAYERS - 1}")
        if not self.enabled(index):
            return self._weights[index].clone()
        c = self._layers[index]
        out = torch.empty((ROWS, COLS), dtype=torch.bfloat16, device=self.device)
        _raise_on(self._lib.lossless_decode_layer(c.plane.data_ptr(), c.headers.data_ptr(), c.raw.data_ptr(),
                                                  out.data_ptr(), torch.cuda.current_stream(self.device).cuda_stream),
                  f"decode layer {index}")
        return out
