"""Fixed-capacity lossless cache of the bf16 gate/up matrices (exponent-delta byte plane) on
MI355X (gfx950).

Drop-in for prime_kernels.lossless_bf16 (reference __init__.py:52-181): `EncodedGUCache(weights)`
encodes 32 contiguous bf16 [5120, 960] gate_up matrices on their device, sizes each layer's escape
table at 1.25x the escapes it found, and exposes the device descriptor table (`table`) the
lossless decode step reads; `refresh(weights)` re-encodes into the same buffers (a layer whose
escapes no longer fit is disabled and decoded from its dense matrix), `statistics()` reports the
state, `decode_layer(i)` rebuilds a matrix bit for bit.  The codec runs in the library's HIP
kernels (include/prime_lossless.h); nothing here computes on the CPU.
"""

from __future__ import annotations

import ctypes
import math

import torch

from prime_kernels_amd import _native

LAYERS = 32
ROWS = 5120
COLS = 960
CHUNKS = ROWS * (COLS // 8)
DESCRIPTOR_BYTES = 5 * ctypes.sizeof(ctypes.c_void_p)


def _check(rc, operation):
    if rc:
        raise RuntimeError(f"{operation} failed: {_native.status_string(rc)}")


class EncodedGUCache:
    """Encode 32 contiguous bf16 [5120, 960] gate/up matrices on their (gfx950) device."""

    def __init__(self, weights):
        if len(weights) != LAYERS:
            raise ValueError(f"weights must contain {LAYERS} layers")
        self.device = weights[0].device
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("EncodedGUCache must be prepared before graph capture")
        self._validate(weights)
        self._lib = _native.library()
        self._stream = torch.cuda.current_stream(self.device)
        self._stream_handle = self._stream.cuda_stream
        self._tables = []
        self._enabled = []
        self._raw_counts = []
        self._raw_capacities = [0] * LAYERS
        self._generation = 0
        self._scan_workspace_bytes = self._lib.lossless_scan_workspace_bytes()
        dev = self.device
        self._scan_workspace = torch.empty(self._scan_workspace_bytes, dtype=torch.uint8, device=dev)
        self._flags = torch.empty((CHUNKS,), dtype=torch.uint32, device=dev)
        self._prefix = torch.empty((CHUNKS,), dtype=torch.uint32, device=dev)
        self._escape_counts = torch.empty((LAYERS,), dtype=torch.uint32, device=dev)
        for _ in range(LAYERS):
            self._tables.append({
                "plane": torch.empty((ROWS, COLS), dtype=torch.uint8, device=dev),
                "headers": torch.empty((ROWS, COLS // 8), dtype=torch.uint32, device=dev),
                "raw": torch.empty((8,), dtype=torch.uint16, device=dev),
                "row_offsets": torch.empty((ROWS + 1,), dtype=torch.uint32, device=dev),
            })
            self._enabled.append(torch.empty((), dtype=torch.uint32, device=dev))
        self.table = torch.empty((LAYERS * DESCRIPTOR_BYTES,), dtype=torch.uint8, device=dev)
        self._weights = tuple(weights)
        self._prime_capacities(self._weights)
        self._pack_all(self._weights)
        self._write_descriptors()
        self._stream.synchronize()
        self._generation = 1

    def _validate(self, weights):
        for i, tensor in enumerate(weights):
            if (not isinstance(tensor, torch.Tensor) or not tensor.is_cuda or tensor.device != self.device
                    or tensor.dtype != torch.bfloat16 or tuple(tensor.shape) != (ROWS, COLS)
                    or not tensor.is_contiguous() or tensor.data_ptr() % 16):
                raise ValueError(f"weights[{i}] must be contiguous 16-byte aligned bf16 [{ROWS}, {COLS}] "
                                 f"on {self.device}")

    def _encode(self, index, tensor):
        t = self._tables[index]
        return self._lib.lossless_encode_layer(
            tensor.data_ptr(), t["plane"].data_ptr(), t["headers"].data_ptr(), t["raw"].data_ptr(),
            t["row_offsets"].data_ptr(), self._flags.data_ptr(), self._prefix.data_ptr(),
            self._scan_workspace.data_ptr(), self._scan_workspace_bytes, self._enabled[index].data_ptr(),
            self._raw_capacities[index], self._stream_handle)

    def _prime_capacities(self, weights):
        # a counting pass with capacity 0, then an escape table of 1.25x the count (at least 1 chunk)
        for i, tensor in enumerate(weights):
            _check(self._encode(i, tensor), f"count escapes for layer {i}")
            self._stream.synchronize()
            count = int(self._prefix[-1].item())
            capacity = max(1, math.ceil(count * 1.25))
            self._tables[i]["raw"] = torch.empty((capacity * 8,), dtype=torch.uint16, device=self.device)
            self._raw_counts.append(count)
            self._raw_capacities[i] = capacity

    def _pack_all(self, weights):
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("EncodedGUCache.refresh cannot run during graph capture")
        self._validate(weights)
        for i, tensor in enumerate(weights):
            _check(self._encode(i, tensor), f"encode layer {i}")
        self._weights = tuple(weights)

    def _write_descriptors(self):
        for i, t in enumerate(self._tables):
            _check(self._lib.lossless_write_descriptor(
                self.table.data_ptr(), i, t["plane"].data_ptr(), t["headers"].data_ptr(), t["raw"].data_ptr(),
                t["row_offsets"].data_ptr(), self._enabled[i].data_ptr(), self._stream_handle),
                f"write descriptor {i}")

    @torch.inference_mode()
    def refresh(self, weights):
        """Synchronously re-encode into the existing buffers after callers quiesce decode."""
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("EncodedGUCache.refresh cannot run during graph capture")
        self._validate(weights)
        torch.cuda.synchronize(self.device)
        self._stream = torch.cuda.current_stream(self.device)
        self._stream_handle = self._stream.cuda_stream
        for i, tensor in enumerate(weights):
            _check(self._encode(i, tensor), f"refresh layer {i}")
            self._escape_counts[i:i + 1].copy_(self._prefix[-1:])
        self._stream.synchronize()
        self._raw_counts = [int(v) for v in self._escape_counts.cpu().tolist()]
        self._weights = tuple(weights)
        self._generation += 1

    def statistics(self):
        active = [int(flag.item()) for flag in self._enabled]
        fixed = sum(t["plane"].numel() + t["headers"].numel() * 4 + t["row_offsets"].numel() * 4
                    + t["raw"].numel() * 2 for t in self._tables)
        return {
            "generation": self._generation,
            "active_layers": sum(active),
            "layers": LAYERS,
            "escape_chunks": list(self._raw_counts),
            "raw_capacities": list(self._raw_capacities),
            "allocated_bytes": fixed + self.table.numel() + self._scan_workspace.numel() + self._flags.numel() * 4
                               + self._prefix.numel() * 4 + self._escape_counts.numel() * 4 + LAYERS * 4,
        }

    def enabled(self, index) -> bool:
        return bool(int(self._enabled[index].item()))

    def buffers(self, index) -> dict:
        """The device buffers of layer `index` (plane, headers, raw, row_offsets) and its flag."""
        return dict(self._tables[index], enabled=self._enabled[index])

    def decode_layer(self, index):
        if not 0 <= index < LAYERS:
            raise IndexError(index)
        if not self.enabled(index):
            return self._weights[index].clone()
        out = torch.empty((ROWS, COLS), dtype=torch.bfloat16, device=self.device)
        t = self._tables[index]
        _check(self._lib.lossless_decode_layer(t["plane"].data_ptr(), t["headers"].data_ptr(), t["raw"].data_ptr(),
                                               out.data_ptr(), torch.cuda.current_stream(self.device).cuda_stream),
               f"decode layer {index}")
        return out
