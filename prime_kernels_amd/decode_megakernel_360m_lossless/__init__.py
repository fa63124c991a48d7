"""Opt-in lossless gate/up SmolLM2-360M decode step on MI355X (gfx950).

Drop-in for prime_kernels.decode_megakernel_360m_lossless (reference __init__.py:83-234):
`prepare_weights(layers)` builds the per-device encoded gate/up cache (before graph capture),
`refresh_weights(layers)` re-encodes it after a weight reload, `cache_statistics(device)` reports
it, and `decode_step(**kw)` has the decode_megakernel_360m contract.  With a prepared cache, the
batch-1 step streams each enabled layer's plane, headers and escapes instead of its dense gate/up
rows (about 1.5 bytes per weight instead of 2) and is bit-identical to the dense step; layers whose
escapes overflowed their table, and batches of 2 or more, read the dense matrices.  The returned
tensor is a view into a shared per-device output buffer, overwritten by the next call.
"""

from __future__ import annotations

import torch

from prime_kernels_amd._decode import SMOLLM2_360M, decode_step as _decode_step, runtime

MODEL = SMOLLM2_360M

MAX_BATCH = MODEL.max_batch
MAX_SEQ = MODEL.max_seq
HIDDEN = MODEL.hidden
INTERMEDIATE = MODEL.inter
LAYERS = MODEL.layers
KV_HEADS = MODEL.kv_heads
HEAD_DIM = MODEL.head_dim
BLOCK_SIZE = 16
EPS = 1e-5

class _PerDevice:
    """One encoded gate/up cache per device, built from one set of gate_up tensors."""

    def __init__(self):
        self._by_device: dict = {}

    def get(self, device):
        return self._by_device.get(torch.device(device))

    def build(self, weights):
        device = weights[0].device
        have = self._by_device.get(device)
        if have is not None:
            if [t.data_ptr() for t in have.weights] != [t.data_ptr() for t in weights]:
                raise RuntimeError("the lossless cache of this device was prepared for other gate_up tensors; "
                                   "re-encode new values in place with refresh_weights")
            return have
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("prepare_weights must be called before graph capture")
        from prime_kernels_amd.lossless_bf16 import EncodedGUCache

        built = EncodedGUCache(weights)
        self._by_device[device] = built
        return built


_caches = _PerDevice()


def _gate_up_of(layers) -> tuple:
    """The gate_up tensor (index 4) of each of the 32 six-tensor layer tuples."""
    layers = list(layers)
    if len(layers) != LAYERS or any(len(layer) != 6 for layer in layers):
        raise ValueError(f"expected {LAYERS} layer tuples of six tensors")
    return tuple(layer[4] for layer in layers)


def prepare_weights(layers):
    """Build (or return) this device's encoded gate/up cache; call it before any graph capture."""
    return _caches.build(_gate_up_of(layers))


def refresh_weights(layers):
    """Re-encode the device's cache after its gate_up tensors were reloaded in place (synchronous).
    Without a prepared cache this does nothing."""
    weights = _gate_up_of(layers)
    cache = _caches.get(weights[0].device)
    if cache is not None:
        cache.refresh(weights)


def cache_statistics(device=None):
    """statistics() of the device's cache (default: the current CUDA device), or None."""
    cache = _caches.get(device if device is not None else torch.device("cuda", torch.cuda.current_device()))
    return None if cache is None else cache.statistics()


def decode_step(**kw):
    """decode_megakernel_360m.decode_step, reading the device's prepared cache when there is one."""
    return _decode_step(MODEL, encoded_gu=_caches.get(kw["input_ids"].device), **kw)


def workspace(device):
    return runtime(MODEL, device)
