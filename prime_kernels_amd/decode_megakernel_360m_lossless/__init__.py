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

_encoded_caches: dict = {}


def _gate_up_weights(layers):
    if len(layers) != LAYERS or any(len(layer) != 6 for layer in layers):
        raise ValueError(f"layers must contain {LAYERS} six-tensor layer tuples")
    return tuple(layer[4] for layer in layers)


def prepare_weights(layers):
    """Prepare the stable encoded gate/up cache eagerly, before graph capture."""
    weights = _gate_up_weights(layers)
    device = weights[0].device
    cache = _encoded_caches.get(device)
    if cache is not None:
        if tuple(t.data_ptr() for t in cache._weights) != tuple(t.data_ptr() for t in weights):
            raise RuntimeError("lossless cache cannot change native GU allocations after preparation")
        return cache
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("prepare_weights must run before graph capture")
    from prime_kernels_amd.lossless_bf16 import EncodedGUCache

    cache = EncodedGUCache(weights)
    _encoded_caches[device] = cache
    return cache


def refresh_weights(layers):
    """Synchronously re-encode the stable cache after a layerwise weight reload."""
    weights = _gate_up_weights(layers)
    cache = _encoded_caches.get(weights[0].device)
    if cache is not None:
        cache.refresh(weights)


def cache_statistics(device=None):
    key = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    cache = _encoded_caches.get(key)
    return cache.statistics() if cache is not None else None


def decode_step(**kw):
    """decode_megakernel_360m.decode_step with this device's prepared cache (if any)."""
    cache = _encoded_caches.get(kw["input_ids"].device)
    return _decode_step(MODEL, encoded_gu=cache, **kw)


def workspace(device):
    return runtime(MODEL, device)
