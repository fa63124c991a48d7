"""torch.ops.prime_decode: the decode step as a registered operator, with a fake (meta) kernel.

The reference registers its compiled ops with TORCH_LIBRARY and adds the fake kernels from
Python (README.md:101-114, pattern flash_moe/__init__.py:34-95); for Python-side ops it names
torch.library.custom_op as the way to define them.  This library's boundary is a C ABI loaded
with ctypes, so the op is defined here with custom_op and calls the same launcher as
`decode_step(**kw)`.  Unlike that function, the op returns fresh tensors (an op's outputs may
not alias a module-owned buffer) and declares the KV caches it appends to as mutated, so it
composes with torch.compile and graph tracing:

    hidden, ids = torch.ops.prime_decode.decode_step(
        360, input_ids, positions, seq_lens, block_table, slot_mapping, embed,
        [w for layer in layers for w in layer], final_norm, kv_caches, cos_sin_cache, 1e-5)
"""

from __future__ import annotations

import torch
from torch import Tensor

from prime_kernels_amd._decode import MODELS, VOCAB, Model, decode_step as _decode_step


def _model(model_id: int) -> Model:
    if model_id not in MODELS:
        raise ValueError(f"model_id must be one of {sorted(MODELS)}, got {model_id}")
    return MODELS[model_id]


def _layers(model: Model, layer_weights: list[Tensor]):
    if len(layer_weights) % 6 or not 1 <= len(layer_weights) // 6 <= model.layers:
        raise ValueError(f"layer_weights must hold 6 tensors per layer for 1..{model.layers} layers")
    return [tuple(layer_weights[6 * i:6 * i + 6]) for i in range(len(layer_weights) // 6)]


@torch.library.custom_op("prime_decode::decode_step", mutates_args=("kv_caches",), device_types="cuda")
def decode_step(model_id: int, input_ids: Tensor, positions: Tensor, seq_lens: Tensor, block_table: Tensor,
                slot_mapping: Tensor, embed: Tensor, layer_weights: list[Tensor], final_norm: Tensor,
                kv_caches: list[Tensor], cos_sin_cache: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """One greedy decode step: (final-normed hidden [B, H] bf16, greedy ids [B] int64)."""
    model = _model(model_id)
    layers = _layers(model, layer_weights)
    hidden, ids = _decode_step(model, input_ids=input_ids, positions=positions, seq_lens=seq_lens,
                               block_table=block_table, slot_mapping=slot_mapping, embed=embed, layers=layers,
                               final_norm=final_norm, kv_caches=kv_caches, cos_sin_cache=cos_sin_cache, eps=eps,
                               return_token_ids=True, num_layers=len(layers))
    return hidden.clone(), ids.clone()


@decode_step.register_fake
def _decode_step_fake(model_id, input_ids, positions, seq_lens, block_table, slot_mapping, embed,
                      layer_weights, final_norm, kv_caches, cos_sin_cache, eps):
    model = _model(model_id)
    _layers(model, layer_weights)
    batch = input_ids.shape[0]
    return (input_ids.new_empty((batch, model.hidden), dtype=torch.bfloat16),
            input_ids.new_empty((batch,), dtype=torch.int64))


@torch.library.custom_op("prime_decode::decode_logits", mutates_args=("kv_caches", "logits"), device_types="cuda")
def decode_logits(model_id: int, input_ids: Tensor, positions: Tensor, seq_lens: Tensor, block_table: Tensor,
                  slot_mapping: Tensor, embed: Tensor, layer_weights: list[Tensor], final_norm: Tensor,
                  kv_caches: list[Tensor], cos_sin_cache: Tensor, eps: float, logits: Tensor) -> Tensor:
    """As decode_step, also writing the bf16 logits [B, 49152] into `logits`; returns the ids."""
    model = _model(model_id)
    layers = _layers(model, layer_weights)
    _, ids = _decode_step(model, input_ids=input_ids, positions=positions, seq_lens=seq_lens,
                          block_table=block_table, slot_mapping=slot_mapping, embed=embed, layers=layers,
                          final_norm=final_norm, kv_caches=kv_caches, cos_sin_cache=cos_sin_cache, eps=eps,
                          return_token_ids=True, logits_out=logits, num_layers=len(layers))
    return ids.clone()


@decode_logits.register_fake
def _decode_logits_fake(model_id, input_ids, positions, seq_lens, block_table, slot_mapping, embed,
                        layer_weights, final_norm, kv_caches, cos_sin_cache, eps, logits):
    model = _model(model_id)
    _layers(model, layer_weights)
    if tuple(logits.shape) != (input_ids.shape[0], VOCAB):
        raise ValueError(f"logits must be [B, {VOCAB}]")
    return input_ids.new_empty((input_ids.shape[0],), dtype=torch.int64)
