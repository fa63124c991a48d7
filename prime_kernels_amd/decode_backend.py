"""Serving integration: route pure-decode batches of a Llama-style serving model through the decode step.

Reference: the vLLM backend patch `research/smollm2_360m_decode/experiments/b2-reproducibility-r1/
decode_backend.after.py` (the prime-rl `decode_backend` module).  Same routing rules, function names
and statistics keys, so a caller of the reference's module finds the same surface:

* geometry routing (`_kernel_name_for_config`, :84-107): an exact SmolLM2-135M or -360M geometry
  selects `decode_megakernel` or `decode_megakernel_360m`;
* model eligibility (`_model_kernel_name`, :110-120): bf16 embedding, fused QKV projection, no
  auxiliary hidden-state layers, one tensor- and pipeline-parallel rank;
* metadata eligibility (`_metadata_eligible`, :128-156): FLASH_ATTN metadata of a pure decode
  batch (one query token per request) within the kernel's batch limit, and KV caches in the
  layout the kernel reads;
* the decode call (`_decode_hidden_states`, :182-207) with the model's weights and caches;
* mixed-batch repair (`_repair_mixed_decode`, :210-241): after the stock forward of a batch
  that mixes prefill and decode requests, the decode rows are recomputed by the decode step so
  their arithmetic does not depend on which prefill joined;
* the lossless route (`refresh_lossless_weights`, :244-270, env PRIME_DECODE_MEGAKERNEL_360M_LOSSLESS);
* the patch itself (`monkey_patch_decode_backend`, :273-338).

vLLM is not a dependency: the model and metadata are read by attribute (the vLLM `LlamaModel`
and `FlashAttentionMetadata` field names), the attention metadata dict is passed in or taken
from vLLM's forward context when vLLM is importable, and `monkey_patch_decode_backend` patches
vLLM's `LlamaModel` or any class passed to it.  Differences from the reference: the batch limit
is the kernels' (16 for both geometries; the reference allows 4 and 2) and the block table may
address up to the kernels' 12288 tokens (reference 8192).
"""

from __future__ import annotations

import importlib.util
import logging
import os
from collections import Counter
from copy import copy

import torch

from . import _decode

logger = logging.getLogger("prime_kernels_amd.decode_backend")

REFERENCE_ENV = "PRIME_DECODE_REFERENCE"
ENABLE_360M_ENV = "PRIME_DECODE_MEGAKERNEL_360M"
ENABLE_360M_LOSSLESS_ENV = "PRIME_DECODE_MEGAKERNEL_360M_LOSSLESS"
KERNEL_NAME_135M = "decode_megakernel"
KERNEL_NAME_360M = "decode_megakernel_360m"
KERNEL_NAME = KERNEL_NAME_135M
BLOCK_SIZE = _decode.BLOCK_SIZE
HEAD_DIM = 64
RMS_EPS = 1e-5
MODELS = {KERNEL_NAME_135M: _decode.SMOLLM2_135M, KERNEL_NAME_360M: _decode.SMOLLM2_360M}
MAX_BATCH_BY_KERNEL = {name: m.max_batch for name, m in MODELS.items()}
MAX_BATCH = MAX_BATCH_BY_KERNEL[KERNEL_NAME_135M]
MAX_SEQ_BY_KERNEL = {name: m.max_seq for name, m in MODELS.items()}

stats: Counter = Counter()
_lossless_module = None
_lossless_route_logged = False
_lossless_decode_logged = False


def _load_reference(path: str):
    """A user-supplied `decode_step` implementation (env PRIME_DECODE_REFERENCE), for A/B runs."""
    module_spec = importlib.util.spec_from_file_location("prime_decode_reference", path)
    module = importlib.util.module_from_spec(module_spec)
    module_spec.loader.exec_module(module)
    return module.decode_step


def _resolve_decode_steps() -> dict:
    """Kernel name -> decode_step callable for the kernels enabled and available on this machine
    (decode_backend.after.py:61-81): the 135M step always; the 360M step when
    PRIME_DECODE_MEGAKERNEL_360M=1; only the 360M lossless step when
    PRIME_DECODE_MEGAKERNEL_360M_LOSSLESS=1; a user file's decode_step when PRIME_DECODE_REFERENCE is set."""
    global _lossless_module
    if os.environ.get(REFERENCE_ENV):
        return {KERNEL_NAME_135M: _load_reference(os.environ[REFERENCE_ENV])}
    import prime_kernels_amd as pk

    if os.environ.get(ENABLE_360M_LOSSLESS_ENV) == "1":
        _lossless_module = pk.load("decode_megakernel_360m_lossless")
        return {KERNEL_NAME_360M: _lossless_module.decode_step}
    names = [KERNEL_NAME_135M]
    if os.environ.get(ENABLE_360M_ENV) == "1":
        names.append(KERNEL_NAME_360M)
    return {name: pk.load(name).decode_step for name in names if name in pk.KERNELS and pk.is_available(name)}


def _kernel_name_for_config(config) -> str | None:
    """Exact geometry match of a HF Llama config (decode_backend.after.py:84-107)."""
    head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
    geometry = (config.hidden_size, config.intermediate_size, config.num_hidden_layers,
                config.num_attention_heads, config.num_key_value_heads, head_dim, config.rms_norm_eps)
    for name, m in MODELS.items():
        if geometry == (m.hidden, m.inter, m.layers, m.heads, m.kv_heads, HEAD_DIM, RMS_EPS):
            return name
    return None


def _vllm_types():
    """(LlamaModel, QKVParallelLinear, tp_world_size, pp_world_size) from vLLM, or None without vLLM."""
    try:
        from vllm.distributed import get_pp_group, get_tensor_model_parallel_world_size
        from vllm.model_executor.layers.linear import QKVParallelLinear
        from vllm.model_executor.models.llama import LlamaModel
    except ImportError:
        return None
    return LlamaModel, QKVParallelLinear, get_tensor_model_parallel_world_size(), get_pp_group().world_size


def _model_kernel_name(model) -> str | None:
    """Model-only eligibility, then the exact geometry (decode_backend.after.py:110-120)."""
    if getattr(model, "aux_hidden_state_layers", None):
        return None
    vt = _vllm_types()
    if vt is not None:
        llama_model, qkv_linear, tp, pp = vt
        if type(model) is not llama_model or tp != 1 or pp != 1:
            return None
        if type(model.layers[0].self_attn.qkv_proj) is not qkv_linear:
            return None
    else:
        layers = getattr(model, "layers", None)
        if not layers or getattr(getattr(layers[0], "self_attn", None), "qkv_proj", None) is None:
            return None
        if getattr(model, "tp_size", 1) != 1 or getattr(model, "pp_size", 1) != 1:
            return None
    if model.embed_tokens.weight.dtype != torch.bfloat16:
        return None
    return _kernel_name_for_config(model.config)


def _model_eligible(model) -> bool:
    """Compatibility alias for the original 135M eligibility predicate (:123-125)."""
    return _model_kernel_name(model) == KERNEL_NAME_135M


def _layer_caches(model) -> list:
    return [layer.self_attn.attn.kv_cache for layer in model.layers]


def _metadata_eligible(meta, model, kernel_name: str, batch: int) -> bool:
    """Pure-decode FLASH_ATTN metadata in the kernel's limits (decode_backend.after.py:128-156).
    The cache layout is checked for both geometries (the kernel reads it for both)."""
    if (type(meta).__name__ != "FlashAttentionMetadata" or meta.max_query_len != 1
            or meta.num_actual_tokens != batch or batch > MAX_BATCH_BY_KERNEL[kernel_name]):
        return False
    m = MODELS[kernel_name]
    caches = _layer_caches(model)
    first = caches[0]
    bt = meta.block_table
    if (first.dtype != torch.bfloat16 or first.ndim != 4 or first.shape[1] != m.kv_heads
            or first.shape[2] != BLOCK_SIZE or first.shape[3] != 2 * HEAD_DIM or first.stride(3) != 1
            or bt.dtype != torch.int32 or bt.shape[0] < batch or bt.stride(1) != 1 or bt.shape[1] < 1
            or bt.shape[1] * BLOCK_SIZE > MAX_SEQ_BY_KERNEL[kernel_name]):
        return False
    return all(kv.dtype == first.dtype and kv.shape == first.shape and kv.stride() == first.stride() for kv in caches)


def _select_decode_step(decode_steps: dict, model, kernel_name: str | None, meta, batch: int):
    """The decode step for this batch, or None to fall through (decode_backend.after.py:159-168)."""
    if (kernel_name is None or kernel_name not in decode_steps
            or not 0 < batch <= MAX_BATCH_BY_KERNEL[kernel_name] or meta is None
            or not _metadata_eligible(meta, model, kernel_name, batch)):
        return None
    return decode_steps[kernel_name]


def _attn_metadata(attn_metadata=None):
    """The forward's attention metadata dict: the one passed in, else vLLM's forward context."""
    if attn_metadata is not None:
        return attn_metadata
    try:
        from vllm.forward_context import get_forward_context
    except ImportError:
        return None
    return get_forward_context().attn_metadata


def _decode_metadata(model, attn_metadata=None):
    """FLASH_ATTN metadata when every request contributes one token, else None (:171-179)."""
    metadata = _attn_metadata(attn_metadata)
    if not isinstance(metadata, dict):
        return None
    meta = metadata.get(model.layers[0].self_attn.attn.layer_name)
    if type(meta).__name__ != "FlashAttentionMetadata" or meta.max_query_len != 1:
        return None
    return meta


def _layer_weights(model) -> list:
    return [(layer.input_layernorm.weight, layer.self_attn.qkv_proj.weight, layer.self_attn.o_proj.weight,
             layer.post_attention_layernorm.weight, layer.mlp.gate_up_proj.weight, layer.mlp.down_proj.weight)
            for layer in model.layers]


def _decode_hidden_states(model, decode_step, input_ids, positions, meta):
    """Final hidden states of the batch from one decode-step call (decode_backend.after.py:182-207)."""
    batch = input_ids.shape[0]
    layers = model.layers
    return decode_step(
        input_ids=input_ids, positions=positions, seq_lens=meta.seq_lens[:batch],
        block_table=meta.block_table[:batch], slot_mapping=meta.slot_mapping[:batch],
        embed=model.embed_tokens.weight, layers=_layer_weights(model), final_norm=model.norm.weight,
        kv_caches=_layer_caches(model), cos_sin_cache=layers[0].self_attn.rotary_emb.cos_sin_cache,
        eps=model.norm.variance_epsilon)


def _repair_mixed_decode(model, decode_steps: dict, input_ids, positions, hidden_states, attn_metadata=None):
    """Recompute the decode rows of a mixed prefill/decode batch with the decode step
    (decode_backend.after.py:210-241): rows of requests with one query token are replaced, and
    their current-token KV entries rewritten by the step, so a joining prefill does not change
    their arithmetic.  Skipped under stream capture (the query layout is read on the host)."""
    metadata = _attn_metadata(attn_metadata)
    if not isinstance(metadata, dict):
        return hidden_states
    meta = metadata.get(model.layers[0].self_attn.attn.layer_name)
    if type(meta).__name__ != "FlashAttentionMetadata" or meta.max_query_len <= 1:
        return hidden_states
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        return hidden_states
    starts = meta.query_start_loc.cpu().tolist()
    requests = [i for i, (start, end) in enumerate(zip(starts, starts[1:])) if end - start == 1]
    if not requests:
        return hidden_states
    dev = input_ids.device
    request_rows = torch.tensor(requests, dtype=torch.long, device=dev)
    token_rows = torch.tensor([starts[i] for i in requests], dtype=torch.long, device=dev)
    decode_meta = copy(meta)
    decode_meta.max_query_len = 1
    decode_meta.num_actual_tokens = len(requests)
    decode_meta.seq_lens = meta.seq_lens.index_select(0, request_rows)
    decode_meta.block_table = meta.block_table.index_select(0, request_rows)
    decode_meta.slot_mapping = meta.slot_mapping.index_select(0, token_rows)
    step = _select_decode_step(decode_steps, model, KERNEL_NAME_360M, decode_meta, len(requests))
    if step is None:
        return hidden_states
    decoded = _decode_hidden_states(model, step, input_ids.index_select(0, token_rows),
                                    positions.index_select(0, token_rows), decode_meta)
    result = hidden_states.clone()
    result.index_copy_(0, token_rows, decoded)
    stats["backend_mixed_decode"] += len(requests)
    return result


def refresh_lossless_weights(model) -> None:
    """Re-encode the gate/up weights after a weight reload when the lossless route is on (:244-270)."""
    global _lossless_module
    llama_model = model if hasattr(model, "layers") else getattr(model, "model", None)
    if (os.environ.get(ENABLE_360M_LOSSLESS_ENV) == "1" and llama_model is not None
            and _kernel_name_for_config(llama_model.config) == KERNEL_NAME_360M):
        if _lossless_module is None:
            import prime_kernels_amd as pk

            _lossless_module = pk.load("decode_megakernel_360m_lossless")
        _lossless_module.refresh_weights(_layer_weights(llama_model))
        cache_stats = _lossless_module.cache_statistics(llama_model.layers[0].mlp.gate_up_proj.weight.device)
        if cache_stats is not None:
            logger.info("Lossless 360M GU cache refreshed: %s", cache_stats)


def make_forward(original_forward, decode_steps: dict, attn_metadata_fn=None):
    """The patched `forward(self, input_ids, positions, intermediate_tensors, inputs_embeds=None,
    **kwargs)` (decode_backend.after.py:285-334).  `attn_metadata_fn(self)` supplies the attention
    metadata dict (default: vLLM's forward context)."""

    def metadata_of(model):
        return attn_metadata_fn(model) if attn_metadata_fn is not None else None

    def forward(self, input_ids, positions, intermediate_tensors=None, inputs_embeds=None, **kwargs):
        global _lossless_decode_logged, _lossless_route_logged
        lossless = os.environ.get(ENABLE_360M_LOSSLESS_ENV) == "1"
        kernel_name = _model_kernel_name(self) if inputs_embeds is None else None
        if kernel_name is not None and kernel_name in decode_steps:
            if kernel_name == KERNEL_NAME_360M and lossless and _lossless_module is not None:
                cache = _lossless_module.prepare_weights(_layer_weights(self))
                if not _lossless_route_logged:
                    logger.info("Lossless 360M decode route prepared: %s", cache.statistics())
                    _lossless_route_logged = True
            meta = _decode_metadata(self, metadata_of(self))
            batch = input_ids.shape[0]
            if meta is None:
                stats["stock_not_pure_decode"] += 1
            elif batch > MAX_BATCH_BY_KERNEL[kernel_name] or meta.num_actual_tokens != batch:
                stats["stock_decode_over_max_batch"] += 1
            else:
                decode_step = _select_decode_step(decode_steps, self, kernel_name, meta, batch)
                if decode_step is None:
                    stats["stock_unsupported_metadata"] += 1
                else:
                    stats["backend_decode"] += 1
                    if kernel_name == KERNEL_NAME_360M and lossless and not _lossless_decode_logged:
                        logger.info("Lossless 360M decode route active: batch=%d", batch)
                        _lossless_decode_logged = True
                    return _decode_hidden_states(self, decode_step, input_ids, positions, meta)
        elif kernel_name is None or inputs_embeds is not None:
            stats["stock_ineligible"] += 1
        else:
            stats["stock_kernel_unavailable"] += 1
        hidden_states = original_forward(self, input_ids, positions, intermediate_tensors, inputs_embeds, **kwargs)
        if kernel_name == KERNEL_NAME_360M and lossless and os.environ.get("VLLM_BATCH_INVARIANT") == "1":
            hidden_states = _repair_mixed_decode(self, decode_steps, input_ids, positions, hidden_states,
                                                 metadata_of(self))
        return hidden_states

    forward._prime_rl_decode_backend = True
    return forward


def monkey_patch_decode_backend(model_cls=None, attn_metadata_fn=None) -> bool:
    """Route pure decode batches through the decode step by patching `model_cls.forward` (vLLM's
    LlamaModel by default; decode_backend.after.py:273-338).  Returns False when no decode step
    is available; installing twice is a no-op.  Graph replays do not re-enter Python, so the path a
    captured graph takes is fixed at capture time."""
    if model_cls is None:
        vt = _vllm_types()
        if vt is None:
            raise ImportError("monkey_patch_decode_backend needs vLLM's LlamaModel (or pass model_cls)")
        model_cls = vt[0]
    if getattr(model_cls.forward, "_prime_rl_decode_backend", False):
        return True
    decode_steps = _resolve_decode_steps()
    if not decode_steps:
        return False
    model_cls.forward = make_forward(model_cls.forward, decode_steps, attn_metadata_fn)
    logger.info("Decode backend installed for supported SmolLM2 geometries: %s", sorted(decode_steps))
    return True
