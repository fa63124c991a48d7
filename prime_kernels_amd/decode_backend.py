"""Serving integration: send the pure-decode batches of a Llama-style serving model to the decode step.

Interface of the reference's vLLM backend module (research/smollm2_360m_decode/experiments/
b2-reproducibility-r1/decode_backend.after.py): `monkey_patch_decode_backend()`,
`refresh_lossless_weights(model)`, the `stats` counter and its keys, the environment switches
PRIME_DECODE_MEGAKERNEL_360M, PRIME_DECODE_MEGAKERNEL_360M_LOSSLESS and PRIME_DECODE_REFERENCE,
and the `_prime_rl_decode_backend` marker on the patched forward.

Design.  A forward call is routed in three steps:

1. the model's kernel (`kernel_for_model`): a SmolLM2-135M or -360M geometry (`_Geometry`, compared
   with the HF config, vocabulary size included) with a bf16 embedding, a fused QKV projection, no
   auxiliary hidden-state layers and a single tensor/pipeline rank;
2. the batch (`route`): FLASH_ATTN metadata of a pure decode batch (one query token per request)
   within the kernel's batch and context limits, over KV caches in the layout the kernel reads
   (`metadata_fits`).  Every decision, taken or not, is counted in `stats`;
3. the call (`_ModelTensors.run`): the decode step with the model's weights and caches.

After a stock forward of a batch that mixes prefill and decode requests, `repair_mixed_batch`
recomputes the decode rows with the 360M step (lossless route, VLLM_BATCH_INVARIANT=1), so that a
joining prefill does not change their arithmetic.

vLLM is optional: models and metadata are read by attribute (vLLM's `LlamaModel` and
`FlashAttentionMetadata` field names), and the attention metadata comes from an `attn_metadata_fn`
or vLLM's forward context.  Limits are the kernels' (batch 16 and 12288 tokens for both geometries;
the reference's are 4 / 2 and 8192).
"""

from __future__ import annotations

import importlib.util
import logging
import os
from collections import Counter
from copy import copy
from dataclasses import dataclass

import torch

from . import _decode

logger = logging.getLogger("prime_kernels_amd.decode_backend")

REFERENCE_ENV = "PRIME_DECODE_REFERENCE"
ENABLE_360M_ENV = "PRIME_DECODE_MEGAKERNEL_360M"
ENABLE_360M_LOSSLESS_ENV = "PRIME_DECODE_MEGAKERNEL_360M_LOSSLESS"
BATCH_INVARIANT_ENV = "VLLM_BATCH_INVARIANT"
KERNEL_NAME_135M = "decode_megakernel"
KERNEL_NAME_360M = "decode_megakernel_360m"
MODELS = {KERNEL_NAME_135M: _decode.SMOLLM2_135M, KERNEL_NAME_360M: _decode.SMOLLM2_360M}
MARKER = "_prime_rl_decode_backend"

stats: Counter = Counter()


@dataclass(frozen=True)
class _Geometry:
    hidden: int
    inter: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    eps: float
    vocab: int

    @classmethod
    def of_config(cls, c) -> "_Geometry":
        head_dim = getattr(c, "head_dim", None) or c.hidden_size // c.num_attention_heads
        return cls(c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.num_attention_heads,
                   c.num_key_value_heads, head_dim, c.rms_norm_eps, c.vocab_size)

    @classmethod
    def of_kernel(cls, m) -> "_Geometry":
        return cls(m.hidden, m.inter, m.layers, m.heads, m.kv_heads, m.head_dim, _decode.EPS, _decode.VOCAB)


_KERNEL_OF_GEOMETRY = {_Geometry.of_kernel(m): name for name, m in MODELS.items()}


def kernel_for_config(config) -> str | None:
    """The kernel whose geometry the HF config has exactly, or None."""
    return _KERNEL_OF_GEOMETRY.get(_Geometry.of_config(config))


def _vllm_types():
    """(LlamaModel, QKVParallelLinear, tensor-parallel size, pipeline-parallel size), or None without vLLM."""
    try:
        from vllm.distributed import get_pp_group, get_tensor_model_parallel_world_size
        from vllm.model_executor.layers.linear import QKVParallelLinear
        from vllm.model_executor.models.llama import LlamaModel
    except ImportError:
        return None
    return LlamaModel, QKVParallelLinear, get_tensor_model_parallel_world_size(), get_pp_group().world_size


def kernel_for_model(model) -> str | None:
    """The kernel for this model object, or None when the model is not one the kernels serve."""
    if getattr(model, "aux_hidden_state_layers", None):
        return None
    vllm = _vllm_types()
    layers = getattr(model, "layers", None)
    if not layers:
        return None
    qkv = getattr(getattr(layers[0], "self_attn", None), "qkv_proj", None)
    if vllm is not None:
        llama_cls, qkv_cls, tp, pp = vllm
        if type(model) is not llama_cls or type(qkv) is not qkv_cls or (tp, pp) != (1, 1):
            return None
    elif qkv is None or (getattr(model, "tp_size", 1), getattr(model, "pp_size", 1)) != (1, 1):
        return None
    if model.embed_tokens.weight.dtype != torch.bfloat16:
        return None
    return kernel_for_config(model.config)


def _kv_caches(model) -> list:
    return [layer.self_attn.attn.kv_cache for layer in model.layers]


def metadata_fits(meta, model, kernel: str, batch: int) -> bool:
    """Whether `meta` describes a pure decode batch of `batch` requests the kernel can take: one query
    token each, within its batch limit, a contiguous-row int32 block table within its context limit,
    and KV caches of one shape and layout [blocks, kv_heads, 16, 128] bf16."""
    m = MODELS[kernel]
    if type(meta).__name__ != "FlashAttentionMetadata" or meta.max_query_len != 1:
        return False
    if meta.num_actual_tokens != batch or not 0 < batch <= m.max_batch:
        return False
    bt = meta.block_table
    if bt.dtype != torch.int32 or bt.stride(1) != 1 or bt.shape[0] < batch:
        return False
    if not 1 <= bt.shape[1] * _decode.BLOCK_SIZE <= m.max_seq:
        return False
    caches = _kv_caches(model)
    c0 = caches[0]
    want = (m.kv_heads, _decode.BLOCK_SIZE, 2 * m.head_dim)
    if c0.dtype != torch.bfloat16 or c0.ndim != 4 or tuple(c0.shape[1:]) != want or c0.stride(3) != 1:
        return False
    return all(c.dtype == c0.dtype and c.shape == c0.shape and c.stride() == c0.stride() for c in caches[1:])


@dataclass
class _ModelTensors:
    """What the decode step reads from a vLLM Llama model."""

    embed: torch.Tensor
    layers: list
    final_norm: torch.Tensor
    kv_caches: list
    cos_sin: torch.Tensor
    eps: float

    @classmethod
    def of(cls, model) -> "_ModelTensors":
        layers = [(l.input_layernorm.weight, l.self_attn.qkv_proj.weight, l.self_attn.o_proj.weight,
                   l.post_attention_layernorm.weight, l.mlp.gate_up_proj.weight, l.mlp.down_proj.weight)
                  for l in model.layers]
        return cls(model.embed_tokens.weight, layers, model.norm.weight, _kv_caches(model),
                   model.layers[0].self_attn.rotary_emb.cos_sin_cache, model.norm.variance_epsilon)

    def run(self, step, input_ids, positions, meta):
        b = input_ids.shape[0]
        return step(input_ids=input_ids, positions=positions, seq_lens=meta.seq_lens[:b],
                    block_table=meta.block_table[:b], slot_mapping=meta.slot_mapping[:b], embed=self.embed,
                    layers=self.layers, final_norm=self.final_norm, kv_caches=self.kv_caches,
                    cos_sin_cache=self.cos_sin, eps=self.eps)


def _layer_metadata(model, attn_metadata):
    """This model's per-layer attention metadata from the forward's metadata dict (vLLM's forward
    context when none is given), or None."""
    if attn_metadata is None:
        try:
            from vllm.forward_context import get_forward_context
        except ImportError:
            return None
        attn_metadata = get_forward_context().attn_metadata
    if not isinstance(attn_metadata, dict):
        return None
    return attn_metadata.get(model.layers[0].self_attn.attn.layer_name)


def route(steps: dict, model, kernel: str | None, meta, batch: int):
    """(decode step, None) when the batch goes to the kernel, else (None, the stats key saying why)."""
    if kernel is None:
        return None, "stock_ineligible"
    if kernel not in steps:
        return None, "stock_kernel_unavailable"
    if type(meta).__name__ != "FlashAttentionMetadata" or meta.max_query_len != 1:
        return None, "stock_not_pure_decode"
    if meta.num_actual_tokens != batch or batch > MODELS[kernel].max_batch:
        return None, "stock_decode_over_max_batch"
    if not metadata_fits(meta, model, kernel, batch):
        return None, "stock_unsupported_metadata"
    return steps[kernel], None


def repair_mixed_batch(model, steps: dict, input_ids, positions, hidden, attn_metadata=None):
    """`hidden` with the rows of the single-token (decode) requests of a mixed prefill/decode batch
    replaced by the 360M decode step's, which also rewrites their current-token KV entries.  Batches
    that are pure decode or pure prefill, and calls under stream capture (the query layout is read
    on the host), return `hidden` itself."""
    meta = _layer_metadata(model, attn_metadata)
    if type(meta).__name__ != "FlashAttentionMetadata" or meta.max_query_len <= 1:
        return hidden
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        return hidden
    starts = meta.query_start_loc.tolist()
    decoding = [(r, s) for r, (s, e) in enumerate(zip(starts, starts[1:])) if e - s == 1]
    if not decoding:
        return hidden
    dev = input_ids.device
    req = torch.tensor([r for r, _ in decoding], dtype=torch.long, device=dev)
    tok = torch.tensor([s for _, s in decoding], dtype=torch.long, device=dev)
    sub = copy(meta)
    sub.max_query_len, sub.num_actual_tokens = 1, len(decoding)
    sub.seq_lens = meta.seq_lens.index_select(0, req)
    sub.block_table = meta.block_table.index_select(0, req)
    sub.slot_mapping = meta.slot_mapping.index_select(0, tok)
    step, _ = route(steps, model, KERNEL_NAME_360M, sub, len(decoding))
    if step is None:
        return hidden
    rows = _ModelTensors.of(model).run(step, input_ids.index_select(0, tok), positions.index_select(0, tok), sub)
    out = hidden.clone()
    out.index_copy_(0, tok, rows)
    stats["backend_mixed_decode"] += len(decoding)
    return out


class _Lossless:
    """The opt-in lossless 360M route (PRIME_DECODE_MEGAKERNEL_360M_LOSSLESS=1): its module, and
    whether its first preparation and first routed step were logged."""

    module = None
    prepared_logged = False
    routed_logged = False

    @classmethod
    def on(cls) -> bool:
        return os.environ.get(ENABLE_360M_LOSSLESS_ENV) == "1"

    @classmethod
    def load(cls):
        if cls.module is None:
            import prime_kernels_amd as pk

            cls.module = pk.load("decode_megakernel_360m_lossless")
        return cls.module


def _user_step(path: str):
    """decode_step of a user's Python file (PRIME_DECODE_REFERENCE), for A/B comparisons."""
    spec = importlib.util.spec_from_file_location("prime_decode_user_step", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.decode_step


def enabled_steps() -> dict:
    """Kernel name -> decode step for the routes the environment enables on this machine: a user's
    step for 135M (PRIME_DECODE_REFERENCE), or the 360M lossless step alone, or the 135M step plus
    the 360M step when PRIME_DECODE_MEGAKERNEL_360M=1."""
    user = os.environ.get(REFERENCE_ENV)
    if user:
        return {KERNEL_NAME_135M: _user_step(user)}
    if _Lossless.on():
        return {KERNEL_NAME_360M: _Lossless.load().decode_step}
    import prime_kernels_amd as pk

    wanted = [KERNEL_NAME_135M] + ([KERNEL_NAME_360M] if os.environ.get(ENABLE_360M_ENV) == "1" else [])
    return {n: pk.load(n).decode_step for n in wanted if n in pk.KERNELS and pk.is_available(n)}


def refresh_lossless_weights(model) -> None:
    """Re-encode the lossless gate/up cache after a weight reload, when that route is on and the
    model (or its `.model`) is SmolLM2-360M."""
    llama = model if hasattr(model, "layers") else getattr(model, "model", None)
    if not _Lossless.on() or llama is None or kernel_for_config(llama.config) != KERNEL_NAME_360M:
        return
    module = _Lossless.load()
    module.refresh_weights(_ModelTensors.of(llama).layers)
    info = module.cache_statistics(llama.layers[0].mlp.gate_up_proj.weight.device)
    if info is not None:
        logger.info("lossless 360M gate/up cache re-encoded: %s", info)


def patched_forward(stock_forward, steps: dict, attn_metadata_fn=None):
    """A `forward(self, input_ids, positions, intermediate_tensors=None, inputs_embeds=None, **kw)`
    that sends routable batches to the decode step and all others to `stock_forward`.
    `attn_metadata_fn(model)` supplies the attention metadata dict (default: vLLM's forward context)."""

    def forward(self, input_ids, positions, intermediate_tensors=None, inputs_embeds=None, **kwargs):
        attn_metadata = attn_metadata_fn(self) if attn_metadata_fn is not None else None
        kernel = kernel_for_model(self) if inputs_embeds is None else None
        lossless = kernel == KERNEL_NAME_360M and _Lossless.on()
        if lossless and kernel in steps and _Lossless.module is not None:
            cache = _Lossless.module.prepare_weights(_ModelTensors.of(self).layers)
            if not _Lossless.prepared_logged:
                logger.info("lossless 360M gate/up cache prepared: %s", cache.statistics())
                _Lossless.prepared_logged = True
        meta = _layer_metadata(self, attn_metadata) if kernel in steps else None
        step, why = route(steps, self, kernel, meta, input_ids.shape[0])
        if step is not None:
            stats["backend_decode"] += 1
            if lossless and not _Lossless.routed_logged:
                logger.info("lossless 360M decode route taken at batch %d", input_ids.shape[0])
                _Lossless.routed_logged = True
            return _ModelTensors.of(self).run(step, input_ids, positions, meta)
        stats[why] += 1
        hidden = stock_forward(self, input_ids, positions, intermediate_tensors, inputs_embeds, **kwargs)
        if lossless and os.environ.get(BATCH_INVARIANT_ENV) == "1":
            hidden = repair_mixed_batch(self, steps, input_ids, positions, hidden, attn_metadata)
        return hidden

    setattr(forward, MARKER, True)
    return forward


def monkey_patch_decode_backend(model_cls=None, attn_metadata_fn=None) -> bool:
    """Patch `model_cls.forward` (vLLM's LlamaModel by default) to route pure decode batches to the
    decode step.  Returns False, patching nothing, when no decode step is available; patching an
    already patched class is a no-op.  A captured graph replays the path taken at capture time."""
    if model_cls is None:
        vllm = _vllm_types()
        if vllm is None:
            raise ImportError("vLLM is not installed: pass the model class to patch as model_cls")
        model_cls = vllm[0]
    if getattr(model_cls.forward, MARKER, False):
        return True
    steps = enabled_steps()
    if not steps:
        return False
    model_cls.forward = patched_forward(model_cls.forward, steps, attn_metadata_fn)
    logger.info("decode backend installed for %s", ", ".join(sorted(steps)))
    return True
