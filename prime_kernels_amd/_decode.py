"""Host wrapper shared by the 360M and 135M decode kernels.

Mirrors the reference wrapper prime_kernels/decode_megakernel_360m/__init__.py:60-234 (contract
checks with the same ValueError messages, per-device runtime with module-owned workspace and
output buffer, device pointer tables rebuilt only when a data_ptr changes and then updated in
place) and calls the C ABI `pk_decode` (include/prime_decode.h) on the current HIP stream.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

from prime_kernels_amd import _native

BLOCK_SIZE = 16
EPS = 1e-5
VOCAB = 49152


@dataclass(frozen=True)
class Model:
    name: str
    model_id: int
    hidden: int
    inter: int
    heads: int
    kv_heads: int
    layers: int
    head_dim: int = 64
    max_batch: int = 16
    max_seq: int = 12288
    weight_format: str = "bf16"   # "bf16", or "mxfp8" (e4m3 projections + e8m0 scale per 32)

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def shapes(self):
        h, i = self.hidden, self.inter
        return ((h,), (self.qkv_rows, h), (h, h), (h,), (2 * i, h), (h, i))

    def layer_spec(self):
        """(name, dtype, shape) of each tensor of one layer tuple, in order."""
        names = ("norm1", "qkv", "o", "norm2", "gate_up", "down")
        if self.weight_format == "bf16":
            return [(n, torch.bfloat16, sh) for n, sh in zip(names, self.shapes())]
        spec = []
        for n, sh in zip(names, self.shapes()):
            if len(sh) == 1:
                spec.append((n, torch.bfloat16, sh))
            else:
                spec.append((n, torch.uint8, sh))
                spec.append((n + "_scales", torch.uint8, (sh[0], mxfp8_scale_stride(sh[1]))))
        return spec


def mxfp8_scale_stride(cols: int) -> int:
    """Bytes per row of an MXFP8 scale array: one e8m0 code per 32 weights, padded to 16 bytes."""
    return ((cols // 32 + 15) // 16) * 16


SMOLLM2_360M = Model("decode_megakernel_360m", 360, hidden=960, inter=2560, heads=15, kv_heads=5, layers=32)
SMOLLM2_135M = Model("decode_megakernel", 135, hidden=576, inter=1536, heads=9, kv_heads=3, layers=30)
SMOLLM2_360M_MXFP8 = Model("decode_megakernel_360m_mxfp8", 360, hidden=960, inter=2560, heads=15, kv_heads=5,
                           layers=32, max_batch=1, weight_format="mxfp8")
MODELS = {m.model_id: m for m in (SMOLLM2_360M, SMOLLM2_135M)}


class _Runtime:
    """Per-device state (reference: decode_megakernel_360m/__init__.py:60-70): the scratch the C ABI
    requires, the output and greedy-id buffers and the pointer tables.  The scratch carries nothing
    between calls -- the library keeps every exchanged word in state of its own per device
    (include/prime_decode.h, pk_workspace_bytes), created here, before any graph capture -- so it is
    plain torch memory, as in the reference."""

    def __init__(self, model: Model, device: torch.device):
        lib = _native.library()
        self.lib = lib
        self.device = device
        with torch.cuda.device(device):
            rc = lib.pk_init()
        if rc != 0:
            raise RuntimeError(f"{model.name}: library state for {device}: {_native.status_string(rc)}")
        nbytes = lib.pk_workspace_bytes(model.model_id)
        self.scratch = torch.empty((nbytes,), dtype=torch.uint8, device=device)
        self.scratch_ptr = self.scratch.data_ptr()
        self.scratch_bytes = nbytes
        self.out = torch.empty((model.max_batch, model.hidden), dtype=torch.bfloat16, device=device)
        self.ids = torch.empty((model.max_batch,), dtype=torch.int64, device=device)
        self.layers_t = None
        self.kv_t = None
        self.table_key = None

    def _stream(self, stream):
        return torch.cuda.current_stream(self.device).cuda_stream if stream is None else stream

    def header(self, n: int = 3, stream=None) -> list:
        """Header words of the device's library state: step epoch, the epoch of the last step that
        gave up a bounded wait, its wait site.  Synchronises `stream` (default: the current one)."""
        buf = (ctypes.c_uint * n)()
        with torch.cuda.device(self.device):
            rc = self.lib.pk_state_read(self._stream(stream), 0, buf, n)
        if rc != 0:
            raise RuntimeError(f"state read failed: {_native.status_string(rc)}")
        return list(buf)

    def take_failure(self, stream=None) -> tuple:
        """pending_failure, clearing the report: the next decode call on the device then does not
        report that step again.  Does not synchronise."""
        buf = (ctypes.c_uint * 2)()
        with torch.cuda.device(self.device):
            rc = self.lib.pk_state_take(self._stream(stream), buf)
        if rc != 0:
            raise RuntimeError(f"state read failed: {_native.status_string(rc)}")
        return buf[0], buf[1]

    def pending_failure(self, stream=None) -> tuple:
        """(epoch, wait site) of a step on the device that gave up a bounded wait and has not been
        reported by a decode call yet; (0, 0) when there is none.  Does not synchronise."""
        buf = (ctypes.c_uint * 2)()
        with torch.cuda.device(self.device):
            rc = self.lib.pk_state_status(self._stream(stream), buf)
        if rc != 0:
            raise RuntimeError(f"state read failed: {_native.status_string(rc)}")
        return buf[0], buf[1]


_runtimes: dict = {}


def runtime(model: Model, device: torch.device) -> _Runtime:
    key = (model.name, device)
    if key not in _runtimes:
        _runtimes[key] = _Runtime(model, device)
    return _runtimes[key]


def check_embed_shape(embed, model: Model) -> None:
    """The embedding table must be [VOCAB, hidden] and contiguous.  The kernels read row `id` of it
    for each input id with the id clamped to 0..VOCAB-1 on the device, and the tied LM head reads every
    row, so a table of another row count would be read past its end or have rows that no id reaches.
    (The reference checks the hidden width only, decode_megakernel_360m/__init__.py:151-152, and its
    kernel indexes the table unchecked.)"""
    if embed.ndim != 2 or tuple(embed.shape) != (VOCAB, model.hidden) or not embed.is_contiguous():
        raise ValueError(f"embed must be contiguous BF16 [{VOCAB}, {model.hidden}], got {tuple(embed.shape)}")


def _check_tensor(tensor, name, *, dtype=None, device=None, shape=None):
    if not isinstance(tensor, torch.Tensor) or not tensor.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor")
    if dtype is not None and tensor.dtype != dtype:
        raise ValueError(f"{name} must have dtype {dtype}")
    if device is not None and tensor.device != device:
        raise ValueError(f"{name} must be on {device}")
    if shape is not None and tuple(tensor.shape) != shape:
        raise ValueError(f"{name} must have shape {shape}")


def _tables(rt: _Runtime, layers, kv_caches):
    """Device pointer tables (reference: decode_megakernel_360m/__init__.py:126-139)."""
    key = (tuple(t.data_ptr() for layer in layers for t in layer), tuple(t.data_ptr() for t in kv_caches))
    if key != rt.table_key:
        layer_table = torch.tensor([[t.data_ptr() for t in layer] for layer in layers], dtype=torch.int64)
        kv_table = torch.tensor([t.data_ptr() for t in kv_caches], dtype=torch.int64)
        if rt.layers_t is None or rt.layers_t.shape != layer_table.shape:
            rt.layers_t = layer_table.to(rt.device)
            rt.kv_t = kv_table.to(rt.device)
        else:
            # in place, so graphs captured with these tables see the new pointers
            rt.layers_t.copy_(layer_table)
            rt.kv_t.copy_(kv_table)
        rt.table_key = key
    return rt.layers_t, rt.kv_t


def _failure_message(model: Model, rc: int) -> str:
    if rc == _native.PK_ERR_ABORTED:
        return (f"{model.name} failed: {_native.status_string(rc)} (an earlier step on this device could not "
                f"complete; its hidden state and logits were set to NaN and its token ids to -1)")
    return f"{model.name} failed: {_native.status_string(rc)}"


def check_failures(model: Model, device: torch.device, stream=None) -> None:
    """Synchronise `device` and raise RuntimeError if a decode step on it gave up a bounded wait
    since the last report (decode calls report such a step at the next call; this reports it now,
    and clears the report, so the next call does not raise for the same step)."""
    rt = runtime(model, device)
    s = rt._stream(stream)
    torch.cuda.synchronize(device)
    epoch, site = rt.take_failure(s)
    if epoch:
        raise RuntimeError(f"{model.name}: the step with epoch {epoch} gave up a bounded wait (site {site}); "
                           f"its outputs were poisoned")


def decode_step(model: Model, *, input_ids, positions, seq_lens, block_table, slot_mapping, embed, layers,
                final_norm, kv_caches, cos_sin_cache, eps, layer_outputs=None, debug=None,
                debug_layer_index=-1, return_token_ids=False, logits_out=None, num_layers=None, encoded_gu=None):
    """One decode step; inputs follow vLLM FLASH_ATTN metadata (reference signature
    decode_megakernel_360m/__init__.py:142-144).

    Returns the final-normed hidden state [B, H] bf16 -- a view of a per-device buffer that the
    next call overwrites.  With `return_token_ids=True` returns (hidden, ids[B] int64) where ids
    are the greedy tokens of the tied LM head (also a reused buffer).  `logits_out` ([B, 49152]
    bf16, caller-owned) receives the LM-head logits.  `num_layers` runs only the first N layers
    (default: all), for tests on truncated models.  `encoded_gu` (a lossless_bf16.EncodedGUCache of
    the same gate_up matrices, SmolLM2-360M only) makes the batch-1 step stream the encoded gate/up
    weights of every enabled layer."""
    nl = model.layers if num_layers is None else int(num_layers)
    batch = input_ids.shape[0]
    if not 1 <= batch <= model.max_batch:
        raise ValueError(f"batch must be 1..{model.max_batch}, got {batch}")
    if eps != EPS:
        raise ValueError(f"the kernel is built for rms eps {EPS}, got {eps}")
    if not 1 <= nl <= model.layers:
        raise ValueError(f"num_layers must be 1..{model.layers}")
    if len(layers) != nl or len(kv_caches) != nl:
        raise ValueError(f"expected {nl} layers and KV caches")
    if debug_layer_index < -1 or debug_layer_index >= model.layers:
        raise ValueError(f"debug_layer_index must be -1 or a layer index 0..{model.layers - 1}")
    if debug is not None:
        if model.model_id != 360 or model.weight_format != "bf16":
            raise ValueError("per-stage debug capture is available for SmolLM2-360M bf16 weights")
        if batch > 2:
            raise ValueError("per-stage debug capture holds at most 2 sequences")

    device = input_ids.device
    _check_tensor(input_ids, "input_ids", device=device)
    if input_ids.dtype not in (torch.int32, torch.int64) or input_ids.ndim != 1:
        raise ValueError("input_ids must be a 1-D int32 or int64 tensor")
    _check_tensor(positions, "positions", dtype=torch.int64, device=device, shape=(batch,))
    _check_tensor(seq_lens, "seq_lens", dtype=torch.int32, device=device, shape=(batch,))
    _check_tensor(slot_mapping, "slot_mapping", dtype=torch.int64, device=device, shape=(batch,))
    if block_table.dtype != torch.int32 or block_table.device != device or block_table.ndim != 2 \
            or block_table.shape[0] < batch:
        raise ValueError("block_table must be int32 [B, width] on the input device")
    if block_table.stride(1) != 1:
        raise ValueError("block_table must have contiguous rows")
    if not 1 <= block_table.shape[1] * BLOCK_SIZE <= model.max_seq:
        raise ValueError(f"block_table context capacity must be 1..{model.max_seq}")
    _check_tensor(embed, "embed", dtype=torch.bfloat16, device=device)
    _check_tensor(final_norm, "final_norm", dtype=torch.bfloat16, device=device, shape=(model.hidden,))
    check_embed_shape(embed, model)
    lm_head = return_token_ids or logits_out is not None
    spec = model.layer_spec()
    for i, layer in enumerate(layers):
        if len(layer) != len(spec):
            raise ValueError(f"layer {i} must contain {'six' if len(spec) == 6 else len(spec)} weight tensors")
        for (name, dtype, shape), tensor in zip(spec, layer):
            _check_tensor(tensor, f"layer {i} {name}", dtype=dtype, device=device, shape=shape)
            if not tensor.is_contiguous():
                raise ValueError(f"layer {i} {name} must be contiguous")
            if tensor.data_ptr() % 16:
                raise ValueError(f"layer {i} {name} must be 16-byte aligned")
    kv0 = kv_caches[0]
    _check_tensor(kv0, "kv_caches[0]", dtype=torch.bfloat16, device=device)
    if kv0.ndim != 4 or kv0.shape[1] != model.kv_heads or kv0.shape[3] != 2 * model.head_dim or kv0.stride(3) != 1:
        raise ValueError(f"KV caches must use vLLM FLASH_ATTN [blocks, {model.kv_heads}, 16, "
                         f"{2 * model.head_dim}] K/V-packed layout")
    if kv0.shape[2] != BLOCK_SIZE:
        raise ValueError("the kernel requires KV block_size=16")
    for i, kv in enumerate(kv_caches):
        _check_tensor(kv, f"kv_caches[{i}]", dtype=torch.bfloat16, device=device, shape=tuple(kv0.shape))
        if kv.stride() != kv0.stride():
            raise ValueError("all KV caches must share strides")
    _check_tensor(cos_sin_cache, "cos_sin_cache", device=device)
    if cos_sin_cache.dtype not in (torch.bfloat16, torch.float32) or cos_sin_cache.ndim != 2 \
            or cos_sin_cache.shape[1] != model.head_dim or not cos_sin_cache.is_contiguous():
        raise ValueError(f"cos_sin_cache must be contiguous BF16 or FP32 [max_position, {model.head_dim}]")
    if layer_outputs is not None:
        _check_tensor(layer_outputs, "layer_outputs", dtype=torch.bfloat16, device=device,
                      shape=(nl, batch, model.hidden))
        if not layer_outputs.is_contiguous():
            raise ValueError("layer_outputs must be contiguous")
    if logits_out is not None:
        _check_tensor(logits_out, "logits_out", dtype=torch.bfloat16, device=device, shape=(batch, VOCAB))
        if not logits_out.is_contiguous():
            raise ValueError("logits_out must be contiguous")
    if debug is not None:  # decode_megakernel_360m/__init__.py:198-213
        _check_tensor(debug, "debug", dtype=torch.uint8, device=device)
        if not debug.is_contiguous():
            raise ValueError("debug must be contiguous raw byte storage")
        if debug.numel() < _native.library().decode360_debug_bytes():
            raise ValueError("debug buffer is too small")
        if debug.data_ptr() % 16:
            raise ValueError("debug buffer must be 16-byte aligned")

    extra = ()
    if encoded_gu is not None:
        if model.model_id != 360 or model.weight_format != "bf16":
            raise ValueError("the lossless gate/up cache is for SmolLM2-360M bf16 weights")
        if encoded_gu.device != device:
            raise ValueError(f"encoded_gu must be on {device}")
        if tuple(t.data_ptr() for t in encoded_gu.weights[:nl]) != tuple(layer[4].data_ptr() for layer in layers):
            raise ValueError("encoded_gu was prepared for other gate_up tensors")

    rt = runtime(model, device)
    layers_t, kv_t = _tables(rt, layers, kv_caches)
    stream = torch.cuda.current_stream(device).cuda_stream
    want_ids = return_token_ids or logits_out is not None
    if debug is not None:
        launch = rt.lib.pk_decode_debug
        extra = (encoded_gu.table.data_ptr() if encoded_gu is not None else None, debug.data_ptr(),
                 debug.numel(), debug_layer_index)
    elif encoded_gu is not None:
        launch = rt.lib.pk_decode_lossless
        extra = (encoded_gu.table.data_ptr(),)
    else:
        launch = rt.lib.pk_decode_mxfp8 if model.weight_format == "mxfp8" else rt.lib.pk_decode
    rc = launch(
        stream, model.model_id, batch, nl, input_ids.data_ptr(), int(input_ids.dtype == torch.int64),
        embed.data_ptr(), final_norm.data_ptr(), positions.data_ptr(), seq_lens.data_ptr(),
        block_table.data_ptr(), block_table.stride(0), slot_mapping.data_ptr(), layers_t.data_ptr(),
        kv_t.data_ptr(), 0, model.head_dim, kv0.stride(0), kv0.stride(2), kv0.stride(1), BLOCK_SIZE,
        cos_sin_cache.data_ptr(), int(cos_sin_cache.dtype == torch.float32), rt.out.data_ptr(),
        layer_outputs.data_ptr() if layer_outputs is not None else None,
        rt.ids.data_ptr() if want_ids else None,
        logits_out.data_ptr() if logits_out is not None else None,
        rt.scratch_ptr, rt.scratch_bytes, block_table.shape[1] * BLOCK_SIZE, *extra)
    if rc != 0:
        raise RuntimeError(_failure_message(model, rc))
    if return_token_ids:
        return rt.out[:batch], rt.ids[:batch]
    return rt.out[:batch]


class StepLauncher:
    """Pre-validated, allocation-free launcher for a run of greedy decode steps of B sequences.

    All per-step metadata lives in device arrays prepared once: step k reads its input ids from
    ids[k] and writes the greedy ids to ids[k+1], so consecutive steps chain on the device with no
    host synchronisation (the way graph-replayed serving steps run, decode_backend.after.py:276-277).
    `first_id` and `start_pos` are one value for every sequence or one per sequence (ragged
    contexts: sequence b decodes positions start_pos[b] .. start_pos[b] + steps - 1).
    """

    def __init__(self, model: Model, *, embed, layers, final_norm, kv_caches, block_table, cos_sin_cache,
                 first_id, start_pos, steps: int, logits: bool = False, batch: int = 1, encoded_gu=None):
        dev = embed.device
        B = batch
        if not 1 <= B <= model.max_batch:
            raise ValueError(f"{model.name}: batch must be 1..{model.max_batch}, got {B}")
        if block_table.shape[0] < B:
            raise ValueError("block table has fewer rows than the batch")
        self.model = model
        self.batch = B
        self.rt = runtime(model, dev)
        self.lib = self.rt.lib
        self.layers_t, self.kv_t = _tables(self.rt, layers, kv_caches)
        self.keep = (embed, layers, final_norm, kv_caches, block_table, cos_sin_cache)
        kv0 = kv_caches[0]
        self.kv_strides = (0, model.head_dim, kv0.stride(0), kv0.stride(2), kv0.stride(1))
        starts = torch.tensor([start_pos] * B if isinstance(start_pos, int) else list(start_pos), dtype=torch.int64)
        firsts = torch.tensor([first_id] * B if isinstance(first_id, int) else list(first_id), dtype=torch.int64)
        if starts.numel() != B or firsts.numel() != B:
            raise ValueError("start_pos / first_id must give one value per sequence")
        pos = starts[None, :] + torch.arange(steps, dtype=torch.int64)[:, None]          # [steps, B]
        bt = block_table[:B].cpu().to(torch.int64)
        self.max_seq = block_table.shape[1] * BLOCK_SIZE
        if int(pos.max()) + 1 > self.max_seq or int(starts.min()) < 0:
            raise ValueError("block table too small for the requested steps")
        self.positions = pos.contiguous().to(dev)
        self.seq_lens = (pos + 1).to(torch.int32).contiguous().to(dev)
        self.slots = (torch.gather(bt, 1, (pos // 16).t()).t() * 16 + pos % 16).contiguous().to(dev)
        self.ids = torch.zeros((steps + 1, B), dtype=torch.int64, device=dev)
        self.ids[0] = firsts.to(dev)
        self.logits = torch.empty((B, VOCAB), dtype=torch.bfloat16, device=dev) if logits else None
        self.steps = steps
        self.encoded_gu = encoded_gu  # lossless_bf16.EncodedGUCache of these gate_up matrices, or None

    def launch(self, k: int, stream: int) -> None:
        m, rt, B = self.model, self.rt, self.batch
        embed, layers, final_norm, kv_caches, block_table, cos_sin = self.keep
        extra = ()
        if self.encoded_gu is not None:
            launch = self.lib.pk_decode_lossless
            extra = (self.encoded_gu.table.data_ptr(),)
        else:
            launch = self.lib.pk_decode_mxfp8 if m.weight_format == "mxfp8" else self.lib.pk_decode
        rc = launch(
            stream, m.model_id, B, len(layers), self.ids.data_ptr() + 8 * B * k, 1, embed.data_ptr(),
            final_norm.data_ptr(), self.positions.data_ptr() + 8 * B * k, self.seq_lens.data_ptr() + 4 * B * k,
            block_table.data_ptr(), block_table.stride(0), self.slots.data_ptr() + 8 * B * k,
            self.layers_t.data_ptr(), self.kv_t.data_ptr(), *self.kv_strides, BLOCK_SIZE,
            cos_sin.data_ptr(), int(cos_sin.dtype == torch.float32), rt.out.data_ptr(), None,
            self.ids.data_ptr() + 8 * B * (k + 1), self.logits.data_ptr() if self.logits is not None else None,
            rt.scratch_ptr, rt.scratch_bytes, self.max_seq, *extra)
        if rc != 0:
            raise RuntimeError(_failure_message(m, rc))
