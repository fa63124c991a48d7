"""CPU checks of the serving integration (prime_kernels_amd.decode_backend), whose routing rules follow
the reference's vLLM backend module (b2-reproducibility-r1/decode_backend.after.py): geometry routing,
model and metadata eligibility, the route and its statistics key, the patched forward's routing and
statistics, and the mixed-batch repair's row selection.  The decode step here is a recording stand-in; the GPU
checks (tests/test_gpu_backend.py) run the real step."""

from dataclasses import dataclass, field
from types import SimpleNamespace as NS

import pytest
import torch

from prime_kernels_amd import decode_backend as D

BF16 = torch.bfloat16


@dataclass
class FlashAttentionMetadata:  # the vLLM class name the backend checks for
    max_query_len: int
    num_actual_tokens: int
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    query_start_loc: torch.Tensor = field(default_factory=lambda: torch.zeros(1, dtype=torch.int32))


class OtherMetadata(FlashAttentionMetadata):
    pass


def _config(name="360m", **over):
    base = dict(hidden_size=960, intermediate_size=2560, num_hidden_layers=32, num_attention_heads=15,
                num_key_value_heads=5, rms_norm_eps=1e-5, vocab_size=49152) if name == "360m" else dict(
        hidden_size=576, intermediate_size=1536, num_hidden_layers=30, num_attention_heads=9,
        num_key_value_heads=3, rms_norm_eps=1e-5, vocab_size=49152)
    base.update(over)
    return NS(**base)


def _model(name="360m", blocks=8, layers=None, embed_dtype=BF16):
    cfg = _config(name)
    L = layers or cfg.num_hidden_layers
    kvh = cfg.num_key_value_heads
    lay = []
    for i in range(L):
        w = lambda: NS(weight=torch.zeros(1, dtype=BF16))  # noqa: E731
        lay.append(NS(input_layernorm=w(), post_attention_layernorm=w(),
                      self_attn=NS(qkv_proj=w(), o_proj=w(),
                                   attn=NS(kv_cache=torch.zeros(blocks, kvh, 16, 128, dtype=BF16), layer_name="l0"),
                                   rotary_emb=NS(cos_sin_cache=torch.zeros(64, 64, dtype=BF16))),
                      mlp=NS(gate_up_proj=w(), down_proj=w())))
    return NS(config=cfg, layers=lay, embed_tokens=NS(weight=torch.zeros(4, dtype=embed_dtype)),
              norm=NS(weight=torch.zeros(1, dtype=BF16), variance_epsilon=1e-5))


def _meta(batch, width=4, qlen=1, **over):
    m = FlashAttentionMetadata(max_query_len=qlen, num_actual_tokens=batch,
                               seq_lens=torch.arange(batch, dtype=torch.int32) + 5,
                               block_table=torch.arange(batch * width, dtype=torch.int32).view(batch, width),
                               slot_mapping=torch.arange(batch, dtype=torch.int64) + 100)
    for k, v in over.items():
        setattr(m, k, v)
    return m


def test_geometry_routing():
    assert D.kernel_for_config(_config("360m")) == D.KERNEL_NAME_360M
    assert D.kernel_for_config(_config("135m")) == D.KERNEL_NAME_135M
    for bad in (dict(num_hidden_layers=31), dict(rms_norm_eps=1e-6), dict(num_key_value_heads=3),
                dict(head_dim=128), dict(intermediate_size=2048), dict(vocab_size=49153), dict(vocab_size=32000)):
        assert D.kernel_for_config(_config("360m", **bad)) is None, bad


def test_geometry_routing_hf_config():
    transformers = pytest.importorskip("transformers")
    c = transformers.LlamaConfig(hidden_size=960, intermediate_size=2560, num_hidden_layers=32,
                                 num_attention_heads=15, num_key_value_heads=5, rms_norm_eps=1e-5,
                                 vocab_size=49152)
    assert D.kernel_for_config(c) == D.KERNEL_NAME_360M


def test_model_eligibility():
    assert D.kernel_for_model(_model("360m")) == D.KERNEL_NAME_360M
    assert D.kernel_for_model(_model("135m")) == D.KERNEL_NAME_135M
    assert D.kernel_for_model(_model("360m", embed_dtype=torch.float16)) is None
    m = _model("360m")
    m.aux_hidden_state_layers = (2,)
    assert D.kernel_for_model(m) is None
    m = _model("360m")
    m.tp_size = 2
    assert D.kernel_for_model(m) is None


def test_metadata_eligibility_rules():
    model = _model("360m")
    K = D.KERNEL_NAME_360M
    assert D.metadata_fits(_meta(3), model, K, 3)
    assert not D.metadata_fits(OtherMetadata(**vars(_meta(3))), model, K, 3)
    assert not D.metadata_fits(_meta(3, qlen=2), model, K, 3)
    assert not D.metadata_fits(_meta(3), model, K, 2)          # num_actual_tokens != batch
    assert not D.metadata_fits(_meta(17), model, K, 17)        # over the batch limit
    assert D.metadata_fits(_meta(16), model, K, 16)
    assert not D.metadata_fits(_meta(3, block_table=_meta(3).block_table.long()), model, K, 3)
    assert not D.metadata_fits(_meta(3, width=12288 // 16 + 1), model, K, 3)
    assert D.metadata_fits(_meta(3, width=12288 // 16), model, K, 3)
    assert not D.metadata_fits(_meta(3, block_table=_meta(3).block_table.t().contiguous().t()), model, K, 3)
    bad = _model("360m")
    bad.layers[5].self_attn.attn.kv_cache = torch.zeros(9, 5, 16, 128, dtype=BF16)   # shapes differ
    assert not D.metadata_fits(_meta(3), bad, K, 3)
    bad = _model("360m")
    for layer in bad.layers:
        layer.self_attn.attn.kv_cache = torch.zeros(8, 16, 5, 128, dtype=BF16)         # heads/tokens swapped
    assert not D.metadata_fits(_meta(3), bad, K, 3)
    # the 135M geometry checks its own KV head count
    assert D.metadata_fits(_meta(2), _model("135m"), D.KERNEL_NAME_135M, 2)
    assert not D.metadata_fits(_meta(2), _model("135m"), K, 2)


def test_route_and_its_reasons():
    model = _model("360m")
    step = object()
    steps = {D.KERNEL_NAME_360M: step}
    assert D.route(steps, model, D.KERNEL_NAME_360M, _meta(2), 2) == (step, None)
    assert D.route(steps, model, None, _meta(2), 2) == (None, "stock_ineligible")
    assert D.route(steps, model, D.KERNEL_NAME_135M, _meta(2), 2) == (None, "stock_kernel_unavailable")
    assert D.route(steps, model, D.KERNEL_NAME_360M, None, 2) == (None, "stock_not_pure_decode")
    assert D.route(steps, model, D.KERNEL_NAME_360M, _meta(2, qlen=2), 2) == (None, "stock_not_pure_decode")
    assert D.route(steps, model, D.KERNEL_NAME_360M, _meta(3), 2) == (None, "stock_decode_over_max_batch")
    assert D.route(steps, model, D.KERNEL_NAME_360M, _meta(17), 17) == (None, "stock_decode_over_max_batch")
    assert D.route(steps, model, D.KERNEL_NAME_360M, _meta(0), 0) == (None, "stock_unsupported_metadata")
    bt64 = _meta(2).block_table.long()
    assert D.route(steps, model, D.KERNEL_NAME_360M, _meta(2, block_table=bt64), 2) == \
        (None, "stock_unsupported_metadata")


class Recorder:
    """A decode_step stand-in: records its kwargs and returns a recognisable [B, H] tensor."""

    def __init__(self, hidden=960):
        self.calls, self.hidden = [], hidden

    def __call__(self, **kw):
        self.calls.append(kw)
        B = kw["input_ids"].shape[0]
        return torch.full((B, self.hidden), 7.0) + kw["input_ids"].float().view(B, 1)


def _patched(model, steps, meta_by_call):
    stock = []

    def original(self, input_ids, positions, intermediate_tensors, inputs_embeds=None, **kw):
        stock.append(input_ids.shape[0])
        return torch.zeros(input_ids.shape[0], 960)

    fwd = D.patched_forward(original, steps, attn_metadata_fn=lambda m: meta_by_call[0])
    return fwd, stock


def test_patched_forward_routes_and_counts(monkeypatch):
    monkeypatch.delenv(D.ENABLE_360M_LOSSLESS_ENV, raising=False)
    D.stats.clear()
    model = _model("360m")
    rec = Recorder()
    current = [None]
    fwd, stock = _patched(model, {D.KERNEL_NAME_360M: rec}, current)
    ids = torch.tensor([3, 4]); pos = torch.tensor([9, 10])
    current[0] = {"l0": _meta(2)}
    out = fwd(model, ids, pos, None)
    assert torch.equal(out, rec(input_ids=ids)) and len(rec.calls) == 2
    kw = rec.calls[0]
    assert kw["eps"] == 1e-5 and len(kw["layers"]) == 32 and len(kw["kv_caches"]) == 32
    assert torch.equal(kw["seq_lens"], current[0]["l0"].seq_lens[:2])
    current[0] = {"l0": _meta(2, qlen=3)}                # a prefill joins: stock forward
    fwd(model, ids, pos, None)
    current[0] = None                                    # no metadata at all
    fwd(model, ids, pos, None)
    current[0] = {"l0": _meta(3)}                        # metadata for 3 tokens, 2 ids
    fwd(model, ids, pos, None)
    current[0] = {"l0": _meta(2, block_table=_meta(2).block_table.long())}
    fwd(model, ids, pos, None)
    fwd(model, ids, pos, None, inputs_embeds=torch.zeros(2, 960))
    assert dict(D.stats) == {"backend_decode": 1, "stock_not_pure_decode": 2, "stock_decode_over_max_batch": 1,
                             "stock_unsupported_metadata": 1, "stock_ineligible": 1}
    assert stock == [2, 2, 2, 2, 2]
    D.stats.clear()
    fwd2, _ = _patched(model, {D.KERNEL_NAME_135M: rec}, [{"l0": _meta(2)}])
    fwd2(model, ids, pos, None)                          # 360M geometry, only the 135M step enabled
    assert dict(D.stats) == {"stock_kernel_unavailable": 1}


def test_repair_mixed_decode_rows():
    """Requests 0 and 2 decode (one query token), request 1 is a 3-token prefill: only token rows
    0 and 4 are recomputed, with the decode rows' sequence metadata."""
    D.stats.clear()
    model = _model("360m")
    rec = Recorder()
    meta = _meta(3, qlen=3, num_actual_tokens=5, query_start_loc=torch.tensor([0, 1, 4, 5], dtype=torch.int32),
                 slot_mapping=torch.arange(5, dtype=torch.int64) + 200)
    ids = torch.tensor([11, 12, 13, 14, 15]); pos = torch.tensor([8, 0, 1, 2, 6])
    hidden = torch.arange(5 * 960, dtype=torch.float32).view(5, 960)
    out = D.repair_mixed_batch(model, {D.KERNEL_NAME_360M: rec}, ids, pos, hidden, {"l0": meta})
    kw = rec.calls[0]
    assert torch.equal(kw["input_ids"], torch.tensor([11, 15])) and torch.equal(kw["positions"], torch.tensor([8, 6]))
    assert torch.equal(kw["seq_lens"], meta.seq_lens[[0, 2]])
    assert torch.equal(kw["block_table"], meta.block_table[[0, 2]])
    assert torch.equal(kw["slot_mapping"], torch.tensor([200, 204]))
    assert torch.equal(out[[0, 4]], rec(input_ids=torch.tensor([11, 15])))
    assert torch.equal(out[1:4], hidden[1:4]) and torch.equal(hidden[0], torch.arange(960, dtype=torch.float32))
    assert D.stats["backend_mixed_decode"] == 2
    # pure decode or pure prefill: nothing to repair
    h2 = hidden[:2].clone()
    assert D.repair_mixed_batch(model, {D.KERNEL_NAME_360M: rec}, ids[:2], pos[:2], h2, {"l0": _meta(2)}) is h2
    pre = _meta(1, qlen=5, num_actual_tokens=5, query_start_loc=torch.tensor([0, 5], dtype=torch.int32))
    h = torch.zeros(5, 960)
    assert D.repair_mixed_batch(model, {D.KERNEL_NAME_360M: rec}, ids, pos, h, {"l0": pre}) is h


def test_monkey_patch_installs_once(tmp_path, monkeypatch):
    ref = tmp_path / "ref_step.py"
    ref.write_text("def decode_step(**kw):\n    return 'reference'\n")
    monkeypatch.setenv(D.REFERENCE_ENV, str(ref))

    class Model:
        def forward(self, input_ids, positions, intermediate_tensors, inputs_embeds=None, **kw):
            return "stock"

    assert D.monkey_patch_decode_backend(Model, attn_metadata_fn=lambda m: None)
    first = Model.forward
    assert first._prime_rl_decode_backend
    assert D.monkey_patch_decode_backend(Model) and Model.forward is first   # idempotent
    m = Model()
    assert m.forward(torch.tensor([1]), torch.tensor([0]), None) == "stock"   # not a SmolLM2 model
    monkeypatch.delenv(D.REFERENCE_ENV)
    if not torch.cuda.is_available():
        class Other:
            def forward(self, *a, **k):
                return "stock"
        assert D.monkey_patch_decode_backend(Other) is False   # no decode step is available here
        assert not getattr(Other.forward, "_prime_rl_decode_backend", False)


def test_monkey_patch_without_vllm_needs_a_class():
    if D._vllm_types() is not None:
        pytest.skip("vLLM is installed")
    with pytest.raises(ImportError, match="model_cls"):
        D.monkey_patch_decode_backend()
