"""GPU checks of the serving integration (prime_kernels_amd.decode_backend) with the real decode step:
a served SmolLM2-360M (vLLM attribute layout, random weights, paged caches) whose patched forward
routes a pure decode batch through the step, bit-identical to calling decode_step directly; and the
mixed-batch repair (b2-reproducibility-r1/decode_backend.after.py:210-241) replacing exactly the
decode rows of a batch that mixes prefill and decode, with those rows' KV appended."""

from dataclasses import dataclass
from types import SimpleNamespace as NS

import pytest
import torch

from prime_kernels_amd import decode_backend as D

pytestmark = pytest.mark.gpu


@dataclass
class FlashAttentionMetadata:
    max_query_len: int
    num_actual_tokens: int
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    query_start_loc: torch.Tensor


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _served(batch, cap, seed=5):
    import prime_kernels_amd as pk
    from prime_kernels_amd import workload as WL

    mod = pk.load("decode_megakernel_360m")
    model = mod.MODEL
    dev = torch.device("cuda:0")
    embed, final_norm, lw = WL.random_weights(model, seed, dev)
    kv = WL.PagedKV(model, batch, cap, device=dev, seed=seed + 1, fill="randn")
    cs = WL.rope_table(cap, device=dev)
    layers = []
    for i, (n1, qkv, o, n2, gu, down) in enumerate(lw):
        layers.append(NS(input_layernorm=NS(weight=n1), post_attention_layernorm=NS(weight=n2),
                         self_attn=NS(qkv_proj=NS(weight=qkv), o_proj=NS(weight=o), rotary_emb=NS(cos_sin_cache=cs),
                                      attn=NS(kv_cache=kv.caches[i], layer_name="model.layers.0.self_attn.attn")),
                         mlp=NS(gate_up_proj=NS(weight=gu), down_proj=NS(weight=down))))
    cfg = NS(hidden_size=960, intermediate_size=2560, num_hidden_layers=32, num_attention_heads=15,
             num_key_value_heads=5, rms_norm_eps=1e-5, vocab_size=49152)
    served = NS(config=cfg, layers=layers, embed_tokens=NS(weight=embed),
                norm=NS(weight=final_norm, variance_epsilon=1e-5))
    return mod, served, kv, cs


def _bits(t):
    return t.contiguous().view(torch.int16)


def test_patched_forward_pure_decode_equals_decode_step():
    _need_gpu()
    ctx = [300, 77, 1025]
    mod, served, kv, cs = _served(3, max(ctx) + 64)
    dev = kv.caches[0].device
    pos = [c for c in ctx]
    meta = FlashAttentionMetadata(
        max_query_len=1, num_actual_tokens=3, seq_lens=torch.tensor([p + 1 for p in pos], dtype=torch.int32, device=dev),
        block_table=kv.block_table, slot_mapping=torch.tensor([kv.slot(b, p) for b, p in enumerate(pos)], device=dev),
        query_start_loc=torch.arange(4, dtype=torch.int32, device=dev))
    ids = torch.tensor([17, 4242, 9], device=dev)
    positions = torch.tensor(pos, device=dev)
    caches0 = [c.clone() for c in kv.caches]

    stock_calls = []

    def stock(self, input_ids, positions, intermediate_tensors, inputs_embeds=None, **kw):
        stock_calls.append(1)
        return torch.zeros(input_ids.shape[0], 960, device=dev)

    D.stats.clear()
    fwd = D.patched_forward(stock, {D.KERNEL_NAME_360M: mod.decode_step},
                         attn_metadata_fn=lambda m: {"model.layers.0.self_attn.attn": meta})
    routed = fwd(served, ids, positions, None).clone()
    torch.cuda.synchronize()
    assert D.stats["backend_decode"] == 1 and not stock_calls
    caches_routed = [c.clone() for c in kv.caches]
    for c, c0 in zip(kv.caches, caches0):
        c.copy_(c0)
    direct = mod.decode_step(input_ids=ids, positions=positions, seq_lens=meta.seq_lens, block_table=kv.block_table,
                             slot_mapping=meta.slot_mapping, embed=served.embed_tokens.weight,
                             layers=[(l.input_layernorm.weight, l.self_attn.qkv_proj.weight, l.self_attn.o_proj.weight,
                                      l.post_attention_layernorm.weight, l.mlp.gate_up_proj.weight,
                                      l.mlp.down_proj.weight) for l in served.layers],
                             final_norm=served.norm.weight, kv_caches=kv.caches, cos_sin_cache=cs, eps=1e-5).clone()
    torch.cuda.synchronize()
    assert torch.equal(_bits(routed), _bits(direct))
    assert all(torch.equal(_bits(a), _bits(b)) for a, b in zip(caches_routed, kv.caches))


def test_mixed_batch_repair_replaces_decode_rows():
    """Requests 0 and 2 decode one token; request 1 is a 3-token prefill.  The repair must give token
    rows 0 and 4 the decode step's hidden states for those two requests, leave rows 1-3 as the
    stock forward left them, and append the two decode tokens' K/V."""
    _need_gpu()
    ctx = [513, 40, 200]
    mod, served, kv, cs = _served(3, max(ctx) + 64, seed=9)
    dev = kv.caches[0].device
    slots = [kv.slot(0, ctx[0]), kv.slot(1, 40), kv.slot(1, 41), kv.slot(1, 42), kv.slot(2, ctx[2])]
    meta = FlashAttentionMetadata(
        max_query_len=3, num_actual_tokens=5,
        seq_lens=torch.tensor([ctx[0] + 1, 43, ctx[2] + 1], dtype=torch.int32, device=dev),
        block_table=kv.block_table, slot_mapping=torch.tensor(slots, device=dev),
        query_start_loc=torch.tensor([0, 1, 4, 5], dtype=torch.int32, device=dev))
    ids = torch.tensor([101, 7, 8, 9, 202], device=dev)
    positions = torch.tensor([ctx[0], 40, 41, 42, ctx[2]], device=dev)
    stock = torch.randn(5, 960, device=dev).to(torch.bfloat16)
    caches0 = [c.clone() for c in kv.caches]
    D.stats.clear()
    out = D.repair_mixed_batch(served, {D.KERNEL_NAME_360M: mod.decode_step}, ids, positions, stock,
                                 {"model.layers.0.self_attn.attn": meta})
    torch.cuda.synchronize()
    out = out.clone()
    assert D.stats["backend_mixed_decode"] == 2
    repaired_caches = [c.clone() for c in kv.caches]
    for c, c0 in zip(kv.caches, caches0):
        c.copy_(c0)
    bt = kv.block_table[[0, 2]].contiguous()
    direct = mod.decode_step(input_ids=ids[[0, 4]], positions=positions[[0, 4]],
                             seq_lens=meta.seq_lens[[0, 2]].contiguous(), block_table=bt,
                             slot_mapping=torch.tensor([slots[0], slots[4]], device=dev),
                             embed=served.embed_tokens.weight,
                             layers=[(l.input_layernorm.weight, l.self_attn.qkv_proj.weight, l.self_attn.o_proj.weight,
                                      l.post_attention_layernorm.weight, l.mlp.gate_up_proj.weight,
                                      l.mlp.down_proj.weight) for l in served.layers],
                             final_norm=served.norm.weight, kv_caches=kv.caches, cos_sin_cache=cs, eps=1e-5).clone()
    torch.cuda.synchronize()
    assert torch.equal(_bits(out[[0, 4]]), _bits(direct))
    assert torch.equal(_bits(out[1:4]), _bits(stock[1:4]))
    for li, (a, b, c0) in enumerate(zip(repaired_caches, kv.caches, caches0)):
        assert torch.equal(_bits(a), _bits(b)), li
        for s in (slots[0], slots[4]):
            assert not torch.equal(_bits(a[s // 16, :, s % 16]), _bits(c0[s // 16, :, s % 16])), (li, s)
        for s in slots[1:4]:   # the prefill's slots are the stock forward's business
            assert torch.equal(_bits(a[s // 16, :, s % 16]), _bits(c0[s // 16, :, s % 16])), (li, s)
