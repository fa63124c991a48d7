"""Write golden vectors for the SmolLM2 decode oracle from HF `transformers` (CPU, eager).

The reference's parity oracle is HF `LlamaForCausalLM` eager decode
(research/smollm2_360m_decode/experiments/r34-packed-full/bench_r30_r34.py:113-140), a
third-party dependency that is not part of /root/reference.  This script imports the installed
copy (transformers 5.15.0, torch CPU) -- never the reference -- and records:

  * `<geom>_greedy.npz`: a 2-layer model of the named geometry with seeded weights
    (oracle.smollm2.make_weights, fingerprinted in the json), a seeded prompt, HF's eager
    prefill KV cache, then `STEPS` greedy eager decode steps: token ids, the final-normed hidden
    state, full bf16 logits of steps 0 and STEPS-1, top-32 logits of every step, and each step's
    per-layer K/V append.
  * `block360_stages.npz`: BASELINE config 1, one SmolLM2-360M decoder layer on a hidden-state
    input N(0,1) with a KV cache pre-filled with 512 positions of N(0,1), every stage output
    captured with forward hooks (the reference debug stages, block360_kernel.inc:1-13).
  * `<config>_full.npz`: BASELINE configs 2 and 3 at full depth (SmolLM2-135M, 30 layers, a
    512-token prompt; SmolLM2-360M, 32 layers, a 1024-token prompt), seeded weights and a seeded
    uniform random prompt, HF's eager prompt pass, then 256 greedy eager decode steps: the prompt,
    the 257 greedy ids (ids[0] from the prompt pass, ids[s+1] from decode step s), the final-normed
    hidden state at steps 0..7 and 255, top-32 logits of the prompt pass and of every step, full
    bf16 logits at steps 0 and 255.  The prompt pass's K/V cache (tens of MB) is not stored: the
    json holds the SHA-256 of every layer's K and V [KVH, P, D] bf16 bits instead.

bf16 arrays are stored as their uint16 bit patterns.  Run from the repo root:
    python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import smollm2 as O  # noqa: E402

OUT = Path(__file__).resolve().parent
STEPS = 6
PROMPT = 24
WEIGHT_SEED = 1234


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def hf_model(geom: O.Geometry, w: O.Weights):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=geom.vocab, hidden_size=geom.hidden, intermediate_size=geom.inter,
                      num_hidden_layers=geom.layers, num_attention_heads=geom.heads,
                      num_key_value_heads=geom.kv_heads, head_dim=geom.head_dim,
                      rms_norm_eps=geom.eps, rope_theta=geom.theta, max_position_embeddings=8704,
                      tie_word_embeddings=True, pad_token_id=None, bos_token_id=None,
                      eos_token_id=None)
    cfg._attn_implementation = "eager"
    model = LlamaForCausalLM(cfg).to(torch.bfloat16).eval()
    # `.to(bfloat16)` also casts the rotary inv_freq buffer; a checkpoint loaded with
    # torch_dtype=bfloat16 keeps it fp32 (it is built with dtype=torch.float), as vLLM's fp32
    # cos_sin_cache construction does.  Restore the fp32 frequencies.
    rot = model.model.rotary_emb
    inv_freq, _ = rot.compute_default_rope_parameters(cfg)
    rot.register_buffer("inv_freq", inv_freq.to(torch.float32), persistent=False)
    H, KVD, I = geom.hidden, geom.kv_heads * geom.head_dim, geom.inter
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(w.embed)
        model.model.norm.weight.copy_(w.final_norm)
        for layer, (n1, qkv, o, n2, gu, d) in zip(model.model.layers, w.layers):
            layer.input_layernorm.weight.copy_(n1)
            layer.self_attn.q_proj.weight.copy_(qkv[:H])
            layer.self_attn.k_proj.weight.copy_(qkv[H:H + KVD])
            layer.self_attn.v_proj.weight.copy_(qkv[H + KVD:])
            layer.self_attn.o_proj.weight.copy_(o)
            layer.post_attention_layernorm.weight.copy_(n2)
            layer.mlp.gate_proj.weight.copy_(gu[:I])
            layer.mlp.up_proj.weight.copy_(gu[I:])
            layer.mlp.down_proj.weight.copy_(d)
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    return model


def cache_kv(cache, layer: int):
    """(K, V) [KVH, S, D] of one layer from an HF DynamicCache."""
    lay = cache.layers[layer]
    return lay.keys[0], lay.values[0]


def greedy_fixture(base: O.Geometry, tag: str, seed: int) -> dict:
    geom = O.with_layers(base, 2)
    w = O.make_weights(geom, seed, norm_jitter=0.05)
    model = hf_model(geom, w)
    g = torch.Generator().manual_seed(seed + 1)
    prompt = torch.randint(0, geom.vocab, (1, PROMPT), generator=g)
    normed = {}
    model.model.norm.register_forward_hook(lambda _m, _i, out: normed.update(h=out.detach()))
    with torch.no_grad():
        out = model(input_ids=prompt, use_cache=True)
        cache = out.past_key_values
        prefill_k = torch.stack([cache_kv(cache, li)[0] for li in range(geom.layers)])
        prefill_v = torch.stack([cache_kv(cache, li)[1] for li in range(geom.layers)])
        tok = out.logits[0, -1].argmax().view(1, 1)
        ids, hidden, top_v, top_i, full, step_k, step_v = [], [], [], [], [], [], []
        for step in range(STEPS):
            pos = PROMPT + step
            o = model(input_ids=tok, past_key_values=cache, use_cache=True,
                      position_ids=torch.tensor([[pos]]))
            lg = o.logits[0, -1]
            ids.append(int(tok))
            hidden.append(bits(normed["h"][0, -1]))
            tv, ti = torch.topk(lg.float(), 32)
            top_v.append(bits(tv)), top_i.append(ti.numpy().astype(np.int32))
            if step in (0, STEPS - 1):
                full.append(bits(lg))
            step_k.append(np.stack([bits(cache_kv(cache, li)[0][:, pos]) for li in range(geom.layers)]))
            step_v.append(np.stack([bits(cache_kv(cache, li)[1][:, pos]) for li in range(geom.layers)]))
            tok = lg.argmax().view(1, 1)
        ids.append(int(tok))
    np.savez_compressed(OUT / f"{tag}_greedy.npz", prompt=prompt[0].numpy().astype(np.int32),
                        prefill_k=bits(prefill_k), prefill_v=bits(prefill_v),
                        ids=np.array(ids, dtype=np.int32), hidden=np.stack(hidden),
                        top_v=np.stack(top_v), top_i=np.stack(top_i), full_logits=np.stack(full),
                        step_k=np.stack(step_k), step_v=np.stack(step_v))
    return {"geometry": geom.__dict__, "seed": seed, "norm_jitter": 0.05, "prompt_len": PROMPT,
            "steps": STEPS, "full_logit_steps": [0, STEPS - 1],
            "weights_sha256": w.fingerprint()}


FULL_STEPS = 256
HIDDEN_STEPS = list(range(8)) + [FULL_STEPS - 1]


def full_fixture(geom: O.Geometry, tag: str, seed: int, prompt_len: int) -> dict:
    """BASELINE config 2 / 3 at full depth: prompt pass, then FULL_STEPS greedy steps."""
    w = O.make_weights(geom, seed)
    model = hf_model(geom, w)
    g = torch.Generator().manual_seed(seed + 1)
    prompt = torch.randint(0, geom.vocab, (1, prompt_len), generator=g)
    normed = {}
    model.model.norm.register_forward_hook(lambda _m, _i, out: normed.update(h=out.detach()))
    with torch.no_grad():
        out = model(input_ids=prompt, use_cache=True)
        cache = out.past_key_values
        kv_sha = {}
        for li in range(geom.layers):
            k, v = cache_kv(cache, li)
            kv_sha[f"layers.{li}.k"] = O.sha256_tensor(k.contiguous())
            kv_sha[f"layers.{li}.v"] = O.sha256_tensor(v.contiguous())
        pv, pi = torch.topk(out.logits[0, -1].float(), 32)
        tok = out.logits[0, -1].argmax().view(1, 1)
        ids, hidden, top_v, top_i, full = [int(tok)], [], [], [], []
        for step in range(FULL_STEPS):
            o = model(input_ids=tok, past_key_values=cache, use_cache=True,
                      position_ids=torch.tensor([[prompt_len + step]]))
            lg = o.logits[0, -1]
            if step in HIDDEN_STEPS:
                hidden.append(bits(normed["h"][0, -1]))
            tv, ti = torch.topk(lg.float(), 32)
            top_v.append(bits(tv)), top_i.append(ti.numpy().astype(np.int32))
            if step in (0, FULL_STEPS - 1):
                full.append(bits(lg))
            tok = lg.argmax().view(1, 1)
            ids.append(int(tok))
    np.savez_compressed(OUT / f"{tag}_full.npz", prompt=prompt[0].numpy().astype(np.int32),
                        ids=np.array(ids, dtype=np.int32), hidden=np.stack(hidden), top_v=np.stack(top_v),
                        top_i=np.stack(top_i), full_logits=np.stack(full), prefill_top_v=bits(pv),
                        prefill_top_i=pi.numpy().astype(np.int32))
    return {"geometry": geom.__dict__, "seed": seed, "norm_jitter": 0.0, "prompt_len": prompt_len,
            "steps": FULL_STEPS, "hidden_steps": HIDDEN_STEPS, "full_logit_steps": [0, FULL_STEPS - 1],
            "prefill_kv_sha256": kv_sha, "weights_sha256": w.fingerprint()}


def block_fixture(seed: int) -> dict:
    """one 360M block, hidden input N(0,1), 512 cached positions N(0,1)."""
    from transformers import DynamicCache

    geom = O.with_layers(O.SMOLLM2_360M, 1)
    w = O.make_weights(geom, seed, norm_jitter=0.05)
    model = hf_model(geom, w)
    layer = model.model.layers[0]
    g = torch.Generator().manual_seed(seed + 7)
    ctx = 512
    x = torch.randn(1, 1, geom.hidden, generator=g).to(torch.bfloat16)
    past_k = torch.randn(1, geom.kv_heads, ctx, geom.head_dim, generator=g).to(torch.bfloat16)
    past_v = torch.randn(1, geom.kv_heads, ctx, geom.head_dim, generator=g).to(torch.bfloat16)
    cache = DynamicCache(config=model.config)
    cache.update(past_k.clone(), past_v.clone(), 0)
    st = {}

    def hook(name):
        return lambda _m, i, out: st.update({name: (out[0] if isinstance(out, tuple) else out).detach(),
                                             name + "_in": i[0].detach() if i else None})

    layer.input_layernorm.register_forward_hook(hook("norm1"))
    layer.self_attn.q_proj.register_forward_hook(hook("q"))
    layer.self_attn.k_proj.register_forward_hook(hook("k"))
    layer.self_attn.v_proj.register_forward_hook(hook("v"))
    layer.self_attn.o_proj.register_forward_hook(hook("o"))
    layer.post_attention_layernorm.register_forward_hook(hook("norm2"))
    layer.mlp.gate_proj.register_forward_hook(hook("gate"))
    layer.mlp.up_proj.register_forward_hook(hook("up"))
    layer.mlp.act_fn.register_forward_hook(hook("silu"))
    layer.mlp.down_proj.register_forward_hook(hook("down"))
    pos = torch.tensor([[ctx]])
    with torch.no_grad():
        cos, sin = model.model.rotary_emb(x, pos)
        out = layer(x, attention_mask=None, position_ids=pos, past_key_values=cache,
                    use_cache=True, position_embeddings=(cos, sin))
        out = out[0] if isinstance(out, tuple) else out
    k_rot, v_new = cache_kv(cache, 0)[0][:, ctx], cache_kv(cache, 0)[1][:, ctx]
    np.savez_compressed(OUT / "block360_stages.npz", x=bits(x[0, 0]), past_k=bits(past_k[0]),
                        past_v=bits(past_v[0]), norm1=bits(st["norm1"][0, 0]), q=bits(st["q"][0, 0]),
                        k=bits(st["k"][0, 0]), v=bits(st["v"][0, 0]), k_rot=bits(k_rot),
                        v_new=bits(v_new), attn=bits(st["o_in"][0, 0]), o=bits(st["o"][0, 0]),
                        norm2=bits(st["norm2"][0, 0]), h1=bits(st["norm2_in"][0, 0]),
                        gate=bits(st["gate"][0, 0]), up=bits(st["up"][0, 0]),
                        silu=bits(st["silu"][0, 0]), act=bits(st["down_in"][0, 0]),
                        down=bits(st["down"][0, 0]), out=bits(out[0, 0]),
                        cos=bits(cos[0, 0]), sin=bits(sin[0, 0]))
    return {"geometry": geom.__dict__, "seed": seed, "norm_jitter": 0.05, "context": ctx,
            "position": ctx, "weights_sha256": w.fingerprint()}


def main() -> None:
    import transformers

    torch.set_num_threads(8)
    meta = {"transformers": transformers.__version__, "torch": torch.__version__, "torch_threads": 8,
            "fixtures": {"smollm2_360m": greedy_fixture(O.SMOLLM2_360M, "smollm2_360m", WEIGHT_SEED),
                         "smollm2_135m": greedy_fixture(O.SMOLLM2_135M, "smollm2_135m", WEIGHT_SEED + 100),
                         "block360": block_fixture(WEIGHT_SEED + 200),
                         "config2_135m": full_fixture(O.SMOLLM2_135M, "config2_135m", 2002, 512),
                         "config3_360m": full_fixture(O.SMOLLM2_360M, "config3_360m", 3003, 1024)}}
    (OUT / "golden.json").write_text(json.dumps(meta, indent=1, sort_keys=True) + "\n")
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))


if __name__ == "__main__":
    main()
