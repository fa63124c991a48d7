"""CPU oracle for the SmolLM2 single-token decode step.

TEST INFRASTRUCTURE ONLY.  Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline`
leg of `bench.py` may import this module, and only as the checker (or the timed CPU
baseline).  The product path (`prime_kernels_amd`) never imports it and has no CPU fallback.

What it restates
----------------
The reference's parity oracle for `decode_megakernel_360m.decode_step` is the PyTorch eager
Llama decode step of HuggingFace `transformers` (the reference harness loads
`LlamaModel` with `attn_implementation="eager"` at
research/smollm2_360m_decode/experiments/r34-packed-full/bench_r30_r34.py:113-140 and takes
`argmax(dim=-1)` at :128).  `transformers` is a third-party dependency that is not vendored in
the reference; the version pinned by this image is 5.15.0.  This file restates its published
algorithm with the same torch ops, shapes and bf16 rounding points, so that on CPU it is
bit-identical to `LlamaForCausalLM` (pinned by tests/golden fixtures written from
transformers 5.15.0):

  RMSNorm        transformers/models/llama/modeling_llama.py:62-67
                 y = w * bf16(x_f32 * rsqrt(mean(x_f32^2) + eps))
  RoPE table     modeling_llama.py:93-127  inv_freq = 1/theta^(2i/D); cos/sin in fp32 -> bf16
  RoPE apply     modeling_llama.py:130-160 q*cos + rotate_half(q)*sin, each op rounded to bf16
  attention      modeling_llama.py:191-214 (eager): bf16(q k^T) * 1/8, fp32 softmax -> bf16,
                 bf16(p v); GQA via repeat_kv (:179-188)
  MLP            modeling_llama.py:174-175 down(silu(gate(x)) * up(x))
  LM head        tied to embed_tokens (modeling_llama.py:422, :480) then argmax (first index)

Reference kernel layout it mirrors (so the oracle takes the kernel's own inputs):
  fused qkv [q;k;v] rows 0..H-1 / H..H+KVH*D-1 / ... and fused gate_up [gate;up]
  (prime_kernels/decode_megakernel_360m/csrc/block360.cu:53-60);
  paged KV cache [blocks, kv_heads, 16, 2*D] with K in [0:D) and V in [D:2D)
  (prime_kernels/decode_megakernel_360m/__init__.py:186-190, block360_kernel.inc:124-135);
  cos_sin_cache [max_pos, D] with cos in [0:D/2) and sin in [D/2:D) (block360.cu:290-307).
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16


@dataclass(frozen=True)
class Geometry:
    """Model constants (reference: decode_megakernel_360m/__init__.py:27-35,
    decode_megakernel/__init__.py:37-43)."""

    name: str
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    layers: int
    vocab: int = 49152
    eps: float = 1e-5
    theta: float = 100000.0

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def layer_shapes(self) -> tuple[tuple[int, ...], ...]:
        h, i = self.hidden, self.inter
        return ((h,), (self.qkv_rows, h), (h, h), (h,), (2 * i, h), (h, i))


SMOLLM2_360M = Geometry("smollm2-360m", 960, 15, 5, 64, 2560, 32)
SMOLLM2_135M = Geometry("smollm2-135m", 576, 9, 3, 64, 1536, 30)


def with_layers(geom: Geometry, layers: int) -> Geometry:
    return Geometry(geom.name + f"-l{layers}", geom.hidden, geom.heads, geom.kv_heads, geom.head_dim,
                    geom.inter, layers, geom.vocab, geom.eps, geom.theta)


# --------------------------------------------------------------------------------------------
# Seeded weights and inputs
# --------------------------------------------------------------------------------------------

@dataclass
class Weights:
    geom: Geometry
    embed: torch.Tensor                      # [V, H] bf16 (also the tied LM head)
    final_norm: torch.Tensor                 # [H] bf16
    layers: list = field(default_factory=list)  # L x (norm1, qkv, o, norm2, gate_up, down)

    def to(self, device) -> "Weights":
        return Weights(self.geom, self.embed.to(device), self.final_norm.to(device),
                       [tuple(t.to(device) for t in layer) for layer in self.layers])

    def fingerprint(self) -> dict[str, str]:
        out = {"embed": sha256_tensor(self.embed), "final_norm": sha256_tensor(self.final_norm)}
        names = ("norm1", "qkv", "o", "norm2", "gate_up", "down")
        for li, layer in enumerate(self.layers):
            for n, t in zip(names, layer):
                out[f"layers.{li}.{n}"] = sha256_tensor(t)
        return out


def sha256_tensor(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().contiguous().cpu().view(torch.uint8).numpy().tobytes()).hexdigest()


def make_weights(geom: Geometry, seed: int, *, norm_jitter: float = 0.0, device="cpu",
                 std: float = 0.02) -> Weights:
    """Random-init weights as HF's Llama init draws them: Linear/Embedding ~ N(0, std) in bf16,
    RMSNorm weight 1.0 (transformers/modeling_utils.py:2391-2420).  `norm_jitter` > 0 draws
    norm weights 1 + N(0, jitter) instead, so tests exercise the norm-weight multiply.

    Draw order is fixed (embed, final_norm, then per layer norm1, qkv, o, norm2, gate_up, down)
    so a seed names one weight set; on CPU the torch generator is deterministic."""
    g = torch.Generator(device=device).manual_seed(seed)

    def normal(shape):
        return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).to(BF16)

    def norm(shape):
        if norm_jitter == 0.0:
            return torch.ones(shape, dtype=BF16, device=device)
        return (1.0 + norm_jitter * torch.randn(shape, generator=g, device=device)).to(BF16)

    embed = normal((geom.vocab, geom.hidden))
    final_norm = norm((geom.hidden,))
    layers = []
    for _ in range(geom.layers):
        shapes = geom.layer_shapes()
        layers.append((norm(shapes[0]), normal(shapes[1]), normal(shapes[2]), norm(shapes[3]),
                       normal(shapes[4]), normal(shapes[5])))
    return Weights(geom, embed, final_norm, layers)


def rope_cos_sin(max_pos: int, head_dim: int = 64, theta: float = 100000.0) -> torch.Tensor:
    """vLLM-layout rotary table [max_pos, D] bf16: cos in [0:D/2), sin in [D/2:D).

    Values are HF's: inv_freq = 1/theta^(arange(0,D,2)/D) (modeling_llama.py:108), then
    freqs = inv_freq @ positions in fp32, cos/sin in fp32, cast to the activation dtype
    (modeling_llama.py:113-127).  HF duplicates freqs over both halves (cat(freqs, freqs)), so the
    half-width table holds every value it uses."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float) / head_dim))
    pos = torch.arange(max_pos, dtype=torch.int64)
    inv_freq_expanded = inv_freq[None, :, None].float()
    position_ids_expanded = pos[None, None, :].float()
    freqs = (inv_freq_expanded @ position_ids_expanded).transpose(1, 2)[0]  # [max_pos, D/2]
    return torch.cat((freqs.cos().to(BF16), freqs.sin().to(BF16)), dim=-1).contiguous()


# --------------------------------------------------------------------------------------------
# Elementwise pieces (each mirrors one HF op and its rounding)
# --------------------------------------------------------------------------------------------

def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """LlamaRMSNorm.forward (modeling_llama.py:62-67)."""
    input_dtype = x.dtype
    hs = x.to(torch.float32)
    variance = hs.pow(2).mean(-1, keepdim=True)
    hs = hs * torch.rsqrt(variance + eps)
    return w * hs.to(input_dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """modeling_llama.py:130-135."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """q*cos + rotate_half(q)*sin in bf16 (modeling_llama.py:138-160); cos/sin are the full-width
    HF tensors [.., D] broadcast over heads."""
    return (x * cos) + (rotate_half(x) * sin)


def full_cos_sin(cos_sin_row: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    half = cos_sin_row.shape[-1] // 2
    c, s = cos_sin_row[..., :half], cos_sin_row[..., half:]
    return torch.cat((c, c), dim=-1), torch.cat((s, s), dim=-1)


def repeat_kv(hs: torch.Tensor, n_rep: int) -> torch.Tensor:
    """modeling_llama.py:179-188."""
    batch, kvh, slen, d = hs.shape
    if n_rep == 1:
        return hs
    hs = hs[:, :, None, :, :].expand(batch, kvh, n_rep, slen, d)
    return hs.reshape(batch, kvh * n_rep, slen, d)


def eager_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, n_rep: int, scaling: float):
    """eager_attention_forward (modeling_llama.py:191-214) without mask (single decode query,
    no padding: the HF causal mask is all zeros there and adding it is exact)."""
    key_states = repeat_kv(k, n_rep)
    value_states = repeat_kv(v, n_rep)
    attn_weights = torch.matmul(q, key_states.transpose(2, 3)) * scaling
    attn_weights = F.softmax(attn_weights, dim=-1, dtype=torch.float32).to(q.dtype)
    attn_output = torch.matmul(attn_weights, value_states)
    return attn_output.transpose(1, 2).contiguous(), attn_weights


# --------------------------------------------------------------------------------------------
# Paged KV helpers (vLLM FLASH_ATTN layout used by the reference ABI)
# --------------------------------------------------------------------------------------------

@dataclass
class PagedKV:
    """Per-layer caches [blocks, kv_heads, block_size, 2*D] bf16 plus per-sequence block tables."""

    caches: list            # L tensors
    block_table: torch.Tensor   # [B, W] int32
    block_size: int = 16

    def slot(self, b: int, pos: int) -> int:
        blk = int(self.block_table[b, pos // self.block_size])
        return blk * self.block_size + pos % self.block_size

    def gather(self, layer: int, b: int, length: int, head_dim: int):
        """K, V of sequence b for positions [0, length) as [1, kv_heads, length, D]."""
        cache = self.caches[layer]
        pos = torch.arange(length)
        blocks = self.block_table[b, (pos // self.block_size)].long()
        offs = pos % self.block_size
        rows = cache[blocks, :, offs, :]            # [length, kv_heads, 2D]
        rows = rows.permute(1, 0, 2).unsqueeze(0)   # [1, kv_heads, length, 2D]
        return rows[..., :head_dim].contiguous(), rows[..., head_dim:].contiguous()

    def write(self, layer: int, slot: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """KV append at slot_mapping (block360_kernel.inc:124-135); slot < 0 skips."""
        if slot < 0:
            return
        blk, off = slot // self.block_size, slot % self.block_size
        d = k.shape[-1]
        self.caches[layer][blk, :, off, :d] = k
        self.caches[layer][blk, :, off, d:] = v


def make_paged_kv(geom: Geometry, batch: int, capacity: int, *, block_size: int = 16,
                  extra_blocks: int = 0, seed: int | None = None, device="cpu",
                  shuffle: bool = True) -> PagedKV:
    """Empty (zero) or random N(0,1) paged caches with a (seeded) permuted block table."""
    width = (capacity + block_size - 1) // block_size
    nblocks = batch * width + extra_blocks
    g = torch.Generator().manual_seed(0 if seed is None else seed)
    perm = torch.randperm(nblocks, generator=g) if shuffle else torch.arange(nblocks)
    block_table = perm[: batch * width].reshape(batch, width).to(torch.int32)
    caches = []
    for _ in range(geom.layers):
        shape = (nblocks, geom.kv_heads, block_size, 2 * geom.head_dim)
        if seed is None:
            caches.append(torch.zeros(shape, dtype=BF16, device=device))
        else:
            caches.append(torch.randn(shape, generator=g, dtype=torch.float32).to(BF16).to(device))
    return PagedKV(caches, block_table.to(device), block_size)


# --------------------------------------------------------------------------------------------
# The decode step
# --------------------------------------------------------------------------------------------

def decoder_layer(geom: Geometry, layer_w, x: torch.Tensor, pos: int, cos_sin: torch.Tensor,
                  past_k: torch.Tensor, past_v: torch.Tensor, stages: dict | None = None):
    """One LlamaDecoderLayer (modeling_llama.py:284-326, attention :243-281) for one sequence, one new token.

    x [1,1,H] bf16; past_k/past_v [1,KVH,S-1,D] bf16 (positions before `pos`).
    Returns (new x, k_rot [KVH,D], v [KVH,D])."""
    norm1, qkv, o_w, norm2, gate_up, down = layer_w
    H, D, NH, KVH, I = geom.hidden, geom.head_dim, geom.heads, geom.kv_heads, geom.inter
    residual = x
    h = rms_norm(x, norm1, geom.eps)
    # q_proj / k_proj / v_proj are separate Linear layers in HF; use the matching row views.
    q = F.linear(h, qkv[:H])
    k = F.linear(h, qkv[H:H + KVH * D])
    v = F.linear(h, qkv[H + KVH * D:])
    q = q.view(1, 1, NH, D).transpose(1, 2)
    k = k.view(1, 1, KVH, D).transpose(1, 2)
    v = v.view(1, 1, KVH, D).transpose(1, 2)
    cos, sin = full_cos_sin(cos_sin[pos].view(1, 1, D))
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    q_rot = apply_rope(q, cos, sin)
    k_rot = apply_rope(k, cos, sin)
    keys = torch.cat((past_k, k_rot), dim=2)
    values = torch.cat((past_v, v), dim=2)
    attn, probs = eager_attention(q_rot, keys, values, NH // KVH, D ** -0.5)
    attn = attn.reshape(1, 1, H).contiguous()
    o = F.linear(attn, o_w)
    x = residual + o
    residual = x
    h2 = rms_norm(x, norm2, geom.eps)
    g = F.linear(h2, gate_up[:I])
    u = F.linear(h2, gate_up[I:])
    silu = F.silu(g)
    act = silu * u
    d = F.linear(act, down)
    x = residual + d
    if stages is not None:
        # bf16(q . k) before the 1/sqrt(D) scale and the scaled scores, by the op eager_attention uses
        qk = torch.matmul(q_rot, repeat_kv(keys, NH // KVH).transpose(2, 3))
        stages.update(norm1=h, qkv=torch.cat([q.reshape(-1), k.reshape(-1), v.reshape(-1)]), q_rot=q_rot,
                      k_rot=k_rot, v=v, qk=qk, scores=qk * D ** -0.5, attn=attn, probs=probs, o=o,
                      h1=residual, norm2=h2, gate=g, up=u, silu=silu, act=act, down=d, out=x)
    return x, k_rot[0, :, 0, :], v[0, :, 0, :]


@torch.no_grad()
def decode_step(w: Weights, ids, positions, kv: PagedKV, cos_sin: torch.Tensor, *,
                slot_mapping=None, seq_lens=None, want_logits: bool = True,
                layer_outputs: bool = False, stages_layer: int = -1) -> dict:
    """One greedy decode step for B independent sequences (each run with B=1 shapes, as HF's
    single-sequence decode).  Appends K/V into `kv` at slot_mapping (default: the slot of
    `positions[b]`).  Attends to positions [0, seq_lens[b]) with the new token last
    (seq_lens defaults to positions+1).

    Returns {hidden: final-normed [B,H] bf16, logits: [B,V] bf16, ids: [B] int64,
             layer_outputs: [L,B,H] bf16 (optional), stages: per-stage dict (optional)}."""
    geom = w.geom
    B = len(ids)
    hidden, logits, out_ids, louts, stages = [], [], [], [], {}
    for b in range(B):
        pos = int(positions[b])
        S = int(seq_lens[b]) if seq_lens is not None else pos + 1
        slot = int(slot_mapping[b]) if slot_mapping is not None else kv.slot(b, S - 1)
        x = w.embed[int(ids[b])].view(1, 1, geom.hidden)
        per_layer = []
        for li in range(geom.layers):
            past_k, past_v = kv.gather(li, b, S - 1, geom.head_dim)
            st = {} if li == stages_layer else None
            x, k_new, v_new = decoder_layer(geom, w.layers[li], x, pos, cos_sin, past_k, past_v, st)
            if st is not None:
                stages[b] = st
            kv.write(li, slot, k_new, v_new)
            per_layer.append(x.view(geom.hidden))
        hf = rms_norm(x, w.final_norm, geom.eps).view(1, geom.hidden)
        hidden.append(hf[0])
        if want_logits:
            lg = F.linear(hf, w.embed)
            logits.append(lg[0])
            out_ids.append(int(torch.argmax(lg[0], dim=-1)))
        if layer_outputs:
            louts.append(torch.stack(per_layer))
    res = {"hidden": torch.stack(hidden)}
    if want_logits:
        res["logits"] = torch.stack(logits)
        res["ids"] = torch.tensor(out_ids, dtype=torch.int64)
    if layer_outputs:
        res["layer_outputs"] = torch.stack(louts, dim=1)
    if stages:
        res["stages"] = stages
    return res


@torch.no_grad()
def prefill(w: Weights, prompt: torch.Tensor, kv: PagedKV, cos_sin: torch.Tensor, b: int = 0,
            start: int = 0) -> None:
    """Fill sequence b's cache for prompt tokens by running the decode step one token at a time
    (slow; for small prompts in tests).  prefill_batched is HF's own prompt pass."""
    for i, tok in enumerate(prompt.tolist()):
        p = start + i
        one = Weights(w.geom, w.embed, w.final_norm, w.layers)
        x = one.embed[int(tok)].view(1, 1, w.geom.hidden)
        slot = kv.slot(b, p)
        for li in range(w.geom.layers):
            past_k, past_v = kv.gather(li, b, p, w.geom.head_dim)
            x, k_new, v_new = decoder_layer(w.geom, w.layers[li], x, p, cos_sin, past_k, past_v)
            kv.write(li, slot, k_new, v_new)


@torch.no_grad()
def prefill_batched(w: Weights, prompt: torch.Tensor, kv: PagedKV, cos_sin: torch.Tensor, b: int = 0) -> dict:
    """HF's prompt pass (LlamaModel.forward over all prompt tokens at once, modeling_llama.py:367-414,
    with the eager attention of :191-214 under the 4-D float causal mask that
    transformers/masking_utils.py:538-604 builds for eager attention: 0 where a position is visible,
    the dtype's minimum elsewhere, added to the scaled scores), writing sequence b's K/V for positions
    0..P-1 into `kv`.  The same batched ops as HF, so on the CPU the cache and the last position's
    logits are HF's bit for bit (pinned by tests/golden fixtures).  Returns the final-normed hidden
    state [H] and the logits [V] of the last prompt position and their argmax (LlamaForCausalLM
    computes the LM head over every position, :479-480, and the greedy pick reads the last row)."""
    geom = w.geom
    H, D, NH, KVH, I = geom.hidden, geom.head_dim, geom.heads, geom.kv_heads, geom.inter
    P = int(prompt.numel())
    x = w.embed[prompt.view(-1).long()].view(1, P, H)
    cos, sin = full_cos_sin(cos_sin[:P])
    cos, sin = cos.view(1, 1, P, D), sin.view(1, 1, P, D)
    visible = torch.ones(P, P, dtype=torch.bool).tril()
    mask = torch.where(visible, torch.tensor(0.0, dtype=BF16), torch.finfo(BF16).min).view(1, 1, P, P)
    slots = [kv.slot(b, p) for p in range(P)]
    blocks = torch.tensor([s // kv.block_size for s in slots])
    offs = torch.tensor([s % kv.block_size for s in slots])
    for li, (norm1, qkv, o_w, norm2, gate_up, down) in enumerate(w.layers):
        residual = x
        h = rms_norm(x, norm1, geom.eps)
        q = F.linear(h, qkv[:H]).view(1, P, NH, D).transpose(1, 2)
        k = F.linear(h, qkv[H:H + KVH * D]).view(1, P, KVH, D).transpose(1, 2)
        v = F.linear(h, qkv[H + KVH * D:]).view(1, P, KVH, D).transpose(1, 2)
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        key_states, value_states = repeat_kv(k, NH // KVH), repeat_kv(v, NH // KVH)
        scores = torch.matmul(q, key_states.transpose(2, 3)) * D ** -0.5
        scores = scores + mask
        probs = F.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
        attn = torch.matmul(probs, value_states).transpose(1, 2).contiguous().reshape(1, P, H).contiguous()
        x = residual + F.linear(attn, o_w)
        residual = x
        h2 = rms_norm(x, norm2, geom.eps)
        x = residual + F.linear(F.silu(F.linear(h2, gate_up[:I])) * F.linear(h2, gate_up[I:]), down)
        # K/V of every prompt position into the paged cache ([KVH, P, D] -> slot rows)
        cache = kv.caches[li]
        cache[blocks, :, offs, :D] = k[0].transpose(0, 1)
        cache[blocks, :, offs, D:] = v[0].transpose(0, 1)
    hf = rms_norm(x, w.final_norm, geom.eps)
    logits = F.linear(hf, w.embed)[0, -1]
    return {"hidden": hf[0, -1], "logits": logits, "id": int(torch.argmax(logits, dim=-1))}


def ordered_bf16(t: torch.Tensor) -> torch.Tensor:
    """Monotone integer map of bf16 bit patterns, for ULP distances
    (research/.../r34-packed-full/bench_r30_r34.py:71-74)."""
    bits = t.to(BF16).contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    return torch.where((bits & 0x8000) != 0, 0xFFFF - bits, bits | 0x8000)


def max_ulp(a: torch.Tensor, b: torch.Tensor) -> int:
    return int((ordered_bf16(a) - ordered_bf16(b)).abs().max().item())
