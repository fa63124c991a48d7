"""Synthetic decode workloads on the GPU: seeded random-init weights, paged KV caches in the
vLLM FLASH_ATTN layout, block tables and the rotary table.  Used by bench.py and the tests.

Weights follow HF's Llama random init (Linear/Embedding ~ N(0, 0.02) in bf16, RMSNorm weight 1;
transformers/modeling_utils.py:2391-2420).  The rotary table is HF's fp32 cos/sin cast to bf16
(transformers/models/llama/modeling_llama.py:93-127) in vLLM's [max_pos, 64] cos|sin layout.
"""

from __future__ import annotations

import torch

BF16 = torch.bfloat16


def rope_table(max_pos: int, head_dim: int = 64, theta: float = 100000.0, device="cpu") -> torch.Tensor:
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float) / head_dim))
    pos = torch.arange(max_pos, dtype=torch.int64)
    freqs = (inv_freq[None, :, None].float() @ pos[None, None, :].float()).transpose(1, 2)[0]
    return torch.cat((freqs.cos().to(BF16), freqs.sin().to(BF16)), dim=-1).contiguous().to(device)


def random_weights(model, seed: int, device, layers: int | None = None, std: float = 0.02):
    """(embed, final_norm, [layer tuples]) drawn on `device` (fast; not bit-identical to CPU draws)."""
    n = model.layers if layers is None else layers
    g = torch.Generator(device=device).manual_seed(seed)

    def normal(shape):
        return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).to(BF16)

    embed = normal((49152, model.hidden))
    final_norm = torch.ones(model.hidden, dtype=BF16, device=device)
    out = []
    for _ in range(n):
        sh = model.shapes()
        out.append((torch.ones(sh[0], dtype=BF16, device=device), normal(sh[1]), normal(sh[2]),
                    torch.ones(sh[3], dtype=BF16, device=device), normal(sh[4]), normal(sh[5])))
    return embed, final_norm, out


class PagedKV:
    """Per-layer caches [blocks, kv_heads, 16, 2*D] bf16 and a block table [B, W] int32."""

    def __init__(self, model, batch: int, capacity: int, layers: int | None = None, device="cuda",
                 seed: int = 0, fill: str = "zeros"):
        n = model.layers if layers is None else layers
        width = (capacity + 15) // 16
        nblocks = batch * width
        g = torch.Generator().manual_seed(seed)
        perm = torch.randperm(nblocks, generator=g)
        self.block_table = perm.reshape(batch, width).to(torch.int32).to(device)
        shape = (nblocks, model.kv_heads, 16, 2 * model.head_dim)
        if fill == "zeros":
            self.caches = [torch.zeros(shape, dtype=BF16, device=device) for _ in range(n)]
        else:
            gd = torch.Generator(device=device).manual_seed(seed + 1)
            self.caches = [torch.randn(shape, generator=gd, device=device).to(BF16) for _ in range(n)]
        self.capacity = width * 16

    def slot(self, b: int, pos: int) -> int:
        return int(self.block_table[b, pos // 16]) * 16 + pos % 16

    def bytes(self) -> int:
        return sum(c.numel() * 2 for c in self.caches)
