"""Pin the CPU oracle (oracle/smollm2.py) against HF transformers golden vectors and against
what the mathematics fixes.  CPU only."""

import json

import numpy as np
import pytest
import torch

from oracle import smollm2 as O

BF16 = torch.bfloat16


def from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.astype(np.uint16).view(np.int16).copy()).view(BF16)


@pytest.fixture(scope="module")
def meta(golden_dir):
    return json.loads((golden_dir / "golden.json").read_text())


def _geom(d: dict) -> O.Geometry:
    return O.Geometry(**d)


def _run_greedy(meta, golden_dir, key):
    fx = meta["fixtures"][key]
    geom = _geom(fx["geometry"])
    w = O.make_weights(geom, fx["seed"], norm_jitter=fx["norm_jitter"])
    fp = w.fingerprint()
    assert fp == fx["weights_sha256"], "seeded weight generator drifted"
    g = np.load(golden_dir / f"{key}_greedy.npz")
    P, steps = fx["prompt_len"], fx["steps"]
    kv = O.make_paged_kv(geom, 1, P + steps + 3, seed=None)
    pk, pv = from_bits(g["prefill_k"]), from_bits(g["prefill_v"])  # [L, KVH, P, D]
    for li in range(geom.layers):
        for p in range(P):
            kv.write(li, kv.slot(0, p), pk[li, :, p], pv[li, :, p])
    cos_sin = O.rope_cos_sin(P + steps + 8, geom.head_dim, geom.theta)
    ids = g["ids"]
    full_i = 0
    for step in range(steps):
        pos = P + step
        res = O.decode_step(w, [int(ids[step])], [pos], kv, cos_sin)
        assert torch.equal(res["hidden"][0], from_bits(g["hidden"][step])), f"hidden step {step}"
        top_v = from_bits(g["top_v"][step])
        top_i = torch.from_numpy(g["top_i"][step].astype(np.int64))
        assert torch.equal(res["logits"][0][top_i], top_v), f"top-32 logits step {step}"
        if step in fx["full_logit_steps"]:
            assert torch.equal(res["logits"][0], from_bits(g["full_logits"][full_i]))
            full_i += 1
        assert int(res["ids"][0]) == int(ids[step + 1]), f"greedy id step {step}"
        slot = kv.slot(0, pos)
        blk, off = slot // 16, slot % 16
        for li in range(geom.layers):
            cache = kv.caches[li][blk, :, off]
            assert torch.equal(cache[:, :geom.head_dim], from_bits(g["step_k"][step][li]))
            assert torch.equal(cache[:, geom.head_dim:], from_bits(g["step_v"][step][li]))


def test_greedy_360m_matches_hf(meta, golden_dir):
    _run_greedy(meta, golden_dir, "smollm2_360m")


def test_greedy_135m_matches_hf(meta, golden_dir):
    _run_greedy(meta, golden_dir, "smollm2_135m")


def full_depth_prefill(meta, golden_dir, key):
    """Weights and the oracle's batched prompt pass of a full-depth HF fixture (BASELINE config 2 or
    3): (fixture meta, geometry, weights, paged cache, rope table, prompt-pass result, fixture
    arrays)."""
    fx = meta["fixtures"][key]
    geom = _geom(fx["geometry"])
    w = O.make_weights(geom, fx["seed"], norm_jitter=fx["norm_jitter"])
    assert w.fingerprint() == fx["weights_sha256"], "seeded weight generator drifted"
    g = np.load(golden_dir / f"{key}_full.npz")
    P, steps = fx["prompt_len"], fx["steps"]
    kv = O.make_paged_kv(geom, 1, P + steps + 16, seed=None)
    cos_sin = O.rope_cos_sin(P + steps + 16, geom.head_dim, geom.theta)
    pre = O.prefill_batched(w, torch.from_numpy(g["prompt"].astype(np.int64)), kv, cos_sin)
    return fx, geom, w, kv, cos_sin, pre, g


@pytest.mark.parametrize("key", ["config2_135m", "config3_360m"])
def test_full_depth_stream_matches_hf(meta, golden_dir, key):
    """BASELINE configs 2 and 3 at full depth against HF transformers 5.15.0 (tests/golden
    config*_full.npz): the oracle's prompt pass gives HF's cache (SHA-256 of every layer's K and V)
    and prompt logits, then 256 free-running greedy steps give HF's ids, its top-32 logits at every
    step, its hidden state at steps 0..7 and 255 and its full logits at steps 0 and 255, bit for bit.
    Run with the thread count the fixtures were written with (CPU GEMM blocking may depend on it)."""
    threads = torch.get_num_threads()
    torch.set_num_threads(meta.get("torch_threads", threads))
    try:
        fx, geom, w, kv, cos_sin, pre, g = full_depth_prefill(meta, golden_dir, key)
        P, steps = fx["prompt_len"], fx["steps"]
        for li in range(geom.layers):
            k, v = kv.gather(li, 0, P, geom.head_dim)
            assert O.sha256_tensor(k[0]) == fx["prefill_kv_sha256"][f"layers.{li}.k"], f"prompt K layer {li}"
            assert O.sha256_tensor(v[0]) == fx["prefill_kv_sha256"][f"layers.{li}.v"], f"prompt V layer {li}"
        pi = torch.from_numpy(g["prefill_top_i"].astype(np.int64))
        assert torch.equal(pre["logits"][pi], from_bits(g["prefill_top_v"]))
        ids = g["ids"]
        assert pre["id"] == int(ids[0])
        hidden_i, full_i = 0, 0
        for step in range(steps):
            res = O.decode_step(w, [int(ids[step])], [P + step], kv, cos_sin)
            top_i = torch.from_numpy(g["top_i"][step].astype(np.int64))
            assert torch.equal(res["logits"][0][top_i], from_bits(g["top_v"][step])), f"top-32 logits step {step}"
            if step in fx["hidden_steps"]:
                assert torch.equal(res["hidden"][0], from_bits(g["hidden"][hidden_i])), f"hidden step {step}"
                hidden_i += 1
            if step in fx["full_logit_steps"]:
                assert torch.equal(res["logits"][0], from_bits(g["full_logits"][full_i])), f"logits step {step}"
                full_i += 1
            assert int(res["ids"][0]) == int(ids[step + 1]), f"greedy id step {step}"
    finally:
        torch.set_num_threads(threads)


def test_block360_stages_match_hf(meta, golden_dir):
    fx = meta["fixtures"]["block360"]
    geom = _geom(fx["geometry"])
    w = O.make_weights(geom, fx["seed"], norm_jitter=fx["norm_jitter"])
    assert w.fingerprint() == fx["weights_sha256"]
    g = np.load(golden_dir / "block360_stages.npz")
    ctx = fx["context"]
    cos_sin = O.rope_cos_sin(ctx + 1, geom.head_dim, geom.theta)
    c, s = O.full_cos_sin(cos_sin[ctx])
    assert torch.equal(c, from_bits(g["cos"])) and torch.equal(s, from_bits(g["sin"]))
    x = from_bits(g["x"]).view(1, 1, -1)
    pk = from_bits(g["past_k"]).unsqueeze(0)
    pv = from_bits(g["past_v"]).unsqueeze(0)
    st = {}
    out, k_new, v_new = O.decoder_layer(geom, w.layers[0], x, ctx, cos_sin, pk, pv, st)
    H, KVD = geom.hidden, geom.kv_heads * geom.head_dim
    assert torch.equal(st["norm1"].flatten(), from_bits(g["norm1"]))
    assert torch.equal(k_new.flatten(), from_bits(g["k_rot"]).flatten())
    assert torch.equal(v_new.flatten(), from_bits(g["v_new"]).flatten())
    assert torch.equal(st["attn"].flatten(), from_bits(g["attn"]))
    for name in ("o", "norm2", "h1", "gate", "up", "silu", "act", "down"):
        assert torch.equal(st[name].flatten(), from_bits(g[name])), name
    assert torch.equal(out.flatten(), from_bits(g["out"]))


# ---- what the mathematics fixes (independent of HF) --------------------------------------------

def test_rms_norm_constant_row_and_scale_invariance():
    # a constant row c with unit weight normalises to sign(c) (up to eps), exactly 1.0 in bf16
    for c in (0.5, -3.0, 17.0):
        x = torch.full((1, 960), c, dtype=BF16)
        y = O.rms_norm(x, torch.ones(960, dtype=BF16), 1e-5)
        assert torch.all(y == torch.tensor(1.0 if c > 0 else -1.0, dtype=BF16))
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 960, generator=g).to(BF16)
    w = (1 + 0.1 * torch.randn(960, generator=g)).to(BF16)
    # scaling by a power of two is exact in bf16 and leaves the normalised value unchanged (eps aside)
    y1 = O.rms_norm(x * 64, w, 0.0)
    y2 = O.rms_norm(x, w, 0.0)
    assert torch.equal(y1, y2)
    # fp64 closed form
    xf = x.double()
    ref = (xf / torch.sqrt((xf ** 2).mean() + 1e-5)).to(BF16).double() * w.double()
    assert torch.allclose(O.rms_norm(x, w, 1e-5).double(), ref, rtol=2 ** -7, atol=0)


def test_rope_table_and_rotation_properties():
    cs = O.rope_cos_sin(4096, 64, 1e5)
    assert cs.shape == (4096, 64) and cs.dtype == BF16
    # position 0: cos = 1, sin = 0 -> identity
    assert torch.all(cs[0, :32] == 1) and torch.all(cs[0, 32:] == 0)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 15, 1, 64, generator=g).to(BF16)
    c, s = O.full_cos_sin(cs[0].view(1, 1, 64))
    assert torch.equal(O.apply_rope(q, c.unsqueeze(1), s.unsqueeze(1)), q)
    # closed form in fp64: angle = pos / theta^(2i/64)
    pos = torch.tensor([1.0, 77.0, 4095.0], dtype=torch.float64)
    inv = 1.0 / (1e5 ** (torch.arange(0, 64, 2, dtype=torch.float64) / 64))
    ang = pos[:, None] * inv[None, :]
    assert torch.allclose(cs[[1, 77, 4095], :32].double(), torch.cos(ang), atol=2 ** -8)
    assert torch.allclose(cs[[1, 77, 4095], 32:].double(), torch.sin(ang), atol=2 ** -8)
    # rotation preserves the pairwise norm up to bf16 rounding
    c, s = O.full_cos_sin(cs[77].view(1, 1, 64))
    r = O.apply_rope(q, c.unsqueeze(1), s.unsqueeze(1)).double()
    qd = q.double()
    n0 = qd[..., :32] ** 2 + qd[..., 32:] ** 2
    n1 = r[..., :32] ** 2 + r[..., 32:] ** 2
    assert torch.allclose(n0, n1, rtol=2e-2, atol=1e-2)


def test_attention_special_cases():
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 15, 1, 64, generator=g).to(BF16)
    v = torch.randn(1, 5, 1, 64, generator=g).to(BF16)
    k = torch.randn(1, 5, 1, 64, generator=g).to(BF16)
    # S = 1: probability 1, output equals v of the kv head of each q head (GQA group of 3)
    out, _ = O.eager_attention(q, k, v, 3, 0.125)
    out = out.view(15, 64)
    for h in range(15):
        assert torch.equal(out[h], v[0, h // 3, 0])
    # identical keys: uniform weights -> mean of V (fp64 closed form within bf16 rounding)
    S = 8
    kk = k.expand(1, 5, S, 64).contiguous()
    vv = torch.randn(1, 5, S, 64, generator=g).to(BF16)
    out, probs = O.eager_attention(q, kk, vv, 3, 0.125)
    assert torch.all(probs == torch.tensor(1.0 / S, dtype=BF16))
    mean = vv.double().mean(dim=2)
    for h in range(15):
        assert torch.allclose(out.view(15, 64)[h].double(), mean[0, h // 3], atol=2 ** -7, rtol=2 ** -7)


def test_argmax_first_index_on_ties():
    x = torch.tensor([0.5, 2.0, 2.0, 1.0], dtype=BF16)
    assert int(torch.argmax(x)) == 1


def test_paged_kv_round_trip():
    geom = O.with_layers(O.SMOLLM2_360M, 1)
    kv = O.make_paged_kv(geom, 2, 40, seed=None)
    g = torch.Generator().manual_seed(1)
    ks = torch.randn(40, 5, 64, generator=g).to(BF16)
    vs = torch.randn(40, 5, 64, generator=g).to(BF16)
    for p in range(40):
        kv.write(0, kv.slot(1, p), ks[p], vs[p])
    k, v = kv.gather(0, 1, 40, 64)
    assert torch.equal(k[0].permute(1, 0, 2), ks) and torch.equal(v[0].permute(1, 0, 2), vs)
    kv.write(0, -1, ks[0] * 0, vs[0] * 0)  # slot -1 skips
    k2, _ = kv.gather(0, 1, 40, 64)
    assert torch.equal(k2, k)


def test_planted_mistake_is_caught(meta, golden_dir):
    """A plausible oracle slip (RoPE sign flipped on the second half) must break the pin."""
    fx = meta["fixtures"]["block360"]
    geom = _geom(fx["geometry"])
    w = O.make_weights(geom, fx["seed"], norm_jitter=fx["norm_jitter"])
    g = np.load(golden_dir / "block360_stages.npz")
    ctx = fx["context"]
    cos_sin = O.rope_cos_sin(ctx + 1, geom.head_dim, geom.theta)
    x = from_bits(g["x"]).view(1, 1, -1)
    pk, pv = from_bits(g["past_k"]).unsqueeze(0), from_bits(g["past_v"]).unsqueeze(0)
    orig = O.rotate_half
    try:
        O.rotate_half = lambda t: torch.cat((t[..., 32:], -t[..., :32]), dim=-1)
        out, k_new, _ = O.decoder_layer(geom, w.layers[0], x, ctx, cos_sin, pk, pv)
    finally:
        O.rotate_half = orig
    assert not torch.equal(k_new.flatten(), from_bits(g["k_rot"]).flatten())
    assert not torch.equal(out.flatten(), from_bits(g["out"]))
