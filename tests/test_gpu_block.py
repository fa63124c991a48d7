"""GPU checks of the research single-block ABI `block360_decode` (hidden states in, block output out):
the BASELINE config-1 block against the HF golden stages (output, debug stages, KV append), two
sequences against the oracle's decoder layer, and agreement with the 1-layer decode path."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import smollm2 as O
from tests import gpu_cases as GC

pytestmark = pytest.mark.gpu
BLK_STAGES = [("norm1", 960), ("qkv", 1600), ("attn", 960), ("h1", 960), ("norm2", 960), ("act", 2560), ("out", 960)]


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _bits(a) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a, dtype=np.uint16).view(np.int16).copy()).view(torch.bfloat16)


def _block(hidden, positions, seq_lens, kv: O.PagedKV, layer_w, cos_sin, *, debug=False):
    """Run block360_decode on GPU copies; returns (out [B, 960], debug stages or None, GPU cache)."""
    import prime_kernels_amd as pk
    from prime_kernels_amd import _native

    pk.load("decode_megakernel_360m")
    lib = _native.library()
    dev = torch.device("cuda:0")
    B = hidden.shape[0]
    hid = hidden.to(dev, torch.bfloat16).contiguous()
    lw = [t.to(dev).contiguous() for t in layer_w]
    table = torch.tensor([t.data_ptr() for t in lw], dtype=torch.int64, device=dev)
    cache = kv.caches[0].to(dev)
    bt = kv.block_table.to(dev)
    cs = cos_sin.to(dev)
    slots = torch.tensor([kv.slot(b, int(positions[b])) for b in range(B)], device=dev)
    # named, so that the allocator cannot hand one tensor's memory to the next before the kernel ran
    pos_t = torch.tensor(positions, dtype=torch.int64, device=dev)
    sl_t = torch.tensor(seq_lens, dtype=torch.int32, device=dev)
    out = torch.empty((B, 960), dtype=torch.bfloat16, device=dev)
    scratch = torch.empty(lib.block360_workspace_bytes(), dtype=torch.uint8, device=dev)
    dbg = torch.full((lib.block360_debug_bytes(),), 0xFF, dtype=torch.uint8, device=dev) if debug else None
    rc = lib.block360_decode(
        torch.cuda.current_stream().cuda_stream, B, hid.data_ptr(), pos_t.data_ptr(), sl_t.data_ptr(),
        bt.data_ptr(), bt.stride(0),
        slots.data_ptr(), table.data_ptr(), cache.data_ptr(), 0, 64, cache.stride(0), cache.stride(2),
        cache.stride(1), 16, cs.data_ptr(), 0, out.data_ptr(), scratch.data_ptr(), scratch.numel(),
        dbg.data_ptr() if debug else None, dbg.numel() if debug else 0, bt.shape[1] * 16)
    assert rc == 0, _native.status_string(rc)
    torch.cuda.synchronize()
    stages = None
    if debug:
        v = dbg.view(torch.bfloat16).cpu()
        stages, off = {}, 0
        for name, n in BLK_STAGES:
            stages[name] = v[off:off + 4 * n].view(4, n)
            off += 4 * n
    return out.cpu(), stages, cache.cpu()


def _close(got, want, label, min_identical=0.9):
    got, want = got.float().flatten(), want.float().flatten()
    frac = GC.identical_fraction(got, want)
    err = (got - want).abs()
    tol = 2 ** -6 * want.abs() + 2e-3 * want.abs().max().clamp(min=1e-6)
    assert frac >= min_identical and bool((err <= tol).all()), (label, frac, err.max().item())
    return frac


def test_config1_block_against_hf_golden():
    _need_gpu()
    gdir = Path(__file__).resolve().parent / "golden"
    meta = json.loads((gdir / "golden.json").read_text())["fixtures"]["block360"]
    geom = O.Geometry(**meta["geometry"])
    w = O.make_weights(geom, meta["seed"], norm_jitter=meta["norm_jitter"])
    g = np.load(gdir / "block360_stages.npz")
    ctx = meta["context"]
    kv = O.make_paged_kv(geom, 1, ctx + 16, seed=None)
    pk_, pv_ = _bits(g["past_k"]), _bits(g["past_v"])
    for p in range(ctx):
        kv.write(0, kv.slot(0, p), pk_[:, p], pv_[:, p])
    cos_sin = O.rope_cos_sin(ctx + 16)
    out, st, cache = _block(_bits(g["x"]).view(1, 960), [ctx], [ctx + 1], kv, w.layers[0], cos_sin, debug=True)
    _close(out[0], _bits(g["out"]), "out")
    want = {"norm1": g["norm1"], "qkv": np.concatenate([g["q"], g["k"], g["v"]]), "attn": g["attn"],
            "h1": g["h1"], "norm2": g["norm2"], "act": g["act"], "out": g["out"]}
    for name, ref in want.items():
        _close(st[name][0], _bits(ref), name)
    assert torch.equal(st["out"][0].view(torch.int16), out[0].view(torch.int16))
    slot = kv.slot(0, ctx)
    got = cache[slot // 16, :, slot % 16].float()
    assert torch.allclose(got[:, :64], _bits(g["k_rot"]).float(), rtol=2 ** -6, atol=2e-2)
    assert torch.allclose(got[:, 64:], _bits(g["v_new"]).float(), rtol=2 ** -6, atol=2e-2)


@pytest.mark.parametrize("contexts", [[8, 32], [1, 129]], ids=["ctx8_32", "ctx1_129"])
def test_two_sequences_against_oracle_layer(contexts):
    """The reference's block fixtures' shapes (B = 2, short contexts): each sequence's block output
    and KV append against the oracle's decoder layer."""
    _need_gpu()
    geom = O.with_layers(O.SMOLLM2_360M, 1)
    w = O.make_weights(geom, 33, norm_jitter=0.05)
    kv = O.make_paged_kv(geom, 2, max(contexts) + 16, seed=34)
    g = torch.Generator().manual_seed(35)
    hidden = torch.randn(2, 960, generator=g).to(torch.bfloat16)
    cos_sin = O.rope_cos_sin(max(contexts) + 16)
    pos = [S - 1 for S in contexts]
    out, st, cache = _block(hidden, pos, contexts, kv, w.layers[0], cos_sin, debug=True)
    for b in range(2):
        S = contexts[b]
        past_k, past_v = kv.gather(0, b, S - 1, 64)
        stages = {}
        x, k_new, v_new = O.decoder_layer(geom, w.layers[0], hidden[b].view(1, 1, 960), pos[b], cos_sin, past_k,
                                          past_v, stages)
        _close(out[b], x.view(960), f"b{b} out", min_identical=0.8)
        _close(st["norm1"][b], stages["norm1"].view(-1), f"b{b} norm1")
        _close(st["qkv"][b], stages["qkv"].view(-1), f"b{b} qkv", min_identical=0.8)
        _close(st["act"][b], stages["act"].view(-1), f"b{b} act", min_identical=0.8)
        slot = kv.slot(b, pos[b])
        got = cache[slot // 16, :, slot % 16]
        assert torch.allclose(got[:, :64].float(), k_new.float(), rtol=2 ** -6, atol=2e-2)
        assert torch.equal(got[:, 64:].view(torch.int16), v_new.reshape(got[:, 64:].shape).view(torch.int16))


def test_block_equals_one_layer_decode_path():
    """block360_decode == the 1-layer decode step of the general kernel (the same arithmetic, so the
    same bits) with the same vector in an embedding row.  The split-role kernel, which takes this
    context by default, sums in another order; its parity is checked against the oracle."""
    _need_gpu()
    from prime_kernels_amd import _native

    geom = O.with_layers(O.SMOLLM2_360M, 1)
    case = GC.random_kv_case(geom, 41, [300])
    x = case.w.embed[123].view(1, 960)
    lib = _native.library()
    old = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, 0)
    try:
        ref = case.kernel_step([123], [299], layer_outputs=True)
    finally:
        lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old)
    case.kv.caches[0].copy_(case.kvd[0].cpu())       # the decode step appended; undo is not needed: same values
    out, _, _ = _block(x, [299], [300], case.kv, case.w.layers[0], case.cos_sin)
    assert torch.equal(out[0].view(torch.int16), ref["layer_outputs"][0, 0].view(torch.int16))


def test_block_captures_and_replays():
    """The single-block ABI under stream capture: after an eager call the same call captures and
    every replay equals the eager result bit for bit (its scratch carries nothing between calls)."""
    _need_gpu()
    import prime_kernels_amd as pk
    from prime_kernels_amd import _native

    pk.load("decode_megakernel_360m")
    lib = _native.library()
    dev = torch.device("cuda:0")
    geom = O.with_layers(O.SMOLLM2_360M, 1)
    w = O.make_weights(geom, 51, norm_jitter=0.05)
    kv = O.make_paged_kv(geom, 1, 80, seed=52)
    hid = torch.randn(1, 960, generator=torch.Generator().manual_seed(53)).to(torch.bfloat16).to(dev)
    lw = [t.to(dev).contiguous() for t in w.layers[0]]
    table = torch.tensor([t.data_ptr() for t in lw], dtype=torch.int64, device=dev)
    cache = kv.caches[0].to(dev)
    bt = kv.block_table.to(dev)
    cs = O.rope_cos_sin(80).to(dev)
    pos_t = torch.tensor([40], dtype=torch.int64, device=dev)
    sl_t = torch.tensor([41], dtype=torch.int32, device=dev)
    slots = torch.tensor([kv.slot(0, 40)], dtype=torch.int64, device=dev)
    out = torch.empty((1, 960), dtype=torch.bfloat16, device=dev)
    scratch = torch.zeros(lib.block360_workspace_bytes(), dtype=torch.uint8, device=dev)

    def call():
        return lib.block360_decode(
            torch.cuda.current_stream().cuda_stream, 1, hid.data_ptr(), pos_t.data_ptr(), sl_t.data_ptr(),
            bt.data_ptr(), bt.stride(0), slots.data_ptr(), table.data_ptr(), cache.data_ptr(), 0, 64,
            cache.stride(0), cache.stride(2), cache.stride(1), 16, cs.data_ptr(), 0, out.data_ptr(),
            scratch.data_ptr(), scratch.numel(), None, 0, bt.shape[1] * 16)

    cache0 = cache.clone()
    assert call() == 0
    torch.cuda.synchronize()
    eager = out.clone()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        assert call() == 0
    for _ in range(3):
        cache.copy_(cache0)
        out.fill_(0)
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
