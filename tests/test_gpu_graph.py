"""The decode step under HIP graph capture (the reference's steady-state contract,
validation-summary.json:186-205): after one eager call, the step is captured into a graph and replayed with new inputs written in place; every replay must equal
the eager step on the same inputs bit for bit.  Eager work and synchronisations run between the
replays."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _setup(batch, ctxs, seed=7, layers=4):
    import prime_kernels_amd as pk
    from prime_kernels_amd import workload as WL

    mod = pk.load("decode_megakernel_360m")
    model = mod.MODEL
    dev = torch.device("cuda:0")
    embed, final_norm, lw = WL.random_weights(model, seed, dev, layers=layers)
    cap = max(ctxs) + 64
    kv = WL.PagedKV(model, batch, cap, layers=layers, device=dev, seed=seed + 1, fill="randn")
    cos_sin = WL.rope_table(cap, device=dev)
    st = dict(
        input_ids=torch.zeros(batch, dtype=torch.int64, device=dev),
        positions=torch.zeros(batch, dtype=torch.int64, device=dev),
        seq_lens=torch.zeros(batch, dtype=torch.int32, device=dev),
        slot_mapping=torch.zeros(batch, dtype=torch.int64, device=dev),
    )
    logits = torch.empty((batch, 49152), dtype=torch.bfloat16, device=dev)
    kw = dict(st, block_table=kv.block_table, embed=embed, layers=lw, final_norm=final_norm, kv_caches=kv.caches,
              cos_sin_cache=cos_sin, eps=1e-5, num_layers=layers, return_token_ids=True, logits_out=logits)
    return mod, kv, st, logits, kw


def _fill(kv, st, ids, positions):
    dev = st["input_ids"].device
    st["input_ids"].copy_(torch.tensor(ids, device=dev))
    st["positions"].copy_(torch.tensor(positions, device=dev))
    st["seq_lens"].copy_(torch.tensor([p + 1 for p in positions], dtype=torch.int32, device=dev))
    st["slot_mapping"].copy_(torch.tensor([kv.slot(b, p) for b, p in enumerate(positions)], device=dev))


@pytest.mark.parametrize("launch", ["ordinary", "cooperative"])
@pytest.mark.parametrize("batch", [1, 2, 3])
def test_decode_step_replays_from_a_graph(batch, launch):
    """Also with the kernels launched cooperatively (PK_OPT_COOPERATIVE), the captured launch
    replaying the eager step bit for bit."""
    _need_gpu()
    from prime_kernels_amd import _native

    lib = _native.library()
    old = lib.pk_set_option(_native.PK_OPT_COOPERATIVE, 1 if launch == "cooperative" else 0)
    try:
        _replay_check(batch)
    finally:
        lib.pk_set_option(_native.PK_OPT_COOPERATIVE, old)


def _replay_check(batch):
    ctxs = [300 + 97 * b for b in range(batch)]
    mod, kv, st, logits, kw = _setup(batch, ctxs)
    kv0 = [c.clone() for c in kv.caches]
    _fill(kv, st, [5] * batch, ctxs)
    mod.decode_step(**kw)                       # first use of the device: outside capture
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        hid_g, ids_g = mod.decode_step(**kw)
    torch.cuda.synchronize()

    for step in range(4):
        ids = [11 * step + 3 + b for b in range(batch)]
        pos = [c + step for c in ctxs]
        # eager reference on a fresh copy of the caches
        for c, c0 in zip(kv.caches, kv0):
            c.copy_(c0)
        _fill(kv, st, ids, pos)
        he, ie = mod.decode_step(**kw)
        he, ie, le = he.clone(), ie.clone(), logits.clone()
        kv_e = [c.clone() for c in kv.caches]
        torch.cuda.synchronize()
        # replay with the same inputs written in place
        for c, c0 in zip(kv.caches, kv0):
            c.copy_(c0)
        _fill(kv, st, ids, pos)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(hid_g.view(torch.int16), he.view(torch.int16)), step
        assert torch.equal(ids_g, ie) and torch.equal(logits.view(torch.int16), le.view(torch.int16)), step
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(kv.caches, kv_e)), step
        _ = (torch.randn(1024, device=hid_g.device) * 2).sum().item()   # unrelated eager work between replays
    assert mod.workspace(hid_g.device).pending_failure() == (0, 0)


def test_one_graph_serves_every_context_range():
    """The kernel choice is made on the device from the context length: one graph captured with a block
    table that reaches 9,800 tokens replays steps at contexts in the split-role kernel's narrow range,
    its wide range and the general kernel's, each bit-identical to the eager step on the same inputs."""
    _need_gpu()
    ranges = [1000, 3000, 9800]
    mod, kv, st, logits, kw = _setup(1, [max(ranges)], layers=2)
    kv0 = [c.clone() for c in kv.caches]
    _fill(kv, st, [5], [ranges[0]])
    mod.decode_step(**kw)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        hid_g, ids_g = mod.decode_step(**kw)
    torch.cuda.synchronize()
    for step, ctx in enumerate(ranges):
        for c, c0 in zip(kv.caches, kv0):
            c.copy_(c0)
        _fill(kv, st, [7 + step], [ctx])
        he, ie = mod.decode_step(**kw)
        he, ie, le = he.clone(), ie.clone(), logits.clone()
        kv_e = [c.clone() for c in kv.caches]
        torch.cuda.synchronize()
        for c, c0 in zip(kv.caches, kv0):
            c.copy_(c0)
        _fill(kv, st, [7 + step], [ctx])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert not torch.isnan(he.float()).any(), ctx
        assert torch.equal(hid_g.view(torch.int16), he.view(torch.int16)), ctx
        assert torch.equal(ids_g, ie) and torch.equal(logits.view(torch.int16), le.view(torch.int16)), ctx
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(kv.caches, kv_e)), ctx
    assert mod.workspace(hid_g.device).pending_failure() == (0, 0)
