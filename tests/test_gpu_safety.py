"""Failure handling and exchange-tag safety of the decode kernels on MI355X.

* A step whose bounded waits give up (forced from the host with pk_test_abort_next, so every wait
  gives up at its first check and every kernel still ends normally) returns NaN hidden state and
  logits and token ids -1, is reported by pk_state_status, makes the next call raise RuntimeError
  (PK_ERR_ABORTED), and leaves the following steps correct.
* Exchange words carry the full 32-bit step epoch: steps that alternate batch sizes (so some words
  are not rewritten every step) give the same bits across the epoch's 32-bit wrap and across jumps
  of 65,536 and 65,535 epochs, where a 16-bit tag (with or without a skipped zero) would accept a
  stale word as current.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _setup(batch_max, contexts, layers=2, seed=5):
    import prime_kernels_amd as pk
    from prime_kernels_amd import workload as WL

    mod = pk.load("decode_megakernel_360m")
    model = mod.MODEL
    dev = torch.device("cuda:0")
    embed, final_norm, lw = WL.random_weights(model, seed, dev, layers=layers)
    cap = max(contexts) + 64
    kv = WL.PagedKV(model, batch_max, cap, layers=layers, device=dev, seed=seed + 1, fill="randn")
    cos_sin = WL.rope_table(cap + 64, device=dev)
    return mod, model, embed, final_norm, lw, kv, cos_sin


def _step(mod, embed, final_norm, lw, kv, cos_sin, ids, positions):
    dev = embed.device
    B = len(ids)
    logits = torch.empty((B, 49152), dtype=BF16, device=dev)
    hid, out_ids = mod.decode_step(
        input_ids=torch.tensor(ids, device=dev), positions=torch.tensor(positions, device=dev),
        seq_lens=torch.tensor([p + 1 for p in positions], dtype=torch.int32, device=dev),
        block_table=kv.block_table[:B].contiguous(),
        slot_mapping=torch.tensor([kv.slot(b, p) for b, p in enumerate(positions)], device=dev),
        embed=embed, layers=lw, final_norm=final_norm, kv_caches=kv.caches, cos_sin_cache=cos_sin, eps=1e-5,
        num_layers=len(lw), return_token_ids=True, logits_out=logits)
    return hid.clone(), out_ids.clone(), logits


@pytest.mark.parametrize("path", ["split_role", "general", "batched"])
def test_abandoned_wait_poisons_outputs_and_is_reported(path):
    _need_gpu()
    from prime_kernels_amd import _native

    lib = _native.library()
    batch = 3 if path == "batched" else 1
    contexts = [300 + 41 * b for b in range(batch)]
    mod, model, embed, final_norm, lw, kv, cos_sin = _setup(batch, contexts)
    rt = mod.workspace(embed.device)
    stream = torch.cuda.current_stream().cuda_stream
    old = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, 0 if path == "general" else 1)
    try:
        kv0 = [c.clone() for c in kv.caches]
        ids = [100 + b for b in range(batch)]

        def restore():
            for c, c0 in zip(kv.caches, kv0):
                c.copy_(c0)

        restore()
        h_ok, i_ok, lg = _step(mod, embed, final_norm, lw, kv, cos_sin, ids, contexts)
        lg_ok = lg.clone()
        torch.cuda.synchronize()
        assert rt.pending_failure() == (0, 0)
        # the next step is marked failed: every bounded wait gives up at its first check
        restore()
        assert lib.pk_test_abort_next(stream) == 0
        h_bad, i_bad, lg_bad = _step(mod, embed, final_norm, lw, kv, cos_sin, ids, contexts)
        torch.cuda.synchronize()
        assert torch.isnan(h_bad.float()).all(), "hidden state not poisoned"
        assert (i_bad == -1).all(), i_bad
        assert torch.isnan(lg_bad.float()).all(), "logits not poisoned"
        epoch, site = rt.pending_failure()
        assert epoch != 0, "no failure report"
        # the next call reports it (and launches nothing)
        with pytest.raises(RuntimeError, match="gave_up_a_bounded_wait"):
            _step(mod, embed, final_norm, lw, kv, cos_sin, ids, contexts)
        assert rt.pending_failure() == (0, 0)
        # and the step after that is correct again
        restore()
        h2, i2, lg2 = _step(mod, embed, final_norm, lw, kv, cos_sin, ids, contexts)
        torch.cuda.synchronize()
        assert torch.equal(h2.view(torch.int16), h_ok.view(torch.int16))
        assert torch.equal(i2, i_ok) and torch.equal(lg2.view(torch.int16), lg_ok.view(torch.int16))
        assert rt.pending_failure() == (0, 0)
    finally:
        lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old)


def test_epoch_wrap_and_16_bit_jumps_with_alternating_batches():
    """A fixed sequence of steps alternating batch 16 (ragged) and batch 1 runs three times on the
    same inputs: from epoch 1000; across the 32-bit wrap; and with the epoch moved forward so that
    every batch-16 step runs 65,536 or 65,535 epochs after the previous one (the slots of sequences
    1..15 are not rewritten by the batch-1 steps in between).  All three give the same bits."""
    _need_gpu()
    from prime_kernels_amd import _native

    lib = _native.library()
    contexts = [40 + 37 * b for b in range(16)]
    mod, model, embed, final_norm, lw, kv, cos_sin = _setup(16, contexts)
    rt = mod.workspace(embed.device)
    stream = torch.cuda.current_stream().cuda_stream
    kv0 = [c.clone() for c in kv.caches]
    plan = [16, 1, 1, 16, 1, 16, 16, 1, 16]

    def run(mode):
        for c, c0 in zip(kv.caches, kv0):
            c.copy_(c0)
        torch.cuda.synchronize()
        assert lib.pk_test_set_epoch(stream, 1000 if mode == "plain" else 0xFFFFFFFF - 4) == 0
        pos = list(contexts)
        outs = []
        last16 = None
        jumps = [65536, 65535, 65536, 65535]
        for k, B in enumerate(plan):
            if mode == "jump" and B == 16 and last16 is not None:
                # the step epoch is the stored one + 1: make it last16 + jump
                assert lib.pk_test_set_epoch(stream, (last16 + jumps.pop(0) - 1) & 0xFFFFFFFF) == 0
            ids = [(7 * k + 3 * b) % 49152 for b in range(B)]
            h, i, lg = _step(mod, embed, final_norm, lw, kv, cos_sin, ids, pos[:B])
            outs.append((h, i, lg.clone()))
            if B == 16:
                last16 = rt.header(1)[0]
            for b in range(B):
                pos[b] += 1
        torch.cuda.synchronize()
        assert rt.pending_failure() == (0, 0), mode
        return outs, [c.clone() for c in kv.caches]

    ref, kv_ref = run("plain")
    for mode in ("wrap", "jump"):
        got, kv_got = run(mode)
        for k, ((h0, i0, l0), (h1, i1, l1)) in enumerate(zip(ref, got)):
            assert torch.equal(h0.view(torch.int16), h1.view(torch.int16)), (mode, k)
            assert torch.equal(i0, i1) and torch.equal(l0.view(torch.int16), l1.view(torch.int16)), (mode, k)
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(kv_ref, kv_got)), mode
