"""Failure handling and exchange-tag safety of the decode kernels on MI355X.

* A step whose bounded waits give up (forced from the host with pk_test_abort_next, so every wait
  gives up at its first check and every kernel still ends normally) returns NaN hidden state and
  logits and token ids -1, is reported by pk_state_status, makes the next call (or check_failures)
  raise RuntimeError once, and leaves the following steps correct.
* Exchange units are never seen torn: a unit whose tag is current carries its own payload
  (pk_test_exchange_units, in every memory kind the kernels use).
* The cooperative launch (PK_OPT_COOPERATIVE) gives the ordinary launch's bits on every kernel.
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


@pytest.mark.parametrize("report", ["next_call", "check_failures"])
@pytest.mark.parametrize("path", ["split_role", "split_wide", "general", "batched"])
def test_abandoned_wait_poisons_outputs_and_is_reported(path, report):
    """The failed step is reported once: by the next decode call (which launches nothing), or by
    check_failures, after which the next call runs normally (split_wide: a context past the narrow
    split-role limit, which the wide layout takes)."""
    _need_gpu()
    from prime_kernels_amd import _native

    lib = _native.library()
    batch = 3 if path == "batched" else 1
    contexts = [3000] if path == "split_wide" else [300 + 41 * b for b in range(batch)]
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
        if report == "next_call":
            # the next call reports it (and launches nothing)
            with pytest.raises(RuntimeError, match="gave_up_a_bounded_wait"):
                _step(mod, embed, final_norm, lw, kv, cos_sin, ids, contexts)
        else:
            from prime_kernels_amd import _decode
            with pytest.raises(RuntimeError, match="gave up a bounded wait"):
                _decode.check_failures(model, embed.device)
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


def test_embed_table_must_have_the_full_vocabulary():
    """The kernels clamp input ids to 0..49151 and the tied LM head reads every row, so decode_step
    refuses an embedding of any other row count (fewer rows would be read past their end), with or
    without the LM head, and one of another width."""
    _need_gpu()
    mod, model, embed, final_norm, lw, kv, cos_sin = _setup(1, [200])
    dev = embed.device

    def step(e, **extra):
        return mod.decode_step(
            input_ids=torch.tensor([999], device=dev), positions=torch.tensor([200], device=dev),
            seq_lens=torch.tensor([201], dtype=torch.int32, device=dev), block_table=kv.block_table[:1].contiguous(),
            slot_mapping=torch.tensor([kv.slot(0, 200)], device=dev), embed=e, layers=lw, final_norm=final_norm,
            kv_caches=kv.caches, cos_sin_cache=cos_sin, eps=1e-5, num_layers=len(lw), **extra)

    bigger = torch.cat([embed, embed[:64]]).contiguous()
    for e in (embed[:1000].contiguous(), bigger, embed[:, :900].contiguous()):
        with pytest.raises(ValueError, match="embed"):
            step(e)
        with pytest.raises(ValueError, match="embed"):
            step(e, return_token_ids=True)
    torch.cuda.synchronize()
    assert mod.workspace(dev).pending_failure() == (0, 0)


@pytest.mark.parametrize("split_role,S", [(1, 900), (1, 3000), (0, 900)], ids=["split_role", "split_wide", "general"])
def test_attention_records_through_uncached_memory_give_the_same_bits(split_role, S):
    """A KV head's chunks exchange their softmax statistics and partials through their XCD's L2 when
    the run-time check finds them on one XCC, else through the uncached workspace.
    PK_OPT_L2_RECORDS=0 forces the second path, the one a placement mismatch takes: same bits."""
    _need_gpu()
    from prime_kernels_amd import _native

    lib = _native.library()
    mod, model, embed, final_norm, lw, kv, cos_sin = _setup(1, [S])
    kv0 = [c.clone() for c in kv.caches]
    old_sr = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, split_role)
    try:
        outs = []
        for l2 in (1, 0):
            old_l2 = lib.pk_set_option(_native.PK_OPT_L2_RECORDS, l2)
            try:
                for c, c0 in zip(kv.caches, kv0):
                    c.copy_(c0)
                h, i, lg = _step(mod, embed, final_norm, lw, kv, cos_sin, [321], [S])
                torch.cuda.synchronize()
                outs.append((h, i, lg.clone(), [c.clone() for c in kv.caches]))
            finally:
                lib.pk_set_option(_native.PK_OPT_L2_RECORDS, old_l2)
        (h0, i0, l0, k0), (h1, i1, l1, k1) = outs
        assert not torch.isnan(h0.float()).any()
        assert torch.equal(h0.view(torch.int16), h1.view(torch.int16)) and torch.equal(i0, i1)
        assert torch.equal(l0.view(torch.int16), l1.view(torch.int16))
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(k0, k1))
        assert mod.workspace(embed.device).pending_failure() == (0, 0)
    finally:
        lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old_sr)


@pytest.mark.parametrize("case", ["b1_split_role", "b1_split_wide", "b1_general", "b16_ragged"])
def test_arrival_skew_leaves_every_bit_unchanged(case):
    """Arrival-skew test of the tagged exchange protocol: with PK_OPT_SKEW every workgroup sleeps a
    pseudo-random 0..23 x 512 cycles (from the seed, the workgroup, the layer and the site) before each
    publish, so exchanged values arrive in orders the hardware rarely produces on its own.  Hidden
    state, greedy ids, logits and the whole KV caches stay bit-identical to the undelayed step, for
    two seeds."""
    _need_gpu()
    from prime_kernels_amd import _native

    lib = _native.library()
    batch = 16 if case == "b16_ragged" else 1
    contexts = [40 + 53 * b for b in range(batch)] if batch > 1 else [3000] if case == "b1_split_wide" else [900]
    mod, model, embed, final_norm, lw, kv, cos_sin = _setup(batch, contexts)
    kv0 = [c.clone() for c in kv.caches]
    ids = [(11 + 97 * b) % 49152 for b in range(batch)]
    old_sr = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, 0 if case == "b1_general" else 1)
    try:
        outs = []
        for seed in (0, 1, 7):
            old = lib.pk_set_option(_native.PK_OPT_SKEW, seed)
            try:
                for c, c0 in zip(kv.caches, kv0):
                    c.copy_(c0)
                h, i, lg = _step(mod, embed, final_norm, lw, kv, cos_sin, ids, contexts)
                torch.cuda.synchronize()
                outs.append((h, i, lg.clone(), [c.clone() for c in kv.caches]))
            finally:
                lib.pk_set_option(_native.PK_OPT_SKEW, old)
            assert mod.workspace(embed.device).pending_failure() == (0, 0), seed
        h0, i0, l0, k0 = outs[0]
        assert not torch.isnan(h0.float()).any()
        for seed, (h, i, lg, kc) in zip((1, 7), outs[1:]):
            assert torch.equal(h.view(torch.int16), h0.view(torch.int16)), seed
            assert torch.equal(i, i0) and torch.equal(lg.view(torch.int16), l0.view(torch.int16)), seed
            assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(kc, k0)), seed
    finally:
        lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old_sr)


@pytest.mark.parametrize("slot", [64, 16])
@pytest.mark.parametrize("mode", [0, 1, 2], ids=["uncached", "cached_sc1", "xcd_l2"])
def test_exchange_units_are_never_torn(mode, slot):
    """The exchanges accept a 16-byte unit {3 payload words, tag} once its tag is current and use the
    payload of that same load, which relies on 16-byte stores never being seen torn.  Workgroups
    publish units whose payload is a function of (tag, unit) with the kernels' stores and read every
    unit back with their polling loads for 400 rounds: no accepted unit may carry another payload, in
    uncached memory (pk_decode's cross-XCD units), ordinary memory with device-scope accesses
    (pk_decode_noalloc's array) and one XCD's L2 (attention records), with one unit per 64-byte
    line (the kernels' placement) and four units from different workgroups per line."""
    _need_gpu()
    import ctypes

    from prime_kernels_amd import _native

    lib = _native.library()
    out = (ctypes.c_uint * 4)()
    rounds = 400
    print(f"mode {mode} slot {slot}", flush=True)
    assert lib.pk_test_exchange_units(mode, rounds, slot, out) == 0
    torn, gave_up, checked, xcc_mask = list(out)
    participants = 32 if mode == 2 else 256
    if mode == 2 and bin(xcc_mask).count("1") != 1:
        pytest.skip(f"the 32 workgroups did not share one XCC (mask {xcc_mask:#x}); the kernels then use uncached records")
    assert torn == 0, (torn, gave_up, checked)
    assert gave_up == 0, (torn, gave_up, checked)
    assert checked == rounds * participants * participants * 4, checked


@pytest.mark.parametrize("path", ["split_role", "split_wide", "general", "batched", "mxfp8", "mxfp8_general"])
def test_cooperative_launch_gives_the_same_bits(path):
    """The decode kernels run with the ordinary launch by default; PK_OPT_COOPERATIVE (or
    PK_LAUNCH=cooperative) launches them with hipLaunchCooperativeKernel as the reference does
    (block360_kernel.inc:914-920).  Both launches give the same hidden state, ids, logits and caches."""
    _need_gpu()
    from prime_kernels_amd import _native

    lib = _native.library()
    batch = 3 if path == "batched" else 1
    contexts = [2100] if path.startswith("mxfp8") or path == "split_wide" else [300 + 41 * b for b in range(batch)]
    mod, model, embed, final_norm, lw, kv, cos_sin = _setup(batch, contexts)
    if path.startswith("mxfp8"):
        import prime_kernels_amd as pk
        from prime_kernels_amd import mxfp8
        mod = pk.load("decode_megakernel_360m_mxfp8")
        lw = mxfp8.quantize_layers(lw)
    kv0 = [c.clone() for c in kv.caches]
    ids = [(57 + 13 * b) % 49152 for b in range(batch)]
    old_sr = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, 0 if path.endswith("general") else 1)
    try:
        outs = []
        for coop in (0, 1):
            old = lib.pk_set_option(_native.PK_OPT_COOPERATIVE, coop)
            try:
                for c, c0 in zip(kv.caches, kv0):
                    c.copy_(c0)
                h, i, lg = _step(mod, embed, final_norm, lw, kv, cos_sin, ids, contexts)
                torch.cuda.synchronize()
                outs.append((h, i, lg.clone(), [c.clone() for c in kv.caches]))
            finally:
                lib.pk_set_option(_native.PK_OPT_COOPERATIVE, old)
            assert mod.workspace(embed.device).pending_failure() == (0, 0), coop
        (h0, i0, l0, k0), (h1, i1, l1, k1) = outs
        assert not torch.isnan(h0.float()).any()
        assert torch.equal(h0.view(torch.int16), h1.view(torch.int16)) and torch.equal(i0, i1)
        assert torch.equal(l0.view(torch.int16), l1.view(torch.int16))
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(k0, k1))
    finally:
        lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old_sr)
