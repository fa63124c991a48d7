"""pk_decode_noalloc (the entry point that allocates nothing) against pk_decode, through the C ABI.

Each model takes two calls in a row, the second with a smaller input (shorter context, narrower
block table, fewer layers).  Both entry points run the split-role kernel on the same inputs, each on
its own copy of the KV caches, so hidden state, greedy ids, logits and the whole caches after the
step must be bit-identical.  Sizes beyond the fixed array's limits are refused on the host with
PK_ERR_NOALLOC.  The first pk_decode_noalloc call comes before any other library call of this
module, so in a fresh process it also covers the entry point's own set-up (symbol address and the
array's clearing fill on the caller's stream).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
PK_ERR_NOALLOC = 9115  # include/prime_decode.h


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


class _Inputs:
    """Random-init weights (all layers), a paged KV cache and the device pointer tables."""

    def __init__(self, model, capacity, seed):
        from prime_kernels_amd import workload as WL

        dev = torch.device("cuda:0")
        self.model = model
        self.embed, self.final_norm, self.layers = WL.random_weights(model, seed, dev)
        self.kv = WL.PagedKV(model, 1, capacity, device=dev, seed=seed + 1, fill="randn")
        self.cos_sin = WL.rope_table(capacity + 64, device=dev)
        self.layer_table = torch.tensor([[t.data_ptr() for t in layer] for layer in self.layers],
                                        dtype=torch.int64, device=dev)

    def call(self, lib, entry, caches, *, token, pos, cap, n_layers, batch=1, scratch=None, bt=None):
        """One step through `entry` on `caches` (a list of per-layer caches) with context capacity
        `cap` (max_seq_len); returns (status, hidden, ids, logits)."""
        dev = self.embed.device
        m = self.model
        kv0 = caches[0]
        if bt is None:
            bt = self.kv.block_table[:batch, : cap // 16].contiguous()
        kv_table = torch.tensor([c.data_ptr() for c in caches], dtype=torch.int64, device=dev)
        ids = torch.full((batch,), token, dtype=torch.int64, device=dev)
        positions = torch.full((batch,), pos, dtype=torch.int64, device=dev)
        seq_lens = torch.full((batch,), pos + 1, dtype=torch.int32, device=dev)
        slots = torch.tensor([self.kv.slot(0, pos)] * batch, dtype=torch.int64, device=dev)
        hid = torch.empty((batch, m.hidden), dtype=BF16, device=dev)
        out_ids = torch.empty((batch,), dtype=torch.int64, device=dev)
        logits = torch.empty((batch, 49152), dtype=BF16, device=dev)
        args = [torch.cuda.current_stream().cuda_stream, m.model_id, batch, n_layers, ids.data_ptr(), 1,
                self.embed.data_ptr(), self.final_norm.data_ptr(), positions.data_ptr(), seq_lens.data_ptr(),
                bt.data_ptr(), bt.stride(0), slots.data_ptr(), self.layer_table.data_ptr(), kv_table.data_ptr(),
                0, m.head_dim, kv0.stride(0), kv0.stride(2), kv0.stride(1), 16, self.cos_sin.data_ptr(), 0,
                hid.data_ptr(), None, out_ids.data_ptr(), logits.data_ptr()]
        if scratch is not None:
            args += [scratch.data_ptr(), scratch.numel()]
        rc = entry(*args, cap)
        torch.cuda.synchronize()
        return rc, hid, out_ids, logits


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("model_name", ["360m", "135m"])
def test_noalloc_matches_pk_decode_on_two_calls(model_name):
    _need_gpu()
    from prime_kernels_amd import _native
    from prime_kernels_amd._decode import SMOLLM2_135M, SMOLLM2_360M

    lib = _native.library()
    if model_name == "360m":
        model, limit, first, second = SMOLLM2_360M, 1537, (1200, 1536, 32), (150, 160, 7)
    else:
        model, limit, first, second = SMOLLM2_135M, 2561, (2400, 2560, 30), (77, 80, 5)
    # pk_decode takes the same split-role kernel for these contexts (its default)
    old_opt = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, 1)
    try:
        _two_calls(lib, model, limit, first, second, seed=11 if model_name == "360m" else 12)
    finally:
        lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old_opt)


def _two_calls(lib, model, limit, first, second, seed):
    from prime_kernels_amd import _native

    x = _Inputs(model, first[1], seed=seed)
    scratch = torch.empty((lib.pk_workspace_bytes(model.model_id),), dtype=torch.uint8, device="cuda:0")
    caches_ref = x.kv.caches
    caches_na = [c.clone() for c in caches_ref]
    torch.cuda.synchronize()
    for k, (pos, cap, n_layers) in enumerate((first, second)):
        token = 1000 + 7 * k
        rc, h_na, i_na, l_na = x.call(lib, lib.pk_decode_noalloc, caches_na, token=token, pos=pos, cap=cap,
                                      n_layers=n_layers)
        assert rc == 0, _native.status_string(rc)
        rc, h_ref, i_ref, l_ref = x.call(lib, lib.pk_decode, caches_ref, token=token, pos=pos, cap=cap,
                                         n_layers=n_layers, scratch=scratch)
        assert rc == 0, _native.status_string(rc)
        assert not torch.isnan(h_ref.float()).any() and int(i_ref[0]) >= 0, "reference step failed"
        assert _same(h_na, h_ref), (k, (h_na.float() - h_ref.float()).abs().max())
        assert torch.equal(i_na, i_ref), (k, i_na, i_ref)
        assert _same(l_na, l_ref), k
        assert all(_same(a, b) for a, b in zip(caches_na, caches_ref)), k
    # sizes beyond the array's limits are refused before any launch: batch 2, and a block table whose
    # capacity (max_seq_len) exceeds the split-role limit
    rc, *_ = x.call(lib, lib.pk_decode_noalloc, caches_na, token=5, pos=10, cap=first[1], n_layers=2, batch=2)
    assert rc == PK_ERR_NOALLOC
    assert "no_alloc" in _native.status_string(rc)
    wide = torch.zeros((1, (limit + 16 + 15) // 16), dtype=torch.int32, device="cuda:0")
    rc, *_ = x.call(lib, lib.pk_decode_noalloc, caches_na, token=5, pos=10, cap=wide.shape[1] * 16, n_layers=2,
                    bt=wide)
    assert rc == PK_ERR_NOALLOC
    # the refused calls changed nothing: one more pair of steps still agrees
    rc, h_na, i_na, _ = x.call(lib, lib.pk_decode_noalloc, caches_na, token=9, pos=second[0] + 1, cap=second[1],
                               n_layers=second[2])
    assert rc == 0
    rc, h_ref, i_ref, _ = x.call(lib, lib.pk_decode, caches_ref, token=9, pos=second[0] + 1, cap=second[1],
                                 n_layers=second[2], scratch=scratch)
    assert rc == 0 and _same(h_na, h_ref) and torch.equal(i_na, i_ref)


def test_noalloc_failure_is_reported_by_status():
    """A pk_decode_noalloc step forced to give up its bounded waits (pk_test_abort_next_noalloc)
    poisons its outputs; pk_noalloc_status reports that step's epoch until cleared; the next step is
    bit-identical to pk_decode again."""
    _need_gpu()
    import ctypes

    from prime_kernels_amd import _native
    from prime_kernels_amd._decode import SMOLLM2_360M

    lib = _native.library()
    model = SMOLLM2_360M
    x = _Inputs(model, 512, seed=21)
    scratch = torch.empty((lib.pk_workspace_bytes(model.model_id),), dtype=torch.uint8, device="cuda:0")
    caches_ref = x.kv.caches
    caches_na = [c.clone() for c in caches_ref]
    stream = torch.cuda.current_stream().cuda_stream
    out = (ctypes.c_uint * 3)()
    old_opt = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, 1)
    try:
        rc, h_ok, i_ok, _ = x.call(lib, lib.pk_decode_noalloc, caches_na, token=3, pos=300, cap=512, n_layers=4)
        assert rc == 0 and int(i_ok[0]) >= 0
        assert lib.pk_noalloc_status(stream, 1, out) == 0  # clear whatever an earlier test left
        assert lib.pk_noalloc_status(stream, 0, out) == 0 and out[0] == 0, list(out)
        assert lib.pk_test_abort_next_noalloc(stream) == 0
        rc, h_bad, i_bad, l_bad = x.call(lib, lib.pk_decode_noalloc, caches_na, token=4, pos=301, cap=512,
                                         n_layers=4)
        assert rc == 0  # the entry point itself cannot see the failure: it does not synchronise
        assert torch.isnan(h_bad.float()).all() and (i_bad == -1).all() and torch.isnan(l_bad.float()).all()
        assert lib.pk_noalloc_status(stream, 0, out) == 0
        assert out[0] != 0 and out[0] == out[2], list(out)  # the failed step is the last one
        assert lib.pk_noalloc_status(stream, 1, out) == 0 and out[0] != 0
        assert lib.pk_noalloc_status(stream, 0, out) == 0 and out[0] == 0, list(out)
        # the next step runs normally: the same bits as pk_decode on its own copy of the caches
        for c_na, c_ref in zip(caches_na, caches_ref):
            c_na.copy_(c_ref)
        rc, h_na, i_na, l_na = x.call(lib, lib.pk_decode_noalloc, caches_na, token=5, pos=302, cap=512, n_layers=4)
        assert rc == 0
        rc, h_ref, i_ref, l_ref = x.call(lib, lib.pk_decode, caches_ref, token=5, pos=302, cap=512, n_layers=4,
                                         scratch=scratch)
        assert rc == 0
        assert _same(h_na, h_ref) and torch.equal(i_na, i_ref) and _same(l_na, l_ref)
        assert lib.pk_noalloc_status(stream, 0, out) == 0 and out[0] == 0, list(out)
    finally:
        lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old_opt)
