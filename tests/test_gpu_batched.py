"""GPU parity of the batched decode kernel (2..16 sequences per launch, ragged contexts, MFMA
projections): every sequence against the oracle (which runs each sequence on its own), KV appends,
agreement with the batch-1 kernel, and the BASELINE config-4 shape (full 360M, 16 sequences,
contexts 128..4096).

Bars as in test_gpu_decode.py.  A free-running step is held to the north-star bound or to twice
the eager-GPU floor of the same sequence, whichever is larger: a single bf16 rounding flip (a
different fp32 summation order in attention or a projection) changes the next RMSNorm scale and so
hundreds of normed values, and random-init layers carry that on.  The eager GPU path shows the same
on other sequences of the same batch.  Layers fed the oracle's own inputs (teacher forced) are held
to the north-star bound itself."""

import numpy as np
import pytest
import torch

from oracle import smollm2 as O
from tests import gpu_cases as GC

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _kv_appends_match(case, contexts, label):
    for li in range(case.geom.layers):
        for b, S in enumerate(contexts):
            slot = case.kv.slot(b, S - 1)
            got = case.kvd[li][slot // 16, :, slot % 16].cpu().float()
            want = case.kv.caches[li][slot // 16, :, slot % 16].float()
            assert torch.allclose(got, want, rtol=2 ** -6, atol=2e-2), (label, li, b)


@pytest.mark.parametrize("contexts", [[37, 300], [1, 2, 65, 129, 1000, 17], [5] * 16],
                         ids=["b2", "b6_edges", "b16_short"])
def test_batched_two_layers(contexts):
    _need_gpu()
    geom = O.with_layers(O.SMOLLM2_360M, 2)
    case = GC.random_kv_case(geom, 60 + len(contexts), contexts)
    ids = [100 + 7 * b for b in range(len(contexts))]
    pos = [S - 1 for S in contexts]
    k = case.kernel_step(ids, pos, layer_outputs=True)
    f = case.eager_gpu_step(ids, pos)
    r = case.oracle_step(ids, pos, layer_outputs=True)
    GC.assert_within_floor(k, r, f, f"batched {contexts}")
    _kv_appends_match(case, contexts, "two layers")


def test_batched_ragged_16_two_layers():
    _need_gpu()
    rng = np.random.default_rng(8)
    contexts = [int(x) for x in rng.integers(1, 2500, 16)]
    geom = O.with_layers(O.SMOLLM2_360M, 2)
    case = GC.random_kv_case(geom, 71, contexts)
    ids = [int(x) for x in rng.integers(0, 49152, 16)]
    pos = [S - 1 for S in contexts]
    k = case.kernel_step(ids, pos)
    f = case.eager_gpu_step(ids, pos)
    r = case.oracle_step(ids, pos)
    GC.assert_within_floor(k, r, f, "ragged16")
    _kv_appends_match(case, contexts, "ragged16")


def test_batched_135m_four_sequences():
    _need_gpu()
    geom = O.with_layers(O.SMOLLM2_135M, 3)
    contexts = [513, 64, 2048, 200]
    case = GC.random_kv_case(geom, 81, contexts)
    ids = [5, 6, 7, 8]
    k = case.kernel_step(ids, [S - 1 for S in contexts])
    f = case.eager_gpu_step(ids, [S - 1 for S in contexts])
    r = case.oracle_step(ids, [S - 1 for S in contexts])
    GC.assert_within_floor(k, r, f, "135m b4")


def test_batched_agrees_with_batch_one_kernel():
    """A sequence decoded inside a batch of 8 gives what the batch-1 kernel gives for it alone,
    within the bf16 bar (the two kernels sum in different orders)."""
    _need_gpu()
    geom = O.with_layers(O.SMOLLM2_360M, 2)
    contexts = [700, 33, 1500, 90, 4, 260, 1024, 2]
    case = GC.random_kv_case(geom, 91, contexts)
    ids = [int(40 + 3 * b) for b in range(8)]
    kb = case.kernel_step(ids, [S - 1 for S in contexts])
    for b in range(8):
        case.sync_kv_from_oracle()
        ks = case.kernel_step([ids[b]], [contexts[b] - 1], seq_lens=[contexts[b]],
                              slot_mapping=[case.kv.slot(b, contexts[b] - 1)], block_rows=[b])
        c = GC.compare_logits(kb["logits"][b], ks["logits"][0])
        assert c["max_abs"] <= GC.LOGIT_ATOL and c["cos"] >= GC.COS_MIN, (b, c)


@pytest.mark.parametrize("base,ids_dtype", [(O.SMOLLM2_360M, torch.int64), (O.SMOLLM2_360M, torch.int32),
                                             (O.SMOLLM2_135M, torch.int64)], ids=["360m-i64", "360m-i32", "135m-i64"])
def test_two_sequences_run_as_two_batch_one_steps(base, ids_dtype):
    """Two sequences without layer_outputs run as two batch-1 steps on the split-role kernel (360M:
    one context on its narrow layout, one on its wide layout; 135M: its 4- and 10-chunk narrow
    builds): within the eager floor of the oracle, the appends where the oracle puts them, and every
    output bit equal to a batch-1 call per sequence."""
    _need_gpu()
    geom = O.with_layers(base, 2)
    contexts = [300, 1700]
    case = GC.random_kv_case(geom, 97, contexts)
    ids = [11, 12]
    pos = [S - 1 for S in contexts]
    k = case.kernel_step(ids, pos, ids_dtype=ids_dtype)
    f = case.eager_gpu_step(ids, pos)
    r = case.oracle_step(ids, pos)
    GC.assert_within_floor(k, r, f, "two sequences")
    _kv_appends_match(case, contexts, "two sequences")
    for b in range(2):
        case.sync_kv_from_oracle()
        one = case.kernel_step([ids[b]], [pos[b]], seq_lens=[contexts[b]],
                               slot_mapping=[case.kv.slot(b, contexts[b] - 1)], block_rows=[b], ids_dtype=ids_dtype)
        assert torch.equal(k["logits"][b], one["logits"][0]), b
        assert torch.equal(k["hidden"][b], one["hidden"][0]), b
        assert int(k["ids"][b]) == int(one["ids"][0]), b


def test_batched_deterministic():
    _need_gpu()
    geom = O.with_layers(O.SMOLLM2_360M, 2)
    contexts = [300, 1200, 45]
    case = GC.random_kv_case(geom, 95, contexts)
    outs = []
    for _ in range(3):
        case.sync_kv_from_oracle()
        outs.append(case.kernel_step([1, 2, 3], [S - 1 for S in contexts]))
    for o in outs[1:]:
        assert torch.equal(o["logits"], outs[0]["logits"]) and torch.equal(o["ids"], outs[0]["ids"])


def test_batched_full_360m_config4_shape():
    """BASELINE config 4 shape: the full 32-layer 360M, 16 sequences with contexts drawn from
    128..4096; each sequence within the eager floor of the oracle."""
    _need_gpu()
    rng = np.random.default_rng(4)
    contexts = [int(x) for x in rng.integers(128, 4097, 16)]
    case = GC.random_kv_case(O.SMOLLM2_360M, 99, contexts, norm_jitter=0.0)
    ids = [int(x) for x in rng.integers(0, 49152, 16)]
    pos = [S - 1 for S in contexts]
    k = case.kernel_step(ids, pos)
    f = case.eager_gpu_step(ids, pos)
    r = case.oracle_step(ids, pos)
    out = GC.assert_within_floor(k, r, f, "config4")
    print("config4 worst", max(v["kernel"]["max_abs"] for v in out.values()),
          "floor worst", max(v["eager_gpu_floor"]["max_abs"] for v in out.values()))


def test_batched_full_360m_config4_teacher_forced_layers():
    """Config 4 shape, every layer of the full 360M fed the oracle's inputs for all 16 sequences at
    once: each layer output within the north-star bound of the oracle's, mostly bit-identical."""
    _need_gpu()
    rng = np.random.default_rng(44)
    contexts = [int(x) for x in rng.integers(128, 4097, 16)]
    geom = O.SMOLLM2_360M
    case = GC.random_kv_case(geom, 98, contexts, norm_jitter=0.0)
    ids = [int(x) for x in rng.integers(16, 49152, 16)]
    pos = [S - 1 for S in contexts]
    r = case.oracle_step(ids, pos, layer_outputs=True)
    lo = r["layer_outputs"]                                  # [L, B, H]
    case.sync_kv_from_oracle()                               # caches the oracle saw, new tokens included
    fracs = []
    for li in range(geom.layers):
        x_in = case.w.embed[ids] if li == 0 else lo[li - 1]
        k = GC.teacher_forced_layer_batch(case, li, x_in, pos, logits=li == geom.layers - 1)
        for b in range(16):
            c = GC.compare_logits(k["out"][b], lo[li, b])
            assert c["max_abs"] <= GC.LOGIT_ATOL and c["cos"] >= GC.COS_MIN, (li, b, c)
            fracs.append(GC.identical_fraction(k["out"][b], lo[li, b]))
    assert sum(fracs) / len(fracs) >= 0.9, sum(fracs) / len(fracs)
    keep = torch.ones(geom.vocab, dtype=torch.bool)
    keep[:16] = False
    for b in range(16):
        c = GC.compare_logits(k["logits"][b][keep], r["logits"][b][keep])
        assert c["max_abs"] <= GC.LOGIT_ATOL and c["cos"] >= GC.COS_MIN, (b, c)
    print("config4 teacher-forced mean bit-identical fraction", round(sum(fracs) / len(fracs), 4))


def test_batched_max_context_and_edges():
    """Batch 3 with one sequence at the longest context (12288), one of 3 tokens and one of 700."""
    _need_gpu()
    geom = O.with_layers(O.SMOLLM2_360M, 2)
    contexts = [12288, 3, 700]
    case = GC.random_kv_case(geom, 303, contexts, capacity=12288)
    ids = [5, 6, 7]
    pos = [S - 1 for S in contexts]
    k = case.kernel_step(ids, pos, layer_outputs=True)
    f = case.eager_gpu_step(ids, pos)
    r = case.oracle_step(ids, pos, layer_outputs=True)
    GC.assert_within_floor(k, r, f, "batched max context")
    _kv_appends_match(case, contexts, "max context")


def test_batched_slot_minus_one_int32_ids_fp32_rope():
    """Batched step: slot_mapping < 0 skips that sequence's K/V write and leaves its result unchanged;
    int32 ids and an fp32 cos/sin table give the identical result."""
    _need_gpu()
    geom = O.with_layers(O.SMOLLM2_360M, 2)
    contexts = [300, 41, 129]
    case = GC.random_kv_case(geom, 305, contexts)
    ids = [11, 12, 13]
    pos = [S - 1 for S in contexts]
    slots = [case.kv.slot(b, pos[b]) for b in range(3)]
    before = [c.clone() for c in case.kvd]
    k1 = case.kernel_step(ids, pos, slot_mapping=[slots[0], -1, slots[2]])
    for li, (a, c) in enumerate(zip(before, case.kvd)):
        s = slots[1]
        assert torch.equal(a[s // 16, :, s % 16], c[s // 16, :, s % 16]), li
        for b in (0, 2):
            s = slots[b]
            assert not torch.equal(a[s // 16, :, s % 16], c[s // 16, :, s % 16]), (li, b)
    k2 = case.kernel_step(ids, pos)
    assert torch.equal(k1["logits"], k2["logits"]) and torch.equal(k1["ids"], k2["ids"])
    k3 = case.kernel_step(ids, pos, ids_dtype=torch.int32, cs_fp32=True)
    assert torch.equal(k3["logits"], k2["logits"]) and torch.equal(k3["hidden"], k2["hidden"])
