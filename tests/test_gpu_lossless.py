"""GPU parity of the lossless gate/up path: the HIP codec against the CPU oracle (oracle/lossless.py)
bit for bit, the encoded cache's lifecycle, and the decode step streaming the encoding, which must
be bit-identical to the dense step (the decoded weights are the same bits and the products are
accumulated in the same order) and within the north-star bound of the oracle."""

import numpy as np
import pytest
import torch

from oracle import lossless as LZ
from oracle import smollm2 as O
from tests import gpu_cases as GC

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["split_role", "general"])
def batch1_kernel(request):
    """Both batch-1 kernels stream the encoding; each must match its own dense step bit for bit."""
    if not torch.cuda.is_available():
        yield request.param
        return
    from prime_kernels_amd import _native

    lib = _native.library()
    old = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, 1 if request.param == "split_role" else 0)
    yield request.param
    lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old)

ROWS, COLS = 5120, 960


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _random_gu(seed: int, std: float = 0.02) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(ROWS, COLS, generator=g) * std).to(torch.bfloat16)


def _crafted_gu(seed: int) -> torch.Tensor:
    """Random weights with rows of edge patterns: the reference's known-answer chunks tiled,
    signed zeros, subnormals, infinities, NaNs, exponent spreads of exactly 7 and 8."""
    w = _random_gu(seed)
    b = _bits(w).copy()
    from tests.test_oracle_lossless import KNOWN_ANSWER

    b[0, :960] = np.tile(KNOWN_ANSWER, 24)
    b[1, :] = 0x8000
    b[2, :] = np.arange(960, dtype=np.uint16) & 0x807F                   # subnormals and zeros
    b[3, :] = np.where(np.arange(960) % 2 == 0, 0x7F80, 0xFF80)          # +-inf
    b[4, :] = 0x7FC0 | (np.arange(960, dtype=np.uint16) & 0x3F)          # NaNs
    for k in range(120):                                                  # spread k % 10 per chunk
        base = 100 + (k % 7)
        e = base + np.array([0, (k % 10)] + [k % 3] * 6)
        b[5, 8 * k:8 * k + 8] = ((e << 7) | (k & 0x7F)).astype(np.uint16)
    b[6, :] = 0x7F00 | (np.arange(960, dtype=np.uint16) & 0x7F)          # exponent 254
    b[7, 8:16] = [0x7F80, 0x7F00, 0x7E80, 0x7E00, 0x7D80, 0x7D00, 0x7C80, 0x7C00]  # 255..248: escaped
    return torch.from_numpy(b.view(np.int16).copy()).view(torch.bfloat16)


def _encode_gpu(w: torch.Tensor, capacity: int):
    import prime_kernels_amd as pk
    from prime_kernels_amd import _native

    pk.load("lossless_bf16")
    lib = _native.library()
    dev = torch.device("cuda:0")
    wd = w.to(dev)
    out = {
        "plane": torch.empty((ROWS, COLS), dtype=torch.uint8, device=dev),
        "headers": torch.empty((ROWS, COLS // 8), dtype=torch.uint32, device=dev),
        "raw": torch.empty((max(capacity, 1) * 8,), dtype=torch.uint16, device=dev),
        "row_offsets": torch.empty((ROWS + 1,), dtype=torch.uint32, device=dev),
        "flags": torch.empty((ROWS * COLS // 8,), dtype=torch.uint32, device=dev),
        "prefix": torch.empty((ROWS * COLS // 8,), dtype=torch.uint32, device=dev),
        "enabled": torch.full((), 7, dtype=torch.uint32, device=dev),
    }
    ws = torch.empty(lib.lossless_scan_workspace_bytes(), dtype=torch.uint8, device=dev)
    rc = lib.lossless_encode_layer(wd.data_ptr(), out["plane"].data_ptr(), out["headers"].data_ptr(),
                                   out["raw"].data_ptr(), out["row_offsets"].data_ptr(), out["flags"].data_ptr(),
                                   out["prefix"].data_ptr(), ws.data_ptr(), ws.numel(), out["enabled"].data_ptr(),
                                   capacity, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return wd, out


def _np(t):
    a = t.cpu()
    if a.dtype == torch.uint32:
        return a.view(torch.int32).numpy().view(np.uint32)
    if a.dtype == torch.uint16:
        return a.view(torch.int16).numpy().view(np.uint16)
    return a.numpy()


@pytest.mark.parametrize("kind", ["random", "crafted"])
def test_encoder_matches_oracle_bit_exact(kind):
    _need_gpu()
    w = _random_gu(11) if kind == "random" else _crafted_gu(12)
    ref = LZ.encode(_bits(w))
    cap = ref["count"] + 5
    _, got = _encode_gpu(w, cap)
    assert np.array_equal(_np(got["plane"]), ref["plane"])
    assert np.array_equal(_np(got["headers"]), ref["headers"])
    assert np.array_equal(_np(got["row_offsets"]), ref["row_offsets"])
    assert np.array_equal(_np(got["flags"]), ref["flags"])
    assert np.array_equal(_np(got["prefix"]), ref["prefix"])
    assert int(_np(got["enabled"])) == 1
    assert np.array_equal(_np(got["raw"])[: 8 * ref["count"]], ref["raw"])
    print(kind, "escaped chunks", ref["count"], "of", ROWS * COLS // 8,
          "bytes per weight %.4f" % (LZ.encoded_bytes(ref) / (ROWS * COLS)))


def test_encoder_capacity_overflow_disables():
    _need_gpu()
    w = _crafted_gu(13)
    ref = LZ.encode(_bits(w), capacity=10)
    assert ref["count"] > 10 and ref["enabled"] == 0
    _, got = _encode_gpu(w, 10)
    assert int(_np(got["enabled"])) == 0
    assert np.array_equal(_np(got["headers"]), ref["headers"])
    assert np.array_equal(_np(got["raw"])[:80], ref["raw"])
    assert int(_np(got["prefix"])[-1]) == ref["count"]
    _, got0 = _encode_gpu(w, 0)                           # the counting pass
    assert int(_np(got0["enabled"])) == 0 and int(_np(got0["prefix"])[-1]) == ref["count"]


@pytest.mark.parametrize("kind", ["random", "crafted"])
def test_decoder_round_trip(kind):
    _need_gpu()
    from prime_kernels_amd import _native

    w = _random_gu(21) if kind == "random" else _crafted_gu(22)
    ref = LZ.encode(_bits(w))
    wd, enc = _encode_gpu(w, ref["count"])
    out = torch.empty_like(wd)
    rc = _native.library().lossless_decode_layer(enc["plane"].data_ptr(), enc["headers"].data_ptr(),
                                                 enc["raw"].data_ptr(), out.data_ptr(),
                                                 torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), _bits(w))
    # and the oracle's decoder on the GPU's buffers
    assert np.array_equal(LZ.decode(_np(enc["plane"]), _np(enc["headers"]), _np(enc["raw"])), _bits(w))


def _model_360m(seed: int):
    import prime_kernels_amd as pk
    from prime_kernels_amd import workload as WL

    model = pk.load("decode_megakernel_360m").MODEL
    dev = torch.device("cuda:0")
    embed, final_norm, layers = WL.random_weights(model, seed, dev)
    return model, embed, final_norm, layers


def test_cache_lifecycle_refresh_and_overflow():
    _need_gpu()
    from prime_kernels_amd.lossless_bf16 import EncodedGUCache

    _, _, _, layers = _model_360m(31)
    gu = [layer[4] for layer in layers]
    cache = EncodedGUCache(gu)
    st = cache.statistics()
    assert st["generation"] == 1 and st["active_layers"] == 32 and st["layers"] == 32
    for i in (0, 17, 31):
        assert torch.equal(cache.decode_layer(i).view(torch.int16), gu[i].view(torch.int16))
        assert st["raw_capacities"][i] >= st["escape_chunks"][i]
    # refresh with new values in the same tensors: layer 5 gets far more escapes than its table holds
    for t in gu:
        t.mul_(-1)
    b = _bits(gu[5]).copy()
    b[:, 0::8] = 0x0001        # a subnormal in every chunk: spread > 7 everywhere
    gu[5].copy_(torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).to(gu[5].device))
    cache.refresh(gu)
    st = cache.statistics()
    assert st["generation"] == 2 and st["active_layers"] == 31 and not cache.enabled(5)
    assert st["escape_chunks"][5] > st["raw_capacities"][5]
    for i in (4, 5, 6):
        assert torch.equal(cache.decode_layer(i).view(torch.int16), gu[i].view(torch.int16))


def _step(mod, model, embed, final_norm, layers, kv, cos_sin, ids, ctx, lossless_cache, logits):
    dev = embed.device
    B = len(ids)
    kw = dict(input_ids=torch.tensor(ids, device=dev), positions=torch.tensor([ctx] * B, device=dev),
              seq_lens=torch.tensor([ctx + 1] * B, dtype=torch.int32, device=dev), block_table=kv.block_table,
              slot_mapping=torch.tensor([kv.slot(b, ctx) for b in range(B)], device=dev), embed=embed,
              layers=layers, final_norm=final_norm, kv_caches=kv.caches, cos_sin_cache=cos_sin, eps=1e-5,
              return_token_ids=True, logits_out=logits, num_layers=len(layers))
    from prime_kernels_amd._decode import decode_step

    hid, out_ids = decode_step(model, encoded_gu=lossless_cache, **kw)
    torch.cuda.synchronize()
    return hid.clone(), out_ids.clone()


@pytest.mark.parametrize("n_layers,ctx", [(2, 300), (32, 1024)])
def test_lossless_step_bit_identical_to_dense(n_layers, ctx, batch1_kernel):
    _need_gpu()
    import prime_kernels_amd as pk
    from prime_kernels_amd import workload as WL
    from prime_kernels_amd.lossless_bf16 import EncodedGUCache

    mod = pk.load("decode_megakernel_360m_lossless")
    model, embed, final_norm, layers = _model_360m(41)
    cache = EncodedGUCache([layer[4] for layer in layers])
    layers = layers[:n_layers]
    dev = embed.device
    kv = WL.PagedKV(model, 1, ctx + 32, layers=n_layers, device=dev, seed=3, fill="randn")
    cos_sin = WL.rope_table(ctx + 32, device=dev)
    kv0 = [c.clone() for c in kv.caches]
    lg_d = torch.empty((1, 49152), dtype=torch.bfloat16, device=dev)
    lg_l = torch.empty_like(lg_d)
    for step in range(3):
        for c, c0 in zip(kv.caches, kv0):
            c.copy_(c0)
        hd, idd = _step(mod, model, embed, final_norm, layers, kv, cos_sin, [100 + step], ctx + step, None, lg_d)
        kv_d = [c.clone() for c in kv.caches]
        for c, c0 in zip(kv.caches, kv0):
            c.copy_(c0)
        hl, idl = _step(mod, model, embed, final_norm, layers, kv, cos_sin, [100 + step], ctx + step, cache, lg_l)
        assert torch.equal(hd.view(torch.int16), hl.view(torch.int16)), step
        assert torch.equal(idd, idl) and torch.equal(lg_d.view(torch.int16), lg_l.view(torch.int16)), step
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(kv_d, kv.caches)), step


def test_lossless_step_with_a_disabled_layer_and_module_api(batch1_kernel):
    """A layer whose escapes overflowed reads its dense matrix; the module's prepare / refresh /
    statistics / decode_step surface; still bit-identical to the dense step."""
    _need_gpu()
    import prime_kernels_amd as pk
    from prime_kernels_amd import workload as WL

    mod = pk.load("decode_megakernel_360m_lossless")
    dense = pk.load("decode_megakernel_360m")
    model, embed, final_norm, layers = _model_360m(51)
    mod._caches._by_device.clear()  # a device's cache is bound to one set of tensors; these are new
    cache = mod.prepare_weights(layers)
    assert mod.prepare_weights(layers) is cache
    gu1 = layers[1][4]
    b = _bits(gu1).copy()
    b[:, 0::8] = 0x0001
    gu1.copy_(torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).to(gu1.device))
    mod.refresh_weights(layers)
    st = mod.cache_statistics(embed.device)
    assert st["active_layers"] == 31 and st["generation"] == 2
    dev = embed.device
    ctx = 700
    kv = WL.PagedKV(model, 1, ctx + 32, device=dev, seed=4, fill="randn")
    cos_sin = WL.rope_table(ctx + 32, device=dev)
    kv0 = [c.clone() for c in kv.caches]
    kw = dict(input_ids=torch.tensor([9], device=dev), positions=torch.tensor([ctx], device=dev),
              seq_lens=torch.tensor([ctx + 1], dtype=torch.int32, device=dev), block_table=kv.block_table,
              slot_mapping=torch.tensor([kv.slot(0, ctx)], device=dev), embed=embed, layers=layers,
              final_norm=final_norm, kv_caches=kv.caches, cos_sin_cache=cos_sin, eps=1e-5)
    hd = dense.decode_step(**kw).clone()
    for c, c0 in zip(kv.caches, kv0):
        c.copy_(c0)
    hl = mod.decode_step(**kw).clone()
    torch.cuda.synchronize()
    assert torch.equal(hd.view(torch.int16), hl.view(torch.int16))


def test_lossless_two_layers_against_oracle(batch1_kernel):
    """The lossless step against the CPU oracle on the same (CPU-drawn) weights and cache."""
    _need_gpu()
    import prime_kernels_amd as pk
    from prime_kernels_amd.lossless_bf16 import EncodedGUCache

    pk.load("decode_megakernel_360m_lossless")
    geom = O.with_layers(O.SMOLLM2_360M, 2)
    case = GC.random_kv_case(geom, 61, [513])
    # a 32-entry cache whose first two matrices are this model's (the rest: copies)
    gu = [case.wd.layers[i % 2][4] for i in range(2)] + [case.wd.layers[1][4].clone() for _ in range(30)]
    cache = EncodedGUCache(gu)
    from prime_kernels_amd._decode import SMOLLM2_360M, decode_step

    dev = case.dev
    lg = torch.empty((1, 49152), dtype=torch.bfloat16, device=dev)
    hid, ids = decode_step(
        SMOLLM2_360M, input_ids=torch.tensor([321], device=dev), positions=torch.tensor([512], device=dev),
        seq_lens=torch.tensor([513], dtype=torch.int32, device=dev), block_table=case.btd,
        slot_mapping=torch.tensor([case.kv.slot(0, 512)], device=dev), embed=case.wd.embed, layers=case.wd.layers,
        final_norm=case.wd.final_norm, kv_caches=case.kvd, cos_sin_cache=case.csd, eps=1e-5, num_layers=2,
        return_token_ids=True, logits_out=lg, encoded_gu=cache)
    torch.cuda.synchronize()
    r = case.oracle_step([321], [512])
    k = {"hidden": hid.cpu(), "ids": ids.cpu(), "logits": lg.cpu()}
    GC.assert_step_parity(k, r, "lossless 2 layers")
