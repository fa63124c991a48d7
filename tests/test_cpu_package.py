"""CPU-side checks of the package: registry surface, manifest, the C ABI library's exports and its
argument validation (which returns before any GPU call), and the wrapper's contract errors."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import prime_kernels_amd as pk
from prime_kernels_amd import _native, _spec

ROOT = Path(__file__).resolve().parents[1]
HEADERS = (ROOT / "include" / "prime_decode.h", ROOT / "include" / "prime_lossless.h")


def test_registry_surface():
    assert pk.KERNELS == ("decode_megakernel_360m", "decode_megakernel", "decode_megakernel_360m_mxfp8",
                          "decode_megakernel_360m_lossless", "lossless_bf16")
    s = pk.spec("decode_megakernel_360m")
    assert s.module == "prime_kernels_amd.decode_megakernel_360m"
    assert [str(a) for a in s.archs] == ["gfx950"] and s.ops == "prime_decode"
    assert s.supports("gfx950:sramecc+:xnack-") and not s.supports("gfx942:sramecc+:xnack-")
    with pytest.raises(KeyError):
        pk.spec("flash_moe")
    st = pk.status()
    assert set(st) == set(pk.KERNELS)
    if not torch.cuda.is_available():
        assert all("HIP device" in v or "not compiled" in v for v in st.values())
        with pytest.raises(RuntimeError):
            pk.load("decode_megakernel_360m")


def test_arch_parse():
    assert str(_spec.Arch.parse("gfx950")) == "gfx950"
    with pytest.raises(ValueError):
        _spec.Arch.parse("8.9")


def _header_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b([a-z_0-9]+)\s*\(", text))
    return sorted(names - {"defined"})


def test_library_exports_every_header_symbol():
    lib = _native.library()
    names = _header_functions()
    assert "decode360" in names and "mk_decode" in names and "pk_decode" in names
    assert "lossless_encode_layer" in names and "decode360_lossless" in names
    for name in names:
        assert hasattr(lib, name), f"libprime_decode.so does not export {name}"
    assert set(names) <= set(_native.SIGNATURES), "ctypes signatures missing for a header function"


def test_status_strings_and_sizes():
    lib = _native.library()
    want = {9101: "batch_out_of_range", 9103: "null_device_pointer", 9104: "cooperative_launch_unsupported",
            9106: "kernel_requires_gfx950", 9107: "kv_offsets_or_pointers_not_16_byte_aligned",
            9108: "scratch_or_debug_buffer_too_small", 9109: "block_size_or_stride_invalid",
            9112: "first_use_of_the_device_under_stream_capture",
            9113: "a_previous_step_on_this_device_gave_up_a_bounded_wait", 9114: "library_state_allocation_failed"}
    for code, s in want.items():
        assert lib.decode360_status_string(code).decode() == s
        assert lib.mk_status_string(code).decode() == s
    assert lib.decode360_workspace_bytes() == lib.pk_workspace_bytes(360) > 0
    assert lib.mk_workspace_bytes(1, 1024) == lib.pk_workspace_bytes(135) > 0
    assert lib.pk_workspace_bytes(7) == 0
    # the reference's layout (block360_kernel.inc:1-20): 32 layers x 37,120 stage values, then the
    # attention internals of one layer (2 x 960 + 3 x 2 x 15 x 8192 + 2 x 960), bf16
    assert lib.decode360_debug_bytes() == 2 * (32 * 37120 + 2 * 960 + 3 * 2 * 15 * 8192 + 2 * 960)


def _args(**over):
    """A pk_decode argument list with plausible (fake, never dereferenced) pointers."""
    a = dict(stream=None, model=360, B=1, n_layers=32, input_ids=16, ids_i64=1, embed=16, final_norm=16,
             positions=16, seq_lens=16, block_table=16, bt_stride=64, slot_mapping=16, layers=16, kv=16,
             k_off=0, v_off=64, block_stride=10240, token_stride=128, head_stride=2048, block_size=16,
             cos_sin=16, cs_fp32=0, out_hidden=16, layer_outputs=None, out_ids=None, out_logits=None,
             scratch=16, scratch_bytes=1 << 40, max_seq_len=1024)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize("over,code", [
    (dict(B=0), 9101), (dict(B=17), 9101), (dict(n_layers=0), 9110), (dict(n_layers=33), 9110),
    (dict(model=7), 9110), (dict(max_seq_len=0), 9102), (dict(max_seq_len=1 << 20), 9102),
    (dict(embed=None), 9103), (dict(scratch=None), 9103), (dict(scratch_bytes=16), 9108),
    (dict(block_size=32), 9109), (dict(bt_stride=1), 9109), (dict(k_off=4), 9107),
    (dict(embed=24), 9107), (dict(out_logits=8), 9107),
])
def test_pk_decode_rejects_bad_arguments_without_gpu(over, code):
    lib = _native.library()
    assert lib.pk_decode(*_args(**over)) == code


def test_mxfp8_decode_is_batch_one():
    lib = _native.library()
    assert lib.pk_decode_mxfp8(*_args(B=2)) == 9101
    assert lib.pk_decode_mxfp8(*_args(model=135)) == 9110


def test_reference_abi_validation():
    lib = _native.library()
    vp = 16
    base = [None, 1, vp, vp, vp, vp, vp, vp, 64, vp, vp, vp, 0, 64, 10240, 128, 2048, 16, vp, 0, vp, None, vp,
            1 << 40, None, 0, 1024, -1]
    bad = list(base); bad[1] = 17  # batch 1..16
    assert lib.decode360(*bad) == 9101
    bad = list(base); bad[-1] = 40
    assert lib.decode360(*bad) == 9109
    dbg = lib.decode360_debug_bytes()
    bad = list(base); bad[24] = vp                       # debug buffer too small
    assert lib.decode360(*bad) == 9108
    bad = list(base); bad[24] = 24; bad[25] = dbg        # misaligned debug buffer
    assert lib.decode360(*bad) == 9107
    bad = list(base); bad[1] = 3; bad[24] = vp; bad[25] = dbg  # capture holds 2 sequences
    assert lib.decode360(*bad) == 9101
    assert lib.pk_decode_debug(*_args(model=135), None, 16, dbg, -1) == 9111
    assert lib.pk_decode_debug(*_args(), None, 16, dbg, 32) == 9109
    mk = [None, 17, vp, 1, vp, vp, vp, 64, vp, vp, vp, vp, vp, 0, 64, 10240, 128, 2048, 16, vp, 0, vp, vp, 1 << 40, 1024]
    assert lib.mk_decode(*mk) == 9101


def test_wrapper_contract_errors_on_cpu_tensors():
    from prime_kernels_amd import decode_megakernel_360m as m
    z = torch.zeros(1, dtype=torch.int64)
    kw = dict(input_ids=z, positions=z, seq_lens=z.int(), block_table=torch.zeros(1, 4, dtype=torch.int32),
              slot_mapping=z, embed=torch.zeros(1), layers=[()] * 32, final_norm=torch.zeros(960),
              kv_caches=[torch.zeros(1)] * 32, cos_sin_cache=torch.zeros(4, 64), eps=1e-5)
    with pytest.raises(ValueError, match="CUDA tensor"):
        m.decode_step(**kw)
    with pytest.raises(ValueError, match="rms eps"):
        m.decode_step(**dict(kw, eps=1e-6))
    with pytest.raises(ValueError, match="batch"):
        m.decode_step(**dict(kw, input_ids=torch.zeros(17, dtype=torch.int64)))
    from prime_kernels_amd import decode_megakernel_360m_mxfp8 as mq
    with pytest.raises(ValueError, match="batch"):
        mq.decode_step(**dict(kw, input_ids=torch.zeros(2, dtype=torch.int64)))
    with pytest.raises(ValueError, match="layers"):
        m.decode_step(**dict(kw, layers=[()] * 3))


def test_embedding_table_must_have_the_full_vocabulary():
    """The kernels clamp input ids to 0..49151 and the tied LM head reads every row, so the wrapper
    takes only a contiguous [49152, hidden] table: fewer rows would be read past their end, more
    would hold rows no id reaches."""
    from prime_kernels_amd import _decode
    for model in (_decode.SMOLLM2_360M, _decode.SMOLLM2_135M):
        _decode.check_embed_shape(torch.zeros(49152, model.hidden, dtype=torch.bfloat16), model)
        for rows in (1, 49151, 49153, 65536):
            with pytest.raises(ValueError, match="embed"):
                _decode.check_embed_shape(torch.zeros(rows, model.hidden, dtype=torch.bfloat16), model)
        with pytest.raises(ValueError, match="embed"):
            _decode.check_embed_shape(torch.zeros(model.hidden, 49152, dtype=torch.bfloat16).t(), model)


def test_manifest_lists_built_sources():
    for name in pk.KERNELS:
        s = pk.spec(name)
        assert all(src.is_file() for src in s.sources)
        assert (pk.LIB_DIR / s.library).is_file(), "run __graft_entry__.build() first"


def test_torch_ops_schema_and_fake_kernels():
    """torch.ops.prime_decode.* exist with their schemas (KV caches and logits marked mutated)
    and the fake kernels give the output shapes without running anything."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode

    import prime_kernels_amd.decode_megakernel_360m  # noqa: F401  (registers the ops)
    s = str(torch.ops.prime_decode.decode_step.default._schema)
    assert "Tensor(a9!)[] kv_caches" in s and s.endswith("-> (Tensor, Tensor)")
    s = str(torch.ops.prime_decode.decode_logits.default._schema)
    assert "Tensor(a12!) logits" in s
    shapes = ((960,), (1600, 960), (960, 960), (960,), (5120, 960), (960, 2560))
    with FakeTensorMode():
        ids = torch.empty(1, dtype=torch.int64)
        lw = [torch.empty(sh, dtype=torch.bfloat16) for _ in range(2) for sh in shapes]
        kv = [torch.empty(8, 5, 16, 128, dtype=torch.bfloat16) for _ in range(2)]
        args = (360, ids, ids, ids.int(), torch.empty(1, 4, dtype=torch.int32), ids,
                torch.empty(49152, 960, dtype=torch.bfloat16), lw, torch.empty(960, dtype=torch.bfloat16), kv,
                torch.empty(80, 64, dtype=torch.bfloat16), 1e-5)
        h, i = torch.ops.prime_decode.decode_step(*args)
        assert h.shape == (1, 960) and h.dtype == torch.bfloat16 and i.shape == (1,) and i.dtype == torch.int64
        i2 = torch.ops.prime_decode.decode_logits(*args, torch.empty(1, 49152, dtype=torch.bfloat16))
        assert i2.shape == (1,)
        with pytest.raises(ValueError):
            torch.ops.prime_decode.decode_step(360, *args[1:7], lw[:5], *args[8:])


def test_lossless_abi_validation_without_gpu():
    """Argument checks of the codec and the lossless decode entry return before any GPU call."""
    lib = _native.library()
    assert lib.lossless_scan_workspace_bytes() == 5120 * 4
    ws = lib.lossless_scan_workspace_bytes()
    def enc(**over):
        a = dict(input=16, plane=16, headers=16, raw=16, row_offsets=16, flags=16, prefix=16, scan=16,
                 scan_bytes=ws, enabled=16, capacity=8, stream=None)
        a.update(over)
        return lib.lossless_encode_layer(*a.values())
    assert enc(input=None) == 9103
    assert enc(raw=None) == 9103                   # capacity > 0 needs an escape table
    assert enc(scan_bytes=ws - 4) == 9108
    assert enc(plane=24) == 9107
    assert lib.lossless_decode_layer(16, 16, None, 16, None) == 9103
    assert lib.lossless_decode_layer(16, 16, 16, 8, None) == 9107
    assert lib.lossless_write_descriptor(None, 0, 16, 16, 16, 16, 16, None) == 9103
    a = _args()
    assert lib.pk_decode_lossless(*_args(model=135), 16) == 9110      # the codec's shape is 360M's
    assert lib.pk_decode_lossless(*a, 24) == 9107                      # misaligned table
    assert lib.pk_decode_lossless(*_args(B=17), 16) == 9101
    d = dict(stream=None, B=1, input_ids=16, embed=16, final_norm=16, positions=16, seq_lens=16, block_table=16,
             bt_stride=64, slot_mapping=16, layers=16, kv=16, k_off=0, v_off=64, block_stride=10240,
             token_stride=128, head_stride=2048, block_size=16, cos_sin=16, cs_fp32=0, out_hidden=16,
             layer_outputs=None, scratch=16, scratch_bytes=1 << 40, debug=16, debug_bytes=1 << 20,
             max_seq_len=1024, debug_layer_index=-1, table=16)
    assert lib.decode360_lossless(*d.values()) == 9108                # debug buffer too small
    d.update(debug=None, debug_layer_index=32)
    assert lib.decode360_lossless(*d.values()) == 9109


def test_lossless_modules_on_cpu():
    from prime_kernels_amd import decode_megakernel_360m_lossless as L
    from prime_kernels_amd import lossless_bf16 as LB

    assert (LB.LAYERS, LB.ROWS, LB.COLS, LB.CHUNKS) == (32, 5120, 960, 614400)
    assert L.cache_statistics("cpu") is None
    with pytest.raises(ValueError):
        L.prepare_weights([()] * 3)
    with pytest.raises(ValueError):
        LB.EncodedGUCache([torch.zeros(5120, 960, dtype=torch.bfloat16)] * 2)


def test_block360_abi_validation_without_gpu():
    """The research single-block ABI: sizes and the checks that return before any GPU call."""
    lib = _native.library()
    assert lib.block360_debug_bytes() == 2 * 4 * (5 * 960 + 1600 + 2560)
    ws = lib.block360_workspace_bytes()
    assert ws >= lib.pk_workspace_bytes(360) + lib.decode360_debug_bytes()
    a = dict(stream=None, B=1, hidden=16, positions=16, seq_lens=16, block_table=16, bt_stride=64, slot_mapping=16,
             layer=16, kv=16, k_off=0, v_off=64, block_stride=10240, token_stride=128, head_stride=2048,
             block_size=16, cos_sin=16, cs_fp32=0, out_hidden=16, scratch=16, scratch_bytes=ws, debug=None,
             debug_bytes=0, max_seq_len=1024)
    call = lambda **o: lib.block360_decode(*dict(a, **o).values())
    assert call(B=3) == 9101
    assert call(max_seq_len=0) == 9102
    assert call(hidden=None) == 9103
    assert call(scratch_bytes=ws - 1) == 9108
    assert call(debug=16, debug_bytes=16) == 9108
    assert call(out_hidden=24) == 9107
    assert lib.block360_status_string(9101).decode() == "batch_out_of_range"
