"""GPU checks of the per-stage debug capture (`debug=` / `debug_layer_index`, the reference's layout
block360_kernel.inc:1-20): every stage of the BASELINE config-1 block against the HF golden stage
vectors, the attention internals of the selected layer against the oracle, the batched kernel's two
capture rows, and unchanged decode outputs with the capture on."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import smollm2 as O
from tests import gpu_cases as GC

# batch-1 steps run on the general kernel, the only one with this path, so that the plain steps
# compared with it bit for bit use the same arithmetic
pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("general_kernel")]

H, QKV, I, NH, SEQ, L = 960, 1600, 2560, 15, 8192, 32
STAGE_SIZES = [("norm1", H), ("qkv", QKV), ("attn", H), ("o", H), ("h1", H), ("norm2", H), ("gate", I),
               ("up", I), ("silu", I), ("act", I), ("down", H), ("out", H)]
LAYER = sum(2 * n for _, n in STAGE_SIZES)


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _bits(a) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a, dtype=np.uint16).view(np.int16).copy()).view(torch.bfloat16)


def layer_stages(buf: torch.Tensor, layer: int) -> dict:
    """Stage name -> [2, N] bf16 rows of `layer` from a capture buffer (uint8)."""
    v = buf.view(torch.bfloat16)
    off = layer * LAYER
    out = {}
    for name, n in STAGE_SIZES:
        out[name] = v[off:off + 2 * n].view(2, n).cpu()
        off += 2 * n
    return out


def attn_stages(buf: torch.Tensor) -> dict:
    v = buf.view(torch.bfloat16)
    off = L * LAYER
    q = v[off:off + 2 * H].view(2, H).cpu()
    off += 2 * H
    res = {"q_rot": q}
    for name in ("qk", "scores", "probs"):
        res[name] = v[off:off + 2 * NH * SEQ].view(2, NH, SEQ).cpu()
        off += 2 * NH * SEQ
    res["pv"] = v[off:off + 2 * H].view(2, H).cpu()
    return res


def _close(got: torch.Tensor, want: torch.Tensor, label: str, min_identical=0.9, rel=2 ** -6):
    got, want = got.float().flatten(), want.float().flatten()
    assert got.shape == want.shape, label
    frac = GC.identical_fraction(got, want)
    err = (got - want).abs()
    tol = rel * want.abs() + 2e-3 * want.abs().max().clamp(min=1e-6)
    assert frac >= min_identical and bool((err <= tol).all()), (label, frac, err.max().item())
    return frac


def _debug_buf(dev):
    from prime_kernels_amd import _native

    n = _native.library().decode360_debug_bytes()
    buf = torch.full((n,), 0xFF, dtype=torch.uint8, device=dev)   # NaN pattern in untouched rows
    return buf


def test_config1_block_stages_match_hf_golden():
    """One 360M block (the HF stage fixture) as a 1-layer model: every captured stage against HF."""
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
    w.embed[5] = _bits(g["x"])
    case = GC.Case(geom, w, kv, ctx + 16)
    dev = case.dev
    buf = _debug_buf(dev)
    case.mod.decode_step(
        input_ids=torch.tensor([5], device=dev), positions=torch.tensor([ctx], device=dev),
        seq_lens=torch.tensor([ctx + 1], dtype=torch.int32, device=dev), block_table=case.btd,
        slot_mapping=torch.tensor([kv.slot(0, ctx)], device=dev), embed=case.wd.embed, layers=case.wd.layers,
        final_norm=case.wd.final_norm, kv_caches=case.kvd, cos_sin_cache=case.csd, eps=1e-5, num_layers=1,
        debug=buf, debug_layer_index=0)
    torch.cuda.synchronize()
    st = layer_stages(buf, 0)
    want = {"norm1": g["norm1"], "qkv": np.concatenate([g["q"], g["k"], g["v"]]), "attn": g["attn"],
            "o": g["o"], "h1": g["h1"], "norm2": g["norm2"], "gate": g["gate"], "up": g["up"],
            "silu": g["silu"], "act": g["act"], "down": g["down"], "out": g["out"]}
    fracs = {}
    for name, ref in want.items():
        fracs[name] = round(_close(st[name][0], _bits(ref), name), 4)
    a = attn_stages(buf)
    _close(a["pv"][0], _bits(g["attn"]), "pv")
    assert torch.equal(a["pv"][0].view(torch.int16), st["attn"][0].view(torch.int16))
    print("config-1 stage bit-identical fractions", fracs)


def _case_two_layers(seed, contexts):
    geom = O.with_layers(O.SMOLLM2_360M, 2)
    return GC.random_kv_case(geom, seed, contexts)


@pytest.mark.parametrize("contexts", [[700], [300, 1025]], ids=["b1", "b2"])
def test_attention_internals_and_stages_match_oracle(contexts):
    """Layer 1 of a 2-layer model: every stage row and the attention internals (rotated q,
    bf16(q.k), scores, probabilities) of each sequence against the oracle's stages."""
    _need_gpu()
    case = _case_two_layers(70 + len(contexts), contexts)
    dev = case.dev
    B = len(contexts)
    ids = [11 + 5 * b for b in range(B)]
    pos = [S - 1 for S in contexts]
    buf = _debug_buf(dev)
    case.mod.decode_step(
        input_ids=torch.tensor(ids, device=dev), positions=torch.tensor(pos, device=dev),
        seq_lens=torch.tensor(contexts, dtype=torch.int32, device=dev), block_table=case.btd,
        slot_mapping=torch.tensor([case.kv.slot(b, pos[b]) for b in range(B)], device=dev), embed=case.wd.embed,
        layers=case.wd.layers, final_norm=case.wd.final_norm, kv_caches=case.kvd, cos_sin_cache=case.csd,
        eps=1e-5, num_layers=2, debug=buf, debug_layer_index=1)
    torch.cuda.synchronize()
    r = O.decode_step(case.w, ids, pos, case.kv, case.cos_sin, stages_layer=1)
    st = layer_stages(buf, 1)
    a = attn_stages(buf)
    for b in range(B):
        ref = r["stages"][b]
        for name in ("norm1", "qkv", "attn", "o", "h1", "norm2", "gate", "up", "silu", "act", "down", "out"):
            _close(st[name][b], ref[name].reshape(-1), f"b{b} {name}", min_identical=0.8)
        S = contexts[b]
        _close(a["q_rot"][b], ref["q_rot"].reshape(-1), f"b{b} q_rot", min_identical=0.9)
        for name in ("qk", "scores", "probs"):
            got = a[name][b, :, :S]
            want = (ref[name] if name != "probs" else ref["probs"]).reshape(NH, S)
            _close(got, want, f"b{b} {name}", min_identical=0.8, rel=2 ** -5)
        # scores are exactly bf16(qk) / 8
        assert torch.equal(a["scores"][b, :, :S].float(), a["qk"][b, :, :S].float() * 0.125)
        assert torch.equal(a["pv"][b].view(torch.int16), st["attn"][b].view(torch.int16))


@pytest.mark.parametrize("contexts", [[513], [200, 64]], ids=["b1", "b2"])
def test_capture_leaves_outputs_unchanged(contexts):
    _need_gpu()
    case = _case_two_layers(90 + len(contexts), contexts)
    pos = [S - 1 for S in contexts]
    ids = [7 + b for b in range(len(contexts))]
    plain = case.kernel_step(ids, pos)
    case.sync_kv_from_oracle()
    buf = _debug_buf(case.dev)
    dev = case.dev
    lg = torch.empty((len(ids), 49152), dtype=torch.bfloat16, device=dev)
    hid, out_ids = case.mod.decode_step(
        input_ids=torch.tensor(ids, device=dev), positions=torch.tensor(pos, device=dev),
        seq_lens=torch.tensor(contexts, dtype=torch.int32, device=dev), block_table=case.btd,
        slot_mapping=torch.tensor([case.kv.slot(b, pos[b]) for b in range(len(ids))], device=dev),
        embed=case.wd.embed, layers=case.wd.layers, final_norm=case.wd.final_norm, kv_caches=case.kvd,
        cos_sin_cache=case.csd, eps=1e-5, num_layers=2, return_token_ids=True, logits_out=lg, debug=buf,
        debug_layer_index=0)
    torch.cuda.synchronize()
    assert torch.equal(hid.cpu().view(torch.int16), plain["hidden"].view(torch.int16))
    assert torch.equal(lg.cpu().view(torch.int16), plain["logits"].view(torch.int16))
    assert torch.equal(out_ids.cpu(), plain["ids"])
    # every layer's out row is the layer output the kernel hands on (layer 1: the pre-norm hidden)
    st = layer_stages(buf, 1)
    lo = case.kernel_step(ids, pos, layer_outputs=True)["layer_outputs"]
    for b in range(len(ids)):
        assert torch.equal(st["out"][b].view(torch.int16), lo[1, b].view(torch.int16))
