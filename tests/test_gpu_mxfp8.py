"""GPU parity of the MXFP8 path: the library's quantisation kernel against the oracle's
(bit-exact), and the MXFP8 decode step against the oracle run on the exact bf16 dequantisation of
the same codes (BASELINE config 5 shape: the full 360M at a context of 8192).  Bars as in
test_gpu_decode.py."""

import numpy as np
import pytest
import torch

from oracle import mxfp8 as MX
from oracle import smollm2 as O
from tests import gpu_cases as GC

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def test_quantizer_matches_oracle_bit_exact():
    """Random weights plus every special case the rule has: all-zero blocks, -0, outliers that
    set the scale, values that saturate or round to e4m3 subnormals, tiny and huge magnitudes."""
    _need_gpu()
    import prime_kernels_amd as pk
    mod = pk.load("decode_megakernel_360m_mxfp8")
    g = torch.Generator().manual_seed(5)
    for rows, cols in ((64, 960), (16, 2560), (8, 576), (3, 32)):
        w = (torch.randn(rows, cols, generator=g) * 0.02).to(torch.bfloat16)
        if cols >= 96:
            w[0, :32] = 0
            w[0, 32:64] = -0.0
            w[1, 40] = 1.0e4   # outlier: the rest of its block rounds to e4m3 subnormals or zero
            w[2, 64:96] = torch.linspace(-3e38, 3e38, 32).to(torch.bfloat16)  # near bf16 max
            w[2, :32] = torch.full((32,), 1e-38).to(torch.bfloat16)            # tiny (bf16 normal)
            w[2, 32:64] = torch.full((32,), 9e-41).to(torch.bfloat16)          # bf16 subnormal
        q, s = mod.quantize(w.cuda())
        torch.cuda.synchronize()
        q_ref, s_ref = MX.quantize(w)
        assert np.array_equal(q.cpu().numpy(), q_ref), (rows, cols)
        assert np.array_equal(s.cpu().numpy(), s_ref), (rows, cols)


@pytest.mark.parametrize("S", [1, 65, 1025, 4097])
def test_mxfp8_two_layers(S):
    """Twelve seeded 2-layer steps per context, held to the seed-set bar (gpu_cases), and at least
    half of them with both layer outputs at least half bit-identical to the oracle's (a bf16
    rounding that flips early in layer 0 spreads one-ulp differences through the rest)."""
    _need_gpu()
    geom = O.with_layers(O.SMOLLM2_360M, 2)
    cases, close = [], 0
    for i in range(12):
        case = GC.mxfp8_case(geom, 40 + S + 1000 * i, [S])
        tok = [77 + S + i]
        k = case.kernel_step(tok, [S - 1], layer_outputs=True)
        e = case.eager_gpu_step(tok, [S - 1])
        r = case.oracle_step(tok, [S - 1], layer_outputs=True)
        cases.append((k, e, r))
        close += all(GC.identical_fraction(k["layer_outputs"][li, 0], r["layer_outputs"][li, 0]) >= 0.5
                     for li in range(2))
    print(GC.assert_seed_set_parity(cases, f"mxfp8 S={S}"), "layer outputs close:", close)
    assert close >= len(cases) // 2, close


def test_mxfp8_full_360m_ctx8192_teacher_forced_layers():
    """BASELINE config 5 shape: 32 layers, 8192 cached tokens; every layer fed the oracle's input."""
    _need_gpu()
    geom = O.SMOLLM2_360M
    S, tok = 8193, 1234
    case = GC.mxfp8_case(geom, 9, [S], norm_jitter=0.0)
    r = case.oracle_step([tok], [S - 1], layer_outputs=True)
    lo = r["layer_outputs"][:, 0]
    fracs = []
    for li in range(geom.layers):
        x_in = case.w.embed[tok] if li == 0 else lo[li - 1]
        k = case.teacher_forced_layer(li, x_in, S - 1, logits=li == geom.layers - 1)
        c = GC.compare_logits(k["out"], lo[li])
        assert c["max_abs"] <= GC.LOGIT_ATOL and c["cos"] >= GC.COS_MIN, (li, c)
        fracs.append(GC.identical_fraction(k["out"], lo[li]))
    assert sum(fracs) / len(fracs) >= 0.9, fracs
    keep = torch.ones(geom.vocab, dtype=torch.bool)
    keep[case.TF_ROW] = False
    c = GC.compare_logits(k["logits"][keep], r["logits"][0][keep])
    assert c["max_abs"] <= GC.LOGIT_ATOL and c["cos"] >= GC.COS_MIN, c
    print("mxfp8 ctx8192 per-layer bit-identical fractions", [round(f, 4) for f in fracs], "logits", c)


def test_mxfp8_full_360m_free_running_within_eager_floor():
    _need_gpu()
    geom = O.SMOLLM2_360M
    S, tok = 1025, 4242
    case = GC.mxfp8_case(geom, 12, [S], norm_jitter=0.0)
    k = case.kernel_step([tok], [S - 1])
    f = case.eager_gpu_step([tok], [S - 1])
    r = case.oracle_step([tok], [S - 1])
    print("mxfp8 360m ctx1024", GC.assert_within_floor(k, r, f, "mxfp8 360m"))
