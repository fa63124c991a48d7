"""MXFP8 weights for the decode kernel: quantisation on the device.

Format (OCP MX v1.0): each projection matrix [rows, cols] becomes e4m3 codes uint8 [rows, cols]
plus e8m0 scale codes uint8 [rows, scale_stride(cols)] -- one per 32 consecutive weights of a row
(w = e4m3(q) * 2^(s-127)), each row zero-padded to a multiple of 16 bytes so that the kernel's
16-byte row segments stay aligned.  The rule is the one the reference applies to MX tensors
(prime_kernels/rmsnorm/test.cu:126-144): s = e8m0(amax/448) rounded toward +inf, saturating;
q = e4m3(bf16(x * 2^(127-s))) rounded to nearest even, saturating at +-448.  Norms, the embedding
and the tied LM head stay bf16.
"""

from __future__ import annotations

import torch

from prime_kernels_amd import _native
from prime_kernels_amd._decode import mxfp8_scale_stride as scale_stride

__all__ = ["quantize", "quantize_layers", "scale_stride"]


def quantize(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 CUDA matrix [rows, cols] -> (e4m3 codes, e8m0 scales) on the same device, computed by
    the library's quantisation kernel on the current stream."""
    if not isinstance(w, torch.Tensor) or not w.is_cuda or w.dtype != torch.bfloat16 or w.ndim != 2:
        raise ValueError("w must be a 2-D bf16 CUDA tensor")
    rows, cols = w.shape
    if cols % 32 or cols < 32:
        raise ValueError("cols must be a positive multiple of 32")
    w = w.contiguous()
    q = torch.empty((rows, cols), dtype=torch.uint8, device=w.device)
    s = torch.empty((rows, scale_stride(cols)), dtype=torch.uint8, device=w.device)
    lib = _native.library()
    with torch.cuda.device(w.device):
        rc = lib.pk_quantize_mxfp8(torch.cuda.current_stream(w.device).cuda_stream, w.data_ptr(), q.data_ptr(),
                                   s.data_ptr(), rows, cols)
    if rc != 0:
        raise RuntimeError(f"MXFP8 quantisation failed: {_native.status_string(rc)}")
    return q, s


def quantize_layers(layers) -> list[tuple]:
    """bf16 layer tuples (norm1, qkv, o, norm2, gate_up, down) -> MXFP8 layer tuples
    (norm1, qkv, qkv_scales, o, o_scales, norm2, gate_up, gate_up_scales, down, down_scales)."""
    out = []
    for norm1, qkv, o, norm2, gate_up, down in layers:
        q1, s1 = quantize(qkv)
        q2, s2 = quantize(o)
        q3, s3 = quantize(gate_up)
        q4, s4 = quantize(down)
        out.append((norm1, q1, s1, q2, s2, norm2, q3, s3, q4, s4))
    return out
