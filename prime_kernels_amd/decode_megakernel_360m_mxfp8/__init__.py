"""SmolLM2-360M decode step on MI355X (gfx950) with MXFP8 projection weights.

The reference has no MXFP8 decode kernel; this is the BASELINE config-5 path.  Same
`decode_step(**kw)` contract as decode_megakernel_360m, except that each entry of `layers` is the
10-tuple (norm1, qkv, qkv_scales, o, o_scales, norm2, gate_up, gate_up_scales, down,
down_scales) produced by `quantize_layers` (e4m3 codes and e8m0 scales, see
prime_kernels_amd.mxfp8).  Norms, the embedding and the tied LM head stay bf16.  The kernel
dequantises in registers (v_cvt_scalef32_pk_bf16_fp8), so a step equals the bf16 step on the
dequantised weights.
"""

from prime_kernels_amd._decode import SMOLLM2_360M_MXFP8, decode_step as _decode_step, runtime
from prime_kernels_amd.mxfp8 import quantize, quantize_layers, scale_stride

MODEL = SMOLLM2_360M_MXFP8

MAX_BATCH = MODEL.max_batch
MAX_SEQ = MODEL.max_seq
HIDDEN = MODEL.hidden
INTERMEDIATE = MODEL.inter
LAYERS = MODEL.layers
KV_HEADS = MODEL.kv_heads
HEAD_DIM = MODEL.head_dim
BLOCK_SIZE = 16
EPS = 1e-5
MODEL_ID = MODEL.model_id


def decode_step(**kw):
    return _decode_step(MODEL, **kw)


def workspace(device):
    return runtime(MODEL, device)


__all__ = ["MODEL", "decode_step", "quantize", "quantize_layers", "scale_stride", "workspace"]
