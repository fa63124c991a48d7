"""SmolLM2-135M decode step on MI355X (gfx950).

Drop-in for prime_kernels.decode_megakernel (reference __init__.py:134-205): same
`decode_step(**kw)` contract, plus the 360M wrapper's optional arguments and extensions.
"""

from prime_kernels_amd import _ops  # registers torch.ops.prime_decode.*
from prime_kernels_amd._decode import SMOLLM2_135M, decode_step as _decode_step, runtime

MODEL = SMOLLM2_135M

MAX_BATCH = MODEL.max_batch
MAX_SEQ = MODEL.max_seq
HIDDEN = MODEL.hidden
INTERMEDIATE = MODEL.inter
LAYERS = MODEL.layers
KV_HEADS = MODEL.kv_heads
HEAD_DIM = MODEL.head_dim
BLOCK_SIZE = 16
EPS = 1e-5


def decode_step(**kw):
    return _decode_step(MODEL, **kw)


def workspace(device):
    return runtime(MODEL, device)


MODEL_ID = MODEL.model_id
decode_step_op = _ops.decode_step      # torch.ops.prime_decode.decode_step(MODEL_ID, ...)
decode_logits_op = _ops.decode_logits  # torch.ops.prime_decode.decode_logits(MODEL_ID, ..., logits)
