"""SmolLM2-360M decode step on MI355X (gfx950).

Drop-in for prime_kernels.decode_megakernel_360m (reference __init__.py:142-234): same
`decode_step(**kw)` contract.  The returned tensor is a view into a shared per-device output
buffer and is overwritten by the next call on that device; consume or copy it before then.
Extensions: `return_token_ids=True` (greedy ids from the fused tied LM head), `logits_out=`,
`num_layers=`.  Batch 1..16 (ragged contexts; B >= 2 runs the batched MFMA kernel); KV block
size 16; contexts up to 12288 tokens.
"""

from prime_kernels_amd import _ops  # registers torch.ops.prime_decode.*
from prime_kernels_amd._decode import SMOLLM2_360M, decode_step as _decode_step, runtime

MODEL = SMOLLM2_360M

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
    """The per-device runtime (workspace, output buffers) -- for diagnostics."""
    return runtime(MODEL, device)


MODEL_ID = MODEL.model_id
decode_step_op = _ops.decode_step      # torch.ops.prime_decode.decode_step(MODEL_ID, ...)
decode_logits_op = _ops.decode_logits  # torch.ops.prime_decode.decode_logits(MODEL_ID, ..., logits)
