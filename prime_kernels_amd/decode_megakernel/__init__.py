"""SmolLM2-135M decode step on MI355X (gfx950).

Drop-in for prime_kernels.decode_megakernel (reference __init__.py:134-205): same
`decode_step(**kw)` contract, plus the 360M wrapper's optional arguments and extensions.
"""

from prime_kernels_amd._decode import Model, decode_step as _decode_step, runtime

MODEL = Model("decode_megakernel", 135, hidden=576, inter=1536, heads=9, kv_heads=3, layers=30)

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
