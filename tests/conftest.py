import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def golden_dir() -> Path:
    return ROOT / "tests" / "golden"


@pytest.fixture
def general_kernel():
    """Batch-1 steps on the general kernel for the test (the split-role kernel, the default for
    contexts up to its limit, sums in another order): for tests that compare a batch-1 step bit for
    bit with a path only the general kernel has (per-stage debug capture, the single-block ABI)."""
    import torch

    if not torch.cuda.is_available():
        yield
        return
    from prime_kernels_amd import _native

    lib = _native.library()
    old = lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, 0)
    yield
    lib.pk_set_option(_native.PK_OPT_SPLIT_ROLE, old)
