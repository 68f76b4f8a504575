"""pytest configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs the oracle, host-logic and C-ABI-symbol tests on any
machine; `-m gpu` runs the parity tests on an MI355X (they call the HIP path
through the torch extension and the C ABI and compare with oracle/).
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP extension")


@pytest.fixture(scope="session")
def torch_gpu():
    """torch with a visible GPU; references computed in fp32 must not use TF32
    or reduced-precision fp16 reductions (scripts/test_quant_linear.py:60-74)."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
    return torch
