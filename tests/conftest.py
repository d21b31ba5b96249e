import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)))) if np.size(a) else 0.0


# tolerances of this path
REL_L2 = 2e-3      # node outputs and committed states vs the fp32 recurrence
MAX_ABS_BF16 = 1e-2  # bf16 outputs


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from dforktree_amd import _lib
    _lib.load()  # fail loudly if the library is missing on a machine with a GPU
    return torch.device("cuda:0")


def announce(msg):
    """Print the case about to run on the GPU, flushed, so a fault names it."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()
    os.fsync(sys.stdout.fileno()) if hasattr(sys.stdout, "fileno") and sys.stdout.isatty() else None
