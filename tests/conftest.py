import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("rust-llm_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP library")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def device():
    if not _gpu_available():
        pytest.skip("no GPU")
    import torch
    return torch.device("cuda:0")


def as_oracle_settings(s):
    """rl_sampler.Sampling -> oracle.Sampling (same layout)."""
    import oracle
    return oracle.Sampling(s.temperature, s.top_p, s.min_p, s.repeat_penalty, s.top_k, s.repeat_last_n, s.seed)
