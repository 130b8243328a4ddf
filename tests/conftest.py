"""Shared fixtures for the test suite.

GPU tests are marked ``gpu``; they call the HIP library through the package
and compare against the CPU oracle in ``oracle/``.
"""

from __future__ import annotations

import json
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def golden():
    from safetensors.torch import load_file
    tensors = load_file(os.path.join(GOLDEN_DIR, "golden.safetensors"))
    with open(os.path.join(GOLDEN_DIR, "golden.json")) as f:
        meta = json.load(f)
    return tensors, meta


@pytest.fixture(scope="session")
def golden_greedy_gpu():
    """Vectors of the reference's GPU greedy backends (low-rank kernel and
    full-rank v2), written by tests/golden/make_golden.py --greedy-gpu."""
    from safetensors.torch import load_file
    tensors = load_file(os.path.join(GOLDEN_DIR, "golden_greedy_gpu.safetensors"))
    with open(os.path.join(GOLDEN_DIR, "golden_greedy_gpu.json")) as f:
        meta = json.load(f)
    return tensors, meta


@pytest.fixture(scope="session")
def golden_rotation():
    """Inputs and outputs of the reference's rotate_weights / rotate_hessian,
    written by tests/golden/make_golden.py --rotation."""
    from safetensors.torch import load_file
    tensors = load_file(os.path.join(GOLDEN_DIR, "golden_rotation.safetensors"))
    with open(os.path.join(GOLDEN_DIR, "golden_rotation.json")) as f:
        meta = json.load(f)
    return tensors, meta


@pytest.fixture
def one_thread():
    """Pin torch to one intra-op thread (MKL rounding depends on blocking)."""
    old = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(old)


def lognormal_hessian(n: int, samples: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    s = torch.exp(torch.randn(n, generator=g))
    X = torch.randn(samples, n, generator=g) * s
    return X.T @ X / samples


@pytest.fixture(scope="session")
def gpu_dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
