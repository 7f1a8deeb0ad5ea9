"""Test configuration.

Seeding mirrors the reference (tests/conftest.py:17-49 of mygitljf/ntops):
`random` and `torch` are reseeded from sha256(module path[::test name]) per
module and per test, so every parametrisation draws the same inputs on every
run.  GPU tests carry the `gpu` marker; everything else runs on the CPU."""

import hashlib
import os
import random
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    import ntops_amd.torch.utils

    ntops_amd.torch.utils.set_default_max_num_configs(3)


def _hash(string):
    return int(hashlib.sha256(string.encode("utf-8")).hexdigest(), 16) % 2**32


def _set_random_seed(seed):
    random.seed(seed)
    torch.manual_seed(seed)


def pytest_collectstart(collector):
    if isinstance(collector, pytest.Module):
        _set_random_seed(_hash(collector.name))


@pytest.fixture(scope="module", autouse=True)
def set_seed_per_module(request):
    _set_random_seed(_hash(f"{request.module.__name__.replace('.', '/')}.py"))


@pytest.fixture(autouse=True)
def set_seed_per_test(request):
    _set_random_seed(_hash(f"{request.module.__name__.replace('.', '/')}.py::{request.node.name}"))
