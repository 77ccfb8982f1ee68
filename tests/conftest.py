"""Test configuration: import paths, the ``gpu`` marker and shared helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for entry in (ROOT / "chomik-grad_amd", ROOT, ROOT / "tests"):
    if str(entry) not in sys.path:
        sys.path.insert(0, str(entry))

import oracle  # noqa: E402,F401  registers the "cpu" oracle compiler

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the hip plugin")


@pytest.fixture(scope="session")
def hip():
    """The hip compiler.  On a GPU box a missing library or device is an
    error, never a skip: these tests must run the native path."""
    from chomikgrad import get_compiler

    return get_compiler("hip")


def tiny_weights(config, seed, dtype=np.float32, scale=0.05):
    """Reference-test style weights: norms are ones, the rest N(0, scale)
    (tests/test_llama.py:100-108 in the reference)."""
    from chomikgrad import Tensor
    from chomikgrad.dtypes import as_dtype
    from chomikgrad.llama import required_weight_shapes

    rng = np.random.default_rng(seed)
    return {
        name: Tensor(as_dtype(np.ones(shape, np.float32) if "norm.weight" in name
                              else rng.normal(0, scale, shape).astype(np.float32), dtype))
        for name, shape in required_weight_shapes(config).items()
    }


@pytest.fixture(scope="session")
def tinyllama_runtime(hip):
    """The C2/C3 model (TinyLlama-1.1B shape, float16 weights from seed 0) on
    the hip plugin, built once per session: generating its 1.1e9 weights on
    the host takes about 20 seconds."""
    from chomikgrad import synthetic
    from chomikgrad.runtime import LlamaRuntime

    spec = synthetic.TINYLLAMA
    host = synthetic.host_weights(spec.config, spec.dtype, seed=0)
    return LlamaRuntime(spec.config, synthetic.weights_as_tensors(host), compiler="hip", dtype=spec.dtype)
