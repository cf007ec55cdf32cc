"""Shared fixtures. CPU tests check the oracle, host logic and the ABI; tests
marked ``gpu`` compare the HIP library with the oracle on a real GPU."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "polarengine-vllm_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    return np.load(os.path.join(ROOT, "tests", "golden", "golden.npz"))


@pytest.fixture
def block_size():
    return 128


@pytest.fixture
def sample_polar_config():
    """Decoder-layer polar_config of the reference fixtures (tests/conftest.py:60-131)."""
    def meta(in_f, out_f, bits, packed):
        return {"in_features": in_f, "out_features": out_f, "in_features_padded": in_f,
                "n_blocks": in_f // 128, "bits": bits, "block_size": 128, "packed": packed,
                "scale_dtype": "float16"}
    return {
        "format": "polar_engine_v4",
        "quantization": "polarengine",
        "block_size": 128,
        "bit_assignment": {"q_proj": 5, "k_proj": 5, "v_proj": 5, "o_proj": 6,
                           "gate_up_proj": 3, "gate_proj": 3, "up_proj": 3, "down_proj": 4,
                           "embed": 5, "lm_head": 6},
        "layers": {
            "model.layers.0.self_attn.q_proj": meta(4096, 4096, 5, False),
            "model.layers.0.self_attn.k_proj": meta(4096, 1024, 5, False),
            "model.layers.0.self_attn.o_proj": meta(4096, 4096, 6, False),
            "model.layers.0.mlp.gate_proj": meta(4096, 12288, 3, True),
            "model.layers.0.mlp.down_proj": meta(12288, 4096, 4, True),
        },
    }
