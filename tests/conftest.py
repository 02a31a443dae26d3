"""Shared fixtures.

The CPU suite pins the oracle (a tiny random Qwen3 from transformers' own Qwen3Config in float64,
as the reference's tests/conftest.py:24-44 does) and checks the host-side logic and the C-ABI
library's exports. GPU tests (``-m gpu``) compare the HIP path with the oracle.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path
from typing import Any

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# The reference's tiny test model (tests/conftest.py:24-35 of the reference).
TINY_CONFIG: dict[str, Any] = {
    "vocab_size": 512,
    "hidden_size": 64,
    "intermediate_size": 128,
    "num_hidden_layers": 2,
    "num_attention_heads": 4,
    "num_key_value_heads": 2,
    "head_dim": 16,
    "max_position_embeddings": 1024,
    "rms_norm_eps": 1e-6,
    "tie_word_embeddings": True,
}

# A small model with Qwen3's real head geometry (head_dim 128, GQA group 2) for kernel parity.
SMALL_QWEN3: dict[str, Any] = {
    "vocab_size": 1024,
    "hidden_size": 256,
    "intermediate_size": 512,
    "num_hidden_layers": 2,
    "num_attention_heads": 4,
    "num_key_value_heads": 2,
    "head_dim": 128,
    "max_position_embeddings": 2048,
    "rms_norm_eps": 1e-6,
    "rope_theta": 1_000_000.0,
    "tie_word_embeddings": True,
}


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def build_hf_model(dtype: torch.dtype = torch.float64, seed: int = 0, **overrides: Any) -> Any:
    from transformers import Qwen3Config, Qwen3ForCausalLM

    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(Qwen3Config(**{**TINY_CONFIG, **overrides}))
    return model.to(dtype).eval()


@pytest.fixture(scope="session")
def tiny_hf() -> Any:
    return build_hf_model()


@pytest.fixture(scope="session")
def gpu_device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


os.environ.setdefault("PYTHONHASHSEED", "0")
