"""Shared fixtures: the package (whose directory name is not an identifier),
the CPU oracle, and the `gpu` marker for tests that need an MI355X."""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PACKAGE = "minimaxh3_on_k100-ai_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libh3mi355x.so")


@pytest.fixture(scope="session")
def pkg():
    return importlib.import_module(PACKAGE)


@pytest.fixture(scope="session")
def oracle():
    from oracle import h3_oracle
    return h3_oracle


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


def assert_bitwise(out: torch.Tensor, ref: torch.Tensor, what: str = ""):
    """Bitwise equality of bf16 tensors, NaN == NaN; reports the worst element."""
    a, b = out.detach().cpu(), ref.detach().cpu()
    assert a.shape == b.shape, f"{what}: shape {tuple(a.shape)} vs {tuple(b.shape)}"
    same = (a.view(torch.int16) == b.view(torch.int16)) | (torch.isnan(a.float()) & torch.isnan(b.float()))
    if not bool(same.all()):
        idx = (~same).nonzero()[0].tolist()
        n = int((~same).sum())
        raise AssertionError(f"{what}: {n} of {a.numel()} elements differ; first at {idx}: "
                             f"{a[tuple(idx)].item()} vs {b[tuple(idx)].item()}")


def attention_error(out: torch.Tensor, ref: torch.Tensor):
    """(max |out - ref|, relative RMS) in fp64."""
    d = out.double() - ref.double()
    return float(d.abs().max()), float(d.norm() / ref.double().norm())
