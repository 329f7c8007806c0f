"""CPU checks of the C ABI: the library loads, exports every declared symbol,
and its host-only logic (constants, config validation, device detection)
behaves. No compute call is made here."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "diffrast_hip.h"


@pytest.fixture(scope="module")
def L():
    from diffrast import _lib

    return _lib


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(drh_[a-z_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_symbols()
    for must in ["drh_create", "drh_destroy", "drh_render", "drh_fused_loss_backward",
                 "drh_backward_from_grad", "drh_adam_project_step", "drh_fit", "drh_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol(L):
    lib = L.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
        assert name in L.SIGNATURES, f"{name} has no ctypes signature"


def test_params_per_triangle(L):
    assert L.params_per_triangle() == 10


@pytest.mark.parametrize("cfg,expected", [
    (dict(), None),
    (dict(sigma_end=0.0), "NonPositiveSigma"),
    (dict(sigma_start=float("nan")), "NonPositiveSigma"),
    (dict(sigma_start=0.001, sigma_end=0.5), "SigmaNotDecreasing"),
    (dict(lr_pos=-1.0), "NonPositiveLearningRate"),
    (dict(lr_alpha=float("inf")), "NonPositiveLearningRate"),
])
def test_fit_config_validation(L, cfg, expected):  # fit.rs:542-564
    assert L.validate_fit_config(16, **cfg) == expected


def test_fit_config_rejects_zero_triangles(L):  # fit.rs:546
    assert L.validate_fit_config(0) == "NoTriangles"


def test_last_error_is_a_string(L):
    assert isinstance(L.last_error(), str)


def test_create_reports_no_device_without_a_gpu(L):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    assert L.lib().drh_create(ctypes.byref(h)) == 1  # NoAdapter
    assert "no HIP device" in L.last_error()
