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
    return sorted(set(re.findall(r"\b(drh_\w+)\s*\(", text)))


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


def test_record_bytes_cover_every_part(L):
    # host-only sizing of the forward record: triangle records (76 floats each),
    # backgrounds, the transmittance (4 bytes per pixel), room for the zero and
    # rescaling counts of every tile lane (8 bytes each, written only for tiles
    # that have any), two counts per tile, T entries of 24 bytes per 8x8 tile,
    # and the block order (one int per 16x16 block), each part rounded up to 256
    # bytes
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    B, T, H, W = 16, 128, 256, 256
    tiles = B * (W // 8) * (H // 8)
    head = 256  # sizes, sigma and math mode of the forward pass
    want = (head + up(B * T * 76 * 4) + up(B * 3 * 4) + up(B * H * W * 4) + up(tiles * 64 * 8) + up(tiles * 8)
            + up(tiles * T * 24) + up(tiles // 4 * 4))
    assert L.record_bytes(B, T, H, W) == want
    assert L.record_bytes(0, T, H, W) == 0
    # odd sizes count the partial tiles of whole 16x16 blocks
    tiles = 3 * 2 * 2 * 4  # 2 x 2 blocks of 2 x 2 tiles per scene
    assert L.record_bytes(3, 5, 17, 30) == (head + up(3 * 5 * 76 * 4) + up(36) + up(3 * 17 * 30 * 4)
                                           + up(tiles * 64 * 8) + up(tiles * 8) + up(tiles * 5 * 24)
                                           + up(tiles // 4 * 4))
    with pytest.raises(L.DiffrastError) as e:
        L.record_bytes(1, 1, 0, 4)
    assert e.value.code == 6


def test_size_limits(L):
    # the kernels address a scene's triangle records by 32-bit byte offsets
    # (76 floats each): at most 2^23 triangles per scene
    assert L.record_bytes(1, 1 << 23, 8, 8) > (1 << 23) * 76 * 4
    for sizes in ((1, (1 << 23) + 1, 8, 8), (65536, 1, 8, 8), (1, 1, 8, (1 << 20) + 1), (4, 1 << 23, 8, 8)):
        with pytest.raises(L.DiffrastError) as e:
            L.record_bytes(*sizes)
        assert e.value.code == 5, sizes


def test_record_keeps_a_bounded_number_of_entries(L, monkeypatch):
    # past 1 GiB of entries the record keeps as many per tile as fit (at least 128)
    B, T, H, W = 16, 4096, 512, 512
    tiles = B * (W // 8) * (H // 8)
    cap = (1 << 30) // (tiles * 24)
    assert cap >= 128
    n = L.record_bytes(B, T, H, W)
    assert n - (1 << 30) < B * T * 76 * 4 + B * H * W * 4 + tiles * 64 * 8 + tiles * 8 + tiles // 4 * 4 + 4096
    monkeypatch.setenv("DRH_MAX_TILE_ENTRIES", "7")
    assert L.record_bytes(2, 50, 16, 16) < L.record_bytes(2, 7, 16, 16) + 2 * 50 * 76 * 4


def test_header_compiles_as_c_and_links_against_the_library(tmp_path):
    # A C consumer's view of the boundary (what a cgo or other FFI binding
    # sees): the header compiles as C99 without warnings, every declared
    # entry point resolves when linked against the built library, and a
    # host-only call answers.
    import shutil
    import subprocess

    from diffrast import _lib

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    libdir = Path(_lib.LIB_PATH).parent
    names = declared_symbols()
    src = tmp_path / "consumer.c"
    src.write_text(
        '#include "diffrast_hip.h"\n#include <stdio.h>\n'
        "typedef void (*fn)(void);\n"
        "static const fn entry_points[] = {\n"
        + "".join(f"    (fn){n},\n" for n in names)
        + "};\n"
        "int main(void) {\n"
        '    printf("%d %d\\n", (int)(sizeof entry_points / sizeof entry_points[0]), drh_params_per_triangle());\n'
        "    return 0;\n"
        "}\n")
    exe = tmp_path / "consumer"
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", f"-I{ROOT / 'include'}", str(src),
                    f"-L{libdir}", "-ldiffrast_hip", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=120).stdout.split()
    assert out == [str(len(names)), "10"]
