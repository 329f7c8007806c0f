"""The oracle under AddressSanitizer + UndefinedBehaviorSanitizer and under
ThreadSanitizer: oracle/sanitize_main.c runs every entry point (renders, loss
and gradients, upstream-gradient forms, finite differences, batches on several
threads, Adam, projection, the fit loop with each stop reason, sRGB) over
ordinary inputs and the edge cases the reference tests (1x1, 1xW, Hx1 canvases,
empty scenes, NaN/inf/huge/degenerate triangles, clamped and NaN alpha). A
sanitizer finding aborts the driver with its report."""

import subprocess
from pathlib import Path

import pytest

ORACLE = Path(__file__).resolve().parents[1] / "oracle"


@pytest.fixture(scope="module")
def built():
    r = subprocess.run(["make", "-s", "-C", str(ORACLE), "sanitize"], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail("sanitizer build failed:\n" + r.stdout + r.stderr)
    return ORACLE / "_san"


@pytest.mark.parametrize("binary", ["asan_ubsan", "tsan"])
def test_oracle_is_clean_under_sanitizers(built, binary):
    r = subprocess.run([str(built / binary)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout[-2000:] + r.stderr[-4000:]
