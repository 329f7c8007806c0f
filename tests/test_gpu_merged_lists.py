"""The one-wave fused kernel's merged lists past their first pass.

A tile's merged list takes candidates until they exceed 64, then the tile's
next pass starts where the box tests stopped (build_list's MERGE mode), so a
tile over many large triangles lists them in several passes with k0 > 0.
The entries hold the triangles' indices themselves, and the backward reads
them back from the tile's region, prefetching the slot after the last entry
(the region holds T + 1 slots or more). A single scene leaves the grid
unordered, so no row lists: these are the merged lists over [0, T).
"""

import numpy as np
import pytest

from bars import assert_grads, check_image, check_losses
from diffrast import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from diffrast import _lib

    c = _lib.Context()
    yield c
    c.close()


# (name, B, H, W, T, sigma): one scene of 960 16x16 blocks (more than the
# device's CUs: the fused kernel, no order) over 300 large triangles, whose
# 8x8 tiles list up to ~180 box candidates (half of them more than 64); and
# the same with 304 = 8 x 38 triangles, whose region (312 slots) ends one
# 64-byte line past them.
CASES = [
    ("300-large", 1, 480, 512, 300, 0.002),
    ("304-large", 1, 480, 512, 304, 0.0025),
]


@pytest.mark.parametrize("name,B,H,W,T,sigma", CASES, ids=[c[0] for c in CASES])
def test_multi_pass_merged_lists_match_oracle(ctx, orc, name, B, H, W, T, sigma):
    params = synth.batch("uniform", B, T, 960)
    bgs = synth.uniforms(967, B * 3).reshape(B, 3).astype(np.float32)
    targets = orc.render_batch(synth.batch("uniform", B, T, 960, target_offset=1000), H, W, sigma, bgs)
    print(f"merged lists {name}", flush=True)
    img = ctx.render(params, H, W, sigma, bgs)
    check_image(img, orc.render_batch(params, H, W, sigma, bgs), label=name)
    want_l, want_g = orc.loss_backward_batch(params, targets, sigma, bgs)
    for det in (False, True):
        losses, grads = ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=det)
        check_losses(losses, want_l, label=f"{name} det={det}")
        assert_grads(grads, want_g, label=f"{name} det={det}")
    gi = np.random.default_rng(5).standard_normal((B, H, W, 3)).astype(np.float32) * 1e-3
    g = ctx.backward_from_grad(params, gi, sigma, bgs)
    assert_grads(g, orc.backward_from_grad_batch(params, gi, sigma, bgs), label=f"{name} from grad")
