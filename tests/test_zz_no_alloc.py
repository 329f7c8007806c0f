"""drh_fused_loss_backward_noalloc: the fused entry point whose buffers live in
the library's fixed scratch array instead of the pool. Its results must equal
drh_fused_loss_backward's: bit for bit with fixed-order sums, to 1e-6 of the
gradient norm with the default float atomics (their order varies run to run)."""

import numpy as np
import pytest

from bars import assert_grads, check_losses
from diffrast import _lib, synth

pytestmark = pytest.mark.gpu

SIGMA = 0.0015


def run_both(ctx, torch, dev, B, H, W, T, kind, seed, flags):
    s = torch.cuda.current_stream(dev).cuda_stream
    params = torch.from_numpy(synth.batch(kind, B, T, seed)).to(dev)
    tp = torch.from_numpy(synth.batch(kind, B, T, seed, target_offset=1000)).to(dev)
    bg = torch.zeros((B, 3), device=dev)
    targets = torch.empty((B, H, W, 3), device=dev)
    ctx.render_ptr(tp.data_ptr(), bg.data_ptr(), B, T, H, W, SIGMA, targets.data_ptr(), s)
    out, pool = {}, {}
    for name in ("pooled", "noalloc"):
        losses = torch.full((B,), float("nan"), device=dev)
        grads = torch.full((B, T, 10), float("nan"), device=dev)
        images = torch.full((B, H, W, 3), float("nan"), device=dev)
        fn = ctx.fused_ptr if name == "pooled" else ctx.fused_noalloc_ptr
        before = ctx.pool_stats()
        fn(params.data_ptr(), bg.data_ptr(), targets.data_ptr(), B, T, H, W, SIGMA, losses.data_ptr(),
           grads.data_ptr(), images.data_ptr(), s, flags)
        after = ctx.pool_stats()
        pool[name] = {k: after[k] - before[k] for k in ("hits", "misses")}
        out[name] = (losses, grads, images)
    torch.cuda.synchronize()
    return out, pool, params, targets


@pytest.mark.parametrize("flags", [_lib.DETERMINISTIC, 0], ids=["fixed-order", "atomic"])
def test_noalloc_matches_the_pooled_entry_point(flags):
    import torch

    dev = torch.device("cuda:0")
    ctx = _lib.Context()
    # two calls in a row, the second smaller (and with T > 128: several triangle chunks)
    for B, H, W, T, kind in [(16, 256, 256, 128, "uniform"), (3, 40, 56, 300, "small")]:
        print(f"noalloc B={B} {H}x{W} T={T} flags={flags}", flush=True)
        out, pool, params, targets = run_both(ctx, torch, dev, B, H, W, T, kind, 7, flags)
        (lp, gp, ip), (ln, gn, inn) = out["pooled"], out["noalloc"]
        assert torch.equal(ip, inn)
        assert torch.equal(lp, ln)  # the losses are summed in a fixed order either way
        if flags & _lib.DETERMINISTIC:
            assert torch.equal(gp, gn)
        else:
            assert_grads(gn.cpu().numpy(), gp.cpu().numpy(), tol=1e-6, label="noalloc vs pooled")
        # the pooled call borrowed its buffers from the pool; the noalloc call took none
        assert pool["pooled"]["hits"] + pool["pooled"]["misses"] > 0
        assert pool["noalloc"] == {"hits": 0, "misses": 0}
    # the smaller call's results also meet the oracle bars
    from oracle import oracle as orc

    cl, cg = orc.loss_backward_batch(params.cpu().numpy(), targets.cpu().numpy(), SIGMA)
    check_losses(ln.cpu().numpy(), cl)
    assert_grads(gn.cpu().numpy(), cg)
    ctx.close()


def test_noalloc_takes_no_pool_buffer_and_refuses_what_it_cannot_do():
    import torch

    dev = torch.device("cuda:0")
    ctx = _lib.Context()
    s = torch.cuda.current_stream(dev).cuda_stream
    B, H, W, T = 2, 32, 32, 20
    p = torch.from_numpy(synth.batch("uniform", B, T, 3)).to(dev)
    bg = torch.zeros((B, 3), device=dev)
    tg = torch.rand((B, H, W, 3), device=dev, generator=torch.Generator(device=dev).manual_seed(1))
    losses, grads = torch.empty(B, device=dev), torch.empty((B, T, 10), device=dev)
    ctx.fused_noalloc_ptr(p.data_ptr(), bg.data_ptr(), tg.data_ptr(), B, T, H, W, SIGMA, losses.data_ptr(),
                          grads.data_ptr(), None, s, _lib.SYNC)
    st = ctx.pool_stats()
    assert st["hits"] == 0 and st["misses"] == 0 and st["bytes"] == 0
    assert torch.isfinite(losses).all() and torch.isfinite(grads).all()
    # host arrays would need staging buffers
    with pytest.raises(_lib.DiffrastError) as e:
        ctx.fused_noalloc_ptr(p.data_ptr(), bg.data_ptr(), tg.data_ptr(), B, T, H, W, SIGMA, losses.data_ptr(),
                              grads.data_ptr(), None, s, _lib.HOST_PTRS)
    assert e.value.code == 6
    # sizes whose buffers exceed the scratch array are refused before any launch
    with pytest.raises(_lib.DiffrastError) as e:
        ctx.fused_noalloc_ptr(p.data_ptr(), bg.data_ptr(), tg.data_ptr(), 16, T, 1024, 1024, SIGMA,
                              losses.data_ptr(), grads.data_ptr(), None, s, 0)
    assert e.value.code == 5 and "scratch" in str(e.value)
    ctx.close()


def test_noalloc_calls_from_two_threads_on_two_streams():
    # The calls on one GPU share its scratch array; the library runs them one
    # after another, so calls made concurrently from two host threads on two
    # streams return what the pooled entry point returns, bit for bit with
    # fixed-order sums. Every job has the same sizes (only the scenes differ).
    import threading

    import torch

    dev = torch.device("cuda:0")
    ctx = _lib.Context()
    s0 = torch.cuda.current_stream(dev).cuda_stream
    B, H, W, T = 4, 96, 80, 64
    jobs = []
    for j in range(8):
        p = torch.from_numpy(synth.batch("uniform", B, T, 100 + j)).to(dev)
        tp = torch.from_numpy(synth.batch("uniform", B, T, 100 + j, target_offset=1000)).to(dev)
        bg = torch.zeros((B, 3), device=dev)
        tg = torch.empty((B, H, W, 3), device=dev)
        ctx.render_ptr(tp.data_ptr(), bg.data_ptr(), B, T, H, W, SIGMA, tg.data_ptr(), s0)
        want_l, want_g = torch.empty(B, device=dev), torch.empty((B, T, 10), device=dev)
        ctx.fused_ptr(p.data_ptr(), bg.data_ptr(), tg.data_ptr(), B, T, H, W, SIGMA, want_l.data_ptr(),
                      want_g.data_ptr(), None, s0, _lib.DETERMINISTIC)
        got_l = torch.full((B,), float("nan"), device=dev)
        got_g = torch.full((B, T, 10), float("nan"), device=dev)
        jobs.append((p, bg, tg, want_l, want_g, got_l, got_g))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(dev) for _ in range(2)]  # default priority
    errors = []

    def worker(k):
        s = streams[k].cuda_stream
        try:
            for rep in range(3):
                for j in range(k, len(jobs), 2):
                    p, bg, tg, _, _, got_l, got_g = jobs[j]
                    ctx.fused_noalloc_ptr(p.data_ptr(), bg.data_ptr(), tg.data_ptr(), B, T, H, W, SIGMA,
                                          got_l.data_ptr(), got_g.data_ptr(), None, s, _lib.DETERMINISTIC)
        except Exception as e:  # reported below, not swallowed
            errors.append(repr(e))

    print(f"noalloc: two threads on two streams, {len(jobs)} jobs x 3, B={B} {H}x{W} T={T}", flush=True)
    threads = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    torch.cuda.synchronize()
    assert not errors, errors
    for j, (_, _, _, want_l, want_g, got_l, got_g) in enumerate(jobs):
        assert torch.equal(got_l, want_l), j
        assert torch.equal(got_g, want_g), j
    ctx.close()
