//! The HIP backend against the CPU crate, in the shape of the reference's own
//! GPU tests (crates/diffrast-gpu/src/lib.rs:1185-1610): same scenes, CPU
//! results from `diffrast`, the library's bars (1e-5 per pixel, 1e-4 relative
//! per loss, 1e-4 of the gradient norm). Each test returns early when no HIP
//! device is present.

use std::sync::OnceLock;

use diffrast_hip::{
    BackwardMode, Canvas, FitConfig, GpuRasterizer, ReduceMode, RenderParams, Scene, StopReason,
};
use rand::rngs::StdRng;
use rand::SeedableRng;

fn gpu() -> Option<&'static GpuRasterizer> {
    static G: OnceLock<Option<GpuRasterizer>> = OnceLock::new();
    G.get_or_init(|| GpuRasterizer::new().ok()).as_ref()
}

fn scene(n: usize, seed: u64) -> Scene {
    let mut rng = StdRng::seed_from_u64(seed);
    Scene::random(n, [0.1, 0.12, 0.15], 0.2, &mut rng)
}

fn max_abs_diff(a: &[f32], b: &[f32]) -> f32 {
    a.iter().zip(b).map(|(x, y)| (x - y).abs()).fold(0.0, f32::max)
}

fn grad_err(want: &[f32], got: &[f32]) -> f32 {
    let norm = want.iter().map(|g| g * g).sum::<f32>().sqrt().max(1e-12);
    max_abs_diff(want, got) / norm
}

fn cpu_backward(s: &Scene, p: RenderParams, target: &Canvas) -> (f32, Vec<f32>) {
    let (rendered, tape) = diffrast::render_with_tape(s, p);
    diffrast::backward(s, p, &tape, &rendered, target)
}

#[test]
fn forward_matches_cpu() {
    let Some(gpu) = gpu() else { return };
    for (w, h, sigma, tris) in [(32, 32, 0.01, 8), (64, 48, 0.004, 24), (37, 19, 0.02, 3)] {
        let s = scene(tris, 7);
        let p = RenderParams::new(w, h, sigma);
        let d = max_abs_diff(&diffrast::render(&s, p).data, &gpu.render(&s, p).expect("render").data);
        assert!(d <= 1e-5, "{w}x{h} sigma {sigma}: max diff {d}");
    }
}

#[test]
fn empty_scene_renders_background() {
    let Some(gpu) = gpu() else { return };
    let img = gpu.render(&Scene::new([0.2, 0.4, 0.6]), RenderParams::new(16, 16, 0.01)).expect("render");
    assert!(max_abs_diff(&img.data, &Canvas::filled(16, 16, [0.2, 0.4, 0.6]).data) <= 1e-6);
}

#[test]
fn backward_matches_cpu_in_both_modes() {
    let Some(gpu) = gpu() else { return };
    let s = scene(12, 7);
    let p = RenderParams::new(48, 48, 0.02);
    let target = Canvas::filled(48, 48, [0.5, 0.3, 0.7]);
    let (cl, cg) = cpu_backward(&s, p, &target);
    for mode in [BackwardMode::Recompute, BackwardMode::Taped] {
        let (gl, gg) = gpu.backward_with(&s, p, &target, mode).expect("backward");
        assert!((cl - gl).abs() <= 1e-4 * cl.abs(), "loss {cl} vs {gl}");
        assert!(grad_err(&cg, &gg) <= 1e-4, "{mode:?}: gradient error {}", grad_err(&cg, &gg));
    }
}

#[test]
fn batches_match_cpu_in_order() {
    let Some(gpu) = gpu() else { return };
    let scenes: Vec<Scene> = (0..5).map(|i| scene(20, 100 + i)).collect();
    let p = RenderParams::new(40, 36, 0.01);
    let targets: Vec<Canvas> = (0..5).map(|i| diffrast::render(&scene(20, 200 + i), p)).collect();
    let imgs = gpu.render_many(&scenes, p).expect("render_many");
    for (s, img) in scenes.iter().zip(&imgs) {
        assert!(max_abs_diff(&diffrast::render(s, p).data, &img.data) <= 1e-5);
    }
    let cpu = diffrast::backward_batch(&scenes, p, &targets);
    for reduce in [ReduceMode::Workgroup, ReduceMode::Deterministic] {
        let (got, t) = gpu.backward_many_full(&scenes, p, &targets, reduce).expect("backward_many_full");
        assert!(t.total_ms() > 0.0);
        for ((cl, cg), (gl, gg)) in cpu.iter().zip(&got) {
            assert!((cl - gl).abs() <= 1e-4 * cl.abs());
            assert!(grad_err(cg, gg) <= 1e-4);
        }
    }
}

#[test]
fn timed_backward_reports_every_phase() {
    let Some(gpu) = gpu() else { return };
    let scenes: Vec<Scene> = (0..4).map(|i| scene(64, 300 + i)).collect();
    let p = RenderParams::new(96, 96, 0.004);
    let targets: Vec<Canvas> = (0..4).map(|_| Canvas::filled(96, 96, [0.4, 0.5, 0.6])).collect();
    let plain = gpu.backward_many_full(&scenes, p, &targets, ReduceMode::Deterministic).expect("plain").0;
    let (timed, t) = gpu.backward_many_timed(&scenes, p, &targets).expect("timed");
    assert!(t.dispatch_ms > 0.0 && t.readback_ms > 0.0 && t.loss_ms == 0.0);
    for ((pl, pg), (tl, tg)) in plain.iter().zip(&timed) {
        assert_eq!(pl, tl);
        assert!(grad_err(pg, tg) <= 1e-6);
    }
}

#[test]
fn ragged_and_mismatched_batches_are_rejected_and_empty_is_empty() {
    let Some(gpu) = gpu() else { return };
    let p = RenderParams::new(16, 16, 0.01);
    assert!(gpu.render_many(&[scene(3, 1), scene(4, 2)], p).is_err());
    assert!(gpu.render_many(&[], p).expect("empty").is_empty());
    let wrong = Canvas::filled(8, 8, [0.0; 3]);
    assert!(gpu.backward_many(&[scene(3, 1)], p, &[wrong]).is_err());
    assert!(gpu.backward_many_from_grad(&[scene(3, 1)], p, &[0.0; 5]).is_err());
}

#[test]
fn gradient_input_mode_matches_target_mode() {
    let Some(gpu) = gpu() else { return };
    let s = scene(10, 9);
    let p = RenderParams::new(32, 32, 0.01);
    let target = Canvas::filled(32, 32, [0.2, 0.6, 0.4]);
    let rendered = gpu.render(&s, p).expect("render");
    let n = rendered.data.len() as f32;
    let dl: Vec<f32> = rendered.data.iter().zip(&target.data).map(|(r, t)| 2.0 * (r - t) / n).collect();
    let from_grad = gpu.backward_many_from_grad(std::slice::from_ref(&s), p, &dl).expect("from_grad");
    let (_, direct) = gpu.backward(&s, p, &target).expect("backward");
    assert!(grad_err(&direct, &from_grad[0]) <= 1e-4);
}

#[test]
fn pool_reuses_buffers() {
    let Some(gpu) = gpu() else { return };
    let s = scene(6, 3);
    let p = RenderParams::new(24, 24, 0.02);
    let target = Canvas::filled(24, 24, [0.5; 3]);
    gpu.backward(&s, p, &target).expect("first");
    let a = gpu.pool_stats();
    gpu.backward(&s, p, &target).expect("second");
    let b = gpu.pool_stats();
    assert_eq!(a.misses, b.misses);
    assert!(b.hits > a.hits);
    assert!(GpuRasterizer::tape_bytes(6, 24, 24) > 0);
}

#[test]
fn fitter_follows_the_cpu_fit() {
    let Some(gpu) = gpu() else { return };
    let target = diffrast::render(&scene(24, 11), RenderParams::new(48, 40, 0.0015));
    let cfg = FitConfig { triangles: 16, iters: 40, patience: None, ..FitConfig::default() };
    let cpu = diffrast::fit(&target, &cfg, |_| {}).expect("cpu fit");
    let mut seen = 0;
    let rep = gpu.fit(&target, &cfg, |pr| {
        assert_eq!(pr.iter, seen);
        assert_eq!(pr.scene.len(), 16);
        seen += 1;
    })
    .expect("gpu fit");
    assert_eq!(seen, 40);
    assert_eq!(rep.stop_reason, StopReason::Completed);
    for (c, g) in cpu.losses.iter().zip(&rep.losses).take(20) {
        assert!((c - g).abs() <= 1e-4 * c, "loss {c} vs {g}");
    }
    let quiet = gpu.fit_quiet(&target, &cfg).expect("fit_quiet");
    assert_eq!(quiet.losses.len(), rep.losses.len());
}

#[test]
fn stepping_stops_once() {
    let Some(gpu) = gpu() else { return };
    let flat = Canvas::filled(24, 24, [0.4; 3]);
    let cfg = FitConfig { triangles: 4, iters: 1000, patience: Some(5), ..FitConfig::default() };
    let mut f = gpu.fitter(flat, cfg).expect("fitter");
    let mut n = 0;
    while f.step().is_some() {
        n += 1;
    }
    assert!(f.is_done() && f.iter() == n && n < 1000);
    assert!(f.step().is_none());
    assert_eq!(f.render_current().data.len(), 24 * 24 * 3);
    assert_eq!(f.into_report().stop_reason, StopReason::Converged);
}
