"""GPU parity of the parts around the blocks (ltx/core_parts.zig), the
distilled scheduler (ltx/scheduler.zig) and the denoising loop
(ltx/e2e_denoise.zig:218-336) against the oracle, through the C ABI.

Gates:
  scheduler (noise init, the fused march step)   bit-exact
  sinusoid-fed outputs (tstab, emb, pts2)        rel-RMS <= 1e-4: f32 on the
      GPU against f64; the f32 sinusoid's phase (t * 1000 * freq, up to
      1000 rad) turns one-ulp differences of exp into ~1e-5 (the reference
      gates its own f32 sinusoid at 1e-5 and these at 2e-3)
  patchify, tail                                  rel-RMS <= 1e-5
  denoised latent per step, mode f16 / f32        2e-3 / 1e-5 (the reference
      gates velocity and latent per step at 2e-3)
"""
import numpy as np
import pytest

from conftest import say

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle  # noqa: E402
from ltx_amd import conditioning  # noqa: E402
from ltx_amd import runtime as rt  # noqa: E402
from ltx_amd import synth  # noqa: E402


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def core_np():
    return conditioning.make_core(7)


@pytest.fixture(scope="module")
def core_dev(ctx, core_np):
    cw = ctx.upload_core(core_np)
    yield cw
    cw.free()


def _latents(T, seed=11):
    g = np.random.default_rng(seed)
    return (g.standard_normal((T, 128)).astype(np.float32), g.standard_normal((T, 128)).astype(np.float32))


@pytest.mark.parametrize("noise_scale", [1.0, 0.909375, 0.3])
def test_noise_init_bit_exact(ctx, noise_scale):
    say(f"sched noise_init scale={noise_scale}")
    T = 1000
    clean, noise = _latents(T)
    # rows: 0 and 1 (endpoints), 0.5 (second branch), 0.25 (first branch)
    mask = np.array([0.0, 0.5, 1.0, 0.25], np.float32)
    tidx = (np.arange(T) % 4).astype(np.int32)
    out = torch.empty((T, 128), dtype=torch.float32, device="cuda")
    ctx.noise_init(dev(clean), dev(noise), dev(mask), dev(tidx), noise_scale, out)
    got = host(out)
    want = oracle.sched_noise_init(clean, noise, mask[tidx], 128, noise_scale).reshape(T, 128)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("stage", [1, 2])
def test_sched_step_bit_exact_every_step(ctx, stage):
    say(f"sched step bit-exact stage {stage}")
    T = 1001
    clean, x = _latents(T, 12)
    vel = np.random.default_rng(13).standard_normal((T, 128)).astype(np.float32)
    mask, tidx = conditioning.mask_rows(T)
    sig = rt.sched_sigmas(stage)
    dx, dv, dc, dm, dt = dev(x), dev(vel), dev(clean), dev(mask), dev(tidx)
    out = torch.empty_like(dx)
    for i in range(len(sig) - 1):
        tk = dev(oracle.sched_timesteps(mask, sig[i]))
        ctx.sched_step(dx, dv, tk, dm, dt, dc, sig[i], sig[i + 1], out)
        _, _, _, want = oracle.sched_step(x, vel, mask, tidx, clean, sig[i], sig[i + 1])
        got = host(out)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"step {i}"
        x = want
        dx.copy_(out)
    # in place (out == x) is the same
    ctx.sched_step(dx, dv, tk, dm, dt, dc, sig[-2], sig[-1], dx)
    _, _, _, want = oracle.sched_step(x, vel, mask, tidx, clean, sig[-2], sig[-1])
    assert np.array_equal(host(dx).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("sigma,striped", [(0.7, True), (1.0, False), (0.421875, True)])
def test_conditioning(ctx, core_np, core_dev, sigma, striped):
    say(f"core conditioning sigma={sigma} striped={striped}")
    mask, _ = conditioning.mask_rows(64, striped)
    t = oracle.sched_timesteps(mask, sigma)
    K = len(t)
    tstab = torch.empty((K, 9, 4096), dtype=torch.float32, device="cuda")
    emb = torch.empty((K, 4096), dtype=torch.float32, device="cuda")
    pts2 = torch.empty((2, 4096), dtype=torch.float32, device="cuda")
    ctx.conditioning(core_dev, dev(t), dev(np.array([sigma], np.float32)), tstab, emb, pts2)
    r = {
        "tstab": oracle.rel_rms(host(tstab), oracle.core_ts9r(core_np, t)),
        "emb": oracle.rel_rms(host(emb), oracle.core_emb(core_np, t)),
        "pts2": oracle.rel_rms(host(pts2), oracle.core_pts2r(core_np, sigma)),
    }
    print("rel-RMS", r, flush=True)
    assert all(v <= 1e-4 for v in r.values()), r


@pytest.mark.parametrize("T", [1024, 1000])
def test_patchify_and_tail(ctx, core_np, core_dev, T):
    say(f"core patchify + tail T={T}")
    lat, _ = _latents(T, 14)
    x = torch.empty((T, 4096), dtype=torch.float32, device="cuda")
    ctx.patchify(core_dev, dev(lat), x)
    r_pat = oracle.rel_rms(host(x), oracle.core_patchify(core_np, lat))
    # tail on a residual stream with a row mean, emb rows from the oracle
    xs = (np.random.default_rng(15).standard_normal((T, 4096)) * 2 + 0.4).astype(np.float32)
    mask, tidx = conditioning.mask_rows(T)
    emb = oracle.core_emb(core_np, oracle.sched_timesteps(mask, 0.7)).astype(np.float32)
    vel = torch.empty((T, 128), dtype=torch.float32, device="cuda")
    ctx.tail(core_dev, dev(xs), dev(emb), dev(tidx), vel)
    got = host(vel)
    want = oracle.core_tail_from_emb(core_np, xs, emb[tidx])
    r_tail = oracle.rel_rms(got, want)
    r_wrong = oracle.rel_rms(got, oracle.core_tail_from_emb(core_np, xs, emb[tidx], wrong_norm=True))
    print(f"patchify {r_pat:.3e} tail {r_tail:.3e} vs wrong-norm {r_wrong:.3e}", flush=True)
    assert r_pat <= 1e-5 and r_tail <= 1e-5
    assert r_wrong > 1e-3


@pytest.fixture(scope="module")
def denoise_case(core_np):
    """Two blocks, the last three stage-2 steps (0.909375 -> 0.725 -> 0.421875
    -> 0), T = 64, S = 32, and the oracle trajectory."""
    T, S = 64, 32
    blocks = [synth.make_block(b, seed=1, dist="t3") for b in (0, 1)]
    clean, noise = _latents(T, 16)
    mask, tidx = conditioning.mask_rows(T)
    sig = rt.sched_sigmas(2)
    lat0 = oracle.sched_noise_init(clean, noise, mask[tidx], 128, sig[0]).reshape(T, 128)
    ctx_tok = synth.rng(2, "ctx").standard_normal((S, 4096), dtype=np.float32)
    cos, sin = rt.rope_tables(synth.grid_for_tokens(T))
    want = oracle.denoise(blocks, core_np, lat0, clean, mask, tidx, ctx_tok, cos, sin, sig)
    return dict(blocks=blocks, clean=clean, mask=mask, tidx=tidx, sig=sig, lat0=lat0, ctx=ctx_tok, cos=cos, sin=sin,
                want=want)


@pytest.mark.parametrize("mode,gate", [("f16", 2e-3), ("f32", 1e-5)])
def test_denoise_loop(ctx, core_dev, denoise_case, mode, gate):
    """The GPU velocity and latent of each step against the oracle
    trajectory, and one 3-step call against three 1-step calls (bitwise)."""
    c = denoise_case
    sig = c["sig"]
    say(f"denoise loop mode={mode} T=64 S=32 blocks=2 steps=3")
    ws = [ctx.upload(b) for b in c["blocks"]]
    dl, dc, dm, dt, dctx, dcos, dsin = (dev(c[k]) for k in ("lat0", "clean", "mask", "tidx", "ctx", "cos", "sin"))
    md = rt.MODES[mode]
    for s in range(len(sig) - 1):
        ctx.denoise(ws, core_dev, dl, dc, dm, dt, dctx, dcos, dsin, sig[s:s + 2], mode=md)
        vel = ctx.stage("velocity").view(torch.float32).reshape(64, 128).cpu().numpy()
        rv = oracle.rel_rms(vel, c["want"][s][0])
        r = oracle.rel_rms(host(dl), c["want"][s][1])
        print(f"step {s} sigma {sig[s]} -> {sig[s + 1]}: velocity rel-RMS {rv:.3e}, latent rel-RMS {r:.3e}",
              flush=True)
        # both gated every step, as ltx/e2e_denoise.zig:314, 331 gate them; in
        # f32 mode the velocity (two f32 blocks, then the f32 LayerNorm tail
        # and its 4096 -> 128 projection) is held to twice the one-block gate
        assert rv <= (2 * gate if mode == "f32" else gate) and r <= gate, f"step {s}"
    stepped = host(dl)
    dl2 = dev(c["lat0"])
    ctx.denoise(ws, core_dev, dl2, dc, dm, dt, dctx, dcos, dsin, sig, mode=md)
    assert np.array_equal(host(dl2).view(np.uint32), stepped.view(np.uint32))
    for w in ws:
        w.free()


def test_denoise_velocity_f32_from_oracle_conditioning(ctx, core_np, core_dev, denoise_case):
    """Mode F32: the first step's velocity computed on the GPU (patchify,
    both blocks, tail) from the oracle's conditioning tables (ts9r, emb,
    pts2r in f64, rounded to f32) is within the 1e-5 gate of the oracle's
    velocity; from the GPU's own f32 sinusoid-fed tables it is not held to
    it (test_denoise_loop). The excess is the conditioning's: t * 1000 *
    freq reaches 1,000 rad, where one ulp of an f32 exp or of the phase moves
    cos and sin by ~1e-5."""
    c = denoise_case
    T = 64
    sig = c["sig"]
    say("denoise velocity f32 from the oracle's conditioning T=64 blocks=2")
    t = oracle.sched_timesteps(c["mask"], sig[0])
    tstab = oracle.core_ts9r(core_np, t).astype(np.float32)
    emb = oracle.core_emb(core_np, t).astype(np.float32)
    pts2 = oracle.core_pts2r(core_np, sig[0]).astype(np.float32)
    want = c["want"][0][0]
    ws = [ctx.upload(b) for b in c["blocks"]]
    bufs = [torch.empty((T, 4096), dtype=torch.float32, device="cuda") for _ in range(2)]
    ctx.patchify(core_dev, dev(c["lat0"]), bufs[0])
    args = [dev(tstab), dev(c["tidx"]), dev(c["ctx"]), dev(pts2), dev(c["cos"]), dev(c["sin"])]
    for b, w in enumerate(ws):
        ctx.forward(w, bufs[b % 2], *args, bufs[(b + 1) % 2], mode=rt.MODES["f32"])
    vel = torch.empty((T, 128), dtype=torch.float32, device="cuda")
    ctx.tail(core_dev, bufs[len(ws) % 2], dev(emb), dev(c["tidx"]), vel)
    r = oracle.rel_rms(host(vel), want)
    for w in ws:
        w.free()
    print(f"velocity from the oracle's conditioning: rel-RMS {r:.3e}", flush=True)
    assert r <= 1e-5
