"""Depth: 48 independently seeded int8 blocks in sequence on the GPU, through
the C ABI, against the oracle.

- Walk: one pass x -> block 0 -> ... -> block 47 at T = 256, S = 64 (mode
  F16 and F32), gated at the block outputs 7, 15, 23, 31, 39 and 47, the
  checkpoints of the reference's 48-block walk (ltx/walk48.zig:231-246).
- Denoise: ltx_denoise over the 48 blocks for the 8 stage-1 steps
  (1.0 -> 0) at T = 64, S = 32, velocity and latent of every step against
  the oracle trajectory, as ltx/e2e_denoise.zig:314, 331 gates them.

Gates (rel-RMS against the f64 oracle, f32 between blocks as on the GPU):
mode F16 2e-3 (the reference's per-checkpoint and per-step gate), mode F32
1e-5 (the fp32 tolerance) for the walk.

Blocks: synth.make_block_q8 (int8 q uniform, fp16 scales, all seven
projections int8). The oracle's cost on the host (f64, 16 threads): the walk
~0.6 s a block (~30 s), the denoise ~0.25 s a block call (384 calls,
~12 s a step); generating the 48 blocks ~35 s, uploading them ~20 s.
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

N_BLOCKS = 48
CHECKPOINTS = (7, 15, 23, 31, 39, 47)
GATE = {"f16": 2e-3, "f32": 1e-5}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def blocks48():
    say(f"depth: generating {N_BLOCKS} int8 blocks")
    return [synth.make_block_q8(b, seed=3) for b in range(N_BLOCKS)]


@pytest.fixture(scope="module")
def weights48(ctx, blocks48):
    say(f"depth: uploading {N_BLOCKS} blocks")
    ws = [ctx.upload(b) for b in blocks48]
    yield ws
    for w in ws:
        w.free()


@pytest.fixture(scope="module")
def walk_case(blocks48):
    T, S = 256, 64
    inp = synth.make_inputs(T, S, seed=5, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    say(f"depth: oracle walk over {N_BLOCKS} blocks T={T} S={S}")
    x = inp["x"]
    want = {}
    for b, bt in enumerate(blocks48):
        x = oracle.block_forward(bt, dict(inp, x=x), cos, sin, chunk=16).astype(np.float32)
        if b in CHECKPOINTS:
            want[b] = x.copy()
    return dict(inp=inp, cos=cos, sin=sin, want=want)


@pytest.mark.parametrize("mode", ["f16", "f32"])
def test_walk48_checkpoints(ctx, weights48, walk_case, mode):
    c = walk_case
    inp = c["inp"]
    T = inp["x"].shape[0]
    say(f"depth: GPU walk mode={mode} T={T}")
    args = [dev(inp[k]) for k in ("tstab", "tidx", "ctx", "pts2")] + [dev(c["cos"]), dev(c["sin"])]
    bufs = [dev(inp["x"]), torch.empty((T, 4096), dtype=torch.float32, device="cuda")]
    r = {}
    for b, w in enumerate(weights48):
        ctx.forward(w, bufs[b % 2], *args, bufs[(b + 1) % 2], mode=rt.MODES[mode])
        if b in CHECKPOINTS:
            r[b] = oracle.rel_rms(host(bufs[(b + 1) % 2]), c["want"][b])
    say("  " + " ".join(f"b{b}={v:.2e}" for b, v in r.items()))
    assert all(v <= GATE[mode] for v in r.values()), r
    # the walk moves the stream: the last checkpoint is not the input
    assert oracle.rel_rms(c["want"][47], inp["x"]) > 0.1


@pytest.fixture(scope="module")
def denoise48():
    """Inputs of the 48-block, 8-step denoise at T = 64, S = 32; the oracle
    trajectory is computed step by step (oracle_step) as the tests need it."""
    T, S = 64, 32
    g = np.random.default_rng(17)
    clean = g.standard_normal((T, 128)).astype(np.float32)
    noise = g.standard_normal((T, 128)).astype(np.float32)
    mask, tidx = conditioning.mask_rows(T)
    sig = rt.sched_sigmas(1)
    lat0 = oracle.sched_noise_init(clean, noise, mask[tidx], 128, sig[0]).reshape(T, 128)
    ctx_tok = synth.rng(6, "ctx").standard_normal((S, 4096), dtype=np.float32)
    cos, sin = rt.rope_tables(synth.grid_for_tokens(T))
    return dict(T=T, clean=clean, mask=mask, tidx=tidx, sig=sig, lat0=lat0, ctx=ctx_tok, cos=cos, sin=sin,
                core=conditioning.make_core(7), traj=[], gpu={})


def oracle_step(c, blocks, s):
    """The oracle trajectory up to step s (velocity, latent after the step)."""
    while len(c["traj"]) <= s:
        k = len(c["traj"])
        lat = c["lat0"] if k == 0 else c["traj"][-1][1]
        say(f"depth: oracle denoise step {k} ({N_BLOCKS} blocks)")
        c["traj"] += oracle.denoise(blocks, c["core"], lat, c["clean"], c["mask"], c["tidx"], c["ctx"], c["cos"],
                                    c["sin"], c["sig"][k:k + 2])
    return c["traj"][s]


@pytest.mark.parametrize("step", range(8))
def test_denoise48_step(ctx, blocks48, weights48, denoise48, step):
    """Step `step` of the GPU's own trajectories in modes F16 and F32 (each
    step starts from that trajectory's latent of the step before) against
    the oracle trajectory. F16: velocity and latent 2e-3. F32: latent 1e-5;
    the velocity is printed and held to 2e-5, since the f32 sinusoid of the
    conditioning (phases up to 1,000 rad) differs from the oracle's by ulps
    (tests/test_gpu_core.py isolates that)."""
    c = denoise48
    g = c["gpu"]
    if "core" not in g:
        g["core"] = ctx.upload_core(c["core"])
        g["done"] = 0
        g.update({k: dev(c[k]) for k in ("clean", "mask", "tidx", "ctx", "cos", "sin")})
        for m in GATE:
            g["lat_" + m] = dev(c["lat0"])
    vel_want, lat_want = oracle_step(c, blocks48, step)
    assert g["done"] == step, "steps run in order"
    r = {}
    for m in GATE:
        say(f"depth: GPU denoise step {step} sigma {c['sig'][step]} -> {c['sig'][step + 1]} mode={m}")
        ctx.denoise(weights48, g["core"], g["lat_" + m], g["clean"], g["mask"], g["tidx"], g["ctx"], g["cos"],
                    g["sin"], c["sig"][step:step + 2], mode=rt.MODES[m])
        vel = ctx.stage("velocity").view(torch.float32).reshape(c["T"], 128).cpu().numpy()
        r[m] = (oracle.rel_rms(vel, vel_want), oracle.rel_rms(host(g["lat_" + m]), lat_want))
        say(f"  {m}: velocity {r[m][0]:.3e} latent {r[m][1]:.3e}")
    g["done"] += 1
    if step == 7:
        g["core"].free()
    assert r["f16"][0] <= GATE["f16"] and r["f16"][1] <= GATE["f16"], r
    assert r["f32"][0] <= 2 * GATE["f32"] and r["f32"][1] <= GATE["f32"], r
