"""Pins of the oracle's restatement of the parts around the blocks
(ltx/core_parts.zig) and of the distilled scheduler (ltx/scheduler.zig).

The reference's bundles for these parts are not in its repository, so each
oracle function is pinned by what fixes it independently:
  - fma_f32 (the lerp's fused multiply-add): libm's correctly rounded fmaf
    and exact rational arithmetic, including cases built so that rounding
    the f64 sum first gives a different f32;
  - sched_lerp: the endpoints, the branch at |w| = 0.5 and the difference
    between the fused and unfused forms that the reference documents
    (ltx/scheduler.zig:20-28);
  - the march: algebraic identities of each operation (mask 1 / 0, dt = 0,
    no snap at sigma_next = 0) and the sigma tables (known answers);
  - the core parts: torch's f64 layer_norm / silu / linear, closed forms of
    the sinusoid, and the reference's wrong-norm control (the RMS-norm tail
    must miss the LayerNorm tail by more than 1e-3, ltx/core_conformance.zig:
    194-212).
"""
import ctypes
from fractions import Fraction

import numpy as np
import pytest

import oracle


def _libm_fmaf():
    m = ctypes.CDLL("libm.so.6")
    m.fmaf.restype = ctypes.c_float
    m.fmaf.argtypes = [ctypes.c_float] * 3
    return m.fmaf


def _exact_round_f32(v: Fraction) -> np.float32:
    """Round a rational to the nearest f32 (ties to even), normal range."""
    if v == 0:
        return np.float32(0.0)
    sgn = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    scale = Fraction(2) ** (23 - e)
    m = round(a * scale)  # Fraction.__round__: half to even
    return np.float32(sgn * float(Fraction(m) / scale))


def _double_rounding_cases(n: int = 64):
    """(a, b, c) with c's last mantissa bit odd and a*b = ulp(c)/2 * (1 - 2^-2k),
    k in [15, 23]: the exact sum lies just below the midpoint above c and
    rounds to c, while the f64 sum lands on the midpoint and then rounds to
    the even neighbour, c + ulp (one rounding against two)."""
    rng = np.random.default_rng(5)
    out = []
    while len(out) < n:
        c = np.float32(rng.uniform(1, 2)) * np.float32(2.0 ** int(rng.integers(-4, 5)))
        if (c.view(np.uint32) & 1) == 0:
            continue
        k = int(rng.integers(15, 24))
        half = np.float64(np.spacing(c)) / 2
        a = np.float32(half * (1 + 2.0 ** -k))
        b = np.float32(1 - 2.0 ** -k)
        sg = np.float32(rng.choice([1, -1]))
        out.append((np.float32(a * sg), b, np.float32(c * sg)))
    return out


def test_fma_f32_matches_libm_and_exact_rationals():
    rng = np.random.default_rng(0)
    a, b, c = (rng.standard_normal(4000).astype(np.float32) for _ in range(3))
    got = oracle.fma_f32(a, b, c)
    fmaf = _libm_fmaf()
    want = np.array([fmaf(float(x), float(y), float(z)) for x, y, z in zip(a, b, c)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for i in range(300):
        ex = _exact_round_f32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i].view(np.uint32) == ex.view(np.uint32), i


def test_fma_f32_hard_cases_differ_from_double_rounding():
    cases = _double_rounding_cases()
    a, b, c = (np.array(v, np.float32) for v in zip(*cases))
    got = oracle.fma_f32(a, b, c)
    fmaf = _libm_fmaf()
    want = np.array([fmaf(float(x), float(y), float(z)) for x, y, z in cases], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for (x, y, z), g in zip(cases, got):
        assert g == _exact_round_f32(Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z)))
    twice = (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)
    assert (twice != got).any(), "the constructed cases must separate one rounding from two"


def test_lerp_endpoints_and_branches():
    rng = np.random.default_rng(1)
    a = rng.standard_normal(5000).astype(np.float32)
    b = rng.standard_normal(5000).astype(np.float32)
    assert np.array_equal(oracle.sched_lerp(a, b, 1.0), b)  # second branch, 1 - w = 0
    assert np.array_equal(oracle.sched_lerp(a, b, 0.0), a)  # first branch, w = 0
    # w = 0.5 is NOT < 0.5: b - (b - a) * 0.5, fused
    d = (b - a).astype(np.float32)
    w05 = oracle.sched_lerp(a, b, 0.5)
    assert np.array_equal(w05, oracle.fma_f32(-d, np.float32(0.5), b))
    for w in (0.3, 0.909375, -0.7):
        fused = oracle.sched_lerp(a, b, w)
        unfused = oracle.sched_lerp(a, b, w, fused=False)
        assert (fused != unfused).any(), f"w={w}: the fused lerp must differ from the two-rounding form"
        exact = (a.astype(np.float64) + w * (b.astype(np.float64) - a))
        assert np.abs(fused - exact).max() <= 2 * np.spacing(np.abs(exact).max().astype(np.float32))


def test_noise_init_mask_rows():
    rng = np.random.default_rng(2)
    T, Cc = 21, 128
    clean = rng.standard_normal((T, Cc)).astype(np.float32)
    noise = rng.standard_normal((T, Cc)).astype(np.float32)
    mtok = np.array([0.0] * 7 + [1.0] * 7 + [0.5] * 7, np.float32)
    out = oracle.sched_noise_init(clean, noise, mtok, Cc, 1.0).reshape(T, Cc)
    assert np.array_equal(out[:7], clean[:7])  # mask 0 keeps the clean latent
    assert np.array_equal(out[7:14], noise[7:14])  # scale 1, mask 1: pure noise
    mid = oracle.sched_lerp(clean[14:], noise[14:], 0.5)
    assert np.array_equal(out[14:], mid)


def test_march_identities():
    rng = np.random.default_rng(3)
    T, Cc = 14, 128
    x = rng.standard_normal((T, Cc)).astype(np.float32)
    v = rng.standard_normal((T, Cc)).astype(np.float32)
    clean = rng.standard_normal((T, Cc)).astype(np.float32)
    mask = np.array([0.0, 1.0], np.float32)
    tidx = np.array([0] * 7 + [1] * 7, np.int32)
    ts, den, post, nxt = oracle.sched_step(x, v, mask, tidx, clean, 0.725, 0.421875)
    assert np.array_equal(ts, np.array([0.0] * 7 + [np.float32(0.725)] * 7, np.float32))
    assert np.array_equal(den[:7], x[:7])  # ts = 0
    assert np.array_equal(post[:7], clean[:7])  # mask 0
    assert np.array_equal(post[7:], den[7:])  # mask 1
    assert np.array_equal(den[7:], x[7:] - v[7:] * np.float32(0.725))
    # dt = 0 leaves the latent unchanged
    _, _, _, same = oracle.sched_step(x, v, mask, tidx, clean, 0.725, 0.725)
    assert np.array_equal(same, x)
    # no snap at the final step: close to the denoised latent, not equal to it
    _, _, post0, last = oracle.sched_step(x, v, mask, tidx, clean, 0.421875, 0.0)
    assert not np.array_equal(last, post0)
    assert np.abs(last - post0).max() <= 4 * np.spacing(np.float32(8.0))


def test_sigma_tables_known_answer():
    from ltx_amd import runtime as rt
    assert np.array_equal(rt.sched_sigmas(1), oracle.SIGMAS_STAGE1)
    assert np.array_equal(rt.sched_sigmas(2), oracle.SIGMAS_STAGE2)
    assert np.array_equal(oracle.SIGMAS_STAGE1[5:], oracle.SIGMAS_STAGE2)
    assert oracle.SIGMAS_STAGE1[0] == 1.0 and oracle.SIGMAS_STAGE1[-1] == 0.0
    assert np.all(np.diff(oracle.SIGMAS_STAGE1) < 0)


def test_sinusoid_closed_forms():
    s = oracle.core_sinusoid(np.array([0.0, 0.5, 0.001], np.float32))
    assert s.shape == (3, 256)
    assert np.array_equal(s[0, :128], np.ones(128, np.float32)) and np.array_equal(s[0, 128:], np.zeros(128))
    # freq 0 is exactly 1: column 0 is cos(1000 t), column 128 sin(1000 t)
    assert s[1, 0] == np.cos(np.float32(500.0)) and s[1, 128] == np.sin(np.float32(500.0))
    assert s[2, 0] == np.cos(np.float32(np.float32(0.001) * np.float32(1000.0)))
    # every column against f64 math with f32 frequencies (phase up to 1000 rad)
    t = np.linspace(0, 1, 33, dtype=np.float32)
    f = np.exp(np.arange(128, dtype=np.float32) * np.float32(-np.log(1e4) / 128)).astype(np.float64)
    arg = (t.astype(np.float64) * 1000.0)[:, None] * f[None, :]
    want = np.concatenate([np.cos(arg), np.sin(arg)], 1)
    got = oracle.core_sinusoid(t)
    assert np.abs(got - want).max() < 2e-4  # f32 phase rounding at |arg| <= 1000
    assert oracle.rel_rms(got, want) < 2e-5


def test_core_layers_match_torch_f64():
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    rng = np.random.default_rng(4)
    x = rng.standard_normal((37, 4096)) * 3 + 0.5
    n = oracle.core_layernorm(x)
    want = F.layer_norm(torch.from_numpy(x), (4096,), eps=1e-6).numpy()
    assert np.abs(n - want).max() < 1e-12
    assert oracle.rel_rms(oracle.core_silu(x), F.silu(torch.from_numpy(x)).numpy()) < 1e-15
    from ltx_amd import conditioning
    cw = conditioning.make_core(7)
    lat = rng.standard_normal((5, 128)).astype(np.float32)
    w = torch.from_numpy(((cw["pat_w"].astype(np.uint32) << 16).view(np.float32)).astype(np.float64))
    b = torch.from_numpy(((cw["pat_b"].astype(np.uint32) << 16).view(np.float32)).astype(np.float64))
    want = F.linear(torch.from_numpy(lat.astype(np.float64)), w, b).numpy()
    assert oracle.rel_rms(oracle.core_patchify(cw, lat), want) < 1e-14


def test_tail_wrong_norm_has_teeth():
    """The RMS-norm tail must miss the LayerNorm tail by > 1e-3 on inputs with
    a non-zero row mean (ltx/core_conformance.zig:194-212)."""
    from ltx_amd import conditioning
    cw = conditioning.make_core(7)
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((64, 4096)) + 0.3).astype(np.float32)
    e = oracle.core_emb(cw, np.array([0.7], np.float32))[np.zeros(64, np.int64)]
    good = oracle.core_tail_from_emb(cw, x, e)
    bad = oracle.core_tail_from_emb(cw, x, e, wrong_norm=True)
    assert oracle.rel_rms(bad, good) > 1e-3


def test_conditioning_helper_matches_oracle():
    """The host-side table synthesis (ltx_amd.conditioning.tables) draws the
    same MLP weights as make_core: its f32 tables agree with the f64 oracle."""
    from ltx_amd import conditioning
    cw = conditioning.make_core(7)
    tstab, tidx, pts2 = conditioning.tables(0.7, 64)
    mask, tidx2 = conditioning.mask_rows(64)
    assert np.array_equal(tidx, tidx2)
    t = oracle.sched_timesteps(mask, 0.7)
    assert oracle.rel_rms(tstab, oracle.core_ts9r(cw, t)) < 1e-5
    assert oracle.rel_rms(pts2, oracle.core_pts2r(cw, 0.7)) < 1e-5
