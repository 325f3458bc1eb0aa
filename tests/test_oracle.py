"""Pins of the oracle (CPU). Each oracle function is checked against
something other than its own formula: golden vectors from the reference's
tools, known answers recorded in the reference, an independent numpy
restatement, closed forms / invariants, brute force on tiny inputs, and
planted mistakes that must be caught.
"""
import json
import pathlib

import numpy as np
import pytest

import oracle
from ltx_amd import blockfmt as bf
from ltx_amd import synth

GOLD = pathlib.Path(__file__).resolve().parent / "golden" / "quant_pack"


# ---- RoPE tables (ltx/block_conformance.zig:87-126) ------------------------

def reference_probe_grid(T=64):
    """The position pattern of the reference's oracle bundle grid
    (tools/make_oracle_bundle.py:55-78): per-axis probes hitting both ends,
    then a mesh; start == end, integer positions."""
    t_probe = [0, 3, 6, 9, 12, 15, 17, 20]
    hw_probe = [0, 292, 585, 877, 1170, 1462, 1755, 2048]
    g = np.zeros((3, T), np.float64)
    g[0, :8] = t_probe
    g[1, 8:16] = hw_probe
    g[2, 16:24] = hw_probe
    for k, i in enumerate(range(24, T)):
        g[0, i] = (k * 3) % 20
        g[1, i] = (k * 97) % 2048
        g[2, i] = (k * 53) % 2048
    return np.stack([g, g], axis=-1).astype(np.float32)


@pytest.mark.parametrize("grid", [reference_probe_grid(), synth.latent_grid(4, 16, 16), synth.latent_grid(2, 3, 5)])
def test_rope_tables_c_equals_numpy(grid):
    c_cos, c_sin = oracle.rope_tables(grid)
    n_cos, n_sin = oracle.rope_tables_np(grid)
    assert np.array_equal(c_cos.view(np.uint32), n_cos.view(np.uint32))
    assert np.array_equal(c_sin.view(np.uint32), n_sin.view(np.uint32))


def test_rope_identity_slots_and_known_answers():
    grid = reference_probe_grid()
    cos, sin = oracle.rope_tables(grid)
    # head 0 slots 0, 1 are the prepended identity pad (ltx/block_conformance.zig:155-163)
    assert (cos[0, :, :2] == 1.0).all() and (sin[0, :, :2] == 0.0).all()
    # freq[0] is f32(pi/2), not pi/2 (the "cos(f32(pi/2))" finding recorded by the reference)
    f = oracle.rope_freqs()
    assert f[0] == float(np.float32(np.pi / 2)) and f[0] != np.pi / 2
    assert f[-1] == float(np.float32(10000.0 * np.pi / 2))
    # token 7 sits at t = 20 = max_pos -> arg_t = +1: slot 2 (k=0, axis t) = cos(f32(pi/2))
    assert cos[0, 7, 2] == np.float32(np.cos(float(np.float32(np.pi / 2))))
    assert sin[0, 7, 2] == np.float32(np.sin(float(np.float32(np.pi / 2))))
    # token 0 at the origin: arg = -1 on every axis
    assert cos[0, 0, 3] == np.float32(np.cos(-f[0])) and sin[0, 0, 4] == np.float32(np.sin(-f[0]))


def test_rope_freq_grid_division_and_linspace_agree():
    """k/681 (the Zig restatement) and k*(1/681) (numpy linspace) give the
    same f32 frequency grid, so the restatement choice cannot matter."""
    div = np.array([np.float32(10000.0 ** (k / 681) * (np.pi / 2)) for k in range(682)], np.float64)
    assert np.array_equal(div, oracle.rope_freqs())


# ---- quantizer (tools/quantize_block.py:51-59) -----------------------------

def _golden_input(name):
    man = json.loads((GOLD / "input" / "manifest.json").read_text())
    e = man["tensors"][name]
    raw = (GOLD / "input" / e["file"]).read_bytes()
    dt = np.uint16 if e["dtype"] == "BF16" else np.float32
    return np.frombuffer(raw, dt).reshape(e["shape"]), e


@pytest.mark.parametrize("name", ["transformer_blocks.0.attn1.to_q.weight", "transformer_blocks.0.ff.net.0.proj.weight"])
def test_quantizer_matches_reference_tool_output(name):
    w, e = _golden_input(name)
    stem = e["file"].removesuffix(".bin")
    gq = np.frombuffer((GOLD / "output" / f"{stem}_q8.bin").read_bytes(), np.int8).reshape(w.shape)
    gs = np.frombuffer((GOLD / "output" / f"{stem}_q8scale.bin").read_bytes(), np.float32).reshape(w.shape[0], -1)
    for q, s in (oracle.quantize(w), oracle.quantize_np(w), bf.quantize_g128(w)):
        assert np.array_equal(q, gq)
        assert np.array_equal(s.view(np.uint32), gs.view(np.uint32))


def test_quantizer_properties():
    rng = np.random.default_rng(5)
    w = bf.bf16_bits((rng.standard_t(3, size=(64, 1024)) * 0.02).astype(np.float32))
    q, s = oracle.quantize(w)
    wf = bf.bf16_to_f32(w).astype(np.float64).reshape(64, 8, 128)
    am = np.abs(wf).max(axis=2)
    assert np.array_equal(s, (am / 127).astype(np.float32))          # s = absmax / 127
    assert np.abs(q).max() <= 127                                      # never -128
    s64 = am / 127  # the f64 scale the quantizer divides by (the file stores its f32 rounding)
    err = np.abs(q.reshape(64, 8, 128) * s64[:, :, None] - wf)
    assert (err <= s64[:, :, None] * (0.5 + 1e-12)).all()             # round to nearest
    # the group maximum maps to exactly +-127
    assert (np.abs(q.reshape(64, 8, 128)).max(axis=2) == 127).all()


# ---- dequant (ltx/block.zig:462-471) ---------------------------------------

def test_dequant_exhaustive():
    q = np.tile(np.arange(-128, 128, dtype=np.int16).astype(np.int8), (64, 1)).reshape(64, 256)
    rng = np.random.default_rng(9)
    s = (10.0 ** rng.uniform(-8, 2, size=(64, 2))).astype(np.float32)
    s[0] = [1.0, 2.0 ** -126]
    want = q.astype(np.float32) * np.repeat(s, 128, axis=1)  # numpy f32 multiply: one IEEE rounding
    got = oracle.dequant(q, s)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = oracle.dequant(q, s.astype(np.float16))
    want16 = q.astype(np.float32) * np.repeat(s.astype(np.float16).astype(np.float32), 128, axis=1)
    assert np.array_equal(got16.view(np.uint32), want16.view(np.uint32))


# ---- attention (ltx/block.zig:105-154 and the dense sdpa) ------------------

def test_sdpa_blockwise_dense_bruteforce():
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((n, 4096)) for n in (8, 64, 64))
    dense = oracle.sdpa(q, k, v, chunk=0)
    for chunk in (16, 32, 64):
        assert oracle.rel_rms(oracle.sdpa(q, k, v, chunk=chunk), dense) < 1e-13
    # brute force, one (query, head) at a time, in plain Python loops
    sc = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))
    for i, h in ((0, 0), (5, 17), (7, 31)):
        s = [sum(q[i, h * 128 + e] * k[j, h * 128 + e] * sc for e in range(128)) for j in range(64)]
        m = max(s)
        p = [np.exp(x - m) for x in s]
        o = [sum(p[j] * v[j, h * 128 + e] for j in range(64)) / sum(p) for e in range(128)]
        assert np.allclose(dense[i, h * 128:(h + 1) * 128], o, rtol=1e-12, atol=1e-13)
    assert oracle.rel_rms(oracle.sdpa_np(q, k, v), dense) < 1e-13


def test_sdpa_special_cases():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((4, 4096))
    k = np.tile(rng.standard_normal((1, 4096)), (32, 1))
    v = rng.standard_normal((32, 4096))
    out = oracle.sdpa(q, k, v, chunk=16)
    assert np.allclose(out, v.mean(0)[None, :], atol=1e-12)  # identical keys -> mean of V
    with pytest.raises(ValueError):
        oracle.sdpa(q, k[:30], v[:30], chunk=16)  # whileSdpaC needs chunk | L


# ---- the block (ltx/block.zig:544-574) -------------------------------------

@pytest.fixture(scope="module")
def small_case(block0):
    inp = synth.make_inputs(16, 8, sigma=0.7)
    c, s = oracle.rope_tables(inp["grid"])
    return block0, inp, np.ascontiguousarray(c.transpose(1, 0, 2)), np.ascontiguousarray(s.transpose(1, 0, 2))


def test_block_c_equals_numpy_restatement(small_case):
    bt, inp, cos, sin = small_case
    c = oracle.block_forward(bt, inp, cos, sin, chunk=16)
    n = oracle.block_np(bt, inp, cos, sin)
    assert oracle.rel_rms(c, n) < 1e-12
    assert oracle.rel_rms(oracle.block_forward(bt, inp, cos, sin, chunk=0), c) < 1e-13  # blockwise == dense
    f32 = oracle.block_forward(bt, inp, cos, sin, chunk=16, real="f32")
    assert oracle.rel_rms(f32, c) < 1e-5  # the f32 twin of the f64 oracle (the reference measured 1.85e-6)


@pytest.mark.parametrize("mistake", ["layernorm", "gate_no_2x", "rope_sign", "kv_scale", "ada_swap"])
def test_block_planted_mistakes_are_caught(small_case, mistake):
    """Teeth: the numpy restatement with one plausible mistake planted must
    fail the f16 block gate (2e-3) by at least 2x. (LayerNorm vs RMSNorm is
    the weakest: rows of N(0, 1) have near-zero mean, ~8e-3.)"""
    bt, inp, cos, sin = small_case
    ref = oracle.block_forward(bt, inp, cos, sin, chunk=16)
    bad = oracle.block_np(bt, inp, cos, sin, mistake=mistake)
    assert oracle.rel_rms(bad, ref) > 4e-3


def test_block_zero_gates_identity(small_case):
    bt, inp, cos, sin = small_case
    inp = dict(inp)
    inp["tidx"] = np.zeros_like(inp["tidx"])
    base = dict(bt.base)
    sst = base["sst"].copy()
    for i in (2, 5, 8):
        sst[i] = -inp["tstab"][0, i]
    base["sst"] = sst
    bt2 = bf.BlockTensors(0, base, bt.q8, bt.q8s)
    out = oracle.block_forward(bt2, inp, cos, sin, chunk=16)
    assert np.array_equal(out, inp["x"].astype(np.float64))


def test_block_chunk_must_divide_keys(block0):
    """The blockwise attention's chunk must divide the key count, as the
    reference asserts (ltx/block.zig:112); the dense softmax (chunk 0) takes
    any length and agrees with a dividing chunk."""
    inp = synth.make_inputs(20, 8, sigma=0.7)
    c, s = oracle.rope_tables(inp["grid"])
    c, s = np.ascontiguousarray(c.transpose(1, 0, 2)), np.ascontiguousarray(s.transpose(1, 0, 2))
    with pytest.raises(ValueError):
        oracle.block_forward(block0, inp, c, s, chunk=16)
    with pytest.raises(ValueError):
        oracle.block_forward(block0, inp, c, s, chunk=10, cross_chunk=3)
    dense = oracle.block_forward(block0, inp, c, s, chunk=0)
    blk = oracle.block_forward(block0, inp, c, s, chunk=10, cross_chunk=4)
    assert np.isfinite(dense).all()
    assert oracle.rel_rms(blk, dense) < 1e-12


def test_block_rows_equal_whole_block(block0):
    """The row-subset oracle (every token's keys and values, the other ops on
    the chosen rows) returns exactly those rows of the whole block, stages
    included."""
    inp = synth.make_inputs(48, 8, sigma=0.7)
    c, s = oracle.rope_tables(inp["grid"])
    c, s = np.ascontiguousarray(c.transpose(1, 0, 2)), np.ascontiguousarray(s.transpose(1, 0, 2))
    full, fst = oracle.block_forward(block0, inp, c, s, chunk=16, stages=True)
    rows = np.array([0, 5, 6, 7, 30, 47])
    part, pst = oracle.block_forward(block0, inp, c, s, chunk=16, stages=True, rows=rows)
    assert np.array_equal(part, full[rows])
    for name in oracle.ST_NAMES:
        want = fst[name] if pst[name].shape[0] != len(rows) else fst[name][rows]
        assert np.array_equal(pst[name], want), name
    with pytest.raises(ValueError):
        oracle.block_forward(block0, inp, c, s, chunk=16, rows=[48])


def test_block_tidx_outside_rows_takes_row_zero(block0):
    """adaVal's select chain (ltx/block.zig:47-67) starts from row 0 and
    replaces it only for an index k in 1 .. K-1, so an index outside that
    range reads row 0."""
    inp = synth.make_inputs(16, 8, sigma=0.7)
    assert inp["tstab"].shape[0] == 3
    c, s = oracle.rope_tables(inp["grid"])
    c, s = np.ascontiguousarray(c.transpose(1, 0, 2)), np.ascontiguousarray(s.transpose(1, 0, 2))
    bad = dict(inp)
    bad["tidx"] = inp["tidx"].copy()
    bad["tidx"][[1, 5, 9, 12]] = [-1, 3, 100, -7]
    fixed = dict(inp)
    fixed["tidx"] = inp["tidx"].copy()
    fixed["tidx"][[1, 5, 9, 12]] = 0
    a = oracle.block_forward(block0, bad, c, s, chunk=16)
    b = oracle.block_forward(block0, fixed, c, s, chunk=16)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, oracle.block_forward(block0, inp, c, s, chunk=16))


# ---- closed forms that pin the block's composition (tests/blockcases.py) ---

@pytest.fixture(scope="module")
def special(block0):
    import blockcases

    bt, inp = blockcases.special_case(block0, 16, 8)
    c, s = oracle.rope_tables(inp["grid"])
    c, s = np.ascontiguousarray(c.transpose(1, 0, 2)), np.ascontiguousarray(s.transpose(1, 0, 2))
    out, st = oracle.block_forward(bt, inp, c, s, chunk=16, stages=True)
    return bt, inp, c, s, out, st


def test_oracle_self_attention_closed_form(special):
    """Scale row ada1 = -1: every token's modulated norm is the shift row
    ada0, every value row is v(ada0), so the gated self-attention output of
    every token is 2 sigmoid(g(ada0)) v(ada0) whatever RoPE and the softmax
    do (pins which AdaLN row is the shift and the 2 sigmoid gate taken from
    the attention input, ltx/block.zig:237-241, 248-252)."""
    import blockcases

    bt, inp, _, _, _, st = special
    merged, sa = blockcases.self_branch(bt, inp)
    T = inp["x"].shape[0]
    assert oracle.rel_rms(st["attn1_merged"], np.tile(merged, (T, 1))) < 1e-12
    assert oracle.rel_rms(st["s4_after_sa"] - inp["x"].astype(np.float64), np.tile(sa, (T, 1))) < 1e-12


def test_oracle_cross_attention_closed_form(special):
    """Identical context rows: every key and value row is the same, so the
    cross output of every query is v2(ctx (1 + kv[1]) + kv[0]) with
    kv = psst + pts2 (pins the K/V modulation, ltx/block.zig:553-556, 291-306)."""
    import blockcases

    bt, inp, _, _, _, st = special
    merged, ca = blockcases.cross_branch(bt, inp, st["attn_in"])
    assert oracle.rel_rms(st["attn2_merged"], merged) < 1e-12
    assert oracle.rel_rms(st["s5_ca_out"], ca) < 1e-12


def test_oracle_ffn_closed_form(special):
    """Scale row ada4 = -1: the FFN input is the shift row ada3 for every
    token, so every FFN row is ff2(gelu(ff1(ada3))) times the gate row ada5
    (ltx/block.zig:320-338, 569-573)."""
    import blockcases

    bt, inp, _, _, out, st = special
    T = inp["x"].shape[0]
    assert oracle.rel_rms(out - st["x_ca"], np.tile(blockcases.ffn_branch(bt, inp), (T, 1))) < 1e-12


@pytest.mark.parametrize("mistake", ["ada_swap", "ca_swap", "ff_swap", "kv_swap", "kv_scale", "gate_no_2x"])
def test_closed_form_catches_planted_mistakes(special, mistake):
    """The oracle equals the closed form of the whole special-case block; the
    numpy restatement with each planted mistake misses it by far more than
    the f16 gate. (A RoPE sign error cannot show here, every value row being
    the same, and LayerNorm for RMSNorm only weakly, through the cross
    queries: the dense restatement and the RoPE table pins catch those.)"""
    import blockcases

    bt, inp, c, s, out, _ = special
    want = blockcases.block_output(bt, inp)
    assert oracle.rel_rms(out, want) < 1e-12
    assert oracle.rel_rms(oracle.block_np(bt, inp, c, s), want) < 1e-12
    assert oracle.rel_rms(oracle.block_np(bt, inp, c, s, mistake=mistake), want) > 4e-3


# ---- RMSNorm, GELU-tanh and the RoPE application ---------------------------
# Pinned by library routines (torch f64) and by invariants of the rotation,
# not by restating the oracle's own expressions. Each check is also run on a
# numpy variant with a planted mistake, which it must reject.

def _bf16_bits(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _rms_rows_input():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((6, D)) * rng.uniform(0.05, 50.0, (6, 1))
    x[0] *= 1e-4  # mean(x^2) ~ 1e-8 < eps: the eps placement decides this row
    x[1, ::7] += 40.0  # outliers
    return x


def _torch_rms(x, w_bits=None):
    import torch
    import torch.nn.functional as F
    w = None if w_bits is None else torch.from_numpy(
        (w_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64))
    return F.rms_norm(torch.from_numpy(x), (D,), weight=w, eps=1e-6).numpy()


D = oracle.D


def test_rms_matches_torch_rms_norm():
    """rmsNoW / rmsW (ltx/block.zig:28-34, ZML nn.rmsNorm with eps 1e-6 and
    the norm weight applied after) against torch.nn.functional.rms_norm."""
    x = _rms_rows_input()
    w = _bf16_bits(np.random.default_rng(12).standard_normal(D))
    for wb in (None, w):
        got, want = oracle.rms(x, wb), _torch_rms(x, wb)
        assert np.abs(got - want).max() <= 1e-14 * np.abs(want).max(), wb is None


@pytest.mark.parametrize("mistake", ["eps_outside", "layernorm", "sum_not_mean"])
def test_rms_torch_check_catches_planted_mistakes(mistake):
    x = _rms_rows_input()
    if mistake == "eps_outside":
        bad = x / (np.sqrt((x * x).mean(-1, keepdims=True)) + 1e-6)
    elif mistake == "layernorm":
        c = x - x.mean(-1, keepdims=True)
        bad = c / np.sqrt((c * c).mean(-1, keepdims=True) + 1e-6)
    else:
        bad = x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)
    want = _torch_rms(x)
    assert np.abs(bad - want).max() > 1e-6 * np.abs(want).max()


def _gelu_input():
    x = np.concatenate([np.linspace(-12, 12, 24001), np.array([0.0, -0.0, 1e-300, -1e-300, 30, -30, 1e3, -1e3])])
    return x


def _torch_gelu_tanh(x):
    import torch
    import torch.nn.functional as F
    return F.gelu(torch.from_numpy(x), approximate="tanh").numpy()


def test_gelu_matches_torch_tanh_form():
    """Tensor.gelu (ltx/block.zig:332), the tanh form, against
    torch.nn.functional.gelu(approximate="tanh") in f64, negative tails
    included (where 1 + tanh cancels)."""
    x = _gelu_input()
    got, want = oracle.gelu(x), _torch_gelu_tanh(x)
    assert np.all(np.abs(got - want) <= 1e-13 * np.abs(x) + 1e-300)
    # odd-part identity of any 0.5 x (1 + tanh(odd u)) form, and the limits
    assert np.abs(got - oracle.gelu(-x) - x).max() <= 1e-12
    assert oracle.gelu(np.array([0.0]))[0] == 0.0
    assert oracle.gelu(np.array([-30.0]))[0] == 0.0 and oracle.gelu(np.array([30.0]))[0] == 30.0


@pytest.mark.parametrize("mistake", ["erf", "kappa", "sqrt_pi"])
def test_gelu_torch_check_catches_planted_mistakes(mistake):
    from scipy.special import erf
    x = _gelu_input()[:24001]
    if mistake == "erf":
        bad = 0.5 * x * (1 + erf(x / np.sqrt(2)))
    elif mistake == "kappa":
        bad = 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.0447 * x ** 3)))
    else:
        bad = 0.5 * x * (1 + np.tanh(np.sqrt(1 / np.pi) * (x + 0.044715 * x ** 3)))
    assert np.abs(bad - _torch_gelu_tanh(x)).max() > 1e-9


def _rope_case():
    grid = reference_probe_grid()
    cos, sin = oracle.rope_tables(grid)  # bundle layout [H, T, 64]
    cs, sn = cos.transpose(1, 0, 2).copy(), sin.transpose(1, 0, 2).copy()  # graph layout [T, H, 64]
    x = np.random.default_rng(13).standard_normal((grid.shape[1], D))
    return x, cs, sn


def _rope_variant(x, cs, sn, mistake):
    """numpy RoPE with one planted mistake (for the checks' teeth)."""
    T = x.shape[0]
    c, s = cs.astype(np.float64), sn.astype(np.float64)
    if mistake == "interleaved":  # pairs (2f, 2f+1) instead of (f, f+64)
        x4 = x.reshape(T, oracle.H, 64, 2)
        a, b = x4[..., 0], x4[..., 1]
        return np.stack([a * c - b * s, b * c + a * s], -1).reshape(T, D)
    x4 = x.reshape(T, oracle.H, 2, 64)
    a, b = x4[:, :, 0], x4[:, :, 1]
    if mistake == "sign":
        out = [a * c + b * s, b * c - a * s]
    elif mistake == "cos_sin_swapped":
        out = [a * s - b * c, b * s + a * c]
    elif mistake == "head_slots_shifted":  # head h reads head h+1's slots
        c, s = np.roll(c, -1, axis=1), np.roll(s, -1, axis=1)
        out = [a * c - b * s, b * c + a * s]
    else:
        raise ValueError(mistake)
    return np.concatenate(out, -1).reshape(T, D)


def _rope_checks(rope, x, cs, sn):
    """The invariants a split-half RoPE (ltx/block.zig:69-77, reshape to
    [.., h, p=2, f=64] at ltx/block.zig:220-226) must satisfy; returns the
    names of the checks that fail."""
    import torch
    T = x.shape[0]
    fails = []
    y = rope(x, cs, sn)
    # 1. z = x[h, f] + i x[h, 64 + f] is multiplied by e^{i theta}, cos/sin = the tables (torch complex)
    x4 = torch.from_numpy(x.reshape(T, oracle.H, 2, 64))
    z = torch.complex(x4[:, :, 0], x4[:, :, 1])
    e = torch.complex(torch.from_numpy(cs.astype(np.float64)), torch.from_numpy(sn.astype(np.float64)))
    r = z * e
    want = torch.cat([r.real, r.imag], -1).reshape(T, D).numpy()
    if np.abs(y - want).max() > 1e-14 * np.abs(want).max():
        fails.append("complex")
    # 2. head 0's identity slots (tables (1, 0)): dimensions 0, 1, 64, 65 pass unchanged
    if not np.array_equal(y[:, [0, 1, 64, 65]], x[:, [0, 1, 64, 65]]):
        fails.append("identity")
    # 3. each (f, f + 64) pair keeps its 2-norm (cos^2 + sin^2 = 1 to f32 rounding)
    n0 = x.reshape(T, oracle.H, 2, 64) ** 2
    n1 = y.reshape(T, oracle.H, 2, 64) ** 2
    if np.abs(n1.sum(2) - n0.sum(2)).max() > 1e-6 * n0.sum(2).max():
        fails.append("pair_norm")
    return fails


def test_rope_apply_pinned_by_rotation_invariants():
    x, cs, sn = _rope_case()
    assert _rope_checks(oracle.rope_apply, x, cs, sn) == []


def test_rope_apply_relative_positions():
    """On a grid that moves along one axis only, the per-head dot product of
    a rotated q and a rotated k depends only on the position difference
    (the angle is linear in the position): q and k read the same slots and
    cos, sin are of one angle."""
    for axis in range(3):
        pos = np.zeros((3, 12), np.float32)
        step = 1.0 if axis == 0 else 32.0
        pos[axis] = np.arange(12) * step
        grid = np.ascontiguousarray(np.stack([pos, pos], -1))
        cos, sin = oracle.rope_tables(grid)
        cs, sn = cos.transpose(1, 0, 2).copy(), sin.transpose(1, 0, 2).copy()
        rng = np.random.default_rng(14 + axis)
        q = np.repeat(rng.standard_normal((1, D)), 12, 0)
        k = np.repeat(rng.standard_normal((1, D)), 12, 0)
        rq, rk = oracle.rope_apply(q, cs, sn), oracle.rope_apply(k, cs, sn)
        dots = np.einsum("thd,shd->hts", rq.reshape(12, oracle.H, 128), rk.reshape(12, oracle.H, 128))
        for d in (1, 3, 5):
            for t in range(12 - d - 2):
                a, b = dots[:, t, t + 2], dots[:, t + d, t + 2 + d]
                assert np.abs(a - b).max() <= 1e-5 * np.abs(dots).max(), (axis, d, t)
        # a shift that changes the difference does change the products
        assert np.abs(dots[:, 0, 2] - dots[:, 0, 5]).max() > 1e-3 * np.abs(dots).max()


@pytest.mark.parametrize("mistake", ["interleaved", "sign", "cos_sin_swapped", "head_slots_shifted"])
def test_rope_checks_catch_planted_mistakes(mistake):
    x, cs, sn = _rope_case()
    fails = _rope_checks(lambda a, c, s: _rope_variant(a, c, s, mistake), x, cs, sn)
    assert fails, mistake
    if mistake == "interleaved":
        assert "identity" in fails and "pair_norm" in fails


def test_linear_small_and_blocked_paths_agree_bitwise(block0):
    """The oracle's GEMM takes a panel path for up to 256 rows and a blocked
    path above; both chain each output's fused multiply-adds over k in
    ascending order, so a row's result does not depend on the path (int8
    with f32 scales, int8 with f16 scales, bf16 weights with a bias)."""
    rng = np.random.default_rng(21)
    x = rng.standard_normal((300, D))
    q, s = block0.q8["f1"][:640], block0.q8s["f1"][:640]
    cases = [dict(q=q, s=s), dict(q=q, s=s.astype(np.float16)),
             dict(w_bf16=block0.base["q1_w"][:600], b_bf16=block0.base["q1_b"][:600])]
    for kw in cases:
        big = oracle.linear(x, **kw)
        for rows in (slice(0, 64), slice(37, 293)):
            small = oracle.linear(x[rows], **kw)
            assert np.array_equal(small.view(np.uint64), big[rows].view(np.uint64))
