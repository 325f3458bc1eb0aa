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
