"""The block at its full size (T = 28,672 tokens on the (14, 32, 64) grid,
S = 256, every projection int8 with f16 scales, fp16 and bf16 MFMA modes,
and with the f32 scales of the reference's own format in fp16 mode),
checked where an f64 reference is affordable:

- self-attention: 64 query rows (spread over the sequence) of the gated,
  head-merged attention output (stage LTX_ST_ATTN1) against f64 softmax
  attention over all 28,672 keys, computed from the kernel's own 16-bit
  Q, K, V^T and f32 gate logits (stages Q1, K1, V1, GLOG1; Q carries
  log2(e)/sqrt(128), divided back exactly here); gate rel-RMS <= 2e-3 in
  fp16 mode, <= 1e-2 in bf16 mode (P and the output rounded to bf16), the
  attention operator's own gates;
- the FFN up-projection: 32 rows of gelu(ff_in . dq(W_f1)^T) (stage FF_H)
  against f64 from the kernel's own 16-bit input rows (stage FF_IN); gate
  2e-3 in fp16 mode, 6e-3 in bf16 mode (one bf16 rounding of each weight
  operand and of the output), the GEMM operator's own gates;
- size-independent properties of the whole block: finite output, two
  forwards bit-identical, and zeroed residual gates returning x exactly.
"""
import numpy as np
import pytest

from conftest import say

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle  # noqa: E402
from ltx_amd import blockfmt as bf  # noqa: E402
from ltx_amd import runtime as rt  # noqa: E402
from ltx_amd import synth  # noqa: E402

T, S = 28672, 256


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def full():
    bt = synth.make_block(0, seed=1, dist="t3", classes=("qkv", "ff", "out"), scale_dtype="F16")
    inp = synth.make_inputs(T, S, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    return bt, inp, cos, sin


@pytest.fixture(scope="module")
def full_s32(full):
    """The same block with the f32 scales of the reference's own format."""
    _, inp, cos, sin = full
    bt = synth.make_block(0, seed=1, dist="t3", classes=("qkv", "ff", "out"), scale_dtype="F32")
    return bt, inp, cos, sin


@pytest.fixture(scope="module")
def full_w16(full):
    """The same block unquantised (every projection in bf16): Block.wBlockOut
    (ltx/block.zig:351-353), the reference's production caller."""
    _, inp, cos, sin = full
    bt = synth.make_block(0, seed=1, dist="t3", classes=())
    return bt, inp, cos, sin


def _run(ctx, w, inp, cos, sin, mode=rt.MODE_F16):
    y = torch.empty((T, 4096), dtype=torch.float32, device="cuda")
    ctx.forward(w, dev(inp["x"]), dev(inp["tstab"]), dev(inp["tidx"]), dev(inp["ctx"]), dev(inp["pts2"]), dev(cos),
                dev(sin), y, mode=mode)
    torch.cuda.synchronize()
    return y


def _stage(ctx, name, dtype, shape, rows=None):
    t = ctx.stage(name).view(dtype).reshape(shape)
    if rows is not None:
        t = t[torch.from_numpy(rows).cuda()]
    return t.float().cpu().numpy().astype(np.float64)  # 16-bit -> f32 is exact


GATES = {"f16": (2e-3, 2e-3), "bf16": (1e-2, 6e-3)}  # attention rows, ff1 rows


@pytest.mark.parametrize("mode,scales", [("f16", "f16"), ("bf16", "f16"), ("f16", "f32")])
def test_full_size_block(ctx, request, mode, scales):
    bt, inp, cos, sin = request.getfixturevalue("full" if scales == "f16" else "full_s32")
    say(f"full-size block T={T} S={S} {mode} operands, {scales} scales: forward, determinism, attention and FFN rows")
    m = rt.MODES[mode]
    dt = torch.float16 if mode == "f16" else torch.bfloat16
    w = ctx.upload(bt)
    y1 = _run(ctx, w, inp, cos, sin, m)
    assert torch.isfinite(y1).all().item()
    # stages of this forward (rows picked on the device)
    rows = np.linspace(0, T - 1, 64).astype(np.int64)
    frows = np.linspace(3, T - 5, 32).astype(np.int64)
    q = (_stage(ctx, "q1", dt, (T, 32, 128)) / rt.ATTN_C).transpose(1, 0, 2)
    k = _stage(ctx, "k1", dt, (T, 32, 128)).transpose(1, 0, 2)
    vt = _stage(ctx, "v1", dt, (32, 128, T))
    glog = _stage(ctx, "glog1", torch.float32, (T, 32), rows)
    att = _stage(ctx, "attn1", dt, (T, 4096), rows)
    ff_in = _stage(ctx, "ff_in", dt, (T, 4096), frows)
    ff_h = _stage(ctx, "ff_h", dt, (T, 16384), frows)
    y2 = _run(ctx, w, inp, cos, sin, m)
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32)), "two forwards differ"
    w.free()

    scale = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))
    want = np.empty((len(rows), 4096))
    for h in range(32):
        s = (q[h, rows] @ k[h].T) * scale  # [64, T]
        p = np.exp(s - s.max(1, keepdims=True))
        o = (p @ vt[h].T) / p.sum(1, keepdims=True)  # [64, 128]
        want[:, 128 * h:128 * h + 128] = o * (2.0 / (1.0 + np.exp(-glog[:, h])))[:, None]
    r_att = oracle.rel_rms(att, want)

    wf = oracle.dequant(bt.q8["f1"], bt.q8s["f1"]).astype(np.float64)
    hpre = ff_in @ wf.T
    hw = 0.5 * hpre * (1 + np.tanh(np.sqrt(2 / np.pi) * (hpre + 0.044715 * hpre ** 3)))
    r_ff = oracle.rel_rms(ff_h, hw)
    print(f"full size {mode}/{scales}: attention rows rel-RMS {r_att:.3e}, ff1+gelu rows rel-RMS {r_ff:.3e}",
          flush=True)
    g_att, g_ff = GATES[mode]
    assert r_att <= g_att and r_ff <= g_ff


def test_full_size_zero_gates_identity(ctx, full):
    """sst rows 2, 5, 8 set to minus the tstab rows of the single mask row:
    every residual gate is zero, so the block returns x exactly (as values:
    x + v * 0 turns an input -0.0, of which the 117 M normal draws hold a
    few, into +0.0)."""
    bt, inp, cos, sin = full
    say(f"full-size zero-gate identity T={T}")
    inp1 = synth.make_inputs(T, S, sigma=0.7, striped=False)
    b2 = bf.BlockTensors(0, dict(bt.base), bt.q8, bt.q8s)
    sst = b2.base["sst"].copy()
    for i in (2, 5, 8):
        sst[i] = -inp1["tstab"][0, i]
    b2.base["sst"] = sst
    w = ctx.upload(b2)
    y = _run(ctx, w, inp1, cos, sin)
    w.free()
    got = y.cpu().numpy()
    assert np.isfinite(got).all() and np.array_equal(got, inp1["x"])
    differ = got.view(np.uint32) != inp1["x"].view(np.uint32)
    assert (inp1["x"][differ] == 0).all()  # only the sign of zeros may change


# ---- whole-block rows against the oracle at the full size -------------------

# 256 output rows spread over the sequence, with the first and last tokens and
# both sides of each change of the striped timestep row (T/7, 2T/7)
ROWS = np.unique(np.concatenate([np.linspace(0, T - 1, 248).astype(np.int64),
                                 [1, T // 7 - 1, T // 7, 2 * T // 7 - 1, 2 * T // 7, T - 2]]))
_ROW_ORACLE = {}


def _oracle_rows(key, bt, inp, cos, sin):
    """The oracle's block rows: the modulated norm, K and V of all 28,672
    tokens (the self-attention's keys), everything else for ROWS only;
    blockwise attention in chunks of 1,024 as the reference runs it."""
    if key not in _ROW_ORACLE:
        say(f"  oracle rows ({len(ROWS)} of {T}, f64, {key} scales)")
        _ROW_ORACLE[key] = oracle.block_forward(bt, inp, cos, sin, chunk=1024, stages=True, rows=ROWS)
    return _ROW_ORACLE[key]


@pytest.mark.parametrize("mode,scales", [("f16", "f16"), ("f16", "f32"), ("bf16", "f16"), ("f16", "w16"),
                                         ("bf16", "w16"), ("f32", "f16"), ("f32", "f32")])
def test_full_size_block_rows(ctx, request, mode, scales):
    """The block at T = 28,672, S = 256, every projection int8 (scales f16 or
    f32) or every projection bf16 (w16, the unquantised block): output rows,
    and the self-attention, cross-attention and FFN residual branches of
    those rows, against the f64 oracle (gate 2e-3 with fp16 operands, 1e-5
    in f32 mode; with bf16 operands the output 2e-3 and the branches
    1.5e-2)."""
    bt, inp, cos, sin = request.getfixturevalue({"f16": "full", "f32": "full_s32", "w16": "full_w16"}[scales])
    say(f"full-size block rows T={T} S={S} {mode} operands, {scales} scales")
    w = ctx.upload(bt)
    y = _run(ctx, w, inp, cos, sin, rt.MODES[mode])
    assert torch.isfinite(y).all().item()
    sel = torch.from_numpy(ROWS).cuda()
    got = y[sel].cpu().numpy().astype(np.float64)
    x_sa = _stage(ctx, "x_sa", torch.float32, (T, 4096), ROWS)
    x_ca = _stage(ctx, "x_ca", torch.float32, (T, 4096), ROWS)
    w.free()
    del y
    want, wst = _oracle_rows(scales, bt, inp, cos, sin)
    x = inp["x"][ROWS].astype(np.float64)
    r = {"y": oracle.rel_rms(got, want),
         "sa_branch": oracle.rel_rms(x_sa - x, wst["s4_after_sa"] - x),
         "ca_branch": oracle.rel_rms(x_ca - x_sa, wst["s5_ca_out"]),
         "ff_branch": oracle.rel_rms(got - x_ca, want - wst["x_ca"])}
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in r.items()))
    gate = {"f16": 2e-3, "f32": 1e-5}.get(mode, 1.5e-2)
    assert all(v <= gate for v in r.values()), r
    if mode == "bf16":  # bf16 operands: the block output holds the 2e-3 gate, its branches cannot
        assert r["y"] <= 2e-3, r
