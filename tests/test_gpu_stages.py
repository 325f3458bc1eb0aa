"""Per-stage GPU parity of the block forward, through the C ABI.

Every intermediate the forward exposes (ltx_block_stage) is compared with the
oracle's dump of the same stage on identical seeded inputs, the way the
reference gates its staged methods one by one at 2e-3
(ltx/block_conformance.zig:311-350). Besides the stored stages, the three
residual branches are gated on their own, so the residual stream cannot
dilute an error in one of them:
  self-attention branch  x_sa - x      (s3Attn1 * ada2)
  cross-attention branch x_ca - x_sa   (s5CaOut)
  FFN branch             y - x_ca      (s7FfOut * ada5)

Gates (rel-RMS): fp16 operands 2e-3, f32 1e-5 per stage. bf16 operands: the
block output 2e-3, the stages printed and held to 1.5e-2. One bf16 rounding
of a value has a relative RMS error of about 2^-9 / sqrt(3) = 1.1e-3, and a
branch sums several: in an f64 simulation of this pipeline's rounding points
at T = 256 (the GPU's bf16 numbers reproduce within 5 %), rounding only the
modulated norms that feed the GEMMs puts the self-attention branch at
2.5e-3, rounding only the dequantised weights at 2.5e-3 too, and every
rounding together at 5.0e-3 (the block output 1.9e-3). The per-stage 2e-3
gate is out of reach with bf16 MFMA operands by construction; fp16 carries
3 more mantissa bits (the same simulation: 6.3e-4).

Also here: the closed-form special case (tests/blockcases.py) on the GPU,
which pins the AdaLN row order, the K/V modulation and the 2 sigmoid gate
independently of the oracle, and the int8 recipe's own error against the
unquantised block with the reference's pre-registered budgets
(ltx/block_conformance.zig:466-494).
"""
import numpy as np
import pytest

from conftest import say

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import blockcases  # noqa: E402
import oracle  # noqa: E402
from ltx_amd import blockfmt as bf  # noqa: E402
from ltx_amd import runtime as rt  # noqa: E402
from ltx_amd import synth  # noqa: E402

D, H, HD, FF = 4096, 32, 128, 16384
GATE = {"f16": 2e-3, "f32": 1e-5, "bf16": 1.5e-2}
TORCH_DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}
_CACHE = {}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def forward(ctx, w, inp, cos, sin, mode):
    T = inp["x"].shape[0]
    y = torch.empty((T, D), dtype=torch.float32, device="cuda")
    ctx.forward(w, dev(inp["x"]), dev(inp["tstab"]), dev(inp["tidx"]), dev(inp["ctx"]), dev(inp["pts2"]), dev(cos),
                dev(sin), y, mode=rt.MODES[mode])
    torch.cuda.synchronize()
    return y.cpu().numpy().astype(np.float64)


def stage(ctx, name, dtype, shape):
    return ctx.stage(name).view(dtype).reshape(shape).float().cpu().numpy().astype(np.float64)


def gpu_stages(ctx, mode, T, S):
    """Every stage of the last forward, in the oracle's layout [rows][cols]
    and scale (Q divided back by log2(e)/sqrt(128))."""
    dt = TORCH_DT[mode]
    f32 = torch.float32
    g = {"norm_msa": stage(ctx, "norm_msa", dt, (T, D)), "glog1": stage(ctx, "glog1", f32, (T, H)),
         "attn1": stage(ctx, "attn1", dt, (T, D)), "x_sa": stage(ctx, "x_sa", f32, (T, D)),
         "attn_in": stage(ctx, "attn_in", dt, (T, D)), "attn2": stage(ctx, "attn2", dt, (T, D)),
         "x_ca": stage(ctx, "x_ca", f32, (T, D)), "ff_in": stage(ctx, "ff_in", dt, (T, D)),
         "ff_h": stage(ctx, "ff_h", dt, (T, FF)), "glog2": stage(ctx, "glog2", f32, (T, H))}
    if mode == "f32":
        for n, rows in (("q1", T), ("k1", T), ("v1", T), ("q2", T), ("k2", S), ("v2", S)):
            g[n] = stage(ctx, n, f32, (rows, D))
    else:
        for n, rows, sc in (("q1", T, rt.ATTN_C), ("k1", T, 1.0), ("q2", T, rt.ATTN_C), ("k2", S, 1.0)):
            g[n] = stage(ctx, n, dt, (rows, D)) / sc
        for n, rows in (("v1", T), ("v2", S)):
            g[n] = stage(ctx, n, dt, (H, HD, rows)).transpose(2, 0, 1).reshape(rows, D)
    return g


# (GPU stage, oracle stage) pairs stored by both sides
PAIRS = [("norm_msa", "s1_norm_msa"), ("q1", "q1_roped"), ("k1", "k1_roped"), ("v1", "v1"), ("glog1", "glog1"),
         ("attn1", "attn1_merged"), ("x_sa", "s4_after_sa"), ("attn_in", "attn_in"), ("q2", "q2_normed"),
         ("k2", "k2_normed"), ("v2", "v2"), ("glog2", "glog2"), ("attn2", "attn2_merged"), ("x_ca", "x_ca"),
         ("ff_in", "s6_ff_in"), ("ff_h", "ff_h")]


def compare_stages(g, y, want, wst, x):
    """rel-RMS of every stage, the three residual branches and y."""
    r = {a: oracle.rel_rms(g[a], wst[b]) for a, b in PAIRS}
    r["sa_branch"] = oracle.rel_rms(g["x_sa"] - x, wst["s4_after_sa"] - x)
    r["ca_branch"] = oracle.rel_rms(g["x_ca"] - g["x_sa"], wst["s5_ca_out"])
    r["ff_branch"] = oracle.rel_rms(y - g["x_ca"], want - wst["x_ca"])
    r["y"] = oracle.rel_rms(y, want)
    return r


@pytest.mark.parametrize("T,S", [(256, 64), (250, 40)])
@pytest.mark.parametrize("mode", ["f16", "f32", "bf16"])
def test_block_stages(ctx, block0, mode, T, S):
    """T = 256, S = 64, and the ragged T = 250, S = 40 (a partial RMSNorm
    group, GEMM row tile and attention tile; the striped mask changes row
    inside a four-row group)."""
    say(f"block stages mode={mode} T={T} S={S}")
    inp = synth.make_inputs(T, S, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    key = ("b0", T, S)
    if key not in _CACHE:
        # the reference's blockwise attention needs a chunk dividing the key
        # count; T = 250 takes the dense softmax (the same softmax in one pass)
        _CACHE[key] = oracle.block_forward(block0, inp, cos, sin, chunk=16 if T % 16 == 0 else 0, stages=True)
    want, wst = _CACHE[key]
    w = ctx.upload(block0)
    y = forward(ctx, w, inp, cos, sin, mode)
    g = gpu_stages(ctx, mode, T, S)
    w.free()
    r = compare_stages(g, y, want, wst, inp["x"].astype(np.float64))
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in r.items()))
    bad = {k: v for k, v in r.items() if not v <= GATE[mode]}
    assert not bad, f"stages over the {GATE[mode]:.0e} gate: {bad}"
    if mode == "bf16":
        assert r["y"] <= 2e-3, r


@pytest.mark.parametrize("T,S", [(256, 64), (2048, 64)])
@pytest.mark.parametrize("mode", ["f16", "bf16"])
def test_unquantised_block_stages(ctx, block0_w16, mode, T, S):
    """The unquantised block (Block.wBlockOut, ltx/block.zig:351-353: every
    projection in bf16 weights, as the reference's production pass calls it,
    ltx/e2e_prod.zig:382-399) in the 16-bit modes, every stage against the
    oracle of the same weights. T = 256 runs the 16-bit-weight GEMMs split
    over K, T = 2,048 whole (256 x 128 tiles fill the CUs). In mode F16 the
    bf16 weights are exact f16 operands (8 significant bits, in range)."""
    say(f"unquantised block stages mode={mode} T={T} S={S}")
    inp = synth.make_inputs(T, S, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    key = ("w16", T, S)
    if key not in _CACHE:
        _CACHE[key] = oracle.block_forward(block0_w16, inp, cos, sin, chunk=64, stages=True)
    want, wst = _CACHE[key]
    w = ctx.upload(block0_w16)
    y = forward(ctx, w, inp, cos, sin, mode)
    g = gpu_stages(ctx, mode, T, S)
    w.free()
    r = compare_stages(g, y, want, wst, inp["x"].astype(np.float64))
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in r.items()))
    bad = {k: v for k, v in r.items() if not v <= GATE[mode]}
    assert not bad, f"stages over the {GATE[mode]:.0e} gate: {bad}"
    if mode == "bf16":
        assert r["y"] <= 2e-3


GEMM_VARIANTS = {
    # every 16-bit GEMM on the four-wave kernel (by default it runs from 4,096
    # rows): the int8 projections dequantised per forward by ltx_gemm_dq16_*,
    # a ragged last row tile, and every epilogue (QKV split with V^T, gated
    # residual, GELU, 16-bit stores)
    "x4": ("LTX_GEMM_X4", "all"),
    # no small-grid kernel: at these sizes the 256 x 256 LDS-DMA kernels with
    # K split over workgroups and the reduce launch
    "s4off": ("LTX_GEMM_S4", "off"),
    # the small-grid kernel (128 x 128 tiles) for every projection, the
    # unquantised ones included, split over K where even its tiles fill at
    # most half the CUs
    "s4all": ("LTX_GEMM_S4", "all"),
    # not a GEMM path: the large-T schedule of the side stream (gate logits
    # after the q|k|v GEMM, the context side on the main stream) at these
    # sizes, where the side stream otherwise starts at the first RMSNorm
    "sideoff": ("LTX_SIDE_EARLY", "off"),
}


@pytest.fixture(scope="module", params=sorted(GEMM_VARIANTS))
def ctx_gemm(request):
    """A context with one GEMM path (or side-stream schedule) forced by its
    environment setting (read when the context is made)."""
    import os
    var, val = GEMM_VARIANTS[request.param]
    old = os.environ.get(var)
    os.environ[var] = val
    try:
        c = rt.Context(0)
    finally:
        if old is None:
            del os.environ[var]
        else:
            os.environ[var] = old
    yield request.param, c
    c.close()


@pytest.mark.parametrize("weights", ["int8", "bf16"])
@pytest.mark.parametrize("T,S", [(256, 64), (250, 40)])
@pytest.mark.parametrize("mode", ["f16", "bf16"])
def test_block_stages_gemm_variants(ctx_gemm, block0, block0_w16, mode, T, S, weights):
    """The block with its projections on another GEMM path: int8 weights and
    the unquantised block, every stage against the oracle under the gates of
    test_block_stages."""
    variant, c = ctx_gemm
    say(f"block stages gemm={variant} mode={mode} T={T} S={S} weights={weights}")
    bt = block0 if weights == "int8" else block0_w16
    inp = synth.make_inputs(T, S, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    key = ("b0" if weights == "int8" else "w16", T, S)
    if key not in _CACHE:
        _CACHE[key] = oracle.block_forward(bt, inp, cos, sin, chunk=16 if T % 16 == 0 else 0, stages=True)
    want, wst = _CACHE[key]
    w = c.upload(bt)
    y = forward(c, w, inp, cos, sin, mode)
    g = gpu_stages(c, mode, T, S)
    w.free()
    r = compare_stages(g, y, want, wst, inp["x"].astype(np.float64))
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in r.items()))
    bad = {k: v for k, v in r.items() if not v <= GATE[mode]}
    assert not bad, f"stages over the {GATE[mode]:.0e} gate: {bad}"
    assert r["y"] <= 2e-3, r


@pytest.mark.parametrize("mode", ["f16", "f32"])
def test_block_closed_form(ctx, block0, mode):
    """The special case of tests/blockcases.py on the GPU: every token's
    gated self-attention output is 2 sigmoid(g(ada0)) v(ada0); the cross
    output is v2 of the modulated context row gated from the GPU's own cross
    queries; the FFN term is ff2(gelu(ff1(ada3))) ada5 for every token."""
    T, S = 64, 16
    say(f"block closed form mode={mode} T={T} S={S}")
    bt, inp = blockcases.special_case(block0, T, S)
    cos, sin = rt.rope_tables(inp["grid"])
    w = ctx.upload(bt)
    y = forward(ctx, w, inp, cos, sin, mode)
    g = gpu_stages(ctx, mode, T, S)
    w.free()
    x = inp["x"].astype(np.float64)
    merged, sa = blockcases.self_branch(bt, inp)
    merged2, ca = blockcases.cross_branch(bt, inp, g["attn_in"])
    ffb = blockcases.ffn_branch(bt, inp)
    r = {"attn1": oracle.rel_rms(g["attn1"], np.tile(merged, (T, 1))),
         "sa_branch": oracle.rel_rms(g["x_sa"] - x, np.tile(sa, (T, 1))),
         "attn2": oracle.rel_rms(g["attn2"], merged2),
         "ca_branch": oracle.rel_rms(g["x_ca"] - g["x_sa"], ca),
         "ff_branch": oracle.rel_rms(y - g["x_ca"], np.tile(ffb, (T, 1))),
         "y": oracle.rel_rms(y, blockcases.block_output(bt, inp))}
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in r.items()))
    bad = {k: v for k, v in r.items() if not v <= GATE[mode]}
    assert not bad, bad


@pytest.mark.parametrize("dist", ["normal", "t3"])
def test_int8_recipe_error_budgets(ctx, dist):
    """The int8 block on the GPU (fp16 operands, the reference's int8 recipe:
    q/k/v and FFN int8, f32 scales) against the f64 oracle of the same block
    with its bf16 weights unquantised, with the budgets the reference
    pre-registers for its own int8 probes (ltx/block_conformance.zig:466-494):
    attention logits 5e-2, attention output (s3Attn1) 2e-2, FFN output
    (s7FfOut) 5e-2, block output 2e-2. Logits: the first 8 heads, all keys.

    Each probe is also measured for the oracle's own int8 block, which is the
    recipe's error with no GPU arithmetic in it: the GPU may add at most 5 %
    of it plus 1e-3. With N(0, 0.02) weights every budget holds. With
    Student-t(3) x 0.02 weights the recipe itself puts the attention output
    at 2.04e-2 (the group-128 absmax scale follows the outliers), just over
    its 2e-2 budget, so that one probe is held to the recipe's own error."""
    T, S = 256, 64
    say(f"int8 recipe error T={T} S={S} f16 weights={dist}")
    bt = synth.make_block(0, seed=1, dist=dist)
    inp = synth.make_inputs(T, S, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    unq = bf.BlockTensors(bt.block, bt.base, {}, {})
    want, wst = oracle.block_forward(unq, inp, cos, sin, chunk=16, stages=True)
    oq, oqst = oracle.block_forward(bt, inp, cos, sin, chunk=16, stages=True)
    w = ctx.upload(bt)
    y = forward(ctx, w, inp, cos, sin, "f16")
    g = gpu_stages(ctx, "f16", T, S)
    w.free()
    x = inp["x"].astype(np.float64)

    def logits(q, k):
        q = q.reshape(T, H, HD)[:, :8].transpose(1, 0, 2)
        k = k.reshape(T, H, HD)[:, :8].transpose(1, 0, 2)
        return q @ k.transpose(0, 2, 1)

    def probes(q1, k1, x_sa, x_ca, yy):
        # the attention output s3Attn1 = (x_sa - x) / ada2 and the FFN output
        # s7FfOut = (y - x_ca) / ada5 are compared through their residual
        # terms (x_sa - x and y - x_ca: the same vectors scaled per channel)
        return {"logits": oracle.rel_rms(logits(q1, k1), logits(wst["q1_roped"], wst["k1_roped"])),
                "attention": oracle.rel_rms(x_sa - x, wst["s4_after_sa"] - x),
                "ffn": oracle.rel_rms(yy - x_ca, want - wst["x_ca"]),
                "block": oracle.rel_rms(yy, want)}

    r = probes(g["q1"], g["k1"], g["x_sa"], g["x_ca"], y)
    rec = probes(oqst["q1_roped"], oqst["k1_roped"], oqst["s4_after_sa"], oqst["x_ca"], oq)
    budget = {"logits": 5e-2, "attention": 2e-2, "ffn": 5e-2, "block": 2e-2}
    say("  " + " ".join(f"{k}: gpu {r[k]:.2e} recipe {rec[k]:.2e} (budget {budget[k]:.0e})" for k in r))
    assert all(r[k] <= 1.05 * rec[k] + 1e-3 for k in r), (r, rec)
    held = [k for k in r if not (dist == "t3" and k == "attention")]
    assert all(r[k] <= budget[k] for k in held), r
    assert r["ffn"] > 1e-3  # the int8 block is not the unquantised one: the probe measures something
