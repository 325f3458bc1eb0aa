"""Range guard of the 16-bit modes (ltx_range_count), through the C ABI.

The reference computes in f32; the fp16 mode stores the MFMA operands in
f16, whose largest finite value is 65504. The block counts, on the device,
every 16-bit store that is not finite or beyond that, and a forward in fp16
mode refuses weights whose f16 operands would exceed it (the streaming
upload counts its unquantised weights' f16 copies on the device instead).
Checked here:
- AdaLN rows of order 1 (instead of the synthetic tables' 0.1) and
  Student-t(3) activations: nothing out of range, and the block still within
  the fp16 gate of the f64 oracle;
- a context row of 1e5 (the modulated K/V input beyond 65504): the fp16
  forward counts it, the bf16 forward (f32 exponent range) counts nothing;
- an f16 scale large enough that 128 |s| > 65504: the fp16 forward is
  refused, the bf16 forward runs.
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

T, S = 256, 64


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def forward(ctx, w, inp, cos, sin, mode):
    y = torch.empty((T, 4096), dtype=torch.float32, device="cuda")
    ctx.forward(w, dev(inp["x"]), dev(inp["tstab"]), dev(inp["tidx"]), dev(inp["ctx"]), dev(inp["pts2"]), dev(cos),
                dev(sin), y, mode=rt.MODES[mode])
    torch.cuda.synchronize()
    return y.cpu().numpy()


def heavy_inputs():
    """Student-t(3) activations and context, AdaLN rows scaled to rms 1."""
    inp = synth.make_inputs(T, S, sigma=0.7)
    g = np.random.default_rng(31)
    inp["x"] = g.standard_t(3, size=(T, 4096)).astype(np.float32)
    inp["ctx"] = g.standard_t(3, size=(S, 4096)).astype(np.float32)
    tab = inp["tstab"].astype(np.float64)
    rms = np.sqrt((tab ** 2).mean(-1, keepdims=True))
    inp["tstab"] = (tab / rms).astype(np.float32)
    return inp


def test_range_guard_heavy_tails_in_range(ctx, block0):
    say(f"range guard: AdaLN rms 1, Student-t(3) activations, T={T} S={S}, f16")
    inp = heavy_inputs()
    cos, sin = rt.rope_tables(inp["grid"])
    w = ctx.upload(block0)
    ctx.range_count(reset=True)
    got = forward(ctx, w, inp, cos, sin, "f16")
    n = ctx.range_count(reset=True)
    w.free()
    want = oracle.block_forward(block0, inp, cos, sin, chunk=16)
    r = oracle.rel_rms(got, want)
    say(f"  out-of-range stores {n}, rel-RMS {r:.3e}, max |x| {np.abs(inp['x']).max():.0f}")
    assert n == 0
    assert r <= 2e-3


def test_range_guard_counts_overflow(ctx, block0):
    say(f"range guard: a context row of 1e5, T={T} S={S}, f16 then bf16")
    inp = synth.make_inputs(T, S, sigma=0.7)
    inp["ctx"] = inp["ctx"].copy()
    inp["ctx"][5] = 1e5
    cos, sin = rt.rope_tables(inp["grid"])
    w = ctx.upload(block0)
    ctx.range_count(reset=True)
    forward(ctx, w, inp, cos, sin, "f16")
    n16 = ctx.range_count(reset=True)
    yb = forward(ctx, w, inp, cos, sin, "bf16")
    nb = ctx.range_count(reset=True)
    w.free()
    say(f"  f16: {n16} out-of-range stores; bf16: {nb}")
    assert n16 >= 4096  # at least the whole modulated context row
    assert nb == 0 and np.isfinite(yb).all()


def test_f16_mode_refuses_weights_beyond_f16(ctx, block0_out):
    """f16 scales of 600: q s reaches 128 * 600 > 65504."""
    say("range guard: f16 scale 600 -> f16 forward refused, bf16 runs")
    q8s = {k: v.astype(np.float16) for k, v in block0_out.q8s.items()}
    s = q8s["f1"].copy()
    s[3, 2] = np.float16(600.0)
    q8s["f1"] = s
    bt = bf.BlockTensors(0, block0_out.base, block0_out.q8, q8s)
    inp = synth.make_inputs(64, 16, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    w = ctx.upload(bt)
    y = torch.empty((64, 4096), dtype=torch.float32, device="cuda")
    args = [dev(inp[k]) for k in ("x", "tstab", "tidx", "ctx", "pts2")] + [dev(cos), dev(sin), y]
    with pytest.raises(rt.LtxError, match="beyond the f16 range"):
        ctx.forward(w, *args, mode=rt.MODE_F16)
    ctx.forward(w, *args, mode=rt.MODE_BF16)
    torch.cuda.synchronize()
    w.free()
    assert torch.isfinite(y).all().item()


def test_async_upload_counts_unquantised_weights_beyond_f16(ctx, block0_w16):
    """The streaming upload makes the f16 copies of unquantised weights on the
    device and counts those that are not finite there (no host pass over
    them); a forward in fp16 mode adds that count to the range guard, one in
    bf16 mode does not. One bf16 weight of 1e5 in ff1: at least that one
    count in fp16 mode; none for the same weights in bf16 mode, and none for
    the unmodified block in fp16 mode."""
    say("range guard: async-uploaded bf16 weight 1e5 -> counted in f16, not in bf16")
    base = dict(block0_w16.base)
    w1 = base["ff1_w"].copy()
    w1[5, 7] = bf.bf16_bits(np.array([1.0e5], np.float32))[0]
    base["ff1_w"] = w1
    big = bf.BlockTensors(0, base, {}, {})
    inp = synth.make_inputs(T, S, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    counts = {}
    for name, bt in (("big", big), ("plain", block0_w16)):
        blob, man = bf.pack(bt)
        pin = torch.empty(len(blob), dtype=torch.uint8).pin_memory()
        pin.numpy()[:] = np.frombuffer(blob, dtype=np.uint8)
        st = torch.cuda.Stream()
        w = ctx.upload_blob_async(pin.data_ptr(), len(blob), bf.manifest_json(man), bt.block, stream=st)
        st.synchronize()
        for mode in ("f16", "bf16"):
            ctx.range_count(reset=True)
            forward(ctx, w, inp, cos, sin, mode)
            counts[(name, mode)] = ctx.range_count(reset=True)
        w.free()
    say(f"  counts {counts}")
    assert counts[("big", "f16")] >= 1
    assert counts[("big", "bf16")] == 0 and counts[("plain", "f16")] == 0
