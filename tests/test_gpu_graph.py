"""The block forward captured as a HIP graph (ltx_block_graph_*): every replay
equals the eager ltx_block_forward bit for bit, with eager forwards and
synchronisations between the replays; a live graph pins the context's
workspace; capture is refused while event profiling is on."""
import numpy as np
import pytest

from conftest import say

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from ltx_amd import runtime as rt  # noqa: E402
from ltx_amd import synth  # noqa: E402


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _inputs(T, S):
    inp = synth.make_inputs(T, S, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    d = {k: dev(inp[k]) for k in ("x", "tstab", "tidx", "ctx", "pts2")}
    return d, dev(cos), dev(sin)


def _eager(ctx, w, d, cos, sin, y, mode):
    ctx.forward(w, d["x"], d["tstab"], d["tidx"], d["ctx"], d["pts2"], cos, sin, y, mode=mode)


@pytest.mark.parametrize("mode,T,S", [("f16", 256, 64), ("f16", 250, 40), ("bf16", 256, 64), ("f32", 128, 32),
                                      ("f16", 8192, 256)])
def test_block_graph_matches_eager(ctx, block0, mode, T, S):
    """T = 8,192 takes the large-T kernel choices and records the marker
    events after the launches around the second stream (from 8,192 tokens)."""
    say(f"block graph mode={mode} T={T} S={S}")
    md = rt.MODES[mode]
    w = ctx.upload(block0)
    d, cos, sin = _inputs(T, S)
    y_ref = torch.empty((T, 4096), dtype=torch.float32, device="cuda")
    _eager(ctx, w, d, cos, sin, y_ref, md)
    torch.cuda.synchronize()
    want = y_ref.clone()
    y = torch.full((T, 4096), float("nan"), dtype=torch.float32, device="cuda")
    g = ctx.block_graph(w, d["x"], d["tstab"], d["tidx"], d["ctx"], d["pts2"], cos, sin, y, mode=md)
    try:
        torch.cuda.synchronize()
        assert torch.isnan(y).all(), "creating the graph ran kernels"
        for i in range(3):
            y.fill_(float("nan"))
            g.launch()
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int32), want.view(torch.int32)), f"replay {i}"
            # the context's own eager work between the replays
            _eager(ctx, w, d, cos, sin, y_ref, md)
            torch.cuda.synchronize()
            assert torch.equal(y_ref.view(torch.int32), want.view(torch.int32)), f"eager after replay {i}"
        # replays back to back on one stream
        for _ in range(3):
            g.launch()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), want.view(torch.int32))
        # after an eager forward of another size, a launch restores the
        # captured forward's intermediates for ltx_block_stage
        d2, cos2, sin2 = _inputs(64, 16)
        y2 = torch.empty((64, 4096), dtype=torch.float32, device="cuda")
        _eager(ctx, w, d2, cos2, sin2, y2, md)
        g.launch()
        torch.cuda.synchronize()
        assert ctx.stage("x_sa").numel() == T * 4096 * 4
    finally:
        g.free()  # a live graph pins the shared context's workspace
        w.free()


def test_block_graph_pins_workspace(block0):
    say("block graph workspace pin")
    c = rt.Context(0)
    try:
        w = c.upload(block0)
        d, cos, sin = _inputs(64, 16)
        y = torch.empty((64, 4096), dtype=torch.float32, device="cuda")
        g = c.block_graph(w, d["x"], d["tstab"], d["tidx"], d["ctx"], d["pts2"], cos, sin, y, mode=rt.MODE_F16)
        g.launch()
        torch.cuda.synchronize()
        d2, cos2, sin2 = _inputs(512, 16)
        y2 = torch.empty((512, 4096), dtype=torch.float32, device="cuda")
        with pytest.raises(rt.LtxError, match="workspace"):
            _eager(c, w, d2, cos2, sin2, y2, rt.MODE_F16)
        g.free()
        _eager(c, w, d2, cos2, sin2, y2, rt.MODE_F16)
        torch.cuda.synchronize()
        assert torch.isfinite(y2).all()
        w.free()
    finally:
        c.close()


def test_block_graph_refused_while_profiling(ctx, block0):
    say("block graph refused while profiling")
    w = ctx.upload(block0)
    d, cos, sin = _inputs(64, 16)
    y = torch.empty((64, 4096), dtype=torch.float32, device="cuda")
    ctx.profile(True)
    try:
        with pytest.raises(rt.LtxError, match="profiling"):
            ctx.block_graph(w, d["x"], d["tstab"], d["tidx"], d["ctx"], d["pts2"], cos, sin, y, mode=rt.MODE_F16)
    finally:
        ctx.profile(False)
    w.free()


def test_graph_capture_failure_leaves_context_usable(ctx, block0, monkeypatch):
    """A forward that throws inside the capture, after its second stream
    joined it (LTX_FAIL_CAPTURE), fails ltx_block_graph_create with that
    error; the capture is ended with the second stream joined back, so the
    context's eager forwards and a later graph still match the forward from
    before, bit for bit."""
    T, S = 256, 64
    say(f"graph capture failure T={T} S={S}")
    md = rt.MODES["f16"]
    w = ctx.upload(block0)
    d, cos, sin = _inputs(T, S)
    want = torch.empty((T, 4096), dtype=torch.float32, device="cuda")
    _eager(ctx, w, d, cos, sin, want, md)
    torch.cuda.synchronize()
    y = torch.empty_like(want)
    monkeypatch.setenv("LTX_FAIL_CAPTURE", "1")
    with pytest.raises(rt.LtxError, match="LTX_FAIL_CAPTURE"):
        ctx.block_graph(w, d["x"], d["tstab"], d["tidx"], d["ctx"], d["pts2"], cos, sin, y, mode=md)
    monkeypatch.delenv("LTX_FAIL_CAPTURE")
    _eager(ctx, w, d, cos, sin, y, md)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), want.view(torch.int32))
    y.fill_(float("nan"))
    g = ctx.block_graph(w, d["x"], d["tstab"], d["tidx"], d["ctx"], d["pts2"], cos, sin, y, mode=md)
    try:
        g.launch()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), want.view(torch.int32))
    finally:
        g.free()
        w.free()
