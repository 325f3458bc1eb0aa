"""The block on both sides of the 4,096-token switch, where the forward
changes GEMM path and schedule together: below it the int8 projections run
the W8A16 / small-grid kernels (split over K where their tiles fill at most
half the CUs) and the second stream starts at the first RMSNorm with the
whole context side; from 4,096 tokens the int8 weights are dequantised once
and run the four-wave 16-bit GEMM (here with a 4-row last M-tile), and the
second stream takes only the gate logits. T = 8,200 adds the launch markers
that a forward records from 8,192 tokens (an 8-row last M-tile). 48 output
rows (with the last tokens) and the three residual branches of those rows
against the f64 row-subset oracle, every projection int8 (the session's
block with f32 scales), fp16 operands: gate rel-RMS 2e-3 (the reference's
per-block gate); bf16 operands at 4,100 tokens: the output 2e-3, its
branches 1.5e-2 (as at the full size)."""
import numpy as np
import pytest

from conftest import say

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle  # noqa: E402
from ltx_amd import runtime as rt  # noqa: E402
from ltx_amd import synth  # noqa: E402

S = 64


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _stage(ctx, name, T, rows):
    t = ctx.stage(name).view(torch.float32).reshape(T, 4096)
    return t[torch.from_numpy(rows).cuda()].cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("T,mode", [(4095, "f16"), (4100, "f16"), (8200, "f16"), (4100, "bf16")])
def test_block_rows_at_size_switch(ctx, block0_out, T, mode):
    block_q8 = block0_out
    say(f"block rows at the size switches T={T} S={S} mode={mode}")
    inp = synth.make_inputs(T, S, sigma=0.7)
    cos, sin = rt.rope_tables(inp["grid"])
    rows = np.unique(np.concatenate([np.linspace(0, T - 1, 44).astype(np.int64), [1, T - 4, T - 3, T - 2]]))
    w = ctx.upload(block_q8)
    y = torch.empty((T, 4096), dtype=torch.float32, device="cuda")
    ctx.forward(w, dev(inp["x"]), dev(inp["tstab"]), dev(inp["tidx"]), dev(inp["ctx"]), dev(inp["pts2"]), dev(cos),
                dev(sin), y, mode=rt.MODES[mode])
    torch.cuda.synchronize()
    assert torch.isfinite(y).all().item()
    got = y[torch.from_numpy(rows).cuda()].cpu().numpy().astype(np.float64)
    x_sa = _stage(ctx, "x_sa", T, rows)
    x_ca = _stage(ctx, "x_ca", T, rows)
    w.free()
    want, wst = oracle.block_forward(block_q8, inp, cos, sin, chunk=0, stages=True, rows=rows)
    x = inp["x"][rows].astype(np.float64)
    r = {"y": oracle.rel_rms(got, want),
         "sa_branch": oracle.rel_rms(x_sa - x, wst["s4_after_sa"] - x),
         "ca_branch": oracle.rel_rms(x_ca - x_sa, wst["s5_ca_out"]),
         "ff_branch": oracle.rel_rms(got - x_ca, want - wst["x_ca"])}
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in r.items()))
    assert r["y"] <= 2e-3, r
    assert all(v <= (2e-3 if mode == "f16" else 1.5e-2) for v in r.values()), r
