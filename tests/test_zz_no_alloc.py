"""ltx_op_linear_q8_noalloc against ltx_op_linear_q8, through the C ABI.

The no-alloc entry point runs the same kernels with its scratch in the
library's static device array, so its output must equal the allocating entry
point's bit for bit. Two calls in a row, the second with a smaller input (so a
stale first-call scratch would show), from a shape on the four-wave GEMM
(weights dequantised into the scratch) down to ones on the W8A16 kernel, in
both 16-bit modes with f16 and f32 scales; the F32 mode (no scratch); and a shape whose scratch exceeds the
array is refused.
"""
import numpy as np
import pytest

from conftest import say

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from ltx_amd import blockfmt as bf  # noqa: E402
from ltx_amd import runtime as rt  # noqa: E402


def _case(M, N, K, seed, scale_f16):
    rng = np.random.default_rng(seed)
    q, s = bf.quantize_g128(bf.bf16_bits((rng.standard_t(3, size=(N, K)) * 0.02).astype(np.float32)))
    if scale_f16:
        s = s.astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    return a, q, s, b


def _both(ctx, mode, M, N, K, seed, scale_f16, gelu, out_f32):
    dt = {rt.MODE_F16: torch.float16, rt.MODE_BF16: torch.bfloat16, rt.MODE_F32: torch.float32}[mode]
    a, q, s, b = _case(M, N, K, seed, scale_f16)
    da = torch.from_numpy(a).to(dt).cuda()
    dq, ds, db = torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(), torch.from_numpy(b).cuda()
    odt = torch.float32 if out_f32 else dt
    y0 = torch.full((M, N), float("nan"), dtype=odt, device="cuda")
    y1 = torch.full((M, N), float("nan"), dtype=odt, device="cuda")
    ctx.linear_q8(da, dq, ds, db, y0, mode=mode, gelu=gelu)
    ctx.linear_q8(da, dq, ds, db, y1, mode=mode, gelu=gelu, noalloc=True)
    torch.cuda.synchronize()
    return y0, y1


@pytest.mark.parametrize("scale_f16", [1, 0])
@pytest.mark.parametrize("mode", [rt.MODE_F16, rt.MODE_BF16])
def test_noalloc_equals_linear_q8(ctx, mode, scale_f16):
    # 4,100 rows: the four-wave GEMM on the weights dequantised into the
    # scratch (ragged last row tile); then smaller calls on the W8A16 kernel
    for M, N, K, gelu, out_f32 in ((4100, 4096, 4096, False, False), (1000, 4096, 4096, True, False),
                                   (300, 512, 1024, False, True)):
        say(f"linear_q8_noalloc mode={mode} scale_f16={scale_f16} M={M} N={N} K={K}")
        y0, y1 = _both(ctx, mode, M, N, K, M + N + K + scale_f16, scale_f16, gelu, out_f32)
        assert torch.isfinite(y0).all().item()
        assert torch.equal(y0.view(torch.int16 if y0.element_size() == 2 else torch.int32),
                           y1.view(torch.int16 if y1.element_size() == 2 else torch.int32))


def test_noalloc_without_scratch_paths(ctx):
    """F32 mode uses no scratch; its results still equal the allocating
    entry point's. A shape both entry points refuse (N not a multiple of 256
    in a 16-bit mode) is refused by both with the same error."""
    M, N, K = 130, 384, 1024
    say(f"linear_q8_noalloc without scratch mode=f32 M={M} N={N} K={K}")
    y0, y1 = _both(ctx, rt.MODE_F32, M, N, K, 7, 1, False, True)
    assert torch.equal(y0.view(torch.int32), y1.view(torch.int32))
    say("linear_q8_noalloc N=320 refused as by linear_q8")
    a = torch.zeros((64, 1024), dtype=torch.float16, device="cuda")
    q = torch.zeros((320, 1024), dtype=torch.int8, device="cuda")
    s = torch.ones((320, 8), dtype=torch.float16, device="cuda")
    y = torch.empty((64, 320), dtype=torch.float32, device="cuda")
    errs = []
    for noalloc in (False, True):
        with pytest.raises(rt.LtxError) as e:
            ctx.linear_q8(a, q, s, None, y, mode=rt.MODE_F16, noalloc=noalloc)
        errs.append(str(e.value).split(": ", 1)[1])
    assert errs[0] == errs[1]


def test_noalloc_refuses_oversized_scratch(ctx):
    """N K + 4 N K / 128 (plus 2 N K from 4,096 rows) beyond the static
    array: refused with an error before any launch (the inputs are never
    read)."""
    say("linear_q8_noalloc oversized shape is refused")
    M, N, K = 256, 32768, 4096  # 128 MiB of weights > the 66 MiB array
    a = torch.empty((M, K), dtype=torch.float16, device="cuda")
    q = torch.empty((N, K), dtype=torch.int8, device="cuda")
    s = torch.empty((N, K // 128), dtype=torch.float16, device="cuda")
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    with pytest.raises(rt.LtxError, match="exceed"):
        ctx.linear_q8(a, q, s, None, y, mode=rt.MODE_F16, noalloc=True)
    # from 4,096 rows the 16-bit weight copy (2 N K) counts too: 32 MiB of
    # weights fit without it (33 MiB) but not with it (97 MiB)
    M, N, K = 4096, 8192, 4096
    say(f"linear_q8_noalloc M={M} N={N} K={K}: no room for the 16-bit weight copy, refused")
    a = torch.empty((M, K), dtype=torch.float16, device="cuda")
    q = torch.empty((N, K), dtype=torch.int8, device="cuda")
    s = torch.empty((N, K // 128), dtype=torch.float16, device="cuda")
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    with pytest.raises(rt.LtxError, match="2 N K bytes"):
        ctx.linear_q8(a, q, s, None, y, mode=rt.MODE_F16, noalloc=True)
