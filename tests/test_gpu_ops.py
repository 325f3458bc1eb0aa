"""GPU parity of the isolated operators against the oracle, through the C ABI.

Tolerances (rel-RMS):
  dequant                     bit-exact (f32 value) / bit-exact RNE to 16-bit
  GEMM vs oracle on the SAME 16-bit operands          <= 1e-5 (accumulation order only)
  GEMM vs exact-weight oracle   f16 <= 1e-3, bf16 <= 6e-3 (one 16-bit rounding of q*s)
  GEMM f32 mode                 <= 1e-5
  attention vs dense f64 oracle on the same 16-bit Q/K/V:  f16 <= 2e-3, bf16 <= 1e-2, f32 <= 1e-5
"""
import numpy as np
import pytest

from conftest import say

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle  # noqa: E402
from ltx_amd import blockfmt as bf  # noqa: E402
from ltx_amd import runtime as rt  # noqa: E402

MODES = {"f16": (rt.MODE_F16, torch.float16), "bf16": (rt.MODE_BF16, torch.bfloat16)}


def to16(a: np.ndarray, dt):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dt)


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("scale_f16", [0, 1])
@pytest.mark.parametrize("mode", ["f16", "bf16"])
def test_dequant_bit_exact(ctx, mode, scale_f16):
    say(f"dequant probe mode={mode} scale_f16={scale_f16}")
    rng = np.random.default_rng(3)
    N, K = 256, 512
    q = np.stack([rng.permutation(np.arange(-128, 128, dtype=np.int16)) for _ in range(N * K // 256)])
    q = q.reshape(N, K).astype(np.int8)
    s = (10.0 ** rng.uniform(-6, 0, size=(N, K // 128))).astype(np.float32)
    s[0, 0], s[1, 1], s[2, 0] = 1.0, 2.0 ** -20, 0.5
    if scale_f16:
        s = s.astype(np.float16)
    want32 = oracle.dequant(q, s)
    m, dt = MODES[mode]
    dq, ds = torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda()
    out32 = torch.empty((N, K), dtype=torch.float32, device="cuda")
    out16 = torch.empty((N, K), dtype=dt, device="cuda")
    ctx.dequant(dq, ds, out32, out16, mode=m)
    torch.cuda.synchronize()
    got32 = out32.cpu().numpy()
    assert np.array_equal(got32.view(np.uint32), want32.view(np.uint32))
    got16 = out16.cpu().view(torch.int16).numpy().view(np.uint16)
    # f16: one round-to-nearest-even of the exact q * s (the fused FMA of the
    # staging path; q * s is exact in f64); bf16: RNE of the f32 value.
    exact = q.astype(np.float64) * np.repeat(s.astype(np.float64), 128, axis=1)
    want16 = exact.astype(np.float16).view(np.uint16) if mode == "f16" else bf.bf16_bits(want32)
    assert np.array_equal(got16, want16)


def _gemm_case(M, N, K, seed, scale_f16=False, t3=True):
    rng = np.random.default_rng(seed)
    w = rng.standard_t(3, size=(N, K)) * 0.02 if t3 else rng.standard_normal((N, K)) * 0.02
    q, s = bf.quantize_g128(bf.bf16_bits(w.astype(np.float32)))
    if scale_f16:
        s = s.astype(np.float16)
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = (rng.standard_normal(N) * 0.1).astype(np.float32)
    return a, q, s, b


@pytest.mark.parametrize("mode", ["f16", "bf16"])
@pytest.mark.parametrize("M,N,K,gelu,out_f32,scale_f16", [
    (256, 512, 4096, False, True, False),
    (300, 256, 4096, True, False, False),   # ragged M, GELU, 16-bit output
    (64, 768, 16384, False, True, True),    # long K, f16 scales
    (512, 1024, 1024, False, False, False),
    (300, 512, 4096, True, False, True),    # f16 scales: ragged M, GELU, 16-bit output
    (768, 1280, 2048, False, True, True),   # f16 scales: several M and N tiles
])
def test_linear_q8(ctx, mode, M, N, K, gelu, out_f32, scale_f16):
    say(f"linear_q8 mode={mode} M={M} N={N} K={K} gelu={gelu} out_f32={out_f32} scale_f16={scale_f16}")
    m, dt = MODES[mode]
    a, q, s, b = _gemm_case(M, N, K, seed=M + N + K, scale_f16=scale_f16)
    da = to16(a, dt).cuda()
    dq, ds = torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda()
    db = torch.from_numpy(b).cuda()
    y = torch.empty((M, N), dtype=torch.float32 if out_f32 else dt, device="cuda")
    ctx.linear_q8(da, dq, ds, db, y, mode=m, gelu=gelu)
    # the 16-bit weight operand, as the GEMM stages it
    w32 = torch.empty((N, K), dtype=torch.float32, device="cuda")
    w16 = torch.empty((N, K), dtype=dt, device="cuda")
    ctx.dequant(dq, ds, w32, w16, mode=m)
    torch.cuda.synchronize()
    a64 = f64(da)

    def post(z):
        z = z + b
        return 0.5 * z * (1 + np.tanh(np.sqrt(2 / np.pi) * (z + 0.044715 * z ** 3))) if gelu else z

    same_ops = post(a64 @ f64(w16).T)
    exact_w = post(a64 @ oracle.dequant(q, s).astype(np.float64).T)
    got = f64(y)
    tol_same = 1e-5 if out_f32 else (1e-3 if mode == "f16" else 6e-3)
    assert oracle.rel_rms(got, same_ops) <= tol_same
    assert oracle.rel_rms(got, exact_w) <= (1e-3 if mode == "f16" else 6e-3)


def _onehot_case(ctx, M, N, K, seed, mode="f16", sf32=False, exp_range=(-4, -1)):
    """y = E . W^T with E[m][k] = (k == m mod K): every output is one weight
    operand times 1, so y must equal the 16-bit operand bit for bit (one
    nonzero product, f32 accumulation): f16 one rounding of the exact q * s,
    bf16 RNE of the f32 value f32(q) * s (as the dequant probe); with f16
    scales q * s is exact in f32 and the two definitions agree."""
    rng = np.random.default_rng(seed)
    q = rng.integers(-128, 128, size=(N, K), dtype=np.int16).astype(np.int8)
    s = (10.0 ** rng.uniform(*exp_range, size=(N, K // 128))).astype(np.float32 if sf32 else np.float16)
    e = np.zeros((M, K), np.float32)
    e[np.arange(M), np.arange(M) % K] = 1.0
    dq, ds = torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    m, dt = MODES[mode]
    ctx.linear_q8(to16(e, dt).cuda(), dq, ds, None, y, mode=m)
    torch.cuda.synchronize()
    exact = q.astype(np.float64) * np.repeat(s.astype(np.float64), 128, axis=1)  # exact: 8 x 24 bits
    if mode == "f16":
        op = exact.astype(np.float16).astype(np.float32)
    else:
        op = bf.bf16_to_f32(bf.bf16_bits(exact.astype(np.float32)))
    want = op[:, np.arange(M) % K].T
    return y.cpu().numpy(), want


@pytest.mark.parametrize("sf32", [False, True])
@pytest.mark.parametrize("mode", ["f16", "bf16"])
@pytest.mark.parametrize("M,N,K", [(1024, 512, 1024), (300, 256, 256)])
def test_linear_q8_onehot_exact(ctx, M, N, K, mode, sf32):
    say(f"linear_q8 one-hot {mode} M={M} N={N} K={K} f32 scales={sf32}")
    got, want = _onehot_case(ctx, M, N, K, seed=M + K, mode=mode, sf32=sf32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("sf32,exp_range", [(True, (-4, -1)), (False, (-4, -1)), (True, (-30, 30))])
def test_linear_q8_onehot_exact_f32_mode(ctx, sf32, exp_range):
    """The f32 MFMA GEMM on one-hot rows: every output is one dequantised
    weight times 1 (one nonzero product, f32 accumulation), so y must equal
    f32(q) * s (dq4 at ltx/block.zig:462-471) bit for bit, f32 or f16 scales,
    and scales across 60 decades."""
    say(f"linear_q8 one-hot f32 mode f32 scales={sf32} 1e{exp_range[0]}..1e{exp_range[1]}")
    M, N, K = 300, 256, 512
    rng = np.random.default_rng(31 + K)
    q = rng.integers(-128, 128, size=(N, K), dtype=np.int16).astype(np.int8)
    s = (10.0 ** rng.uniform(*exp_range, size=(N, K // 128))).astype(np.float32 if sf32 else np.float16)
    e = np.zeros((M, K), np.float32)
    e[np.arange(M), np.arange(M) % K] = 1.0
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ctx.linear_q8(torch.from_numpy(e).cuda(), torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(), None, y,
                  mode=rt.MODE_F32)
    torch.cuda.synchronize()
    want = oracle.dequant(q, s)[:, np.arange(M) % K].T
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(want).view(np.uint32))


@pytest.mark.parametrize("mode,exp_range", [
    ("f16", (-9, -5)),   # q * s among the f16 subnormals: one rounding into them
    ("bf16", (20, 36)),  # q * s up to 1.3e38: the bf16 path keeps the whole f32 range
])
def test_linear_q8_onehot_extreme_f32_scales(ctx, mode, exp_range):
    """Values, not bits: an operand that underflows to -0 leaves the f32
    accumulation (+0 + 1 * -0) as +0."""
    say(f"linear_q8 one-hot {mode} f32 scales 1e{exp_range[0]}..1e{exp_range[1]}")
    got, want = _onehot_case(ctx, 1024, 512, 1024, seed=21, mode=mode, sf32=True, exp_range=exp_range)
    assert np.isfinite(want).all()
    assert np.array_equal(got, want)
    if mode == "f16":
        assert ((want != 0) & (np.abs(want) < 6.1e-5)).sum() > 1000  # subnormal operands were exercised


VARIANT_ENV = {"reg": ("LTX_GEMM_Q8", "reg"), "x4": ("LTX_GEMM_X4", "all"), "s4off": ("LTX_GEMM_S4", "off"),
               "s4all": ("LTX_GEMM_S4", "all")}


@pytest.mark.parametrize("variant", ["reg", "x4", "s4off", "s4all"])
def test_linear_q8_variants(monkeypatch, variant):
    """Other GEMM kernels forced everywhere, in a context of their own:
    - reg: the register-staged int8 GEMM (the fallback of the LDS-DMA one);
    - x4: the four-wave 16-bit GEMM after the per-call dequantisation
      (ltx_gemm_dq16_*), which the block uses from 4,096 rows;
    - s4off: no small-grid kernel, so these shapes (below 4,096 rows, most
      of which take it by default) run the 256 x 256 LDS-DMA int8 kernel;
    - s4all: the small-grid kernel (128 x 128 tiles) at every shape.
    The one-hot exactness check (every output one weight operand, bit for
    bit: the dequantised operands, f16 and f32 scales, both operand types),
    then GEMMs against the oracle: ragged M with a bias, and for x4 also GELU
    into a 16-bit output in bf16 with f32 scales."""
    say(f"linear_q8 variant={variant}")
    monkeypatch.setenv(*VARIANT_ENV[variant])
    c = rt.Context(0)
    try:
        for mode in ("f16", "bf16"):
            for sf32 in (False, True):
                got, want = _onehot_case(c, 1024, 512, 1024, seed=9, mode=mode, sf32=sf32)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (mode, sf32)
        if variant == "x4":
            got, want = _onehot_case(c, 300, 256, 256, seed=10, mode="f16", sf32=False)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        a, q, s, b = _gemm_case(300, 768, 4096, seed=11, scale_f16=True)
        y = torch.empty((300, 768), dtype=torch.float32, device="cuda")
        c.linear_q8(to16(a, torch.float16).cuda(), torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(),
                    torch.from_numpy(b).cuda(), y, mode=rt.MODE_F16)
        torch.cuda.synchronize()
        want = f64(to16(a, torch.float16)) @ oracle.dequant(q, s).astype(np.float64).T + b
        assert oracle.rel_rms(f64(y), want) <= 1e-3
        if variant == "x4":
            a, q, s, b = _gemm_case(300, 512, 4096, seed=12, scale_f16=False)
            da = to16(a, torch.bfloat16).cuda()
            y = torch.empty((300, 512), dtype=torch.bfloat16, device="cuda")
            c.linear_q8(da, torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(), torch.from_numpy(b).cuda(), y,
                        mode=rt.MODE_BF16, gelu=True)
            torch.cuda.synchronize()
            z = f64(da) @ oracle.dequant(q, s).astype(np.float64).T + b
            want = 0.5 * z * (1 + np.tanh(np.sqrt(2 / np.pi) * (z + 0.044715 * z ** 3)))
            assert oracle.rel_rms(f64(y), want) <= 6e-3
    finally:
        c.close()


# the f32 MFMA GEMM: f32 and f16 scales, ragged M and N (partial 128 x 128
# tiles), GELU, one row and one K group
@pytest.mark.parametrize("M,N,K,scale_f16,gelu", [(200, 384, 2048, False, False), (200, 384, 2048, True, False),
                                                  (333, 200, 4096, True, True), (1, 130, 128, False, False)])
def test_linear_q8_f32_mode(ctx, M, N, K, scale_f16, gelu):
    say(f"linear_q8 mode=f32 M={M} N={N} K={K} scale_f16={scale_f16} gelu={gelu}")
    a, q, s, b = _gemm_case(M, N, K, seed=5 + M + N, scale_f16=scale_f16)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    ctx.linear_q8(torch.from_numpy(a).cuda(), torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(),
                  torch.from_numpy(b).cuda(), y, mode=rt.MODE_F32, gelu=gelu)
    torch.cuda.synchronize()
    z = oracle.linear(a, q=q, s=s.astype(np.float32)) + b
    want = 0.5 * z * (1 + np.tanh(np.sqrt(2 / np.pi) * (z + 0.044715 * z ** 3))) if gelu else z
    # the products alone to 1e-6; the device GELU (tanh through the fast exp
    # and reciprocal) to the f32 mode's 1e-5
    assert oracle.rel_rms(f64(y), want) <= (1e-5 if gelu else 1e-6)


def _heads(x, L):  # [L, D] -> [H, L, 128]
    return np.ascontiguousarray(x.reshape(L, 32, 128).transpose(1, 0, 2))


@pytest.mark.parametrize("mode", ["f16", "bf16"])
@pytest.mark.parametrize("lq,lkv,gated", [(256, 256, True), (300, 200, True), (256, 32, False), (512, 1024, True),
                                          (64, 77, True),
                                          # the ping-pong kernel's shortest loop (two 64-key tiles) and
                                          # key counts the any-length kernel masks
                                          (100, 128, True), (300, 160, True), (256, 480, False),
                                          # resident K/V (64-256 keys): several query tiles per workgroup,
                                          # a ragged last tile, one to four key tiles
                                          (4000, 256, True), (3000, 64, True), (2100, 192, False),
                                          # one key tile and a single ragged query tile per head
                                          (200, 64, True)])
@pytest.mark.parametrize("q_scaled", [False, True])
def test_attention(ctx, mode, lq, lkv, gated, q_scaled):
    """q_scaled: q arrives multiplied by log2(e)/sqrt(128), as the block's
    qk-norm writes it; the oracle then takes that q divided back (exactly)."""
    say(f"attention mode={mode} lq={lq} lkv={lkv} gated={gated} q_scaled={q_scaled}")
    m, dt = MODES[mode]
    rng = np.random.default_rng(lq * 7 + lkv)
    q = rng.standard_normal((lq, 4096)).astype(np.float32)
    k = rng.standard_normal((lkv, 4096)).astype(np.float32)
    v = rng.standard_normal((lkv, 4096)).astype(np.float32)
    glog = rng.standard_normal((lq, 32)).astype(np.float32) if gated else None
    cq = rt.ATTN_C if q_scaled else 1.0
    dq = to16(_heads(q * np.float32(cq), lq), dt).cuda()
    dk = to16(_heads(k, lkv), dt).cuda()
    dv = to16(np.ascontiguousarray(v.reshape(lkv, 32, 128).transpose(1, 2, 0)), dt).cuda()  # [H][128][L]
    dg = torch.from_numpy(glog).cuda() if gated else None
    out = torch.empty((lq, 4096), dtype=dt, device="cuda")
    ctx.attention(dq, dk, dv, dg, out, lq, lkv, mode=m, q_scaled=q_scaled)
    torch.cuda.synchronize()
    q64 = f64(dq).transpose(1, 0, 2).reshape(lq, 4096) / cq
    k64 = f64(dk).transpose(1, 0, 2).reshape(lkv, 4096)
    v64 = f64(dv).transpose(2, 0, 1).reshape(lkv, 4096)
    want = oracle.sdpa(q64, k64, v64, chunk=0)
    if gated:
        g = 2.0 / (1.0 + np.exp(-glog.astype(np.float64)))
        want = (want.reshape(lq, 32, 128) * g[:, :, None]).reshape(lq, 4096)
    assert oracle.rel_rms(f64(out), want) <= (2e-3 if mode == "f16" else 1e-2)


@pytest.mark.parametrize("lq,lkv", [(130, 70), (1000, 1000), (257, 193), (64, 1)])
def test_attention_f32_mode(ctx, lq, lkv):
    say(f"attention mode=f32 lq={lq} lkv={lkv}")
    rng = np.random.default_rng(11 + lq + lkv)
    q, k, v = (rng.standard_normal((n, 4096)).astype(np.float32) for n in (lq, lkv, lkv))
    glog = rng.standard_normal((lq, 32)).astype(np.float32)
    out = torch.empty((lq, 4096), dtype=torch.float32, device="cuda")
    ctx.attention(*(torch.from_numpy(a).cuda() for a in (q, k, v)), torch.from_numpy(glog).cuda(), out, lq, lkv,
                  mode=rt.MODE_F32)
    torch.cuda.synchronize()
    want = oracle.sdpa(q, k, v, chunk=0)
    g = 2.0 / (1.0 + np.exp(-glog.astype(np.float64)))
    want = (want.reshape(lq, 32, 128) * g[:, :, None]).reshape(lq, 4096)
    assert oracle.rel_rms(f64(out), want) <= 1e-5


@pytest.mark.parametrize("lkv,dom", [(96, 37), (160, 130), (256, 200)])
@pytest.mark.parametrize("q_scaled", [False, True])
def test_attention_special_cases(ctx, lkv, dom, q_scaled):
    """Identical keys -> mean of V; one dominant key -> that V row (placed
    past the first tiles, so the running max must move and rescale O)."""
    say(f"attention special cases f16 lkv={lkv} dominant key={dom} q_scaled={q_scaled}")
    cq = np.float32(rt.ATTN_C if q_scaled else 1.0)
    rng = np.random.default_rng(12)
    lq = 64
    q = rng.standard_normal((lq, 4096)).astype(np.float32)
    k = np.tile(rng.standard_normal((1, 4096)).astype(np.float32), (lkv, 1))
    v = rng.standard_normal((lkv, 4096)).astype(np.float32)
    dt = torch.float16
    args = [to16(_heads(q * cq, lq), dt).cuda(), to16(_heads(k, lkv), dt).cuda(),
            to16(np.ascontiguousarray(v.reshape(lkv, 32, 128).transpose(1, 2, 0)), dt).cuda()]
    out = torch.empty((lq, 4096), dtype=dt, device="cuda")
    ctx.attention(*args, None, out, lq, lkv, mode=rt.MODE_F16, q_scaled=q_scaled)
    torch.cuda.synchronize()
    vm = f64(args[2]).transpose(2, 0, 1).reshape(lkv, 4096).mean(0)
    assert np.abs(f64(out) - vm[None, :]).max() < 2e-3
    # dominant key: key 37 equals 8 * q-direction for every head -> softmax ~ one-hot
    k2 = rng.standard_normal((lkv, 4096)).astype(np.float32) * 0.01
    qq = np.tile(rng.standard_normal((1, 4096)).astype(np.float32), (lq, 1))
    k2[dom] = qq[0] * 4.0
    args2 = [to16(_heads(qq * cq, lq), dt).cuda(), to16(_heads(k2, lkv), dt).cuda(), args[2]]
    ctx.attention(*args2, None, out, lq, lkv, mode=rt.MODE_F16, q_scaled=q_scaled)
    torch.cuda.synchronize()
    vd = f64(args[2]).transpose(2, 0, 1).reshape(lkv, 4096)[dom]
    assert np.abs(f64(out) - vd[None, :]).max() < 5e-3


@pytest.mark.parametrize("lkv,dom", [(96, 70), (200, 130), (256, 200), (1000, 900)])
def test_attention_f32_special_cases(ctx, lkv, dom):
    """The f32 MFMA attention: identical keys -> the mean of V; one dominant
    key past the first 64-key tiles -> that V row (the running max moves and
    O is rescaled); key counts that are not multiples of 64 mask the last
    tile."""
    say(f"attention special cases f32 lkv={lkv} dominant key={dom}")
    rng = np.random.default_rng(13 + lkv)
    lq = 70
    q = rng.standard_normal((lq, 4096)).astype(np.float32)
    k = np.tile(rng.standard_normal((1, 4096)).astype(np.float32), (lkv, 1))
    v = rng.standard_normal((lkv, 4096)).astype(np.float32)
    out = torch.empty((lq, 4096), dtype=torch.float32, device="cuda")
    dv = torch.from_numpy(v).cuda()
    ctx.attention(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), dv, None, out, lq, lkv, mode=rt.MODE_F32)
    torch.cuda.synchronize()
    vm = v.astype(np.float64).mean(0)
    assert np.abs(f64(out) - vm[None, :]).max() < 1e-5
    # key `dom` is 4 q in every head: its score leads the others by ~45 in
    # natural-log units, so the softmax is one-hot to f32 precision
    k2 = rng.standard_normal((lkv, 4096)).astype(np.float32) * 0.01
    qq = np.tile(rng.standard_normal((1, 4096)).astype(np.float32), (lq, 1))
    k2[dom] = qq[0] * 4.0
    ctx.attention(torch.from_numpy(qq).cuda(), torch.from_numpy(k2).cuda(), dv, None, out, lq, lkv, mode=rt.MODE_F32)
    torch.cuda.synchronize()
    assert np.abs(f64(out) - v[dom].astype(np.float64)[None, :]).max() < 1e-5


@pytest.mark.parametrize("variant,lq,lkv", [("w8", 384, 2048), ("default", 384, 2048), ("pp", 1000, 256),
                                            ("default", 1000, 256)])
def test_attention_variants(monkeypatch, variant, lq, lkv):
    """The any-length attention kernel forced everywhere (w8), the streaming
    ping-pong kernel forced for 256 keys (pp) and the defaults (streaming
    ping-pong for 2048 keys, resident K/V for 256) against the dense f64
    oracle."""
    say(f"attention variant={variant} lq={lq} lkv={lkv}")
    if variant == "default":
        monkeypatch.delenv("LTX_ATTN_VARIANT", raising=False)
    else:
        monkeypatch.setenv("LTX_ATTN_VARIANT", variant)
    c = rt.Context(0)
    try:
        rng = np.random.default_rng(21)
        q, k, v = (rng.standard_normal((n, 4096)).astype(np.float32) for n in (lq, lkv, lkv))
        glog = rng.standard_normal((lq, 32)).astype(np.float32)
        dt = torch.float16
        dq, dk = to16(_heads(q, lq), dt).cuda(), to16(_heads(k, lkv), dt).cuda()
        dv = to16(np.ascontiguousarray(v.reshape(lkv, 32, 128).transpose(1, 2, 0)), dt).cuda()
        out = torch.empty((lq, 4096), dtype=dt, device="cuda")
        c.attention(dq, dk, dv, torch.from_numpy(glog).cuda(), out, lq, lkv, mode=rt.MODE_F16)
        torch.cuda.synchronize()
        want = oracle.sdpa(f64(dq).transpose(1, 0, 2).reshape(lq, 4096), f64(dk).transpose(1, 0, 2).reshape(lkv, 4096),
                           f64(dv).transpose(2, 0, 1).reshape(lkv, 4096), chunk=0)
        g = 2.0 / (1.0 + np.exp(-glog.astype(np.float64)))
        want = (want.reshape(lq, 32, 128) * g[:, :, None]).reshape(lq, 4096)
        assert oracle.rel_rms(f64(out), want) <= 2e-3
    finally:
        c.close()


# ---- the microbenchmark shapes (isolated GEMM and attention configurations) ----

@pytest.mark.parametrize("mode", ["f16", "bf16"])
def test_linear_q8_square_4096(ctx, mode):
    """The 4096 x 4096 x 4096 W8A16 GEMM of the sweep: A N(0, 1) 16-bit,
    W Student-t(3) x 0.02 int8 grouped-128 with fp16 scales, 16-bit output;
    96 output rows against f64 with the exact weights (rel-RMS f16 <= 1e-3,
    bf16 <= 6e-3: one rounding of the operands and of the output)."""
    M = N = K = 4096
    say(f"linear_q8 {M}x{K}x{N} mode={mode}")
    m, dt = MODES[mode]
    a, q, s, _ = _gemm_case(M, N, K, seed=44, scale_f16=True)
    da = to16(a, dt).cuda()
    y = torch.empty((M, N), dtype=dt, device="cuda")
    ctx.linear_q8(da, torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(), None, y, mode=m)
    torch.cuda.synchronize()
    rows = np.linspace(0, M - 1, 96).astype(np.int64)
    sel = torch.from_numpy(rows).cuda()
    want = f64(da[sel]) @ oracle.dequant(q, s).astype(np.float64).T
    r = oracle.rel_rms(f64(y[sel]), want)
    say(f"  rel-RMS {r:.3e}")
    assert r <= (1e-3 if mode == "f16" else 6e-3)


@pytest.mark.parametrize("mode", ["f16", "bf16"])
@pytest.mark.parametrize("L", [4096, 16384])
def test_attention_long(ctx, mode, L):
    """Self-attention at L = 4,096 and 16,384 (the sweep's tile-size lengths),
    Q/K/V N(0, 1) 16-bit, no gate: 48 query rows of every head against f64
    softmax attention over all L keys from the same 16-bit operands."""
    say(f"attention L={L} mode={mode}")
    m, dt = MODES[mode]
    g = torch.Generator(device="cuda").manual_seed(L)
    q = torch.randn((H_, L, 128), generator=g, device="cuda").to(dt)
    k = torch.randn((H_, L, 128), generator=g, device="cuda").to(dt)
    vt = torch.randn((H_, 128, L), generator=g, device="cuda").to(dt)
    out = torch.empty((L, 4096), dtype=dt, device="cuda")
    ctx.attention(q, k, vt, None, out, L, L, mode=m)
    torch.cuda.synchronize()
    rows = np.linspace(0, L - 1, 48).astype(np.int64)
    sel = torch.from_numpy(rows).cuda()
    q64, k64, v64 = f64(q[:, sel]), f64(k), f64(vt)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))
    want = np.empty((len(rows), 4096))
    for h in range(H_):
        sc = (q64[h] @ k64[h].T) * scale
        p = np.exp(sc - sc.max(1, keepdims=True))
        want[:, 128 * h:128 * h + 128] = (p @ v64[h].T) / p.sum(1, keepdims=True)
    r = oracle.rel_rms(f64(out[sel]), want)
    say(f"  rel-RMS {r:.3e}")
    assert r <= (2e-3 if mode == "f16" else 1e-2)


H_ = 32


def test_linear_q8_large_f32_scale_zero_group(ctx):
    """fp16 operands with f32 scales up to 2^99 (s 2^24 still finite): for
    every fourth column the first group's q are all 0 under a scale of
    1e25..1e29.8, and its operands must be exactly 0, not NaN (0 * s formed
    as fma((q + 128) 2^-24, s 2^24, -128 s)); every other group keeps small
    scales, so the one-hot outputs stay finite and exact."""
    say("linear_q8 one-hot f16 with huge f32 scales over all-zero groups")
    M, N, K = 1024, 512, 1024
    rng = np.random.default_rng(23)
    q = rng.integers(-128, 128, size=(N, K), dtype=np.int16).astype(np.int8)
    s = (10.0 ** rng.uniform(-4, -1, size=(N, K // 128))).astype(np.float32)
    q[::4, :128] = 0
    s[::4, 0] = (10.0 ** rng.uniform(25, 29.8, size=N // 4)).astype(np.float32)
    e = np.zeros((M, K), np.float32)
    e[np.arange(M), np.arange(M) % K] = 1.0
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ctx.linear_q8(to16(e, torch.float16).cuda(), torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(), None, y,
                  mode=rt.MODE_F16)
    torch.cuda.synchronize()
    exact = q.astype(np.float64) * np.repeat(s.astype(np.float64), 128, axis=1)
    want = exact.astype(np.float16).astype(np.float32)[:, np.arange(M) % K].T
    got = y.cpu().numpy()
    assert np.isfinite(want).all()
    assert np.array_equal(got, want)


def test_upload_refuses_f32_scales_out_of_range(ctx, block0):
    """An f32 scale that is not finite or has magnitude >= 2^100 is refused at
    upload (error ScaleRange)."""
    say("upload with an out-of-range f32 scale")
    for bad in (np.float32(2.0 ** 100), np.float32(np.inf), np.float32(np.nan), np.float32(-(2.0 ** 101))):
        q8s = dict(block0.q8s)
        s = q8s["k1"].copy()
        s[7, 3] = bad
        q8s["k1"] = s
        with pytest.raises(rt.LtxError, match="ScaleRange"):
            ctx.upload(bf.BlockTensors(0, block0.base, block0.q8, q8s))


@pytest.mark.parametrize("noalloc", [False, True])
def test_linear_q8_rejects_bad_arguments_before_allocating(ctx, noalloc):
    """Invalid shapes and modes are refused by name before N and K size any
    scratch (a negative N once reached the allocation as a wrapped size).
    Nothing is launched: every call fails its checks first."""
    say(f"linear_q8 argument checks noalloc={noalloc}")
    a = torch.zeros((4, 128), dtype=torch.float16, device="cuda")
    q = torch.zeros((256, 128), dtype=torch.int8, device="cuda")
    s = torch.ones((256, 1), dtype=torch.float16, device="cuda")
    y = torch.empty((4, 256), dtype=torch.float16, device="cuda")
    name = "ltx_op_linear_q8_noalloc" if noalloc else "ltx_op_linear_q8"
    fn = getattr(rt.lib(), name)
    st = torch.cuda.current_stream().cuda_stream
    cases = [(4, -256, 128, rt.MODE_F16, "bad GEMM shape"), (4, 256, 0, rt.MODE_F16, "bad GEMM shape"),
             (4, 256, 100, rt.MODE_F16, "bad GEMM shape"), (0, 256, 128, rt.MODE_F16, "bad GEMM shape"),
             (4, 256, 128, 7, "unknown mode")]
    for M, N, K, mode, msg in cases:
        with pytest.raises(rt.LtxError, match=msg):
            ctx._check(fn(ctx.handle, a.data_ptr(), q.data_ptr(), s.data_ptr(), 1, None, y.data_ptr(), 0, M, N, K, 0,
                          mode, st), name)
