"""The oracle — TEST INFRASTRUCTURE ONLY.

A CPU restatement of the reference's block forward (QBlock.qBlockOutAll,
ltx/block.zig:544-574, with the blockwise attention of ltx/block.zig:105-154)
and of its host contracts (RoPE tables ltx/block_conformance.zig:87-126, the
int8-g128 quantizer tools/quantize_block.py:51-59, dq4 ltx/block.zig:462-471).
Only tests, the smoke check and the benchmark's CPU-baseline leg may use it,
and only as the checker / baseline; the product never imports it.

Two layers:
- ``ltx_oracle.c`` (built by ``oracle/build.py``): f64 parity oracle and the
  f32 CPU-baseline build of the same source;
- the numpy restatements below, written independently of the C code, used to
  pin it (``rope_tables_np``, ``quantize_np``, ``sdpa_np``, ``block_np``).

Parity status of each function is documented where it is pinned (tests/).
"""
from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
D, H, HD, FF = 4096, 32, 128, 16384
NF = 682
MAXPOS = (20.0, 2048.0, 2048.0)
ST_NAMES = ["s1_norm_msa", "q1_roped", "k1_roped", "v1", "attn1_merged", "s3_attn1", "s4_after_sa", "s4_normed",
            "attn_in", "enc", "q2_normed", "k2_normed", "v2", "attn2_merged", "s5_ca_out", "x_ca", "s6_ff_in",
            "ff_h", "s7_ff_out", "glog1", "glog2"]
BASE_ORDER = ["q1_w", "q1_b", "k1_w", "k1_b", "v1_w", "v1_b", "o1_w", "o1_b", "qn1", "kn1", "g1_w", "g1_b",
              "q2_w", "q2_b", "k2_w", "k2_b", "v2_w", "v2_b", "o2_w", "o2_b", "qn2", "kn2", "g2_w", "g2_b",
              "ff1_w", "ff2_w", "sst", "psst"]
Q_ORDER = ["q1", "k1", "v1", "q2", "k2", "v2", "f1", "f2", "o1", "o2"]

_libs: dict = {}


def lib(real: str = "f64") -> C.CDLL:
    if real in _libs:
        return _libs[real]
    p = HERE / "_build" / f"liboracle_{real}.so"
    if not p.exists():
        raise RuntimeError(f"{p} not built; run `python oracle/build.py`")
    L = C.CDLL(str(p))
    vp, i32 = C.c_void_p, C.c_int
    L.orc_block_forward.restype = i32
    L.orc_block_forward.argtypes = [C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), i32, vp, vp, i32, vp, vp, i32, vp,
                                    vp, vp, i32, i32, i32, vp, C.POINTER(vp)]
    L.orc_block_rows.restype = i32
    L.orc_block_rows.argtypes = [C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), i32, vp, vp, i32, vp, vp, i32, vp,
                                 vp, vp, i32, i32, i32, vp, i32, vp, C.POINTER(vp)]
    L.orc_rope_tables.argtypes = [vp, i32, vp, vp]
    L.orc_rope_freqs.argtypes = [vp]
    L.orc_quantize.argtypes = [vp, i32, i32, i32, i32, vp, vp]
    L.orc_dequant.argtypes = [vp, vp, i32, i32, i32, vp]
    L.orc_sdpa.argtypes = [vp, i32, vp, vp, i32, i32, vp]
    L.orc_sdpa.restype = i32
    L.orc_linear.argtypes = [vp, i32, i32, vp, vp, vp, i32, vp, i32, vp]
    L.orc_rms.argtypes = [vp, i32, i32, vp, vp]
    L.orc_rope_apply.argtypes = [vp, i32, vp, vp]
    L.orc_gelu.argtypes = [vp, C.c_long, vp]
    _libs[real] = L
    return L


def _rdt(real):
    return np.float64 if real == "f64" else np.float32


def _p(a):
    return None if a is None else a.ctypes.data


# ---- C oracle wrappers ------------------------------------------------------

def rope_tables(grid: np.ndarray):
    """Bundle layout [H][T][64] cos, sin (f32)."""
    grid = np.ascontiguousarray(grid, np.float32)
    T = grid.shape[1]
    cos, sin = np.empty((H, T, 64), np.float32), np.empty((H, T, 64), np.float32)
    lib().orc_rope_tables(grid.ctypes.data, T, cos.ctypes.data, sin.ctypes.data)
    return cos, sin


def rope_freqs() -> np.ndarray:
    f = np.empty(NF, np.float64)
    lib().orc_rope_freqs(f.ctypes.data)
    return f


def quantize(w_bf16: np.ndarray, gs: int = 128, bits: int = 8):
    w_bf16 = np.ascontiguousarray(w_bf16, np.uint16)
    O, I = w_bf16.shape
    q, s = np.empty((O, I), np.int8), np.empty((O, I // gs), np.float32)
    lib().orc_quantize(w_bf16.ctypes.data, O, I, gs, bits, q.ctypes.data, s.ctypes.data)
    return q, s


def dequant(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(s)
    out = np.empty(q.shape, np.float32)
    lib().orc_dequant(q.ctypes.data, s.ctypes.data, int(s.dtype == np.float16), q.shape[0], q.shape[1],
                      out.ctypes.data)
    return out


def sdpa(q, k, v, chunk: int, real: str = "f64"):
    """q [Lq, D], k/v [Lkv, D] -> [Lq, D]; chunk 0 = dense softmax."""
    dt = _rdt(real)
    q, k, v = (np.ascontiguousarray(a, dt) for a in (q, k, v))
    out = np.empty_like(q)
    if not lib(real).orc_sdpa(q.ctypes.data, q.shape[0], k.ctypes.data, v.ctypes.data, k.shape[0], chunk,
                              out.ctypes.data):
        raise ValueError(f"chunk {chunk} does not divide the key count {k.shape[0]}")
    return out


def linear(x, w_bf16=None, q=None, s=None, b_bf16=None, real: str = "f64"):
    dt = _rdt(real)
    x = np.ascontiguousarray(x, dt)
    M, K = x.shape
    N = (q if q is not None else w_bf16).shape[0]
    y = np.empty((M, N), dt)
    sf16 = int(s is not None and s.dtype == np.float16)
    lib(real).orc_linear(x.ctypes.data, M, K, _p(w_bf16), _p(q), _p(s), sf16, _p(b_bf16), N, y.ctypes.data)
    return y


def rms(x, w_bf16=None, real: str = "f64"):
    """rmsNoW / rmsW rows (ltx/block.zig:28-34); w_bf16 the norm weight as bf16 bits."""
    dt = _rdt(real)
    x = np.ascontiguousarray(x, dt)
    y = np.empty_like(x)
    w = None if w_bf16 is None else np.ascontiguousarray(w_bf16, np.uint16)
    lib(real).orc_rms(x.ctypes.data, x.shape[0], x.shape[1], _p(w), y.ctypes.data)
    return y


def rope_apply(x, cos_thf, sin_thf, real: str = "f64"):
    """Split-half RoPE (ltx/block.zig:69-77) of x [T, 4096] with graph-layout
    cos/sin [T, 32, 64] f32; returns a new array."""
    dt = _rdt(real)
    y = np.array(x, dt, order="C", copy=True)
    cs = np.ascontiguousarray(cos_thf, np.float32)
    sn = np.ascontiguousarray(sin_thf, np.float32)
    assert y.shape[1] == D and cs.shape == (y.shape[0], H, 64) == sn.shape
    lib(real).orc_rope_apply(y.ctypes.data, y.shape[0], cs.ctypes.data, sn.ctypes.data)
    return y


def gelu(x, real: str = "f64"):
    """Tensor.gelu, tanh form (ltx/block.zig:332), elementwise."""
    dt = _rdt(real)
    x = np.ascontiguousarray(x, dt)
    y = np.empty_like(x)
    lib(real).orc_gelu(x.ctypes.data, x.size, y.ctypes.data)
    return y


def block_forward(bt, inp: dict, cos_thf: np.ndarray, sin_thf: np.ndarray, chunk: int = 16, cross_chunk: int = 0,
                  real: str = "f64", stages: bool = False, rows=None):
    """QBlock.qBlockOutAll on the CPU. ``bt`` is a BlockTensors (numpy),
    ``inp`` holds x, ctx, tstab, tidx, pts2; cos/sin in graph layout [T][H][64].

    ``rows``: None for every token, or token indices whose output rows alone
    are computed (the keys and values of every token are still computed for
    the self-attention); each returned row equals that row of the whole
    block. Stage dumps (``stages=True``) then have one row per entry of
    ``rows``, except k1_roped / v1 (every token) and enc / k2_normed / v2
    (the S context tokens)."""
    L = lib(real)
    dt = _rdt(real)
    base = (C.c_void_p * 28)(*[bt.base[f].ctypes.data for f in BASE_ORDER])
    q8 = (C.c_void_p * 10)(*[bt.q8[n].ctypes.data if n in bt.q8 else None for n in Q_ORDER])
    q8s = (C.c_void_p * 10)(*[bt.q8s[n].ctypes.data if n in bt.q8s else None for n in Q_ORDER])
    x = np.ascontiguousarray(inp["x"], np.float32)
    T, S = x.shape[0], inp["ctx"].shape[0]
    # the blockwise attention's chunk must divide the key count
    # (ltx/block.zig:112); the C code would return NaN rows
    if chunk > 0 and T % chunk:
        raise ValueError(f"chunk {chunk} does not divide the token count {T}")
    if cross_chunk > 0 and S % cross_chunk:
        raise ValueError(f"cross_chunk {cross_chunk} does not divide the context length {S}")
    if rows is not None:
        rows = np.ascontiguousarray(rows, np.int32)
        if rows.ndim != 1 or rows.size == 0 or rows.min() < 0 or rows.max() >= T:
            raise ValueError("rows must be a non-empty list of token indices")
    nr = T if rows is None else rows.size
    out = np.empty((nr, D), dt)
    st_bufs = {}
    st_arr = None
    if stages:
        shapes = {"ff_h": (nr, FF), "enc": (S, D), "k2_normed": (S, D), "v2": (S, D), "k1_roped": (T, D),
                  "v1": (T, D), "glog1": (nr, H), "glog2": (nr, H)}
        st_bufs = {n: np.empty(shapes.get(n, (nr, D)), dt) for n in ST_NAMES}
        st_arr = (C.c_void_p * len(ST_NAMES))(*[st_bufs[n].ctypes.data for n in ST_NAMES])
    tstab = np.ascontiguousarray(inp["tstab"], np.float32)
    tidx = np.ascontiguousarray(inp["tidx"], np.int32)
    ctx = np.ascontiguousarray(inp["ctx"], np.float32)
    pts2 = np.ascontiguousarray(inp["pts2"], np.float32)
    cos_thf = np.ascontiguousarray(cos_thf, np.float32)
    sin_thf = np.ascontiguousarray(sin_thf, np.float32)
    args = (base, q8, q8s, int(bt.scale_f16), x.ctypes.data, tstab.ctypes.data, tstab.shape[0], tidx.ctypes.data,
            ctx.ctypes.data, S, pts2.ctypes.data, cos_thf.ctypes.data, sin_thf.ctypes.data, T, chunk, cross_chunk)
    if rows is None:
        ok = L.orc_block_forward(*args, out.ctypes.data, st_arr)
    else:
        ok = L.orc_block_rows(*args, rows.ctypes.data, nr, out.ctypes.data, st_arr)
    if not ok:
        raise RuntimeError("oracle block forward failed")
    return (out, st_bufs) if stages else out


# ---- numpy restatements (independent of the C code) -----------------------

def rope_freqs_np() -> np.ndarray:
    """theta ** linspace(0, 1, 682) * pi / 2 in f64, rounded to f32."""
    return (10000.0 ** np.linspace(0.0, 1.0, NF, dtype=np.float64) * np.pi / 2).astype(np.float32).astype(np.float64)


def rope_tables_np(grid: np.ndarray):
    """precompute_freqs_cis(SPLIT) semantics, numpy f64: [H][T][64] f32."""
    g = np.asarray(grid, np.float64)  # [3, T, 2]
    mid = (g[..., 0] + g[..., 1]) / 2.0  # [3, T]
    frac = mid / np.array(MAXPOS)[:, None]
    arg = frac * 2.0 - 1.0  # [3, T]
    f = rope_freqs_np()  # [NF]
    th = f[None, :, None] * arg.T[:, None, :]  # [T, NF, 3]
    th = th.reshape(th.shape[0], NF * 3)  # axis triplets adjacent, freq-major
    cos = np.concatenate([np.ones((th.shape[0], 2)), np.cos(th)], axis=1)
    sin = np.concatenate([np.zeros((th.shape[0], 2)), np.sin(th)], axis=1)
    T = th.shape[0]
    cos = cos.reshape(T, H, 64).transpose(1, 0, 2).astype(np.float32)
    sin = sin.reshape(T, H, 64).transpose(1, 0, 2).astype(np.float32)
    return np.ascontiguousarray(cos), np.ascontiguousarray(sin)


def quantize_np(w_bf16: np.ndarray, gs: int = 128, bits: int = 8):
    qmax, lo = (7, -8) if bits == 4 else (127, -128)
    w = (np.asarray(w_bf16, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    o, i = w.shape
    wg = w.reshape(o, i // gs, gs)
    am = np.abs(wg).max(axis=2, keepdims=True)
    sc = np.where(am > 0, am / qmax, 1.0)
    q = np.clip(np.round(wg / sc), lo, qmax).astype(np.int8).reshape(o, i)
    return q, sc.squeeze(2).astype(np.float32)


def sdpa_np(q, k, v):
    """Dense softmax attention, f64, K scaled by f32(1/sqrt(128))."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    Lq, Lk = q.shape[0], k.shape[0]
    qh = q.reshape(Lq, H, HD).transpose(1, 0, 2)
    kh = k.reshape(Lk, H, HD).transpose(1, 0, 2) * float(np.float32(1.0) / np.sqrt(np.float32(128.0)))
    vh = v.reshape(Lk, H, HD).transpose(1, 0, 2)
    s = qh @ kh.transpose(0, 2, 1)
    s = np.exp(s - s.max(-1, keepdims=True))
    o = (s / s.sum(-1, keepdims=True)) @ vh
    return o.transpose(1, 0, 2).reshape(Lq, D)


def _bf(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


_W_CACHE: dict = {}


def _weights_np(bt) -> dict:
    """f64 weights of a block (dq4 of the int8 companions, else bf16),
    cached by the identity of the tensors they come from."""
    key = tuple(id(bt.base[f]) for f in BASE_ORDER[:-2]) + tuple(id(a) for a in bt.q8.values())
    if key not in _W_CACHE:
        W = {}
        for f in BASE_ORDER[:-2]:
            W[f] = _bf(bt.base[f])
        for n, wf in {"q1": "q1_w", "k1": "k1_w", "v1": "v1_w", "q2": "q2_w", "k2": "k2_w", "v2": "v2_w",
                      "f1": "ff1_w", "f2": "ff2_w", "o1": "o1_w", "o2": "o2_w"}.items():
            if n in bt.q8:
                q = bt.q8[n].astype(np.float32)
                s = bt.q8s[n].astype(np.float32)
                W[wf] = (q.reshape(q.shape[0], -1, 128) * s[:, :, None]).reshape(q.shape).astype(np.float64)
        _W_CACHE.clear()
        _W_CACHE[key] = (W, (bt.base, bt.q8))  # the tensors stay referenced while cached
    return _W_CACHE[key][0]


def block_np(bt, inp: dict, cos_thf, sin_thf, mistake: str | None = None):
    """Dense-attention numpy restatement of qBlockOutAll (f64). `mistake`
    plants one deliberate error (tests use it to show the gates have teeth):
    layernorm | gate_no_2x | rope_sign | kv_scale | ada_swap (self-attention
    shift and scale rows exchanged) | ca_swap (cross-attention query rows) |
    ff_swap (FFN rows) | kv_swap (the K/V modulation rows)."""
    W = dict(_weights_np(bt))
    sst = bt.base["sst"].astype(np.float64)
    psst = bt.base["psst"].astype(np.float64)
    x = inp["x"].astype(np.float64)
    ctx = inp["ctx"].astype(np.float64)
    tab = inp["tstab"].astype(np.float64)[inp["tidx"]]  # [T, 9, D]
    ada = [tab[:, i, :] + sst[i] for i in range(9)]
    cs, sn = cos_thf.astype(np.float64), sin_thf.astype(np.float64)

    def rms(a, w=None):
        if mistake == "layernorm" and w is None:  # mean-subtracting norm instead of RMS
            a = a - a.mean(-1, keepdims=True)
        r = a / np.sqrt((a * a).mean(-1, keepdims=True) + 1e-6)
        return r * w if w is not None else r

    def rope(a):
        T = a.shape[0]
        a4 = a.reshape(T, H, 2, 64)
        u, v = a4[:, :, 0], a4[:, :, 1]
        sg = -1.0 if mistake == "rope_sign" else 1.0
        return np.concatenate([u * cs - sg * v * sn, v * cs + sg * u * sn], -1).reshape(T, D)

    def attn(xq, xkv, p, use_rope):
        q = rms(xq @ W[p + "q_w"].T + W[p + "q_b"], W["qn" + p[-1]])
        k = rms(xkv @ W[p + "k_w"].T + W[p + "k_b"], W["kn" + p[-1]])
        v = xkv @ W[p + "v_w"].T + W[p + "v_b"]
        if use_rope:
            q, k = rope(q), rope(k)
        o = sdpa_np(q, k, v)
        g = (1.0 if mistake == "gate_no_2x" else 2.0) / (1.0 + np.exp(-(xq @ W["g" + p[-1] + "_w"].T
                                                                         + W["g" + p[-1] + "_b"])))
        o = (o.reshape(-1, H, HD) * g[:, :, None]).reshape(-1, D)
        return o @ W[p + "o_w"].T + W[p + "o_b"]

    # weight names in W use q1_w etc.; adapt the prefix scheme
    W2 = {}
    for a in ("1", "2"):
        for t in ("q", "k", "v", "o"):
            W2[f"a{a}{t}_w"] = W[f"{t}{a}_w"]
            W2[f"a{a}{t}_b"] = W[f"{t}{a}_b"]
    W.update(W2)
    swaps = {"ada_swap": (0, 1), "ca_swap": (6, 7), "ff_swap": (3, 4)}
    if mistake in swaps:  # shift and scale rows exchanged
        i, j = swaps[mistake]
        ada[i], ada[j] = ada[j], ada[i]
    n = rms(x) * (1 + ada[1]) + ada[0]
    x_sa = x + attn(n, n, "a1", True) * ada[2]
    ai = rms(x_sa) * (1 + ada[7]) + ada[6]
    kv = psst + inp["pts2"].astype(np.float64)
    if mistake == "kv_swap":
        kv = kv[::-1]
    enc = ctx * (kv[1] if mistake == "kv_scale" else 1 + kv[1]) + kv[0]
    x_ca = x_sa + attn(ai, enc, "a2", False) * ada[8]
    fi = rms(x_ca) * (1 + ada[4]) + ada[3]
    h = fi @ W["ff1_w"].T
    h = 0.5 * h * (1 + np.tanh(np.sqrt(2 / np.pi) * (h + 0.044715 * h ** 3)))
    return x_ca + (h @ W["ff2_w"].T) * ada[5]


def rel_rms(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.sqrt(((got - want) ** 2).sum() / ((want ** 2).sum() + 1e-300)))


# ---- parts around the blocks (ltx/core_parts.zig), numpy -------------------
# The sinusoid is f32 as in the reference (ltx/core_parts.zig:37-49: the
# embedding is computed in f32 even under the f64 torch oracle); everything
# after it is f64. Core tensors are a dict field -> array in CORE_SPECS order
# (bf16 bits as uint16, fsst f32).

CORE_EPS = 1e-6
TE, HALF, IN_CH = 256, 128, 128


def core_sinusoid(t) -> np.ndarray:
    """ltx/core_parts.zig:42-49: freqs = exp(arange(128) * f32(-ln(1e4)/128)),
    arg = (t * 1000) * freqs, [cos(arg) | sin(arg)], all f32."""
    t = np.asarray(t, np.float32).reshape(-1, 1)
    idx = np.arange(HALF, dtype=np.float32)
    freqs = np.exp(idx * np.float32(-np.log(1e4) / HALF))
    arg = (t * np.float32(1000.0)) * freqs[None, :]
    return np.concatenate([np.cos(arg), np.sin(arg)], axis=1).astype(np.float32)


def core_lin(x, cw: dict, name: str) -> np.ndarray:
    """lin (ltx/block.zig:22-26): x . f32(W)^T + f32(b), in f64."""
    return np.asarray(x, np.float64) @ _bf(cw[name + "_w"]).T + _bf(cw[name + "_b"])


def core_silu(x):
    return x / (1.0 + np.exp(-x))


def core_emb(cw: dict, t) -> np.ndarray:
    """embedded_timestep [K, D] (ltx/core_parts.zig:115-117)."""
    return core_lin(core_silu(core_lin(core_sinusoid(t), cw, "ada_l1")), cw, "ada_l2")


def core_ts9r(cw: dict, t) -> np.ndarray:
    """ts9r [K, 9, D] (ltx/core_parts.zig:119-136)."""
    ts9 = core_lin(core_silu(core_emb(cw, t)), cw, "ada_out")
    return ts9.reshape(-1, 9, D)


def core_pts2r(cw: dict, sigma: float) -> np.ndarray:
    """pts2r [2, D] from scalar sigma (ltx/core_parts.zig:124-141)."""
    e = core_lin(core_silu(core_lin(core_sinusoid([sigma]), cw, "pada_l1")), cw, "pada_l2")
    return core_lin(core_silu(e), cw, "pada_out").reshape(2, D)


def core_patchify(cw: dict, latent) -> np.ndarray:
    """ltx/core_parts.zig:143-145: [T, 128] -> [T, D]."""
    return core_lin(latent, cw, "pat")


def core_layernorm(x) -> np.ndarray:
    """LayerNorm without weight, biased variance, eps 1e-6 (ltx/core_parts.zig:30-35)."""
    x = np.asarray(x, np.float64)
    c = x - x.mean(-1, keepdims=True)
    return c / np.sqrt((c * c).mean(-1, keepdims=True) + CORE_EPS)


def core_tail_from_emb(cw: dict, x, e_tok, wrong_norm: bool = False) -> np.ndarray:
    """tailFrom (ltx/core_parts.zig:147-166): shift = fsst[0] + e,
    scale = fsst[1] + e, proj_out(norm(x) * (1 + scale) + shift). e_tok is
    the per-token embedded_timestep [T, D]. wrong_norm: the reference's
    RMS-norm control (ltx/core_parts.zig:175-180)."""
    x = np.asarray(x, np.float64)
    fsst = np.asarray(cw["fsst"], np.float64)
    e = np.asarray(e_tok, np.float64)
    n = x / np.sqrt((x * x).mean(-1, keepdims=True) + CORE_EPS) if wrong_norm else core_layernorm(x)
    return core_lin(n * (1.0 + (fsst[1] + e)) + (fsst[0] + e), cw, "po")


# ---- distilled scheduler (ltx/scheduler.zig), exact f32 ---------------------
# numpy evaluates each f32 operation with one rounding and never contracts,
# which is the reference's operation order; the lerp's fused multiply-add is
# emulated exactly (fma_f32).

SIGMAS_STAGE1 = np.array([1.0, 0.99375, 0.9875, 0.98125, 0.975, 0.909375, 0.725, 0.421875, 0.0], np.float32)
SIGMAS_STAGE2 = np.array([0.909375, 0.725, 0.421875, 0.0], np.float32)


def fma_f32(a, b, c) -> np.ndarray:
    """Correctly rounded f32 a*b + c. The product of two f32 is exact in f64;
    the f64 sum is taken with round-to-odd (TwoSum error term, then a step to
    the odd neighbour toward the error), which makes the final rounding to
    f32 equal the single rounding of the exact value."""
    a = np.asarray(a, np.float32).astype(np.float64)
    b = np.asarray(b, np.float32).astype(np.float64)
    c = np.asarray(c, np.float32).astype(np.float64)
    p = a * b
    s = p + c
    bb = s - p
    e = (p - (s - bb)) + (c - bb)
    even = (np.asarray(s, np.float64).view(np.int64) & 1) == 0
    adj = (e != 0) & even
    s = np.where(adj, np.nextafter(s, np.where(e > 0, np.inf, -np.inf)), s)
    return s.astype(np.float32)


def sched_lerp(a, b, w, fused: bool = True) -> np.ndarray:
    """torch.lerp as ltx/scheduler.zig:29-35 computes it: d = b - a; |w| < 0.5
    -> fma(w, d, a), else fma(-d, 1 - w, b). fused=False evaluates the same
    forms with two roundings (the reference notes that this differs)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    w = np.broadcast_to(np.asarray(w, np.float32), np.broadcast(a, b).shape)
    d = (b - a).astype(np.float32)
    one_m = (np.float32(1.0) - w).astype(np.float32)
    if fused:
        lo, hi = fma_f32(w, d, a), fma_f32(-d, one_m, b)
    else:
        lo = (w * d).astype(np.float32) + a
        hi = ((-d) * one_m).astype(np.float32) + b
    return np.where(np.abs(w) < np.float32(0.5), lo, hi).astype(np.float32)


def sched_noise_init(clean, noise, mask_tok, stride: int, noise_scale: float) -> np.ndarray:
    """noiseInit (ltx/scheduler.zig:41-46); mask_tok [T] per token."""
    clean = np.asarray(clean, np.float32).reshape(-1)
    noise = np.asarray(noise, np.float32).reshape(-1)
    m = np.repeat(np.asarray(mask_tok, np.float32), stride)
    x = sched_lerp(clean, noise, np.float32(noise_scale))
    return sched_lerp(clean, x, m)


def sched_timesteps(mask, sigma) -> np.ndarray:
    """ltx/scheduler.zig:49-51."""
    return (np.asarray(mask, np.float32) * np.float32(sigma)).astype(np.float32)


def sched_to_denoised(x, v, ts_tok, stride: int) -> np.ndarray:
    """ltx/scheduler.zig:57-59."""
    ts = np.repeat(np.asarray(ts_tok, np.float32), stride)
    return (np.asarray(x, np.float32).reshape(-1) - (np.asarray(v, np.float32).reshape(-1) * ts)).astype(np.float32)


def sched_post_process(den, clean, mask_tok, stride: int) -> np.ndarray:
    """ltx/scheduler.zig:62-67."""
    m = np.repeat(np.asarray(mask_tok, np.float32), stride)
    c = np.asarray(clean, np.float32).reshape(-1)
    return ((np.asarray(den, np.float32) * m) + (c * (np.float32(1.0) - m))).astype(np.float32)


def sched_euler_step(x, post, sigma, sigma_next) -> np.ndarray:
    """ltx/scheduler.zig:74-80, no snap at sigma_next == 0."""
    x = np.asarray(x, np.float32).reshape(-1)
    dt = np.float32(sigma_next) - np.float32(sigma)
    v = ((x - np.asarray(post, np.float32)) / np.float32(sigma)).astype(np.float32)
    return (x + (v * dt)).astype(np.float32)


def sched_step(x, vel, mask, tidx, clean, sigma, sigma_next):
    """One march of the loop (ltx/e2e_denoise.zig:321-326) for a latent
    [T, C] with mask rows `mask` [K] and token rows `tidx` [T]: returns
    (ts, den, post, next)."""
    x = np.asarray(x, np.float32)
    T, Cc = x.shape
    mask_tok = np.asarray(mask, np.float32)[np.asarray(tidx)]
    ts = sched_timesteps(mask_tok, sigma)
    den = sched_to_denoised(x, vel, ts, Cc)
    post = sched_post_process(den, clean, mask_tok, Cc)
    nxt = sched_euler_step(x, post, sigma, sigma_next)
    return ts, den.reshape(T, Cc), post.reshape(T, Cc), nxt.reshape(T, Cc)


def denoise(blocks: list, cw: dict, latent, clean, mask, tidx, ctx, cos_thf, sin_thf, sigmas, chunk: int = 16):
    """The denoising loop (ltx/e2e_denoise.zig:218-336) with K distinct mask
    rows: per step timesteps -> ts9r / emb / pts2r -> patchify -> blocks (the
    C oracle, f64 inside, f32 between blocks) -> tail -> the f32 march.
    Returns the list of (velocity f32 [T, 128], next latent f32 [T, 128])."""
    lat = np.asarray(latent, np.float32).copy()
    out = []
    for s in range(len(sigmas) - 1):
        sigma, sn = np.float32(sigmas[s]), np.float32(sigmas[s + 1])
        t = sched_timesteps(mask, sigma)
        emb = core_emb(cw, t)
        inp = dict(ctx=ctx, tstab=core_ts9r(cw, t).astype(np.float32), tidx=tidx,
                   pts2=core_pts2r(cw, sigma).astype(np.float32))
        x = core_patchify(cw, lat).astype(np.float32)
        for bt in blocks:
            inp["x"] = x
            x = block_forward(bt, inp, cos_thf, sin_thf, chunk=chunk).astype(np.float32)
        vel = core_tail_from_emb(cw, x, emb[np.asarray(tidx)]).astype(np.float32)
        _, _, _, lat = sched_step(lat, vel, mask, tidx, clean, sigma, sn)
        out.append((vel, lat.copy()))
    return out
