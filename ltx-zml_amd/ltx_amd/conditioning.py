"""Timestep conditioning: sigma -> the block's AdaLN inputs.

The block consumes precomputed tables, tstab [K, 9, D] + tidx [T] and
pts2 [2, D] (ltx/block.zig:47-67, ltx/e2e_prod.zig:243-246). They come from
sigma through the model's adaln_single / prompt_adaln_single MLPs
(ltx/core_parts.zig:42-49, 112-141):

  sinusoid(t) = [cos(1000 t f), sin(1000 t f)],  f_k = exp(-ln(1e4) k / 128)
  emb  = lin2(silu(lin1(sinusoid(t))))            (256 -> 4096 -> 4096)
  ts9  = lin_out(silu(emb))                       (4096 -> 9 * 4096)
  pts2 = p_out(silu(p_lin2(silu(p_lin1(sinusoid(sigma))))))   (-> 2 * 4096)

Real checkpoint weights are unavailable offline, so the MLP weights are drawn
here (seeded N(0, 0.02), rounded to bf16 like checkpoint tensors). Per-token
timesteps are mask * sigma with the production pass's striped mask
(ltx/e2e_prod.zig:218-229): mask 0 for the first T/7 tokens, 0.5 for the
next T/7, 1 for the rest — K = 3 distinct rows gathered through tidx.
"""
from __future__ import annotations

import zlib
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from .blockfmt import D

TE, HALF = 256, 128


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


_CHUNK = 1 << 20


def _draw_bf16(seed: int, name: str, shape) -> np.ndarray:
    """N(0, 1) * 0.02 rounded to bf16 (nearest even), as f32 values.

    Drawn and rounded in chunks in place: the generator's stream does not
    depend on how the draws are split, and the values are finite, so this
    equals bf16_to_f32(bf16_bits(standard_normal(shape) * 0.02))."""
    g = _rng(seed, name)
    out = np.empty(int(np.prod(shape)), dtype=np.float32)
    u = out.view(np.uint32)
    for i in range(0, out.size, _CHUNK):
        c = out[i:i + _CHUNK]
        g.standard_normal(out=c, dtype=np.float32)
        c *= np.float32(0.02)
        cu = u[i:i + _CHUNK]
        r = (cu >> 16) & np.uint32(1)
        r += np.uint32(0x7FFF)
        cu += r
        cu &= np.uint32(0xFFFF0000)
    return out.reshape(shape)


def _bits(seed: int, name: str, shape) -> np.ndarray:
    return (_draw_bf16(seed, name, shape).view(np.uint32) >> 16).astype(np.uint16)


def _w(seed: int, name: str, shape) -> np.ndarray:
    return _draw_bf16(seed, name, shape)


def _parallel(fn, jobs):
    """{name: fn(seed, name, shape)} for jobs [(seed, name, shape)], the
    tensors drawn on worker threads (each has its own generator)."""
    with ThreadPoolExecutor(max_workers=8) as ex:
        futs = {j[1]: ex.submit(fn, *j) for j in jobs}
        return {k: f.result() for k, f in futs.items()}


# The core tensors in CORE_SPECS order (ltx/core_parts.zig:53-72): name,
# shape. All bf16 except the f32 scale_shift_table "fsst".
IN_CH = 128
CORE_SPECS = [
    ("ada_l1_w", (D, TE)), ("ada_l1_b", (D,)), ("ada_l2_w", (D, D)), ("ada_l2_b", (D,)),
    ("ada_out_w", (9 * D, D)), ("ada_out_b", (9 * D,)),
    ("pada_l1_w", (D, TE)), ("pada_l1_b", (D,)), ("pada_l2_w", (D, D)), ("pada_l2_b", (D,)),
    ("pada_out_w", (2 * D, D)), ("pada_out_b", (2 * D,)),
    ("pat_w", (D, IN_CH)), ("pat_b", (D,)), ("po_w", (IN_CH, D)), ("po_b", (IN_CH,)),
    ("fsst", (2, D)),
]
CORE_FIELDS = [n for n, _ in CORE_SPECS]


def make_core(seed: int = 7) -> dict:
    """Seeded core tensors: bf16 bits (uint16) ~ N(0, 0.02) for the linear
    layers, the same draws ``tables`` uses for the conditioning MLPs; fsst
    f32 ~ N(0, 1) / sqrt(D)."""
    bits = _parallel(_bits, [(seed, name, shape) for name, shape in CORE_SPECS if name != "fsst"])
    out = {}
    for name, shape in CORE_SPECS:
        if name == "fsst":
            g = _rng(seed, name)
            out[name] = (g.standard_normal(shape, dtype=np.float32) / np.float32(np.sqrt(D))).astype(np.float32)
        else:
            out[name] = bits[name]
    return out


def mask_rows(T: int, striped: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """Distinct denoise-mask values [K] f32 and the per-token row index
    tidx [T] i32. Striped: the production pass's mask (ltx/e2e_prod.zig:
    218-229), 0 for the first T/7 tokens, 0.5 for the next T/7, 1 for the
    rest; else one row of 1."""
    if striped:
        mask = np.array([0.0, 0.5, 1.0], dtype=np.float32)
        tidx = np.full(T, 2, dtype=np.int32)
        tidx[: T // 7] = 0
        tidx[T // 7: 2 * T // 7] = 1
    else:
        mask = np.array([1.0], dtype=np.float32)
        tidx = np.zeros(T, dtype=np.int32)
    return mask, tidx


def sinusoid(t: np.ndarray) -> np.ndarray:
    """f32 sinusoid of t * 1000, cos half first (ltx/core_parts.zig:42-49)."""
    t = np.asarray(t, dtype=np.float32).reshape(-1, 1)
    freqs = np.exp(np.arange(HALF, dtype=np.float32) * np.float32(-np.log(1e4) / HALF)).astype(np.float32)
    arg = (t * np.float32(1000.0)) * freqs[None, :]
    return np.concatenate([np.cos(arg), np.sin(arg)], axis=1).astype(np.float32)


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _mlp_tables(seed: int):
    jobs = []
    for pfx in ("ada", "pada"):
        jobs += [(seed, pfx + "_l1_w", (D, TE)), (seed, pfx + "_l1_b", (D,)),
                 (seed, pfx + "_l2_w", (D, D)), (seed, pfx + "_l2_b", (D,))]
    jobs += [(seed, "ada_out_w", (9 * D, D)), (seed, "ada_out_b", (9 * D,)),
             (seed, "pada_out_w", (2 * D, D)), (seed, "pada_out_b", (2 * D,))]
    return _parallel(_w, jobs)


_CACHE: dict = {}


def tables(sigma: float, T: int, seed: int = 7, striped: bool = True):
    """(tstab [K, 9, D] f32, tidx [T] i32, pts2 [2, D] f32) for noise level sigma."""
    if seed not in _CACHE:
        _CACHE[seed] = _mlp_tables(seed)
    w = _CACHE[seed]
    mask, tidx = mask_rows(T, striped)
    t = (mask * np.float32(sigma)).astype(np.float32)
    e = sinusoid(t)
    h = _silu(e @ w["ada_l1_w"].T + w["ada_l1_b"])
    emb = h @ w["ada_l2_w"].T + w["ada_l2_b"]
    ts9 = _silu(emb) @ w["ada_out_w"].T + w["ada_out_b"]
    tstab = np.ascontiguousarray(ts9.reshape(len(t), 9, D), dtype=np.float32)
    ps = sinusoid(np.array([sigma], dtype=np.float32))
    ph = _silu(ps @ w["pada_l1_w"].T + w["pada_l1_b"])
    pe = ph @ w["pada_l2_w"].T + w["pada_l2_b"]
    p2 = _silu(pe) @ w["pada_out_w"].T + w["pada_out_b"]
    pts2 = np.ascontiguousarray(p2.reshape(2, D), dtype=np.float32)
    return tstab, tidx, pts2
