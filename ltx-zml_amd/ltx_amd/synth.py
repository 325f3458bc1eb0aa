"""Seeded synthetic blocks and inputs (no checkpoint or dataset is available
offline). Every tensor has its own generator, seeded by (seed, crc32(name)),
numpy PCG64, so any subset can be regenerated independently.

Weights (the block's 28 base tensors, ltx/block.zig:377-406):
  matrices and biases ~ dist * 0.02, dist = Student-t(nu = 3) or N(0, 1),
  rounded to bf16; q/k RMS-norm weights = bf16(1 + dist * 0.02);
  sst [9, D], psst [2, D] ~ N(0, 1) / sqrt(D) in f32.
Inputs: x, ctx ~ N(0, 1) f32; RoPE positions on a latent (F, H, W) grid.
"""
from __future__ import annotations

import zlib

import numpy as np

from . import blockfmt as bf
from . import conditioning

D, H, FF = bf.D, bf.H, bf.FF


def rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def _draw(g: np.random.Generator, shape, dist: str) -> np.ndarray:
    z = g.standard_normal(shape, dtype=np.float32)
    if dist == "t3":  # Student-t(3) = Z / sqrt(chi2_3 / 3), chi2_3 = 2 Gamma(1.5)
        chi = g.standard_gamma(1.5, size=shape, dtype=np.float32) * np.float32(2.0)
        z = z / np.sqrt(chi / np.float32(3.0))
    return z


def _tensor(block: int, seed: int, field: str, shape, dist: str, std: float) -> np.ndarray:
    g = rng(seed, f"{block}:{field}")
    if field in ("sst", "psst"):
        return (g.standard_normal(shape, dtype=np.float32) / np.float32(np.sqrt(D))).astype(np.float32)
    if field in ("qn1", "kn1", "qn2", "kn2"):
        return bf.bf16_bits(np.float32(1.0) + _draw(g, shape, dist) * np.float32(std))
    return bf.bf16_bits(_draw(g, shape, dist) * np.float32(std))


def make_block(block: int = 0, seed: int = 1, dist: str = "t3", std: float = 0.02,
               classes=("qkv", "ff"), scale_dtype: str = "F32", workers: int = 8) -> bf.BlockTensors:
    """Tensors are independent streams, drawn (and quantised) in parallel
    threads; the result does not depend on `workers`."""
    from concurrent.futures import ThreadPoolExecutor

    specs = bf.BASE_SPECS
    with ThreadPoolExecutor(max_workers=workers) as ex:
        arrs = list(ex.map(lambda s: _tensor(block, seed, s[0], s[2], dist, std), specs))
        base = {s[0]: a for s, a in zip(specs, arrs)}
        bt = bf.BlockTensors(block, base, {}, {})
        names = [qn for c in classes for qn in bf.CLASSES[c]]
        qs = list(ex.map(lambda qn: bf.quantize_g128(base[bf.Q8_BASE[qn]]), names))
    for qn, (q, s) in zip(names, qs):
        bt.q8[qn] = q
        bt.q8s[qn] = s.astype(np.float16) if scale_dtype == "F16" else s
    return bt


_ZERO_BF16 = {}


def make_block_q8(block: int, seed: int = 3, scale_dtype: str = "F16") -> bf.BlockTensors:
    """A seeded block whose seven projections are int8 from the start: q
    uniform over [-127, 127] and one scale per group of 128 drawn as
    0.02 / std(q) x U(0.5, 1.5) (weights of std ~0.02, the magnitude of
    make_block's), rounded to the scale type. The small tensors (biases,
    norm and gate weights, sst, psst) are drawn as in make_block with
    N(0, 1). The bf16 tensors of the int8 projections are never read when
    the int8 companions are present (neither by the upload nor by the
    oracle); they share one read-only zero array. About 0.5 s a block,
    against ~40 s for quantising drawn weights, which is what lets a test
    hold 48 independently seeded blocks."""
    base = {}
    q8, q8s = {}, {}
    qbase = set(bf.Q8_BASE.values())
    for field, _, shape, _ in bf.BASE_SPECS:
        if field in qbase:
            if shape not in _ZERO_BF16:
                z = np.zeros(shape, np.uint16)
                z.setflags(write=False)
                _ZERO_BF16[shape] = z
            base[field] = _ZERO_BF16[shape]
        else:
            base[field] = _tensor(block, seed, field, shape, "normal", 0.02)
    qstd = np.float32(np.sqrt((255 ** 2 - 1) / 12.0))  # std of the uniform integers -127..127
    for qn, field in bf.Q8_BASE.items():
        O, I = dict((s[0], s[2]) for s in bf.BASE_SPECS)[field]
        g = rng(seed, f"{block}:{qn}:q8")
        q8[qn] = g.integers(-127, 128, size=(O, I), dtype=np.int8)
        sc = (np.float32(0.02) / qstd) * g.uniform(0.5, 1.5, size=(O, I // bf.GROUP)).astype(np.float32)
        q8s[qn] = sc.astype(np.float16) if scale_dtype == "F16" else sc
    return bf.BlockTensors(block, base, q8, q8s)


def latent_grid(frames: int, height: int, width: int) -> np.ndarray:
    """[3, T, 2] f32 (start, end) positions, tokens frame-major. Positions are
    integers so the f32 grid is exact: frame index, and pixel coordinates
    32 * y, 32 * x of the latent cell (all < max_pos = (20, 2048, 2048))."""
    f, y, x = np.meshgrid(np.arange(frames), np.arange(height), np.arange(width), indexing="ij")
    pos = np.stack([f.ravel(), 32 * y.ravel(), 32 * x.ravel()]).astype(np.float32)  # [3, T]
    return np.ascontiguousarray(np.stack([pos, pos], axis=-1))


def grid_for_tokens(T: int) -> np.ndarray:
    """A latent grid with T tokens: (14, 32, 64) at 28,672, (4, 16, 16) at 1,024,
    else frames x 8 x (T / frames / 8) or a single row."""
    for fr, hh, ww in ((14, 32, 64), (4, 16, 16)):
        if fr * hh * ww == T:
            return latent_grid(fr, hh, ww)
    if T % 64 == 0:
        return latent_grid(T // 64, 8, 8)
    return latent_grid(1, 1, T)


def make_inputs(T: int, S: int, seed: int = 2, sigma: float = 0.7, striped: bool = True):
    x = rng(seed, "x").standard_normal((T, D), dtype=np.float32)
    ctx = rng(seed, "ctx").standard_normal((S, D), dtype=np.float32)
    tstab, tidx, pts2 = conditioning.tables(sigma, T, striped=striped)
    return dict(x=x, ctx=ctx, tstab=tstab, tidx=tidx, pts2=pts2, grid=grid_for_tokens(T))
