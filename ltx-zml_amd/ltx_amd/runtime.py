"""ctypes bindings of libltx_amd.so (include/ltx_block.h, include/ltx_loader.h).

Device memory and streams come from PyTorch (plumbing only); every compute
call goes through the C ABI into the gfx950 kernels. There is no fallback:
a missing library or a failed call raises.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import weakref

import numpy as np

from . import blockfmt as bf

PKG_DIR = pathlib.Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "libltx_amd.so"

MODE_F16, MODE_BF16, MODE_F32 = 0, 1, 2
ATTN_Q_SCALED = 0x100  # ltx_op_attention mode flag
ATTN_C = float(np.float32(1.4426950408889634 / 11.313708498984761))  # log2(e) / sqrt(128)
MODES = {"f16": MODE_F16, "bf16": MODE_BF16, "f32": MODE_F32}
STAGES = ["norm_msa", "q1", "k1", "v1", "glog1", "attn1", "x_sa", "attn_in", "attn2", "x_ca", "ff_in", "ff_h",
          "glog2", "q2", "k2", "v2", "velocity"]

W_COUNT, Q_COUNT = 28, 10

_lib = None


class LtxError(RuntimeError):
    pass


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise LtxError(f"{LIB_PATH} is not built; run `python ltx-zml_amd/build.py`")
    L = C.CDLL(str(LIB_PATH))
    vp, i32, i64, u64 = C.c_void_p, C.c_int, C.c_int64, C.c_uint64
    sig = {
        "ltx_init": (i32, [i32, C.POINTER(vp)]),
        "ltx_destroy": (None, [vp]),
        "ltx_last_error": (C.c_char_p, [vp]),
        "ltx_version": (C.c_char_p, []),
        "ltx_block_weights_from_blob": (i32, [vp, vp, u64, C.c_char_p, i64, C.POINTER(vp)]),
        "ltx_block_weights_from_host": (i32, [vp, C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), i32, C.POINTER(vp)]),
        "ltx_block_weights_from_blob_async": (i32, [vp, vp, u64, C.c_char_p, i64, vp, vp, C.POINTER(vp)]),
        "ltx_block_weights_free": (None, [vp, vp]),
        "ltx_block_weights_bytes": (u64, [vp]),
        "ltx_block_forward": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, vp, vp, vp, i32, vp, i32, vp]),
        "ltx_block_graph_create": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, vp, vp, vp, i32, vp, i32, C.POINTER(vp)]),
        "ltx_block_graph_launch": (i32, [vp, vp]),
        "ltx_block_graph_destroy": (None, [vp]),
        "ltx_block_stage": (i32, [vp, i32, C.POINTER(vp), C.POINTER(u64)]),
        "ltx_range_count": (i32, [vp, vp, C.POINTER(u64), i32]),
        "ltx_op_linear_q8": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32, i32, i32, vp]),
        "ltx_op_linear_q8_noalloc": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32, i32, i32, vp]),
        "ltx_op_attention": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, vp]),
        "ltx_op_dequant": (i32, [vp, vp, vp, i32, i32, i32, vp, vp, i32, vp]),
        "ltx_rope_tables": (i32, [vp, i32, vp, vp, i32]),
        "ltx_profile_enable": (i32, [vp, i32]),
        "ltx_profile_read": (i32, [vp, C.c_char_p, C.POINTER(C.c_double), C.POINTER(i32)]),
        "ltx_profile_reset": (i32, [vp]),
        "ltx_blob_open": (i32, [C.c_char_p, C.POINTER(vp)]),
        "ltx_blob_close": (None, [vp]),
        "ltx_blob_check_layout": (i32, [vp]),
        "ltx_blob_verify": (i32, [vp]),
        "ltx_blob_data": (vp, [vp, C.POINTER(u64)]),
        "ltx_blob_manifest_text": (C.c_char_p, [vp]),
        "ltx_blob_block_index": (i64, [vp]),
        "ltx_blob_find": (i32, [vp, C.c_char_p, C.POINTER(u64), C.POINTER(u64), C.c_char_p, i32]),
        "ltx_ring_create": (i32, [C.POINTER(vp), i32, C.POINTER(i32), i32, i32, u64, i32, C.POINTER(vp)]),
        "ltx_ring_static_check": (i32, [vp]),
        "ltx_ring_start": (i32, [vp]),
        "ltx_ring_acquire": (i32, [vp, i32, C.POINTER(vp), C.POINTER(u64)]),
        "ltx_ring_release": (i32, [vp, i32]),
        "ltx_ring_abort": (None, [vp]),
        "ltx_ring_stats": (i32, [vp, C.POINTER(u64), C.POINTER(u64), C.POINTER(u64), C.POINTER(u64)]),
        "ltx_ring_set_reader_delay_us": (i32, [vp, C.c_uint32]),
        "ltx_ring_destroy": (None, [vp]),
        "ltx_loader_last_error": (C.c_char_p, []),
        "ltx_sha256_hex": (i32, [vp, u64, C.c_char_p]),
        "ltx_core_weights_from_host": (i32, [vp, C.POINTER(vp), C.POINTER(vp)]),
        "ltx_core_weights_free": (None, [vp, vp]),
        "ltx_core_conditioning": (i32, [vp, vp, vp, i32, vp, vp, vp, vp, vp]),
        "ltx_core_patchify": (i32, [vp, vp, vp, i32, vp, vp]),
        "ltx_core_tail": (i32, [vp, vp, vp, vp, vp, i32, vp, vp]),
        "ltx_sched_sigmas": (i32, [i32, vp, C.POINTER(i32)]),
        "ltx_sched_noise_init": (i32, [vp, vp, vp, vp, vp, i32, i32, C.c_float, vp, vp]),
        "ltx_sched_step": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, i32, C.c_float, C.c_float, vp, vp]),
        "ltx_denoise": (i32, [vp, C.POINTER(vp), i32, vp, vp, vp, vp, vp, i32, vp, i32, vp, vp, i32, vp, i32, i32,
                              vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _ptr(t) -> int | None:
    """Device/host address of a torch tensor or numpy array (None -> NULL)."""
    if t is None:
        return None
    if isinstance(t, np.ndarray):
        return t.ctypes.data
    return t.data_ptr()


def rope_tables(grid: np.ndarray, graph_layout: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """Host f64 3D-RoPE tables (ltx/block_conformance.zig:87-126)."""
    grid = np.ascontiguousarray(grid, dtype=np.float32)
    T = grid.shape[1]
    shape = (T, 32, 64) if graph_layout else (32, T, 64)
    cos, sin = np.empty(shape, np.float32), np.empty(shape, np.float32)
    if not lib().ltx_rope_tables(_ptr(grid), T, _ptr(cos), _ptr(sin), int(graph_layout)):
        raise LtxError(lib().ltx_last_error(None).decode())
    return cos, sin


def sha256_hex(data: bytes) -> str:
    out = C.create_string_buffer(65)
    lib().ltx_sha256_hex(data, len(data), out)
    return out.value.decode()


def sched_sigmas(stage: int = 1) -> np.ndarray:
    """The distilled sigma list of a stage (ltx/scheduler.zig:15-18)."""
    n = C.c_int()
    if not lib().ltx_sched_sigmas(stage, None, C.byref(n)):
        raise LtxError(lib().ltx_last_error(None).decode())
    out = np.empty(n.value, np.float32)
    lib().ltx_sched_sigmas(stage, out.ctypes.data, C.byref(n))
    return out


class CoreWeights:
    """Device copy of the parts around the blocks (ltx/core_parts.zig:86-104)."""

    def __init__(self, ctx: "Context", handle: int):
        self.ctx, self.handle = ctx, handle

    def free(self):
        if self.handle:
            lib().ltx_core_weights_free(self.ctx.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weights:
    def __init__(self, ctx: "Context", handle: int):
        self.ctx, self.handle = ctx, handle

    @property
    def nbytes(self) -> int:
        return lib().ltx_block_weights_bytes(self.handle)

    def free(self):
        if self.handle:
            lib().ltx_block_weights_free(self.ctx.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class BlockGraph:
    """One block forward captured with its buffers bound (ltx_block_graph_*);
    launch() replays it on a stream."""

    def __init__(self, ctx: "Context", handle: int, keep: tuple):
        self.ctx, self.handle = ctx, handle
        self._keep = keep  # the bound tensors stay alive with the graph

    def launch(self, stream=None):
        st = stream.cuda_stream if stream is not None else _current_stream()
        self.ctx._check(lib().ltx_block_graph_launch(self.handle, st), "ltx_block_graph_launch")

    def free(self):
        if self.handle:
            lib().ltx_block_graph_destroy(self.handle)
            self.handle = None
            self._keep = ()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One device context (ltx_init). Not thread-safe."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        if not lib().ltx_init(device, C.byref(h)):
            raise LtxError("ltx_init: " + lib().ltx_last_error(None).decode())
        self.handle = h.value
        self.device = device
        self._graphs = weakref.WeakSet()

    def _check(self, ok: int, what: str):
        if not ok:
            raise LtxError(f"{what}: " + lib().ltx_last_error(self.handle).decode())

    def close(self):
        if self.handle:
            for g in list(self._graphs):  # graphs hold the context's workspace
                g.free()
            lib().ltx_destroy(self.handle)
            self.handle = None

    # ---- weights ----
    def upload(self, bt: bf.BlockTensors) -> Weights:
        base = (C.c_void_p * W_COUNT)()
        for i, f in enumerate(bf.FIELDS):
            base[i] = bt.base[f].ctypes.data
        q8 = (C.c_void_p * Q_COUNT)()
        q8s = (C.c_void_p * Q_COUNT)()
        for i, qn in enumerate(bf.Q8_FIELDS):
            if qn in bt.q8:
                q8[i] = bt.q8[qn].ctypes.data
                q8s[i] = bt.q8s[qn].ctypes.data
        h = C.c_void_p()
        self._check(lib().ltx_block_weights_from_host(self.handle, base, q8, q8s, int(bt.scale_f16), C.byref(h)),
                    "ltx_block_weights_from_host")
        return Weights(self, h.value)

    def upload_blob(self, blob: bytes | np.ndarray, manifest_json: str, block: int) -> Weights:
        buf = np.frombuffer(blob, dtype=np.uint8) if not isinstance(blob, np.ndarray) else blob
        h = C.c_void_p()
        self._check(lib().ltx_block_weights_from_blob(self.handle, buf.ctypes.data, buf.nbytes,
                                                      manifest_json.encode(), block, C.byref(h)),
                    "ltx_block_weights_from_blob")
        return Weights(self, h.value)

    def upload_blob_async(self, mem_ptr: int, nbytes: int, manifest_json: str, block: int, reuse: Weights | None = None,
                          stream=None) -> Weights:
        """Streaming upload from `mem_ptr` (pinned host memory, e.g. a ring
        slot) on `stream`; returns at once. Keep the memory unchanged until
        the stream passes this call."""
        st = stream.cuda_stream if stream is not None else _current_stream()
        h = C.c_void_p()
        self._check(lib().ltx_block_weights_from_blob_async(self.handle, mem_ptr, nbytes, manifest_json.encode(),
                                                            block, reuse.handle if reuse else None, st, C.byref(h)),
                    "ltx_block_weights_from_blob_async")
        return reuse if reuse is not None else Weights(self, h.value)

    # ---- forward ----
    def forward(self, w: Weights, x, tstab, tidx, ctx, pts2, cos, sin, y, mode: int = MODE_F16, stream=None):
        T, S, K = x.shape[0], ctx.shape[0], tstab.shape[0]
        st = stream.cuda_stream if stream is not None else _current_stream()
        self._check(lib().ltx_block_forward(self.handle, w.handle, _ptr(x), _ptr(tstab), K, _ptr(tidx), _ptr(ctx), S,
                                            _ptr(pts2), _ptr(cos), _ptr(sin), T, _ptr(y), mode, st),
                    "ltx_block_forward")
        return y

    def block_graph(self, w: Weights, x, tstab, tidx, ctx, pts2, cos, sin, y, mode: int = MODE_F16) -> BlockGraph:
        """The forward of ``forward`` with these tensors, captured once
        (ltx_block_graph_create); BlockGraph.launch() runs it."""
        T, S, K = x.shape[0], ctx.shape[0], tstab.shape[0]
        h = C.c_void_p()
        self._check(lib().ltx_block_graph_create(self.handle, w.handle, _ptr(x), _ptr(tstab), K, _ptr(tidx), _ptr(ctx),
                                                 S, _ptr(pts2), _ptr(cos), _ptr(sin), T, _ptr(y), mode, C.byref(h)),
                    "ltx_block_graph_create")
        g = BlockGraph(self, h.value, (w, x, tstab, tidx, ctx, pts2, cos, sin, y))
        self._graphs.add(g)
        return g

    def range_count(self, reset: bool = True, stream=None) -> int:
        """16-bit stores out of range since the last reset (ltx_range_count)."""
        st = stream.cuda_stream if stream is not None else _current_stream()
        n = C.c_uint64()
        self._check(lib().ltx_range_count(self.handle, st, C.byref(n), int(reset)), "ltx_range_count")
        return n.value

    def stage(self, name: str):
        import torch
        p, n = C.c_void_p(), C.c_uint64()
        self._check(lib().ltx_block_stage(self.handle, STAGES.index(name), C.byref(p), C.byref(n)), "ltx_block_stage")
        out = torch.empty(n.value, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        _memcpy_dtod(out.data_ptr(), p.value, n.value)
        return out

    # ---- operators ----
    def linear_q8(self, a, q, s, bias, y, mode=MODE_F16, gelu=False, stream=None, noalloc=False):
        """noalloc: the entry point with its scratch in the library's static
        device array (ltx_op_linear_q8_noalloc)."""
        M, K = a.shape
        N = q.shape[0]
        import torch
        st = stream.cuda_stream if stream is not None else _current_stream()
        name = "ltx_op_linear_q8_noalloc" if noalloc else "ltx_op_linear_q8"
        self._check(getattr(lib(), name)(self.handle, _ptr(a), _ptr(q), _ptr(s), int(s.dtype == torch.float16),
                                         _ptr(bias), _ptr(y), int(y.dtype == torch.float32), M, N, K, int(gelu),
                                         mode, st), name)
        return y

    def attention(self, q, k, v, glog, out, lq, lkv, mode=MODE_F16, stream=None, q_scaled=False):
        """q_scaled: q already holds q * log2(e) / sqrt(128) (LTX_ATTN_Q_SCALED)."""
        st = stream.cuda_stream if stream is not None else _current_stream()
        m = mode | (ATTN_Q_SCALED if q_scaled else 0)
        self._check(lib().ltx_op_attention(self.handle, _ptr(q), _ptr(k), _ptr(v), _ptr(glog), _ptr(out), lq, lkv,
                                           m, st), "ltx_op_attention")
        return out

    def dequant(self, q, s, out32, out16, mode=MODE_F16, stream=None):
        import torch
        N, K = q.shape
        st = stream.cuda_stream if stream is not None else _current_stream()
        self._check(lib().ltx_op_dequant(self.handle, _ptr(q), _ptr(s), int(s.dtype == torch.float16), N, K,
                                         _ptr(out32), _ptr(out16), mode, st), "ltx_op_dequant")

    # ---- parts around the blocks and the scheduler ----
    def upload_core(self, tensors: dict) -> CoreWeights:
        """tensors: field -> numpy array in CORE_SPECS order (bf16 bits as
        uint16, fsst f32), e.g. conditioning.make_core()."""
        from .conditioning import CORE_FIELDS
        arrs = [np.ascontiguousarray(tensors[f]) for f in CORE_FIELDS]
        ptrs = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
        h = C.c_void_p()
        self._check(lib().ltx_core_weights_from_host(self.handle, ptrs, C.byref(h)), "ltx_core_weights_from_host")
        return CoreWeights(self, h.value)

    def conditioning(self, cw: CoreWeights, t, sigma, tstab, emb, pts2, stream=None):
        """t [K] f32, sigma [1] f32 (device) -> tstab [K, 9, D], emb [K, D], pts2 [2, D]."""
        st = stream.cuda_stream if stream is not None else _current_stream()
        self._check(lib().ltx_core_conditioning(self.handle, cw.handle, _ptr(t), t.shape[0], _ptr(sigma), _ptr(tstab),
                                                _ptr(emb), _ptr(pts2), st), "ltx_core_conditioning")

    def patchify(self, cw: CoreWeights, latent, x, stream=None):
        st = stream.cuda_stream if stream is not None else _current_stream()
        self._check(lib().ltx_core_patchify(self.handle, cw.handle, _ptr(latent), latent.shape[0], _ptr(x), st),
                    "ltx_core_patchify")
        return x

    def tail(self, cw: CoreWeights, x, emb, tidx, vel, stream=None):
        st = stream.cuda_stream if stream is not None else _current_stream()
        self._check(lib().ltx_core_tail(self.handle, cw.handle, _ptr(x), _ptr(emb), _ptr(tidx), x.shape[0], _ptr(vel),
                                        st), "ltx_core_tail")
        return vel

    def noise_init(self, clean, noise, maskk, tidx, noise_scale: float, out, stream=None):
        T, Cc = clean.shape
        st = stream.cuda_stream if stream is not None else _current_stream()
        self._check(lib().ltx_sched_noise_init(self.handle, _ptr(clean), _ptr(noise), _ptr(maskk), _ptr(tidx), T, Cc,
                                               float(noise_scale), _ptr(out), st), "ltx_sched_noise_init")
        return out

    def sched_step(self, x, vel, tk, maskk, tidx, clean, sigma: float, sigma_next: float, out, stream=None):
        T, Cc = x.shape
        st = stream.cuda_stream if stream is not None else _current_stream()
        self._check(lib().ltx_sched_step(self.handle, _ptr(x), _ptr(vel), _ptr(tk), _ptr(maskk), _ptr(tidx),
                                         _ptr(clean), T, Cc, float(sigma), float(sigma_next), _ptr(out), st),
                    "ltx_sched_step")
        return out

    def denoise(self, blocks: list, cw: CoreWeights, latent, clean, maskk, tidx, ctx, cos, sin, sigmas,
                mode: int = MODE_F16, stream=None):
        """Runs len(sigmas) - 1 steps over the resident blocks; latent [T, 128]
        is updated in place."""
        sig = np.ascontiguousarray(sigmas, np.float32)
        hs = (C.c_void_p * len(blocks))(*[b.handle for b in blocks])
        st = stream.cuda_stream if stream is not None else _current_stream()
        self._check(lib().ltx_denoise(self.handle, hs, len(blocks), cw.handle, _ptr(latent), _ptr(clean), _ptr(maskk),
                                      _ptr(tidx), maskk.shape[0], _ptr(ctx), ctx.shape[0], _ptr(cos), _ptr(sin),
                                      latent.shape[0], sig.ctypes.data, len(sig) - 1, mode, st), "ltx_denoise")
        return latent

    # ---- profiling ----
    def profile(self, enable: bool):
        self._check(lib().ltx_profile_enable(self.handle, int(enable)), "ltx_profile_enable")

    def profile_reset(self):
        self._check(lib().ltx_profile_reset(self.handle), "ltx_profile_reset")

    def profile_read(self, substr: str = "") -> tuple[float, int]:
        ms, n = C.c_double(), C.c_int()
        self._check(lib().ltx_profile_read(self.handle, substr.encode(), C.byref(ms), C.byref(n)), "ltx_profile_read")
        return ms.value, n.value


def _current_stream() -> int:
    import torch
    return torch.cuda.current_stream().cuda_stream


def _memcpy_dtod(dst: int, src: int, n: int):
    import torch
    # a uint8 view of the source allocation through torch's storage API is not
    # available for foreign pointers; use hipMemcpy from the HIP runtime.
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipMemcpy.restype = C.c_int
    rc = hip.hipMemcpy(dst, src, n, 3)  # hipMemcpyDeviceToDevice
    if rc != 0:
        raise LtxError(f"hipMemcpy failed ({rc})")
    torch.cuda.synchronize()
