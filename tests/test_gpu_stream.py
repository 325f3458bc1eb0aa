"""GPU checks of the streaming upload (ltx_block_weights_from_blob_async):
one DMA of a blob image into the context's staging buffer, carved on the
device into the same form the synchronous upload builds
(ltx/loader.zig:133-172), and its use behind the pinned two-slot ring
(ltx/loader.zig:176-321) with the copy on its own stream.

Gate: bit-identical block outputs against the synchronous blob upload
(the weights are the same bytes, so every kernel sees identical operands).
"""
import ctypes as C
import json
import time

import numpy as np
import pytest

from conftest import say

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from ltx_amd import blockfmt as bf  # noqa: E402
from ltx_amd import runtime as rt  # noqa: E402
from ltx_amd import synth  # noqa: E402


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _forward(ctx, w, inp, cos, sin, stream=None):
    T = inp["x"].shape[0]
    y = torch.empty((T, 4096), dtype=torch.float32, device="cuda")
    ctx.forward(w, dev(inp["x"]), dev(inp["tstab"]), dev(inp["tidx"]), dev(inp["ctx"]), dev(inp["pts2"]), dev(cos),
                dev(sin), y, stream=stream)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _pinned(blob: bytes):
    t = torch.empty(len(blob), dtype=torch.uint8).pin_memory()
    t.numpy()[:] = np.frombuffer(blob, dtype=np.uint8)
    return t


@pytest.fixture(scope="module")
def blocks():
    """Block 0 in the reference recipe (q/k/v + ff int8, f32 scales, bf16
    out-projections) and block 1 with every projection int8 and f16 scales."""
    b0 = synth.make_block(0, seed=1, dist="t3")
    b1 = synth.make_block(1, seed=3, dist="t3", classes=("qkv", "ff", "out"), scale_dtype="F16")
    return b0, b1


@pytest.mark.parametrize("which", [0, 1])
def test_async_upload_equals_sync(ctx, blocks, which):
    bt = blocks[which]
    say(f"streaming upload vs synchronous, block {which}")
    blob, man = bf.pack(bt)
    mj = bf.manifest_json(man)
    inp = synth.make_inputs(256, 64)
    cos, sin = rt.rope_tables(inp["grid"])
    ws = ctx.upload_blob(blob, mj, bt.block)
    pin = _pinned(blob)
    st = torch.cuda.Stream()
    wa = ctx.upload_blob_async(pin.data_ptr(), len(blob), mj, bt.block, stream=st)
    st.synchronize()
    assert wa.nbytes == ws.nbytes
    a = _forward(ctx, ws, inp, cos, sin)
    b = _forward(ctx, wa, inp, cos, sin)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ws.free()
    wa.free()


def test_async_upload_reuse_and_errors(ctx, blocks):
    """A handle reused for another block of the same layout holds exactly
    that block; a handle of another layout is refused; manifest errors are
    the synchronous call's."""
    say("streaming upload: reuse of a handle, layout and manifest errors")
    b0, b1 = blocks
    bt1 = bf.BlockTensors(2, dict(b1.base), b1.q8, b1.q8s)
    blob1, man1 = bf.pack(b1)
    blob2, man2 = bf.pack(bt1)
    inp = synth.make_inputs(64, 32)
    cos, sin = rt.rope_tables(inp["grid"])
    st = torch.cuda.Stream()
    p1, p2 = _pinned(blob1), _pinned(blob2)
    w = ctx.upload_blob_async(p1.data_ptr(), len(blob1), bf.manifest_json(man1), 1, stream=st)
    w2 = ctx.upload_blob_async(p2.data_ptr(), len(blob2), bf.manifest_json(man2), 2, reuse=w, stream=st)
    st.synchronize()
    assert w2 is w
    ref = ctx.upload_blob(blob2, bf.manifest_json(man2), 2)
    a = _forward(ctx, w, inp, cos, sin)
    b = _forward(ctx, ref, inp, cos, sin)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # block 0's layout (bf16 out-projections, f32 scales) differs from block 1's
    blob0, man0 = bf.pack(b0)
    p0 = _pinned(blob0)
    with pytest.raises(rt.LtxError, match="different layout"):
        ctx.upload_blob_async(p0.data_ptr(), len(blob0), bf.manifest_json(man0), 0, reuse=w, stream=st)
    with pytest.raises(rt.LtxError, match="no entry named"):
        ctx.upload_blob_async(p0.data_ptr(), len(blob0), bf.manifest_json(man0), 5, stream=st)
    st.synchronize()
    for h in (w, ref):
        h.free()


def _write_blob(d, blob: bytes, man: dict):
    d.mkdir(parents=True, exist_ok=True)
    (d / "blob.bin").write_bytes(blob)
    (d / "blob_manifest.json").write_text(json.dumps(man))


def test_ring_streams_blocks_through_async_uploads(ctx, blocks, tmp_path):
    """Two blobs on disk, the pinned ring staging a schedule of block
    executions, each slot uploaded with one DMA on a copy stream (double
    buffered handles) while the previous block computes on the compute
    stream; the slot is released once its copy has passed. The chained output
    equals the chain over synchronously uploaded weights, bit for bit."""
    say("ring + streaming uploads: schedule 0 1 0 1 0 1, T=256 S=64")
    b0 = blocks[1]
    b1 = bf.BlockTensors(2, dict(b0.base), b0.q8, b0.q8s)
    bts = [b0, b1]
    L = rt.lib()
    hs, mans, sizes = [], [], []
    for i, bt in enumerate(bts):
        blob, man = bf.pack(bt)
        _write_blob(tmp_path / f"b{i}", blob, man)
        h = C.c_void_p()
        assert L.ltx_blob_open(str(tmp_path / f"b{i}").encode(), C.byref(h)), L.ltx_loader_last_error()
        hs.append(h.value)
        mans.append(bf.manifest_json(man))
        sizes.append(len(blob))
    sched = [0, 1, 0, 1, 0, 1]
    arr = (C.c_void_p * 2)(*hs)
    sc = (C.c_int * len(sched))(*sched)
    r = C.c_void_p()
    assert L.ltx_ring_create(arr, 2, sc, len(sched), 0, max(sizes), 1, C.byref(r)), L.ltx_loader_last_error()
    inp = synth.make_inputs(256, 64)
    cos, sin = rt.rope_tables(inp["grid"])
    dcos, dsin = dev(cos), dev(sin)
    args = [dev(inp[k]) for k in ("tstab", "tidx", "ctx", "pts2")]
    copy_st, comp_st = torch.cuda.Stream(), torch.cuda.Stream()
    handles = [None, None]
    x = dev(inp["x"])
    ys = [torch.empty_like(x), torch.empty_like(x)]
    done = [None, None]  # event after the last forward that read handle i
    try:
        assert L.ltx_ring_static_check(r.value)
        assert L.ltx_ring_start(r.value)
        t0 = time.time()
        for pos, bi in enumerate(sched):
            p, n = C.c_void_p(), C.c_uint64()
            assert L.ltx_ring_acquire(r.value, pos, C.byref(p), C.byref(n)), L.ltx_loader_last_error()
            k = pos & 1
            if done[k] is not None:
                copy_st.wait_event(done[k])  # the handle's previous forward has read it
            handles[k] = ctx.upload_blob_async(p.value, n.value, mans[bi], bts[bi].block, reuse=handles[k],
                                               stream=copy_st)
            copied = torch.cuda.Event()
            copied.record(copy_st)
            comp_st.wait_event(copied)
            y = ys[pos & 1]
            ctx.forward(handles[k], x, *args[:2], args[2], args[3], dcos, dsin, y, stream=comp_st)
            done[k] = torch.cuda.Event()
            done[k].record(comp_st)
            copied.synchronize()  # the slot's bytes have been copied
            assert L.ltx_ring_release(r.value, pos)
            x = y
        comp_st.synchronize()
        got = x.cpu().numpy()
        print(f"ring streaming: {len(sched)} block executions in {time.time() - t0:.2f} s", flush=True)
    finally:
        L.ltx_ring_destroy(r.value)
        for h in hs:
            L.ltx_blob_close(h)
    # reference chain over synchronously uploaded weights
    ws = [ctx.upload(bt) for bt in bts]
    xr = dev(inp["x"])
    for bi in sched:
        yr = torch.empty_like(xr)
        ctx.forward(ws[bi], xr, *args[:2], args[2], args[3], dcos, dsin, yr)
        xr = yr
    torch.cuda.synchronize()
    want = xr.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for h in handles + ws:
        h.free()
