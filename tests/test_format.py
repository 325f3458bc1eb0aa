"""The blob format and the loader (CPU): packer byte-identity with the
reference tool's output, the C++ Blob (mmap, layout check, digest, lookup)
and Ring (slot state machine, reader thread, abort) through the C ABI.
Error names follow ltx/loader.zig."""
import ctypes as C
import json
import pathlib
import shutil

import numpy as np
import pytest

from ltx_amd import blockfmt as bf
from ltx_amd import runtime as rt

GOLD = pathlib.Path(__file__).resolve().parent / "golden" / "quant_pack"


def test_pack_dir_matches_reference_tool(tmp_path):
    """quantize_dir + pack_dir on the golden input reproduce the reference
    tools' blob.bin and blob_manifest.json byte for byte."""
    d = tmp_path / "blk"
    shutil.copytree(GOLD / "input", d)
    bf.quantize_dir(d, "qkv")
    bf.quantize_dir(d, "ff")
    bf.pack_dir(d, packer_commit="unknown")
    for f in sorted((GOLD / "output").iterdir()):
        assert (d / f.name).read_bytes() == f.read_bytes(), f.name


def test_pack_block_layout_and_determinism(block0):
    blob, man = bf.pack(block0)
    assert len(man["entries"]) == 44  # 28 base + 8 q8 + 8 q8scale (EXPECTED_ENTRIES, tools/assemble_blocks.py:28)
    bf.check_layout(man)
    names = [e["name"] for e in man["entries"]]
    assert names == sorted(names)
    assert all(e["offset"] % 64 == 0 for e in man["entries"])
    blob2, man2 = bf.pack(block0)
    assert man2["blob_sha256"] == man["blob_sha256"] and blob2 == blob
    back = bf.unpack(blob, man)
    for f in bf.FIELDS:
        assert np.array_equal(back.base[f], block0.base[f])
    for qn in block0.q8:
        assert np.array_equal(back.q8[qn], block0.q8[qn])
        assert np.array_equal(back.q8s[qn], block0.q8s[qn])


def test_normalize_name():
    assert bf.normalize_name("transformer_blocks.3.attn1.to_q.weight::q8scale") == \
        "transformer_blocks_3_attn1_to_q_weight_q8scale"
    assert bf.normalize_name("transformer_blocks.3.ff.net.0.proj.weight::q8") == \
        "transformer_blocks_3_ff_net_0_proj_weight_q8"


def test_check_layout_errors():
    man = json.loads((GOLD / "output" / "blob_manifest.json").read_text())
    bf.check_layout(man)
    for mutate, err in ((lambda m: m["entries"][1].__setitem__("offset", m["entries"][1]["offset"] + 1), "Misaligned"),
                        (lambda m: m["entries"][1].__setitem__("offset", m["entries"][1]["offset"] + 64), "LayoutGap"),
                        (lambda m: m.__setitem__("total_bytes", m["total_bytes"] + 1), "TrailingBytes")):
        m = json.loads(json.dumps(man))
        mutate(m)
        with pytest.raises(ValueError, match=err):
            bf.check_layout(m)


# ---- C++ Blob --------------------------------------------------------------

def _write_blob(dirpath: pathlib.Path, blob: bytes, man: dict):
    dirpath.mkdir(parents=True, exist_ok=True)
    (dirpath / "blob.bin").write_bytes(blob)
    (dirpath / "blob_manifest.json").write_text(bf.manifest_json(man))


def _open(d):
    L = rt.lib()
    h = C.c_void_p()
    ok = L.ltx_blob_open(str(d).encode(), C.byref(h))
    return ok, h.value, L.ltx_loader_last_error().decode()


def test_blob_open_check_find_verify(tmp_path):
    blob = (GOLD / "output" / "blob.bin").read_bytes()
    man = json.loads((GOLD / "output" / "blob_manifest.json").read_text())
    _write_blob(tmp_path / "b", blob, man)
    L = rt.lib()
    ok, h, err = _open(tmp_path / "b")
    assert ok, err
    try:
        assert L.ltx_blob_check_layout(h) and L.ltx_blob_verify(h)
        assert L.ltx_blob_block_index(h) == 0
        n = C.c_uint64()
        p = L.ltx_blob_data(h, C.byref(n))
        assert n.value == len(blob) and C.string_at(p, n.value) == blob
        off, nb = C.c_uint64(), C.c_uint64()
        dt = C.create_string_buffer(8)
        assert L.ltx_blob_find(h, b"transformer_blocks_0_attn1_to_q_weight_q8scale", C.byref(off), C.byref(nb), dt, 8)
        e = [e for e in man["entries"] if e["name"].endswith("to_q.weight::q8scale")][0]
        assert (off.value, nb.value, dt.value) == (e["offset"], e["nbytes"], b"F32")
        assert not L.ltx_blob_find(h, b"transformer_blocks_0_nope", None, None, None, 0)
        assert "MissingEntry" in L.ltx_loader_last_error().decode()
        assert json.loads(L.ltx_blob_manifest_text(h).decode()) == man
    finally:
        L.ltx_blob_close(h)


def test_blob_error_paths(tmp_path):
    blob = bytearray((GOLD / "output" / "blob.bin").read_bytes())
    man = json.loads((GOLD / "output" / "blob_manifest.json").read_text())
    L = rt.lib()
    # truncated -> BlobSizeMismatch
    _write_blob(tmp_path / "t", bytes(blob[:-1]), man)
    ok, h, err = _open(tmp_path / "t")
    assert not ok and "BlobSizeMismatch" in err
    # one corrupted byte -> BlobDigestMismatch on verify
    bad = bytearray(blob)
    bad[100] ^= 0xFF
    _write_blob(tmp_path / "c", bytes(bad), man)
    ok, h, err = _open(tmp_path / "c")
    assert ok
    assert not L.ltx_blob_verify(h) and "BlobDigestMismatch" in L.ltx_loader_last_error().decode()
    L.ltx_blob_close(h)
    # manifest layout errors
    for key, delta, name in (("offset", 1, "Misaligned"), ("offset", 64, "LayoutGap")):
        m = json.loads(json.dumps(man))
        m["entries"][2][key] += delta
        _write_blob(tmp_path / name, bytes(blob), m)
        ok, h, err = _open(tmp_path / name)
        assert ok
        assert not L.ltx_blob_check_layout(h) and name in L.ltx_loader_last_error().decode()
        L.ltx_blob_close(h)


def test_blob_manifest_bounds(tmp_path):
    """Offsets and sizes that do not lie inside the blob (negative, or whose
    sum would wrap past 2^64) and a non-positive alignment are refused when
    the manifest is read."""
    blob = (GOLD / "output" / "blob.bin").read_bytes()
    man = json.loads((GOLD / "output" / "blob_manifest.json").read_text())
    cases = [("neg_offset", lambda m: m["entries"][1].update(offset=-64), "TrailingBytes"),
             ("neg_nbytes", lambda m: m["entries"][1].update(nbytes=-1), "TrailingBytes"),
             ("wrap", lambda m: m["entries"][1].update(offset=64, nbytes=2 ** 63 - 1), "TrailingBytes"),
             ("past_end", lambda m: m["entries"][-1].update(nbytes=m["entries"][-1]["nbytes"] + 1), "TrailingBytes"),
             ("align0", lambda m: m.update(align=0), "Misaligned"),
             ("align_neg", lambda m: m.update(align=-64), "Misaligned")]
    for name, edit, err_name in cases:
        m = json.loads(json.dumps(man))
        edit(m)
        _write_blob(tmp_path / name, blob, m)
        ok, h, err = _open(tmp_path / name)
        assert not ok and err_name in err, (name, err)


def test_sha256_matches_hashlib():
    import hashlib
    for n in (0, 1, 55, 56, 63, 64, 65, 1000):
        data = bytes(range(256)) * 4
        assert rt.sha256_hex(data[:n]) == hashlib.sha256(data[:n]).hexdigest()


# ---- C++ Ring --------------------------------------------------------------

def _two_blobs(tmp_path):
    L = rt.lib()
    hs, datas = [], []
    for i in range(2):
        rng = np.random.default_rng(i)
        arr = rng.integers(0, 255, size=4096 + 64 * i, dtype=np.uint8).tobytes()
        blob, man = bf.pack_entries([(f"transformer_blocks.{i}.x", arr, "I8", [len(arr)])], i, "r", "v", "f", "", "c")
        _write_blob(tmp_path / f"b{i}", blob, man)
        ok, h, err = _open(tmp_path / f"b{i}")
        assert ok, err
        hs.append(h)
        datas.append(blob)
    return hs, datas


def _ring(hs, sched, verify=1, slot=1 << 16):
    L = rt.lib()
    arr = (C.c_void_p * len(hs))(*hs)
    s = (C.c_int * len(sched))(*sched)
    r = C.c_void_p()
    ok = L.ltx_ring_create(arr, len(hs), s, len(sched), verify, slot, 0, C.byref(r))
    assert ok, L.ltx_loader_last_error()
    return r.value


@pytest.mark.parametrize("delay_us", [0, 2000])
def test_ring_stages_schedule_in_order(tmp_path, delay_us):
    L = rt.lib()
    hs, datas = _two_blobs(tmp_path)
    sched = [0, 1, 1, 0, 1, 0, 0]
    r = _ring(hs, sched)
    try:
        assert L.ltx_ring_static_check(r)
        L.ltx_ring_set_reader_delay_us(r, delay_us)
        assert L.ltx_ring_start(r)
        for pos, bi in enumerate(sched):
            p, n = C.c_void_p(), C.c_uint64()
            assert L.ltx_ring_acquire(r, pos, C.byref(p), C.byref(n)), L.ltx_loader_last_error()
            assert C.string_at(p, n.value) == datas[bi]
            assert L.ltx_ring_release(r, pos)
        stats = [C.c_uint64() for _ in range(4)]
        L.ltx_ring_stats(r, *(C.byref(x) for x in stats))
        if delay_us:
            assert stats[1].value > 0  # the consumer waited on the slow reader
    finally:
        L.ltx_ring_destroy(r)
        for h in hs:
            L.ltx_blob_close(h)


def test_ring_static_check_errors(tmp_path):
    L = rt.lib()
    hs, _ = _two_blobs(tmp_path)
    r = _ring(hs, [0, 2])
    assert not L.ltx_ring_static_check(r) and "ScheduleOutOfRange" in L.ltx_loader_last_error().decode()
    L.ltx_ring_destroy(r)
    r = _ring(hs, [0, 1], slot=1024)
    assert not L.ltx_ring_static_check(r) and "SlotTooSmall" in L.ltx_loader_last_error().decode()
    L.ltx_ring_destroy(r)
    for h in hs:
        L.ltx_blob_close(h)


def test_ring_abort_with_parked_reader_does_not_hang(tmp_path):
    """The consumer holds a slot and errors out; the reader is parked on a full
    ring. abort + join must return (the deadlock fixed at ltx/loader.zig:199-202)."""
    L = rt.lib()
    hs, _ = _two_blobs(tmp_path)
    r = _ring(hs, [0, 1, 0, 1, 0])
    L.ltx_ring_start(r)
    p, n = C.c_void_p(), C.c_uint64()
    assert L.ltx_ring_acquire(r, 0, C.byref(p), C.byref(n))
    L.ltx_ring_destroy(r)  # never released slot 0: reader parked; destroy = abort + join
    for h in hs:
        L.ltx_blob_close(h)


def test_ring_reader_error_reaches_consumer(tmp_path):
    """A digest mismatch found by the reader on first touch surfaces at acquire."""
    L = rt.lib()
    rng = np.random.default_rng(0)
    arr = rng.integers(0, 255, size=4096, dtype=np.uint8).tobytes()
    blob, man = bf.pack_entries([("transformer_blocks.0.x", arr, "I8", [4096])], 0, "r", "v", "f", "", "c")
    bad = bytearray(blob)
    bad[7] ^= 1
    _write_blob(tmp_path / "x", bytes(bad), man)
    ok, h, err = _open(tmp_path / "x")
    assert ok
    r = _ring([h], [0, 0], verify=1)
    L.ltx_ring_start(r)
    p, n = C.c_void_p(), C.c_uint64()
    assert not L.ltx_ring_acquire(r, 0, C.byref(p), C.byref(n))
    assert "BlobDigestMismatch" in L.ltx_loader_last_error().decode()
    L.ltx_ring_destroy(r)
    L.ltx_blob_close(h)


# ---- format versions ----------------------------------------------------------

def _tiny_entries(scale_dtype="F32", out_q8=False):
    """A few named entries (small shapes) exercising the version rule."""
    q = np.arange(256, dtype=np.int16).astype(np.int8).reshape(2, 128)
    s = np.ones((2, 1), dtype=np.float16 if scale_dtype == "F16" else np.float32)
    ents = [("transformer_blocks.0.attn1.to_q.weight", b"\x00" * 8, "BF16", [2, 2]),
            ("transformer_blocks.0.attn1.to_q.weight::q8", q.tobytes(), "I8", [2, 128]),
            ("transformer_blocks.0.attn1.to_q.weight::q8scale", s.tobytes(), scale_dtype, [2, 1])]
    if out_q8:
        ents += [("transformer_blocks.0.attn1.to_out.0.weight::q8", q.tobytes(), "I8", [2, 128]),
                 ("transformer_blocks.0.attn1.to_out.0.weight::q8scale", s.tobytes(), scale_dtype, [2, 1])]
    return ents


@pytest.mark.parametrize("scale_dtype,out_q8,version", [("F32", False, 1), ("F16", False, 2), ("F32", True, 2),
                                                        ("F16", True, 2)])
def test_packer_version_follows_extensions(tmp_path, scale_dtype, out_q8, version):
    blob, man = bf.pack_entries(_tiny_entries(scale_dtype, out_q8), 0, "r", "v", "f", "", "c")
    assert man["packer_version"] == version
    bf.check_version(man)
    _write_blob(tmp_path / "ok", blob, man)
    ok, h, err = _open(tmp_path / "ok")
    assert ok, err
    rt.lib().ltx_blob_close(h)


def test_version1_manifest_with_extension_is_refused(tmp_path):
    blob, man = bf.pack_entries(_tiny_entries("F16", True), 0, "r", "v", "f", "", "c")
    for v, what in ((1, "version-1 manifest"), (3, "unsupported packer_version 3")):
        m = dict(man, packer_version=v)
        with pytest.raises(ValueError, match="FormatVersion"):
            bf.check_version(m)
        _write_blob(tmp_path / f"v{v}", blob, m)
        ok, h, err = _open(tmp_path / f"v{v}")
        assert not ok and "FormatVersion" in err and what in err


def test_reference_golden_blob_is_version1():
    man = json.loads((GOLD / "output" / "blob_manifest.json").read_text())
    assert man["packer_version"] == bf.PACKER_VERSION == 1
    bf.check_version(man)
