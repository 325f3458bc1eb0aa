"""The packed int8-g128 block format.

Restates the reference's offline weight tooling so blobs produced here are
byte-compatible with its loader:

- tensor names / shapes / dtypes of one video block (ltx/block.zig:377-406,
  ltx/loader.zig:146-156; names as fetched, tools/fetch_block.py:160-170);
- ``quantize_g128``: symmetric int8 (or int4) per group of 128 along K,
  arithmetic in f64, ``np.round`` (half-to-even), clip, f32 scales
  (tools/quantize_block.py:28-73);
- ``pack``: entries = base tensors + ``::q8`` (I8 [O, I]) + ``::q8scale``
  (F32 [O, I/128]), sorted by name, 64-byte aligned with zero fill, per-entry
  and whole-blob sha256 (tools/pack_block.py:33-95);
- ``normalize_name`` (ltx/loader.zig:100-119).

Format versions. ``packer_version`` 1 is the reference format exactly
(F32 scales, int8 companions for the q/k/v and ff classes only). A blob that
uses either extension — F16 scale entries (``scale_dtype="F16"``, the
half-size form the GEMM kernels read natively) or int8 companions of the
out-projections (class "out") — is written as version 2; every version-1
blob still packs byte for byte as the reference tool does, and readers
refuse a version-1 manifest that carries an extension (``check_version``).
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass

import numpy as np

D, H, FF, GROUP = 4096, 32, 16384, 128
PACKER_VERSION = 1  # the reference format (tools/pack_block.py:27)
PACKER_VERSION_EXT = 2  # F16 scales and / or int8 out-projections
ALIGN = 64

# (field, tensor suffix after "transformer_blocks.{i}.", shape, dtype) in
# WEIGHT_SPECS order (ltx/block.zig:377-406).
BASE_SPECS = [
    ("q1_w", "attn1.to_q.weight", (D, D), "BF16"),
    ("q1_b", "attn1.to_q.bias", (D,), "BF16"),
    ("k1_w", "attn1.to_k.weight", (D, D), "BF16"),
    ("k1_b", "attn1.to_k.bias", (D,), "BF16"),
    ("v1_w", "attn1.to_v.weight", (D, D), "BF16"),
    ("v1_b", "attn1.to_v.bias", (D,), "BF16"),
    ("o1_w", "attn1.to_out.0.weight", (D, D), "BF16"),
    ("o1_b", "attn1.to_out.0.bias", (D,), "BF16"),
    ("qn1", "attn1.q_norm.weight", (D,), "BF16"),
    ("kn1", "attn1.k_norm.weight", (D,), "BF16"),
    ("g1_w", "attn1.to_gate_logits.weight", (H, D), "BF16"),
    ("g1_b", "attn1.to_gate_logits.bias", (H,), "BF16"),
    ("q2_w", "attn2.to_q.weight", (D, D), "BF16"),
    ("q2_b", "attn2.to_q.bias", (D,), "BF16"),
    ("k2_w", "attn2.to_k.weight", (D, D), "BF16"),
    ("k2_b", "attn2.to_k.bias", (D,), "BF16"),
    ("v2_w", "attn2.to_v.weight", (D, D), "BF16"),
    ("v2_b", "attn2.to_v.bias", (D,), "BF16"),
    ("o2_w", "attn2.to_out.0.weight", (D, D), "BF16"),
    ("o2_b", "attn2.to_out.0.bias", (D,), "BF16"),
    ("qn2", "attn2.q_norm.weight", (D,), "BF16"),
    ("kn2", "attn2.k_norm.weight", (D,), "BF16"),
    ("g2_w", "attn2.to_gate_logits.weight", (H, D), "BF16"),
    ("g2_b", "attn2.to_gate_logits.bias", (H,), "BF16"),
    ("ff1_w", "ff.net.0.proj.weight", (FF, D), "BF16"),
    ("ff2_w", "ff.net.2.weight", (D, FF), "BF16"),
    ("sst", "scale_shift_table", (9, D), "F32"),
    ("psst", "prompt_scale_shift_table", (2, D), "F32"),
]
FIELDS = [s[0] for s in BASE_SPECS]

# int8 companions in Q8_SPECS order (ltx/loader.zig:147-156) + out class.
Q8_FIELDS = ["q1", "k1", "v1", "q2", "k2", "v2", "f1", "f2", "o1", "o2"]
Q8_BASE = {"q1": "q1_w", "k1": "k1_w", "v1": "v1_w", "q2": "q2_w", "k2": "k2_w", "v2": "v2_w",
           "f1": "ff1_w", "f2": "ff2_w", "o1": "o1_w", "o2": "o2_w"}
# quantisation classes (tools/quantize_block.py:20-25)
CLASSES = {"qkv": ["q1", "k1", "v1", "q2", "k2", "v2"], "out": ["o1", "o2"], "ff": ["f1", "f2"]}
REFERENCE_RECIPE = CLASSES["qkv"] + CLASSES["ff"]  # tools/assemble_blocks.py:80-81


def tensor_name(block: int, field: str) -> str:
    return f"transformer_blocks.{block}." + dict((s[0], s[1]) for s in BASE_SPECS)[field]


def normalize_name(name: str) -> str:
    """'.' -> '_' and '::' -> '_' (ltx/loader.zig:100-119)."""
    return name.replace("::", "_").replace(".", "_")


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = np.isnan(x)
    r = (u >> 16) & np.uint32(1)
    r += u
    r += np.uint32(0x7FFF)  # cannot wrap for finite inputs (|u| <= 0xff7fffff)
    r >>= 16
    out = r.astype(np.uint16)
    if nan.any():
        out[nan] = 0x7FC0
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> f32 by the <<16 widening of tools/quantize_block.py:28-30."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize_g128(w_bf16: np.ndarray, gs: int = GROUP, bits: int = 8) -> tuple[np.ndarray, np.ndarray]:
    """(tools/quantize_block.py:51-59) f64 group absmax, s = absmax/qmax (1.0
    for an all-zero group), q = clip(round-half-even(w/s), lo, qmax)."""
    qmax, lo = (7, -8) if bits == 4 else (127, -128)
    w = bf16_to_f32(w_bf16).astype(np.float64)
    o, i = w.shape
    wg = w.reshape(o, i // gs, gs)
    absmax = np.abs(wg).max(axis=2, keepdims=True)
    scale3 = np.where(absmax > 0, absmax / qmax, 1.0)
    q = np.clip(np.round(wg / scale3), lo, qmax).astype(np.int8).reshape(o, i)
    return q, scale3.squeeze(2).astype(np.float32)


@dataclass
class BlockTensors:
    """One block's tensors as numpy arrays: ``base[field]`` (uint16 bf16 bits
    or f32), ``q8[name]`` int8 [O, I] and ``q8s[name]`` f32/f16 [O, I/128]."""
    block: int
    base: dict
    q8: dict
    q8s: dict

    @property
    def scale_f16(self) -> bool:
        return any(v.dtype == np.float16 for v in self.q8s.values())


def quantize_block(bt: BlockTensors, classes=("qkv", "ff"), scale_dtype: str = "F32") -> BlockTensors:
    for c in classes:
        for qn in CLASSES[c]:
            q, s = quantize_g128(bt.base[Q8_BASE[qn]])
            bt.q8[qn] = q
            bt.q8s[qn] = s.astype(np.float16) if scale_dtype == "F16" else s
    return bt


def pack(bt: BlockTensors, repo: str = "synthetic", revision: str = "synthetic", source_file: str = "synthetic",
         model_version: str = "", packer_commit: str = "ltx-mi355x") -> tuple[bytes, dict]:
    """Blob bytes + manifest dict (tools/pack_block.py:33-92)."""
    entries = []
    for field, suffix, shape, dtype in BASE_SPECS:
        name = f"transformer_blocks.{bt.block}.{suffix}"
        arr = bt.base[field]
        entries.append((name, np.ascontiguousarray(arr).tobytes(), dtype, list(shape)))
    for qn, q in bt.q8.items():
        name = tensor_name(bt.block, Q8_BASE[qn])
        o, i = q.shape
        s = bt.q8s[qn]
        entries.append((name + "::q8", np.ascontiguousarray(q).tobytes(), "I8", [o, i]))
        entries.append((name + "::q8scale", np.ascontiguousarray(s).tobytes(),
                        "F16" if s.dtype == np.float16 else "F32", [o, i // GROUP]))
    return pack_entries(entries, bt.block, repo, revision, source_file, model_version, packer_commit)


_OUT_SUFFIXES = ("attn1.to_out.0.weight", "attn2.to_out.0.weight")


def _extensions(entries) -> list:
    """Version-2 features among (name, dtype) pairs."""
    ext = []
    for name, dtype in entries:
        if name.endswith("::q8scale") and dtype == "F16":
            ext.append(f"F16 scales ({name})")
        if name.endswith("::q8") and name[:-4].endswith(_OUT_SUFFIXES):
            ext.append(f"int8 out-projection ({name})")
    return ext


def check_version(manifest: dict) -> None:
    """packer_version 1 or 2; a version-1 manifest may not use the
    version-2 extensions."""
    v = manifest.get("packer_version", PACKER_VERSION)
    if v not in (PACKER_VERSION, PACKER_VERSION_EXT):
        raise ValueError(f"FormatVersion: unsupported packer_version {v}")
    ext = _extensions((e["name"], e["dtype"]) for e in manifest["entries"])
    if v == PACKER_VERSION and ext:
        raise ValueError(f"FormatVersion: version-1 manifest with a version-2 extension: {ext[0]}")


def pack_entries(entries: list, block: int, repo: str, revision: str, source_file: str, model_version: str,
                 packer_commit: str) -> tuple[bytes, dict]:
    """Canonical blob from (name, bytes, dtype, shape) entries: name-sorted,
    64-byte aligned with zero fill (tools/pack_block.py:54-91). Version 2
    when an extension is present, else 1."""
    entries = sorted(entries, key=lambda t: t[0])
    version = PACKER_VERSION_EXT if _extensions((n, d) for n, _, d, _ in entries) else PACKER_VERSION
    blob = bytearray()
    mentries = []
    for name, data, dtype, shape in entries:
        if len(blob) % ALIGN:
            blob.extend(b"\x00" * (ALIGN - len(blob) % ALIGN))
        off = len(blob)
        blob.extend(data)
        mentries.append({"name": name, "dtype": dtype, "shape": shape, "offset": off, "nbytes": len(data),
                         "sha256": hashlib.sha256(data).hexdigest()})
    manifest = {
        "packer_version": version, "packer_commit": packer_commit, "align": ALIGN, "block": block,
        "repo": repo, "revision": revision, "source_file": source_file, "model_version": model_version,
        "total_bytes": len(blob), "blob_sha256": hashlib.sha256(bytes(blob)).hexdigest(), "entries": mentries,
    }
    return bytes(blob), manifest


def check_layout(manifest: dict) -> None:
    """Blob.checkLayout (ltx/loader.zig:73-82)."""
    end = 0
    al = manifest["align"]
    for e in manifest["entries"]:
        if e["offset"] % al:
            raise ValueError(f"Misaligned: {e['name']}")
        if e["offset"] < end or e["offset"] - end >= al:
            raise ValueError(f"LayoutGap: {e['name']}")
        end = e["offset"] + e["nbytes"]
    if end != manifest["total_bytes"]:
        raise ValueError("TrailingBytes")


def unpack(blob: bytes, manifest: dict, block: int | None = None) -> BlockTensors:
    """Inverse of ``pack``: numpy views of every entry (buildBlockBufs /
    buildQuantBufs lookups, ltx/loader.zig:133-172)."""
    check_version(manifest)
    block = manifest["block"] if block is None else block
    byname = {normalize_name(e["name"]): e for e in manifest["entries"]}
    mv = memoryview(blob)
    dt = {"BF16": np.uint16, "F32": np.float32, "F16": np.float16, "I8": np.int8}
    base, q8, q8s = {}, {}, {}
    for field, suffix, shape, dtype in BASE_SPECS:
        e = byname.get(normalize_name(f"transformer_blocks.{block}.{suffix}"))
        if e is None:
            raise KeyError(f"MissingEntry: {suffix}")
        base[field] = np.frombuffer(mv[e["offset"]:e["offset"] + e["nbytes"]], dtype=dt[e["dtype"]]).reshape(shape)
    for qn, bf in Q8_BASE.items():
        stem = normalize_name(tensor_name(block, bf))
        eq, es = byname.get(stem + "_q8"), byname.get(stem + "_q8scale")
        if eq is None or es is None:
            continue
        q8[qn] = np.frombuffer(mv[eq["offset"]:eq["offset"] + eq["nbytes"]], dtype=np.int8).reshape(eq["shape"])
        q8s[qn] = np.frombuffer(mv[es["offset"]:es["offset"] + es["nbytes"]], dtype=dt[es["dtype"]]).reshape(es["shape"])
    return BlockTensors(block, base, q8, q8s)


def manifest_json(manifest: dict) -> str:
    return json.dumps(manifest, indent=1)


# ---- block directories (the fetch_block.py layout) -------------------------

def quantize_dir(wdir, cls: str = "qkv", gs: int = GROUP, bits: int = 8, scale_dtype: str = "F32") -> list[str]:
    """Quantise the tensors of class `cls` in a block directory, writing
    NAME_q8.bin / NAME_q8scale.bin beside the source (tools/quantize_block.py:
    45-73; the int4 form writes NAME_q4.bin (u4 stored as q + 8) and
    NAME_q4scale.bin)."""
    import pathlib

    wdir = pathlib.Path(wdir)
    man = json.loads((wdir / "manifest.json").read_text())
    suffixes = [dict((s[0], s[1]) for s in BASE_SPECS)[Q8_BASE[q]] for q in CLASSES[cls]]
    done = []
    for name, e in man["tensors"].items():
        if not any(name.endswith(f"transformer_blocks.{man['block']}.{s}") or name.split(".", 2)[-1] == s
                   for s in suffixes):
            continue
        if e["dtype"] != "BF16":
            raise ValueError(f"{name}: expected BF16, got {e['dtype']}")
        raw = np.frombuffer((wdir / e["file"]).read_bytes(), dtype=np.uint16).reshape(e["shape"])
        q, s = quantize_g128(raw, gs, bits)
        stem = e["file"].removesuffix(".bin")
        if bits == 4:
            (wdir / f"{stem}_q4.bin").write_bytes((q.astype(np.int16) + 8).astype(np.uint8).tobytes())
            (wdir / f"{stem}_q4scale.bin").write_bytes(s.astype(np.float32).tobytes())
        else:
            (wdir / f"{stem}_q8.bin").write_bytes(q.tobytes())
            sd = s.astype(np.float16) if scale_dtype == "F16" else s.astype(np.float32)
            (wdir / f"{stem}_q8scale.bin").write_bytes(sd.tobytes())
        done.append(name)
    return done


def pack_dir(wdir, packer_commit: str = "ltx-mi355x") -> dict:
    """Pack a block directory into blob.bin + blob_manifest.json
    (tools/pack_block.py:33-95). A *_q8scale.bin of half the f32 size is
    recorded as F16."""
    import pathlib

    wdir = pathlib.Path(wdir)
    man = json.loads((wdir / "manifest.json").read_text())
    entries = []
    for name, e in man["tensors"].items():
        entries.append((name, (wdir / e["file"]).read_bytes(), e["dtype"], e["shape"]))
        stem = e["file"].removesuffix(".bin")
        q8 = wdir / f"{stem}_q8.bin"
        if q8.exists():
            o, i = e["shape"]
            sraw = (wdir / f"{stem}_q8scale.bin").read_bytes()
            sdt = "F16" if len(sraw) == o * (i // GROUP) * 2 else "F32"
            entries.append((name + "::q8", q8.read_bytes(), "I8", [o, i]))
            entries.append((name + "::q8scale", sraw, sdt, [o, i // GROUP]))
    blob, out = pack_entries(entries, man["block"], man["repo"], man["revision"], man["file"],
                             man.get("model_version", ""), packer_commit)
    (wdir / "blob.bin").write_bytes(blob)
    (wdir / "blob_manifest.json").write_text(manifest_json(out))
    return out


def _main(argv=None) -> int:
    import argparse

    ap = argparse.ArgumentParser(prog="python -m ltx_amd.blockfmt")
    sub = ap.add_subparsers(dest="cmd", required=True)
    q = sub.add_parser("quantize", help="quantise one class of a block directory")
    q.add_argument("wdir")
    q.add_argument("--cls", default="qkv", choices=list(CLASSES))
    q.add_argument("--gs", type=int, default=GROUP)
    q.add_argument("--bits", type=int, default=8, choices=(4, 8))
    q.add_argument("--scale-dtype", default="F32", choices=("F32", "F16"))
    p = sub.add_parser("pack", help="pack a block directory into blob.bin + blob_manifest.json")
    p.add_argument("wdir")
    a = ap.parse_args(argv)
    if a.cmd == "quantize":
        for n in quantize_dir(a.wdir, a.cls, a.gs, a.bits, a.scale_dtype):
            print(f"  quantized {n}")
    else:
        m = pack_dir(a.wdir)
        print(f"block {m['block']}: {len(m['entries'])} entries, {m['total_bytes']} bytes, "
              f"sha256 {m['blob_sha256'][:16]}")
    return 0


if __name__ == "__main__":
    raise SystemExit(_main())
