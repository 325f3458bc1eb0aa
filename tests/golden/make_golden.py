"""Write golden vectors for the int8-g128 quantizer and the blob packer by
running the reference's own tools (tools/quantize_block.py,
tools/pack_block.py) on a tiny synthetic block directory.

Run in the build container only (the reference is not on the GPU box):
    python tests/golden/make_golden.py /root/reference
Outputs tests/golden/quant_pack/: the input directory (manifest.json +
per-tensor .bin), and the tools' outputs (*_q8.bin, *_q8scale.bin, blob.bin,
blob_manifest.json). Inputs include exact rounding ties, an all-zero group,
a negative-extreme group and denormal-range values.
"""
import json
import pathlib
import shutil
import subprocess
import sys
import tempfile

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
OUT = HERE / "quant_pack"


def bf16(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def main(ref: str) -> int:
    ref = pathlib.Path(ref)
    rng = np.random.default_rng(2024)
    tensors = {}
    # q weight [8, 256]: row 0 = exact ties (w/s = k + 0.5 for s = absmax/127 = 1/127 * 127/127 ...)
    w = rng.standard_t(3, size=(8, 256)).astype(np.float32) * 0.02
    # row 0 group 0: absmax 127 -> s = 1.0; values k + 0.5 are exact half-way cases
    w[0, :128] = np.concatenate([[127.0], np.arange(-63, 63) + 0.5, [-127.0]])[:128]
    w[1, :128] = 0.0                      # all-zero group -> scale 1.0, q = 0
    w[2, 128:] = -np.abs(w[2, 128:])      # negative-extreme group
    w[2, 200] = -3.0
    w[3, :128] = np.float32(1e-38) * rng.standard_normal(128).astype(np.float32)  # tiny values
    tensors["transformer_blocks.0.attn1.to_q.weight"] = ("BF16", [8, 256], bf16(w))
    tensors["transformer_blocks.0.attn1.to_q.bias"] = ("BF16", [8], bf16(rng.standard_normal(8) * 0.02))
    f = rng.standard_normal((4, 384)).astype(np.float32) * 0.05
    tensors["transformer_blocks.0.ff.net.0.proj.weight"] = ("BF16", [4, 384], bf16(f))
    tensors["transformer_blocks.0.attn2.to_out.0.weight"] = ("BF16", [4, 128], bf16(rng.standard_normal((4, 128))))
    tensors["transformer_blocks.0.scale_shift_table"] = ("F32", [9, 16],
                                                         rng.standard_normal((9, 16)).astype(np.float32))
    with tempfile.TemporaryDirectory() as td:
        d = pathlib.Path(td)
        man = {"repo": "synthetic", "revision": "golden", "file": "synthetic.safetensors", "block": 0,
               "model_version": "golden", "tensors": {}}
        for name, (dt, shape, arr) in tensors.items():
            short = name
            fname = short.replace(".", "_") + ".bin"
            (d / fname).write_bytes(np.ascontiguousarray(arr).tobytes())
            man["tensors"][short] = {"file": fname, "shape": shape, "dtype": dt}
        (d / "manifest.json").write_text(json.dumps(man, indent=1))
        if OUT.exists():
            shutil.rmtree(OUT)
        shutil.copytree(d, OUT / "input")
        py = sys.executable
        for cls in ("qkv", "ff"):
            subprocess.run([py, str(ref / "tools" / "quantize_block.py"), str(d), "--cls", cls, "--gs", "128",
                            "--bits", "8"], check=True)
        subprocess.run([py, str(ref / "tools" / "pack_block.py"), str(d)], check=True)
        (OUT / "output").mkdir()
        for p in sorted(d.iterdir()):
            if p.name.endswith(("_q8.bin", "_q8scale.bin")) or p.name in ("blob.bin", "blob_manifest.json"):
                shutil.copy(p, OUT / "output" / p.name)
    print(f"wrote {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
