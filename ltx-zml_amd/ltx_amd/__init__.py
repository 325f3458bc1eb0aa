"""MI355X-native LTX-2.5 DiT block forward: host-side Python tooling.

- ``blockfmt``: the packed int8-g128 blob format (quantizer, packer, names)
- ``synth``: seeded synthetic blocks and inputs
- ``conditioning``: sigma -> AdaLN tables (tstab, tidx, pts2)
- ``runtime``: ctypes bindings of libltx_amd.so (the C ABI in include/)
"""
from . import blockfmt, conditioning, synth  # noqa: F401
