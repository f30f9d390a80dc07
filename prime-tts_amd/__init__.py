"""prime-tts_amd: MI355X-native (gfx950) conv hot path of the PrimeTTS v2.1 MB-iSTFT decoder.

The product is the C-ABI shared library ``libptconv_hip.so`` built from ``csrc/`` (HIP kernels +
a C gnu11 host layer exporting the reference's ``pt_v21_*`` device entry points).  This Python
module only loads that library for tests and bench.py; ``synth`` holds the packed-layout helpers
and the seeded synthetic decoder inputs.
"""
from . import synth  # noqa: F401
