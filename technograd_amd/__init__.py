"""MI355X (gfx950) batch backend for Technograd's quantized `tgc batch` path.

The product is the C-ABI library lib/libtg_hip.so (include/tg_hip.h) and the
bin/tgc-hip driver, both built in-tree from csrc/ by technograd_amd/Makefile.
This package holds the ctypes binding (hip.py) and the host-side synthetic
model/row generators used by the benchmark (synth.py).
"""
from . import hip, synth  # noqa: F401
