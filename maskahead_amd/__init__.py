"""maskahead_amd: MI355X-native (gfx950 HIP) implementation of MaskAhead's KV read/keep path.

Host code mirrors the reference's Python interface (maskahead.kernels.splitk,
maskahead.kernels.ops, the session's value score and the eviction keep set); every
operation runs in hand-written kernels of libmaskahead_hip.so, bound with ctypes.
"""

__version__ = "0.1.0"
