"""MI355X-native (gfx950) backend for Channel's Q4 inference hot path.

The compute path is libchannel_hip.so: hand-written HIP kernels behind the
C-ABI declared in include/channel_hip.h.  This package only binds it
(ctypes) for tests, benchmarks and Python callers.
"""
from ._abi import HEADER_PATH, LIB_PATH, PROTOTYPES, ChannelError, lib
from .device import Buffer, Context, device_count

Q4_BLOCK_BYTES = 20
Q8_BLOCK_BYTES = 36


def q4_bytes(rows, K):
    """getQuantizedSizeBytes(rows, K, .q4) (src/quant.zig:181-183)."""
    return rows * ((K + 31) // 32) * Q4_BLOCK_BYTES


def q4r_bytes(rows, K):
    """Bytes of a repacked (Q4R) matrix: 16 B of nibbles + 2 B of f16 scale
    per 32 weights."""
    return rows * (K // 32) * 18


def xplanes_bytes(K):
    """Bytes of the activation digit planes of K values (chn_xplanes): 20
    plane words and one float scale per 32 values."""
    return (K // 32) * 21 * 4


def q8_bytes(rows, K):
    """getQuantizedSizeBytes(rows, K, .q8) (src/quant.zig:181-183)."""
    return rows * ((K + 31) // 32) * Q8_BLOCK_BYTES


__all__ = ["Buffer", "ChannelError", "Context", "HEADER_PATH", "LIB_PATH", "PROTOTYPES",
           "device_count", "lib", "q4_bytes", "q4r_bytes", "q8_bytes"]
