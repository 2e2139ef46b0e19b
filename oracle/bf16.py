"""bfloat16 as uint16 bit patterns in numpy (numpy has no bf16 dtype).

TEST INFRASTRUCTURE (see oracle/__init__.py).  The reference widens bf16 exactly and
rounds fp32 results to bf16 with round-to-nearest-even (Mojo's ``.cast``,
cpu_attention/_mojo/src/paged_attn.mojo:316-319); torch's ``.bfloat16()`` is the
library routine the tests pin these two functions against.
"""

import numpy as np


def to_float(bits):
    """bf16 bit patterns (uint16) -> exact float32 values."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def from_float(x):
    """float32 values -> bf16 bit patterns, round to nearest even; NaN stays NaN."""
    u = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32)
    rounded = (u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)
    out = rounded.astype(np.uint16)
    nan = np.isnan(np.asarray(x, np.float32))
    out[nan] = np.uint16(0x7FC0)
    return out


def round_float(x):
    """float32 values rounded to the nearest bf16 value (as float32)."""
    return to_float(from_float(x))
