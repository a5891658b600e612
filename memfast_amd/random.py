"""Address-keyed random samples: the schedule never changes a physical event.

Same functions as memfast/random.py:8-33.  ``mix`` and ``event_seed`` are
pure integer functions (Python ints or integer tensors on any device).
``uniform`` and ``normal`` evaluate on the GPU through the same device RNG the
kernels use (libmemfast_hip.so); address tensors must be HIP tensors.
"""

from . import hip


def mix(value):
    """Integer avalanche hash of the low 32 bits (lowbias32 constants)."""
    value = value & 0xFFFFFFFF
    value = ((value ^ (value >> 16)) * 0x7FEB352D) & 0xFFFFFFFF
    value = ((value ^ (value >> 15)) * 0x846CA68B) & 0xFFFFFFFF
    return value ^ (value >> 16)


def event_seed(seed, event):
    """64-bit read seed: low word seed ^ mix(lo(event)), high word mix(hi(event))."""
    return (seed ^ mix(event & 0xFFFFFFFF)) | (mix(event >> 32) << 32)


def uniform(address, seed, stream):
    """24-bit uniform sample in (0, 1) for each int64 address (HIP tensor)."""
    return hip.rng(address, seed, stream, "uniform")


def normal(address, seed, stream):
    """Box-Muller standard normal from streams (stream, stream + 1) (HIP tensor)."""
    return hip.rng(address, seed, stream, "normal")


__all__ = ["mix", "event_seed", "uniform", "normal"]
