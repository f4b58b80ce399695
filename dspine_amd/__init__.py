"""MI355X-native draft verification for DSpine's speculative decoding.

Hand-written HIP kernels for gfx950 behind a thin C ABI (include/dspine_verify.h), with host
modules that keep the call signatures of the reference's sglang_dspine.{kernels, sampling,
verification, runtime} entry points on this path.
"""

from dspine_amd import _lib  # noqa: F401

__all__ = ["_lib"]
