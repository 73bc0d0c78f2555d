"""MI355X (gfx950) DEQ forward path of AIDEEN behind a C ABI (include/aideen_hip.h).

The compute lives in ``libaideen_hip.so`` (hand-written HIP kernels); ``backend`` mirrors the
reference's Rust GPU surfaces over that ABI and ``synth`` makes deterministic synthetic models.
"""

__all__ = ["backend", "synth"]
