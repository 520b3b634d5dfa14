"""MI355X-native (gfx950) build of MoEArc's paged grouped-query attention hot path.

The compute is HIP behind the C ABI in include/moearc_attn.h; this package holds the host-side
mirror of the reference wrapper (context.py), the ctypes binding (native.py), the build recipe
(build.py) and the seeded synthetic-input generator (synth.py).
"""
from .context import (BadArgument, BufferTooSmall, Context, DeviceBuffer, Failed, KernelError,  # noqa: F401
                      AttnBlockDesc, DeviceView, KvType, NoDevice, OutOfMemory, OUT_F16, OUT_F32, QuantType,
                      RopeKind, RopeScaling)
