"""MI355X-native (gfx950) sparse INT4 / turbo decode attention for flashquest.

Operators keep the reference's names and signatures (flashquest.kernel.*,
flashquest.eager.*, flashquest.cache.*) and run on hand-written HIP kernels in
libfq_hip.so through a C ABI (include/fq_hip.h).
"""
from ._lib import LIB_PATH, load_library  # noqa: F401

__all__ = ["LIB_PATH", "load_library"]
