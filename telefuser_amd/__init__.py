"""MI355X-native quantized attention backend (INT8 Q.K^T, FP8 P.V) for TeleFuser's Wan-style DiT.

``telefuser_amd.sageattn2`` is the drop-in for the module TeleFuser loads as
``backends.sageattention``; ``telefuser_amd.attention`` mirrors ``telefuser.ops.attention.attention``.
The kernels live in libqattn.so (C ABI: include/qattn.h), built in-tree by ``telefuser_amd.build``.
"""

__version__ = "0.1.0"
