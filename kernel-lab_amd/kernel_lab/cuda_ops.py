"""Drop-in name for the original project's native-op module.

Code written against kernel_lab/cuda_ops.py (``available``, ``why_unavailable``,
``rms_norm``, ``fused_add_rms_norm``, ``paged_decode_attention``) keeps
working unchanged; the functions are those of ``kernel_lab.ops``, which run
the gfx950 HIP kernels.
"""

from kernel_lab.ops import (  # noqa: F401
    available,
    fused_add_rms_norm,
    paged_decode_attention,
    rms_norm,
    why_unavailable,
)
