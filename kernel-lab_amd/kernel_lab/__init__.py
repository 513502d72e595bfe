"""kernel_lab for AMD Instinct MI355X: paged-KV decode attention and fused
residual-add + RMSNorm as hand-written gfx950 HIP kernels.

The operators register as ``torch.ops.kernel_lab.*`` (same schemas as the
original project's CUDA extension) when ``kernel_lab.ops`` is imported; the
same kernels are reachable without PyTorch through the C-ABI in
``include/kernel_lab.h`` (``libkernel_lab.so``).
"""

__version__ = "0.1.0"
