"""MI355X (gfx950) batched-decode hot path of TensorForge.

Hand-written HIP kernels for paged GQA decode attention, the paged KV append,
fused residual+RMSNorm and SwiGLU, exposed through the C ABI declared in
``include/tensorforge_amd.h`` and wrapped behind the reference's
``tensorforge.kernels`` call signatures (``tensorforge_amd.kernels``).
"""

__version__ = "0.1.0"
