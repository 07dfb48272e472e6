"""mlx_motif (MI355X): the Motif decode-attention hot path on gfx950.

Drop-in for the kernel API of junhoyeo/mlx-motif (``mlx_motif.kernels``) and
its 4-slot KV caches (``mlx_motif.cache``), with torch ROCm tensors in place
of ``mx.array`` and hand-written HIP kernels behind one C ABI
(``include/motif_hip.h``, loaded by ``mlx_motif._native``).
"""

__version__ = "0.1.0"
