"""opaque_amd: MI355X-native DP-SGD clip + noise core.

The public surface mirrors the reference's drop-in names (``clipped_grad``,
``auto_clipped_grad``, ``per_group``, ``gaussian_noise`` and the DP wrapper
types); the work runs in hand-written HIP kernels for gfx950 behind the C ABI
declared in ``include/opaque_dp.h``.
"""

__version__ = "0.1.0"
