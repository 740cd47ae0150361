"""MI355X-native fused linear cross-entropy (Cut Cross-Entropy) for Chronicals.

``chronicals_amd.kernels.cut_cross_entropy`` mirrors the reference module
``chronicals.kernels.cut_cross_entropy``; the compute runs in hand-written
gfx950 HIP kernels from ``libchronicals_cce.so`` (built by
``chronicals_amd.build``).
"""

__version__ = "0.1.0"
