"""Kernel entry points (mirrors ``chronicals.kernels``)."""
