"""Kernel boundary: ctypes binding of the C ABI and the operators built on it."""
