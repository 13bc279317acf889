"""Greedy selection under the reference's module path (tokserve/generation/greedy.py)."""

from tokserve_amd.generation.sampling import select_greedy

__all__ = ["select_greedy"]
