"""Host-side mirror of the matching tokserve package."""
