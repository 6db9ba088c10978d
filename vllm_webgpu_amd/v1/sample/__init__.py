"""Sampling metadata and the ``Sampler`` facade over the gfx950 library."""
