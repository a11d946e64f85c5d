"""spikeinfer_amd: MI355X-native (gfx950) spiking decode hot path.

Drop-in kernels for spikeinfer's paged popcount decode attention and fused
LIF -> bit-pack -> paged-cache write, behind the reference's call signatures.
"""
__version__ = "0.1.0"
