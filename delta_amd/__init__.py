"""MI355X (gfx950) selective-KV decode hot path of DELTA, behind DELTA's engine surface.

Importing the package never touches the GPU; the HIP library
(``delta_amd/_delta_hip.so``) is loaded on the first kernel call and there is
no CPU fallback.
"""
__version__ = "0.1.0"
