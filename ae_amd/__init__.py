"""ae_amd: SpecMoE's verify-step MoE hot path, rebuilt for MI355X (gfx950).

The kernels live in libspecmoe_mi355x.so (HIP, C ABI in include/specmoe_mi355x.h); the
``ae_amd.layers`` modules keep the reference's specmoe/layers operator interface.
"""
__version__ = "0.1.0"
