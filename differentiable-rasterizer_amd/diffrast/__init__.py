"""MI355X-native soft-triangle rasterizer (gfx950 HIP kernels behind a C ABI).

`diffrast.torch_layer` is the drop-in for the reference's PyTorch op
(python/diffrast/torch_layer.py); `diffrast._lib` is the ctypes binding of
libdiffrast_hip.so; `diffrast.synth` generates the seeded benchmark inputs.
"""
