"""molten_amd: MI355X-native (gfx950) quantized-matmul hot path of molten.

- `molten_amd.hip`    ctypes binding of libmolten_hip.so (the C ABI in
                      include/molten_hip.h), one function per reference
                      operator.
- `molten_amd.layout` MLX affine weight layout helpers and synthetic inputs.
"""
__all__ = ["hip", "layout"]
