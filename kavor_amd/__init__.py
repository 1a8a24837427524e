"""MI355X-native paged KV-cache path of the Kavor inference engine.

The product path is libkvpath.so (hand-written gfx950 HIP kernels behind the C ABI in
include/kvpath.h) and its Python boundary kavor_amd.layers.attention, which mirrors
kavor/layers/attention/flash_attention_kvcache.py.
"""

__version__ = "0.1.0"
