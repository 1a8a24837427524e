"""MI355X-native paged KV-cache path of the Kavor inference engine.

The product path is libkvpath.so (hand-written gfx950 HIP kernels behind the C ABI in
include/kvpath.h) and its Python boundary kavor_amd.layers.attention, which mirrors
kavor/layers/attention/flash_attention_kvcache.py.
"""

__version__ = "0.1.0"

__all__ = ["LLM", "SamplingParams"]


def __getattr__(name):
    # lazy, so that importing the package (e.g. for the C-ABI binding) stays light
    if name == "LLM":
        from kavor_amd.engine.llm_engine import LLM

        return LLM
    if name == "SamplingParams":
        from kavor_amd.sampling_params import SamplingParams

        return SamplingParams
    raise AttributeError(name)
