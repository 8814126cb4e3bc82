"""cajeta-llm's KV-cached greedy decode path, MI355X-native.

Host surface (mirroring the reference's names): LlmEngine, EngineOptions,
SampleParams, KernelCap, LlmException. The compute is the gfx950 code object
kernels.hsaco driven through the C-ABI library libcajeta_mi355x.so
(include/cajeta_mi355x.h); `native` is the thin ctypes binding of it.
"""
from . import native
from .engine import EngineOptions, KernelCap, LlmEngine, Request, SampleParams, image_bytes, image_free, synth_gguf
from .native import Buffer, LlmException

__all__ = ["native", "EngineOptions", "KernelCap", "LlmEngine", "Request", "SampleParams", "LlmException", "Buffer",
           "synth_gguf", "image_bytes", "image_free"]
