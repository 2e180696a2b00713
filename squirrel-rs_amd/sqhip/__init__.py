"""squirrel-hip: MI355X implementation of squirrel-rs's Llama token loop.

Python mirror of the reference's ops / model API over the C ABI of
libsquirrel_hip.so.  All compute runs in the HIP kernels of that library.
"""
from ._lib import (KernelError, LLMError, SqError, SQ_BF16, SQ_Q4_0, SQ_Q8_0, check, lib)
from .model import (GreedySampler, Llama3_2, ModelContext, TextTokenGenerator, LLAMA_1B,
                    write_synthetic_gguf)
from . import ops

__all__ = ["KernelError", "LLMError", "SqError", "SQ_BF16", "SQ_Q4_0", "SQ_Q8_0", "check", "lib",
           "GreedySampler", "Llama3_2", "ModelContext", "TextTokenGenerator", "LLAMA_1B",
           "write_synthetic_gguf", "ops"]
