"""zerollm_amd — MI355X-native speculative-decoding step of zerollm (draft k tokens, verify k+1 in one target pass,
rejection-sampling acceptance with KV rollback), behind zerollm's model interface. Host side in Python over the C ABI
of libzerollm_hip.so (include/zerollm_hip.h); the kernels are hand-written HIP for gfx950."""
from . import gguf  # noqa: F401

__all__ = ["gguf", "model", "sampler", "speculative", "generate", "synth"]
