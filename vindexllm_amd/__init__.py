"""MI355X (gfx950) token sampler for VindexLLM: a drop-in for TVdxSampler.

The product is libvdxsampler.so (HIP kernels + C ABI, include/vdx_sampler.h);
``vindexllm_amd.sampler`` mirrors the reference's Pascal interface over it.
"""
from .sampler import (ROW_FALLBACK, ROW_FULL, ROW_GREEDY, ROW_NAN, ROW_TOPK_FAST,  # noqa: F401
                      ROW_TOPK_REPLAY, VDX_RNG_PHILOX, VDX_RNG_XOSHIRO, VDX_TENSOR_F16,
                      VDX_TENSOR_Q4_0, VDX_TENSOR_Q8_0, TVdxSampler, TVdxSamplerConfig,
                      VdxSamplerError, lmhead, lmhead_q4_0, load_library, version)
from .sampler import VDX_LMHEAD_PACKED, lmhead_pack, lmhead_packed_bytes, sample_device_noalloc  # noqa: F401
from .gguf import TVdxGGUFReader, TVdxGGUFTensorInfo, lm_head_from_gguf  # noqa: F401
