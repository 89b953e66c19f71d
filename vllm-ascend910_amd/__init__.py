"""MI355X (gfx950) W4A8 per-group quantized linear.

A drop-in for the W4A8 dynamic linear of GongCheng1919/vllm-ascend910:
dynamic per-token int8 activation quant, int4 per-group weight GEMM with exact
int32 per-group accumulation on the CDNA4 i8 MFMA, and an fp32 scale epilogue
to bf16.  Importing the package registers ``torch.ops.npu.*``; the HIP library
itself is loaded on first use (``_abi.lib()``) and must have been built.

The directory name is not a Python identifier, so the package is imported as
``vllm_ascend910_amd`` through ``__graft_entry__.package()``.
"""
from . import checkpoint, decoder, geometry, packing, synth, vllm_plugin  # noqa: F401
from . import ops  # noqa: F401
from .linear import MidGroupW4A8Linear, W4A8Linear, linear, linear_swiglu, midgroup_linear  # noqa: F401

__all__ = ["W4A8Linear", "MidGroupW4A8Linear", "linear", "linear_swiglu", "midgroup_linear", "geometry",
           "packing", "ops", "synth", "decoder", "checkpoint", "vllm_plugin"]
