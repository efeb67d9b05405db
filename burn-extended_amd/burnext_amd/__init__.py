"""burnext_amd -- MI355X-native GPT-OSS MoE feed-forward (MXFP4 experts) behind burn-extended's
MoE / quant-loader API.  The compute is libburnext_moe.so (HIP, gfx950); this package holds the
Python front-end over its C ABI, the seeded synthetic-layer generator and the on-disk loaders
(model.bin and safetensors MoE weights)."""
from . import _native, loaders, synth  # noqa: F401

__all__ = ["_native", "loaders", "synth"]
