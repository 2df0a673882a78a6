"""MI355X (gfx950) FP8 hot path: quantizers and scaled FP8 BMM.

Public API (drop-in for xuOAO/practice_cuda's fp8_training/fp8_bench):

* registry: QuantResult, register_quant, register_bmm, get_quant, get_bmm,
  bmm_impl_names, load_builtin_impls
* quantizers: per_block_quant, per_channel_quant, per_tensor_quant
* BMMs: per_block_bmm, per_channel_bmm, per_tensor_bmm

The kernels live in the in-tree HIP library built by
``python -m practice_cuda_amd.build``; every entry point raises if it is
missing.
"""
from .registry import (  # noqa: F401
    BMM_IMPLS,
    QUANT_IMPLS,
    BMMImpl,
    QuantImpl,
    QuantResult,
    bmm_impl_names,
    get_bmm,
    get_quant,
    load_builtin_impls,
    register_bmm,
    register_quant,
)


def __getattr__(name):
    # the kernel wrappers import torch.cuda helpers; load them lazily
    aliases = {
        "per_block_quant": ("hip_per_block", "hip_per_block_quant"),
        "per_block_bmm": ("hip_per_block", "hip_per_block_bmm"),
        "per_channel_quant": ("hip_per_channel", "hip_per_channel_quant"),
        "per_channel_bmm": ("hip_per_channel", "hip_per_channel_bmm"),
        "per_tensor_quant": ("hip_per_tensor", "hip_per_tensor_quant"),
        "per_tensor_bmm": ("hip_per_tensor", "hip_per_tensor_bmm"),
    }
    if name in aliases:
        import importlib
        mod, attr = aliases[name]
        load_builtin_impls()
        return getattr(importlib.import_module(f"practice_cuda_amd.impls.{mod}"), attr)
    raise AttributeError(name)
