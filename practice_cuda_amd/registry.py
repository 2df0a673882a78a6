"""Plugin registry and the QuantResult container.

Drop-in for ``fp8_training/fp8_bench/registry.py`` of xuOAO/practice_cuda:
the same public names (QuantResult, QuantImpl, BMMImpl, QUANT_IMPLS,
BMM_IMPLS, register_quant, register_bmm, load_builtin_impls,
bmm_impl_names, get_quant, get_bmm), the same fields and argument meaning,
and the same error types (ValueError for duplicates and bad layouts,
KeyError listing the choices for unknown names). Importing
``practice_cuda_amd.impls`` registers the built-in HIP implementations.
"""
from __future__ import annotations

import importlib
from dataclasses import dataclass, field
from typing import Any, Callable

import torch


@dataclass
class QuantResult:
    """FP8 tensor plus fp32 *dequant* scale (multiply to recover values).

    granularity is "tensor", "channel" (meta["channel_axis"] in {-1, -2}) or
    "block" (meta["block_m"], meta["block_n"]); see registry.py:10-70 of the
    reference for the layout contract this mirrors.
    """

    tensor: torch.Tensor
    dequant_scale: torch.Tensor
    impl: str
    granularity: str
    meta: dict[str, Any] = field(default_factory=dict)

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        scale = self.dequant_scale.to(dtype)
        values = self.tensor.to(dtype)
        kind = self.granularity
        if kind == "tensor":
            return values * scale
        if kind == "channel":
            axis = self.meta["channel_axis"]
            if axis not in (-1, -2):
                raise ValueError(f"unknown channel_axis for per-channel dequant: {axis}")
            if scale.ndim != values.ndim - 1:
                raise ValueError(
                    "per-channel dequant scale must have one fewer dimension than its "
                    f"tensor: tensor={tuple(values.shape)}, scale={tuple(scale.shape)}")
            # a row scale (axis -2) broadcasts along the last dim, a column
            # scale (axis -1) along the row dim
            return values * scale.unsqueeze(-1 if axis == -2 else -2)
        if kind == "block":
            if "block_m" not in self.meta or "block_n" not in self.meta:
                raise ValueError("block_m and block_n must be specified in meta for block dequant")
            bm, bn = self.meta["block_m"], self.meta["block_n"]
            if bm <= 0 or bn <= 0:
                raise ValueError("block_m and block_n must be positive for block granularity")
            rows, cols = values.shape[-2:]
            want = tuple(values.shape[:-2]) + (-(-rows // bm), -(-cols // bn))
            if tuple(scale.shape) != want:
                raise ValueError(
                    f"per-block dequant scale must have shape {want}, got {tuple(scale.shape)}")
            row_ids = torch.arange(rows, device=scale.device) // bm
            col_ids = torch.arange(cols, device=scale.device) // bn
            expanded = scale.index_select(-2, row_ids).index_select(-1, col_ids)
            return values.mul_(expanded)
        raise ValueError(f"unknown quantization granularity: {kind}")


@dataclass(frozen=True)
class QuantImpl:
    name: str
    fn: Callable[..., QuantResult]
    description: str = ""
    get_best_config: Callable[[], Any | None] = lambda: None


@dataclass(frozen=True)
class BMMImpl:
    name: str
    fn: Callable[..., torch.Tensor]
    quant_impl: str
    a_layout: str
    layout: str
    prepare_a: Callable[[QuantResult], QuantResult]
    prepare_b: Callable[[QuantResult], QuantResult]
    quant_a_kwargs: dict[str, Any]
    quant_b_kwargs: dict[str, Any]
    prepare_call_kwargs: Callable[[QuantResult, QuantResult], dict[str, Any]]
    description: str = ""
    get_best_config: Callable[[bool], Any | None] = lambda _use_tma: None


QUANT_IMPLS: dict[str, QuantImpl] = {}
BMM_IMPLS: dict[str, BMMImpl] = {}
_BUILTINS_LOADED = False

# listing order used by bmm_impl_names(): scaling scheme, then layout
_QUANT_ORDER = ("hip_per_block_1d", "hip_per_block_2d", "hip_per_channel", "hip_per_tensor")
_LAYOUT_ORDER = ("a_k_b_k", "a_k_b_n", "a_k_b_n_transpose", "a_m_b_n", "a_m_transpose_b_n_transpose")


def register_quant(
    name: str,
    fn: Callable[..., QuantResult],
    description: str = "",
    *,
    get_best_config: Callable[[], Any | None] | None = None,
) -> None:
    if name in QUANT_IMPLS:
        raise ValueError(f"duplicate quant implementation: {name}")
    QUANT_IMPLS[name] = QuantImpl(name, fn, description, get_best_config or (lambda: None))


def register_bmm(
    name: str,
    fn: Callable[..., torch.Tensor],
    *,
    quant_impl: str,
    layout: str,
    prepare_b: Callable[[QuantResult], QuantResult],
    a_layout: str = "k",
    prepare_a: Callable[[QuantResult], QuantResult] | None = None,
    quant_a_kwargs: dict[str, Any] | None = None,
    quant_b_kwargs: dict[str, Any] | None = None,
    prepare_call_kwargs: Callable[[QuantResult, QuantResult], dict[str, Any]] | None = None,
    description: str = "",
    get_best_config: Callable[[bool], Any | None] | None = None,
) -> None:
    if name in BMM_IMPLS:
        raise ValueError(f"duplicate BMM implementation: {name}")
    if a_layout not in ("m", "k"):
        raise ValueError(f"a_layout must be 'm' or 'k', got {a_layout}")
    if layout not in ("n", "k"):
        raise ValueError(f"layout must be 'n' or 'k', got {layout}")
    BMM_IMPLS[name] = BMMImpl(
        name=name,
        fn=fn,
        quant_impl=quant_impl,
        a_layout=a_layout,
        layout=layout,
        prepare_a=prepare_a or (lambda value: value),
        prepare_b=prepare_b,
        quant_a_kwargs=dict(quant_a_kwargs or {}),
        quant_b_kwargs=dict(quant_b_kwargs or {}),
        prepare_call_kwargs=prepare_call_kwargs or (lambda _a, _b: {}),
        description=description,
        get_best_config=get_best_config or (lambda _use_tma: None),
    )


def load_builtin_impls() -> None:
    global _BUILTINS_LOADED
    if not _BUILTINS_LOADED:
        importlib.import_module("practice_cuda_amd.impls")
        _BUILTINS_LOADED = True


def bmm_impl_names() -> list[str]:
    """Registered BMMs grouped by scaling scheme, then by operand layout."""
    load_builtin_impls()

    def rank(seq: tuple[str, ...], key: str) -> int:
        return seq.index(key) if key in seq else len(seq)

    def sort_key(name: str):
        impl = BMM_IMPLS[name]
        layout_name = name.removeprefix(f"{impl.quant_impl}_")
        return (rank(_QUANT_ORDER, impl.quant_impl), impl.quant_impl,
                rank(_LAYOUT_ORDER, layout_name), name)

    return sorted(BMM_IMPLS, key=sort_key)


def get_quant(name: str) -> QuantImpl:
    load_builtin_impls()
    if name not in QUANT_IMPLS:
        raise KeyError(f"unknown quant implementation {name}; choices={sorted(QUANT_IMPLS)}")
    return QUANT_IMPLS[name]


def get_bmm(name: str) -> BMMImpl:
    load_builtin_impls()
    if name not in BMM_IMPLS:
        raise KeyError(f"unknown BMM implementation {name}; choices={sorted(BMM_IMPLS)}")
    return BMM_IMPLS[name]
