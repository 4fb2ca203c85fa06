"""QuantizedTensor: a torch.Tensor subclass that presents a logical (dequantized) tensor
while holding quantized storage plus a layout's typed parameters.

Interface kept from the reference (tensor/base.py:1-511), because checkpoints, layouts
and callers depend on it: the layout registry (`register_layout_class`,
`get_layout_class`), the frozen `BaseLayoutParams` dataclass with its `scale`,
`orig_dtype`, `orig_shape` fields and `to_device` / `clone` / `copy_from`, the
`QuantizedLayout` class methods (`quantize`, `dequantize`, `get_plain_tensors`,
`state_dict_tensors`, `supports_fast_matmul`, `get_requirements`), the
`QuantizedTensor(qdata, layout_name, params)` constructor with `_qdata`, `_layout_cls`,
`_params`, `from_float`, `dequantize`, `state_dict`, the set of aten ops it intercepts,
`register_layout_op`, and the dequantize fallback for every other op.

Design of this implementation:
  * Params rebuild themselves through one map over their tensor-valued fields (found by
    value, so a layout adds tensor fields without listing them).
  * Each layout class carries its own op table, filled by `register_layout_op`; a call
    looks the op up along the layout's MRO, so a sub-layout inherits and may override.
  * The layout-independent ops (detach, clone, to, _to_copy, contiguous, is_contiguous,
    copy_, empty_like) are QuantizedTensor methods.  Their arguments are bound to names
    through the aten op's schema, so every `to` overload reads the same `dtype` and
    `device` names.
  * "Fast matmul" support is decided by the device architecture (gfx950, where the hip
    backend's GEMMs run), not by a CUDA SM version.
"""
from __future__ import annotations

import dataclasses
import logging
from abc import ABC, abstractmethod
from dataclasses import dataclass
from functools import lru_cache
from typing import Any, Callable

import torch

logger = logging.getLogger(__name__)
aten = torch.ops.aten

# ----------------------------------------------------------------------------- layouts
LAYOUTS: dict[str, type] = {}


def register_layout_class(name: str, cls) -> None:
    """Make layout class `cls` reachable by `name` (the string QuantizedTensors store)."""
    LAYOUTS[name] = cls


def get_layout_class(name: str):
    return LAYOUTS[name]


@lru_cache(maxsize=1)
def get_cuda_capability() -> tuple[int, int] | None:
    """torch's device capability of the current GPU (on ROCm, gfx950 reports (9, 5))."""
    return torch.cuda.get_device_capability() if torch.cuda.is_available() else None


@lru_cache(maxsize=1)
def get_device_arch() -> str | None:
    """gcnArchName of the current GPU, e.g. 'gfx950:sramecc+:xnack-'."""
    if not torch.cuda.is_available():
        return None
    props = torch.cuda.get_device_properties(torch.cuda.current_device())
    return getattr(props, "gcnArchName", None)


@dataclass(frozen=True)
class BaseLayoutParams:
    """Parameters every layout has: the scale tensor and the logical dtype / shape.

    Layouts subclass it (as frozen dataclasses) to add fields.  Any field whose value is
    a tensor travels with device moves, clones and in-place copies.
    """

    scale: torch.Tensor
    orig_dtype: torch.dtype
    orig_shape: tuple[int, ...]

    def __post_init__(self):
        self._validate_tensor_fields()

    def _validate_tensor_fields(self):
        """Hook run after construction (and after every rebuild): normalise tensor fields."""

    def _tensor_fields(self) -> list[str]:
        """Names of the fields holding tensors, in declaration order."""
        return [f.name for f in dataclasses.fields(self) if isinstance(getattr(self, f.name), torch.Tensor)]

    def _map_tensors(self, fn: Callable[[torch.Tensor], torch.Tensor], **changes) -> BaseLayoutParams:
        """A copy with fn applied to every tensor field and `changes` applied on top."""
        new = {name: fn(getattr(self, name)) for name in self._tensor_fields()}
        new.update(changes)
        return dataclasses.replace(self, **new)

    def to_device(self, device: torch.device) -> BaseLayoutParams:
        return self._map_tensors(lambda t: t.to(device=device))

    def clone(self) -> BaseLayoutParams:
        return self._map_tensors(torch.Tensor.clone)

    def copy_from(self, src: BaseLayoutParams, non_blocking: bool = False) -> None:
        """Take src's values in place: tensors are copied into this object's own tensors
        (their memory is reused), every other field is rebound."""
        tensors = set(self._tensor_fields())
        for f in dataclasses.fields(self):
            value = getattr(src, f.name)
            if f.name in tensors:
                getattr(self, f.name).copy_(value, non_blocking=non_blocking)
            else:
                object.__setattr__(self, f.name, value)


def _op_table(layout_cls: type, create: bool = False) -> dict | None:
    """The op table a layout class owns itself (not one inherited from a base)."""
    table = layout_cls.__dict__.get("_layout_ops")
    if table is None and create:
        table = {}
        setattr(layout_cls, "_layout_ops", table)
    return table


class QuantizedLayout(ABC):
    """A quantization format: how to quantize, dequantize and serialise one tensor."""

    Params: type[Any]

    # Kept for interface compatibility with the reference; not used for gating here.
    MIN_SM_VERSION: tuple[int, int] | None = None
    # Architectures whose hip kernels implement this layout's matmul.
    REQUIRED_ARCH: tuple[str, ...] = ("gfx950",)

    @classmethod
    @abstractmethod
    def quantize(cls, tensor: torch.Tensor, **kwargs) -> tuple[torch.Tensor, Any]:
        raise NotImplementedError

    @classmethod
    @abstractmethod
    def dequantize(cls, qdata: torch.Tensor, params: Any) -> torch.Tensor:
        raise NotImplementedError

    @classmethod
    @abstractmethod
    def get_plain_tensors(cls, qtensor: QuantizedTensor) -> tuple[torch.Tensor, ...]:
        raise NotImplementedError

    @classmethod
    @abstractmethod
    def state_dict_tensors(cls, qdata: torch.Tensor, params: Any) -> dict[str, torch.Tensor]:
        raise NotImplementedError

    @classmethod
    def handler_for(cls, op) -> Callable | None:
        """The handler registered for aten `op` on this layout or the nearest base layout."""
        for klass in cls.__mro__:
            table = _op_table(klass)
            if table and op in table:
                return table[op]
        return None

    @classmethod
    def supports_fast_matmul(cls) -> bool:
        """True when the current GPU runs this layout's matmul on the hip kernels."""
        arch = get_device_arch()
        if arch is None or not arch.startswith(cls.REQUIRED_ARCH):
            return False
        from ..registry import registry

        return registry.is_available("hip")

    @classmethod
    def get_requirements(cls) -> dict[str, Any]:
        return {
            "layout": cls.__name__,
            "min_sm_version": cls.MIN_SM_VERSION,
            "current_sm_version": get_cuda_capability(),
            "required_arch": cls.REQUIRED_ARCH,
            "current_arch": get_device_arch(),
            "fast_matmul_supported": cls.supports_fast_matmul(),
        }


def register_layout_op(torch_op: Any, layout_cls: type[QuantizedLayout]):
    """Decorator: `handler(qt, args, kwargs)` serves `torch_op` for QuantizedTensors of
    `layout_cls` and of layouts derived from it (unless they register their own)."""

    def decorator(handler):
        _op_table(layout_cls, create=True)[torch_op] = handler
        return handler

    return decorator


def _bind(func, args, kwargs) -> dict[str, Any]:
    """An aten call's arguments by schema name (positional and keyword alike)."""
    names = [a.name for a in func._schema.arguments]
    bound = dict(zip(names, args))
    bound.update(kwargs)
    return bound


# ----------------------------------------------------------------------------- tensor
class QuantizedTensor(torch.Tensor):
    """Quantized storage (`_qdata`) + layout name (`_layout_cls`) + typed params (`_params`),
    presenting the logical (unpadded) shape and the original dtype to torch.

    `storage_shape` is the shape of the stored codes (padded, and for NVFP4 packed two
    per byte); `is_padded` tells whether the logical shape differs from the padded one.
    """

    @staticmethod
    def __new__(cls, qdata: torch.Tensor, layout_cls: str, params: Any):
        return torch.Tensor._make_wrapper_subclass(
            cls, params.orig_shape, device=qdata.device, dtype=params.orig_dtype, requires_grad=False)

    def __init__(self, qdata: torch.Tensor, layout_cls: str, params: Any):
        if not isinstance(layout_cls, str):
            raise TypeError(f"layout_cls must be a layout name, got {type(layout_cls).__name__}")
        self._qdata = qdata
        self._layout_cls = layout_cls
        self._params = params

    def __repr__(self) -> str:
        return (f"QuantizedTensor(shape={tuple(self.shape)}, storage_shape={self.storage_shape}, "
                f"layout={self._layout_cls}, dtype={self._params.orig_dtype})")

    # ------------------------------------------------------------ properties
    @property
    def storage_shape(self) -> tuple[int, ...]:
        return tuple(self._qdata.shape)

    @property
    def storage_dtype(self) -> torch.dtype:
        return self._qdata.dtype

    @property
    def nbytes(self) -> int:
        """Bytes of the quantized storage (not of the logical orig_dtype tensor)."""
        return self._qdata.nbytes

    @property
    def padded_shape(self) -> tuple[int, ...]:
        to_logical = getattr(self.layout_cls, "get_logical_shape_from_storage", None)
        return to_logical(self.storage_shape) if to_logical else self.storage_shape

    @property
    def is_padded(self) -> bool:
        return self._params.orig_shape != self.padded_shape

    @property
    def layout_cls(self) -> type[QuantizedLayout]:
        return get_layout_class(self._layout_cls)

    @property
    def params(self) -> Any:
        return self._params

    # ------------------------------------------------------------ construction
    @classmethod
    def from_float(cls, tensor: torch.Tensor, layout_cls: str, **kwargs) -> QuantizedTensor:
        qdata, params = get_layout_class(layout_cls).quantize(tensor, **kwargs)
        return cls(qdata, layout_cls, params)

    def _rewrap(self, qdata: torch.Tensor, params: Any) -> QuantizedTensor:
        return QuantizedTensor(qdata, self._layout_cls, params)

    # ------------------------------------------------------------ storage access
    def data_ptr(self):
        return self._qdata.data_ptr()

    def is_pinned(self):
        return self._qdata.is_pinned()

    def storage(self):
        return self._qdata.storage()

    def dequantize(self) -> torch.Tensor:
        """The logical tensor in orig_dtype: padding cropped, a deferred transpose applied."""
        full = self.layout_cls.dequantize(self._qdata.contiguous(), self._params)
        rows_cols = tuple(self._params.orig_shape)
        transposed = getattr(self._params, "transposed", False)
        stored = rows_cols[::-1] if transposed else rows_cols
        if tuple(full.shape) != stored:
            full = full[tuple(slice(0, n) for n in stored)]
        return full.t() if transposed else full

    def state_dict(self, prefix: str = "") -> dict[str, torch.Tensor]:
        tensors = self.layout_cls.state_dict_tensors(self._qdata, self._params)
        return {f"{prefix}{suffix}": t for suffix, t in tensors.items()}

    # ------------------------------------------------------------ flatten protocol
    # Inner tensors: the codes, then each tensor-valued param field under "_pt_<field>".
    # The context holds the layout name, the params class, the tensor field names and
    # the values of every other field.
    def __tensor_flatten__(self):
        tensor_fields = tuple(self._params._tensor_fields())
        for name in tensor_fields:
            object.__setattr__(self, f"_pt_{name}", getattr(self._params, name))
        others = tuple((f.name, getattr(self._params, f.name)) for f in dataclasses.fields(self._params)
                       if f.name not in tensor_fields)
        ctx = (self._layout_cls, type(self._params), tensor_fields, others)
        return ["_qdata", *(f"_pt_{n}" for n in tensor_fields)], ctx

    @staticmethod
    def __tensor_unflatten__(inner_tensors, ctx, outer_size, outer_stride):
        layout_name, params_cls, tensor_fields, others = ctx
        values = dict(others)
        values.update({n: inner_tensors[f"_pt_{n}"] for n in tensor_fields})
        return QuantizedTensor(inner_tensors["_qdata"], layout_name, params_cls(**values))

    # ------------------------------------------------------------ generic ops
    def _op_detach(self, a):
        return self._rewrap(self._qdata.detach(), self._params._map_tensors(torch.Tensor.detach))

    def _op_clone(self, a):
        return self._rewrap(self._qdata.clone(), self._params.clone())

    def _op_to(self, a, always_copy: bool = False):
        device, dtype = a.get("device"), a.get("dtype")
        device = torch.device(device) if isinstance(device, str) else device
        move = device is not None and device != self._qdata.device
        recast = dtype is not None and dtype != self._params.orig_dtype
        if not (move or recast or always_copy):
            return self
        if move:
            qdata, params = self._qdata.to(device=device), self._params.to_device(device)
        else:
            qdata, params = (self._qdata.clone() if always_copy else self._qdata), self._params.clone()
        if recast:  # only the logical (dequantized) dtype changes; the codes stay
            params = dataclasses.replace(params, orig_dtype=dtype)
        return self._rewrap(qdata, params)

    def _op_to_copy(self, a):
        return self._op_to(a, always_copy=True)

    def _op_contiguous(self, a):
        return self if self._qdata.is_contiguous() else self._rewrap(self._qdata.contiguous(), self._params)

    def _op_is_contiguous(self, a):
        return self._qdata.is_contiguous()

    def _op_copy_(self, a):
        src = a["src"]
        if not isinstance(src, QuantizedTensor):
            raise TypeError(f"Cannot copy {type(src).__name__} to QuantizedTensor")
        if src._layout_cls != self._layout_cls:
            raise TypeError(f"Layout mismatch: {self._layout_cls} vs {src._layout_cls}")
        non_blocking = bool(a.get("non_blocking", False))
        keep = self._params.orig_dtype  # the destination keeps its logical dtype
        self._qdata.copy_(src._qdata, non_blocking=non_blocking)
        self._params.copy_from(src._params, non_blocking=non_blocking)
        self._params = dataclasses.replace(self._params, orig_dtype=keep)
        return self

    def _op_empty_like(self, a):
        device, dtype = a.get("device"), a.get("dtype")
        params = self._params.clone() if device is None else self._params.to_device(device)
        if dtype is not None:
            params = dataclasses.replace(params, orig_dtype=dtype)
        return self._rewrap(torch.empty_like(self._qdata, device=device), params)

    def _op_shallow_copy_ok(self, a):
        return True

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        method = _GENERIC_OPS.get(func)
        if method is not None and args and isinstance(args[0], QuantizedTensor):
            return getattr(args[0], method)(_bind(func, args, kwargs))
        layout = _first_layout(args)
        handler = layout.handler_for(func) if layout is not None else None
        if handler is not None:
            return handler(args[0] if args else None, args, kwargs)
        logger.debug("%s has no handler for %s: dequantizing", getattr(layout, "__name__", "?"), func)
        return func(*dequantize_args(args), **dequantize_args(kwargs))


_GENERIC_OPS: dict[Any, str] = {
    aten.detach.default: "_op_detach",
    aten.clone.default: "_op_clone",
    aten.to.dtype_layout: "_op_to",
    aten.to.dtype: "_op_to",
    aten.to.device: "_op_to",
    aten._to_copy.default: "_op_to_copy",
    aten.contiguous.default: "_op_contiguous",
    aten.is_contiguous.default: "_op_is_contiguous",
    aten.copy_.default: "_op_copy_",
    aten.empty_like.default: "_op_empty_like",
    aten._has_compatible_shallow_copy_type.default: "_op_shallow_copy_ok",
}


def dequantize_args(args):
    """`args` with every QuantizedTensor inside (nested lists, tuples, dicts) dequantized."""
    if isinstance(args, QuantizedTensor):
        return args.dequantize()
    if isinstance(args, dict):
        return {k: dequantize_args(v) for k, v in args.items()}
    if isinstance(args, (list, tuple)):
        return type(args)(dequantize_args(a) for a in args)
    return args


def _first_layout(args) -> type[QuantizedLayout] | None:
    """Layout class of the first QuantizedTensor among args (one level of nesting)."""
    for a in args:
        for t in (a if isinstance(a, (list, tuple)) else (a,)):
            if isinstance(t, QuantizedTensor):
                return get_layout_class(t._layout_cls)
    return None


def slice_to(result: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """Cut a padded matmul result back to [rows, cols]."""
    if result.shape[0] != rows or result.shape[1] != cols:
        return result[:rows, :cols]
    return result
