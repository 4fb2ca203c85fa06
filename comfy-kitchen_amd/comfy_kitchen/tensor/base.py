"""QuantizedTensor: a torch.Tensor subclass holding quantized storage plus typed layout
parameters, with layout-specific handlers for the aten ops it intercepts.

Mirrors the reference's interface (tensor/base.py:1-511): the layout registry, the
frozen `BaseLayoutParams` dataclass, the `QuantizedLayout` protocol, the
`QuantizedTensor` wrapper subclass (`from_float`, `dequantize`, `state_dict`,
`__tensor_flatten__` / `__tensor_unflatten__`), the generic handlers (detach, clone,
to, _to_copy, contiguous, is_contiguous, copy_, empty_like), the per-layout handler
table filled through `register_layout_op`, and the dequantize fallback for any other
op.  The one deliberate difference: "fast matmul" support is decided by the device
architecture (the hip backend's gfx950 kernels), not by a CUDA SM version.
"""
from __future__ import annotations

import contextlib
import dataclasses
import logging
from abc import ABC, abstractmethod
from dataclasses import dataclass
from functools import lru_cache
from typing import Any, Callable

import torch

logger = logging.getLogger(__name__)

# ----------------------------------------------------------------------------- layouts
LAYOUTS: dict[str, type] = {}


def register_layout_class(name: str, cls) -> None:
    LAYOUTS[name] = cls


def get_layout_class(name: str):
    return LAYOUTS[name]


@lru_cache(maxsize=1)
def get_cuda_capability() -> tuple[int, int] | None:
    """torch's device capability of the current GPU (on ROCm, gfx950 reports (9, 5))."""
    if not torch.cuda.is_available():
        return None
    return torch.cuda.get_device_capability()


@lru_cache(maxsize=1)
def get_device_arch() -> str | None:
    """gcnArchName of the current GPU, e.g. 'gfx950:sramecc+:xnack-'."""
    if not torch.cuda.is_available():
        return None
    return getattr(torch.cuda.get_device_properties(torch.cuda.current_device()), "gcnArchName", None)


@dataclass(frozen=True)
class BaseLayoutParams:
    """Parameters shared by every layout: the scale tensor and the logical dtype/shape.

    Subclasses add fields; `_tensor_fields` names every field holding a tensor so that
    device moves, clones and in-place copies cover them all.
    """

    scale: torch.Tensor
    orig_dtype: torch.dtype
    orig_shape: tuple[int, ...]

    def __post_init__(self):
        self._validate_tensor_fields()

    def _validate_tensor_fields(self):
        pass

    def _tensor_fields(self) -> list[str]:
        return ["scale"]

    def _fields(self) -> dict[str, Any]:
        return {f.name: getattr(self, f.name) for f in dataclasses.fields(self)}

    def to_device(self, device: torch.device) -> BaseLayoutParams:
        kw = self._fields()
        for name in self._tensor_fields():
            kw[name] = kw[name].to(device=device)
        return type(self)(**kw)

    def clone(self) -> BaseLayoutParams:
        kw = self._fields()
        for name in self._tensor_fields():
            kw[name] = kw[name].clone()
        return type(self)(**kw)

    def copy_from(self, src: BaseLayoutParams, non_blocking: bool = False) -> None:
        """Copy src's fields into self: tensors in place (reusing memory), others rebound."""
        tensor_fields = set(self._tensor_fields())
        for f in dataclasses.fields(self):
            value = getattr(src, f.name)
            if f.name in tensor_fields:
                getattr(self, f.name).copy_(value, non_blocking=non_blocking)
            else:
                object.__setattr__(self, f.name, value)


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
    def supports_fast_matmul(cls) -> bool:
        """True when the current GPU runs this layout's matmul on the hip kernels."""
        arch = get_device_arch()
        if arch is None or not any(arch.startswith(a) for a in cls.REQUIRED_ARCH):
            return False
        from ..registry import registry

        return bool(registry.list_backends().get("hip", {}).get("available", False))

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


# ----------------------------------------------------------------------------- tensor
class QuantizedTensor(torch.Tensor):
    """Quantized storage (`_qdata`) + layout name + typed params, presenting the logical
    (unpadded) shape and the original dtype to torch.

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
        layout = self.layout_cls
        if hasattr(layout, "get_logical_shape_from_storage"):
            return layout.get_logical_shape_from_storage(self.storage_shape)
        return self.storage_shape

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

    def _copy_with(self, qdata: torch.Tensor | None = None, params: Any | None = None,
                   clone_params: bool = True) -> QuantizedTensor:
        if params is None:
            params = self._params.clone() if clone_params else self._params
        return QuantizedTensor(self._qdata if qdata is None else qdata, self._layout_cls, params)

    # ------------------------------------------------------------ core operations
    def data_ptr(self):
        return self._qdata.data_ptr()

    def is_pinned(self):
        return self._qdata.is_pinned()

    def storage(self):
        return self._qdata.storage()

    def dequantize(self) -> torch.Tensor:
        """The logical tensor in orig_dtype (padding sliced off; deferred transposes applied)."""
        qdata = self._qdata if self._qdata.is_contiguous() else self._qdata.contiguous()
        full = self.layout_cls.dequantize(qdata, self._params)
        shape = self._params.orig_shape
        if getattr(self._params, "transposed", False):
            physical = (shape[1], shape[0])
            if tuple(full.shape[:2]) != physical:
                full = full[: physical[0], : physical[1]]
            return full.t()
        if tuple(full.shape) != tuple(shape):
            full = full[tuple(slice(0, s) for s in shape)]
        return full

    def state_dict(self, prefix: str = "") -> dict[str, torch.Tensor]:
        return {prefix + k: v for k, v in self.layout_cls.state_dict_tensors(self._qdata, self._params).items()}

    # ------------------------------------------------------------ flatten protocol
    def __tensor_flatten__(self):
        inner = ["_qdata"]
        tensor_fields, other_fields = {}, {}
        for f in dataclasses.fields(self._params):
            value = getattr(self._params, f.name)
            if isinstance(value, torch.Tensor):
                attr = f"_param_{f.name}"
                object.__setattr__(self, attr, value)
                inner.append(attr)
                tensor_fields[f.name] = attr
            else:
                other_fields[f.name] = value
        return inner, {"layout_cls": self._layout_cls, "params_class": type(self._params),
                       "tensor_fields": tensor_fields, "non_tensor_fields": other_fields}

    @staticmethod
    def __tensor_unflatten__(inner_tensors, ctx, outer_size, outer_stride):
        kw = dict(ctx["non_tensor_fields"])
        kw.update({name: inner_tensors[attr] for name, attr in ctx["tensor_fields"].items()})
        return QuantizedTensor(inner_tensors["_qdata"], ctx["layout_cls"], ctx["params_class"](**kw))

    # ------------------------------------------------------------ dispatch
    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        qt = args[0] if args else None
        generic = _GENERIC_HANDLERS.get(func)
        if generic is not None:
            return generic(qt, args, kwargs)
        layout = _layout_of(args)
        if layout is not None:
            per_layout = _LAYOUT_HANDLERS.get(func)
            if per_layout:
                for klass in layout.__mro__:
                    handler = per_layout.get(klass)
                    if handler is not None:
                        return handler(qt, args, kwargs)
        logger.debug("unhandled %s for %s: dequantizing", func, layout.__name__ if layout else "?")
        return func(*dequantize_args(args), **dequantize_args(kwargs))


def dequantize_args(args):
    """Replace every QuantizedTensor inside (nested) args by its dequantized tensor."""
    if isinstance(args, QuantizedTensor):
        return args.dequantize()
    if isinstance(args, dict):
        return {k: dequantize_args(v) for k, v in args.items()}
    if isinstance(args, (list, tuple)):
        return type(args)(dequantize_args(a) for a in args)
    return args


def _layout_of(args) -> type[QuantizedLayout] | None:
    for a in args:
        if isinstance(a, QuantizedTensor):
            return get_layout_class(a._layout_cls)
        if isinstance(a, (list, tuple)):
            for b in a:
                if isinstance(b, QuantizedTensor):
                    return get_layout_class(b._layout_cls)
    return None


# ----------------------------------------------------------------------------- generic handlers
def _to_target(args, kwargs) -> tuple[torch.device | None, torch.dtype | None]:
    """(device, dtype) requested by a .to(...) call's positional and keyword arguments."""
    device, dtype = kwargs.get("device"), kwargs.get("dtype")
    for a in args[1:]:
        if isinstance(a, torch.device):
            device = a
        elif isinstance(a, torch.dtype):
            dtype = a
        elif isinstance(a, str):
            with contextlib.suppress(RuntimeError, ValueError):
                device = torch.device(a)
    if isinstance(device, str):
        device = torch.device(device)
    return device, dtype


def _to(qt: QuantizedTensor, args, kwargs, force_copy: bool = False):
    device, dtype = _to_target(args, kwargs)
    move = device is not None and device != qt._qdata.device
    recast = dtype is not None and dtype != qt._params.orig_dtype
    if not (move or recast or force_copy):
        return qt
    if move:
        qdata, params = qt._qdata.to(device=device), qt._params.to_device(device)
    else:
        qdata, params = (qt._qdata.clone() if force_copy else qt._qdata), qt._params.clone()
    if recast:  # the codes stay; only the logical (dequantized) dtype changes
        params = dataclasses.replace(params, orig_dtype=dtype)
    return qt._copy_with(qdata=qdata, params=params, clone_params=False)


def _copy_(qt, args, kwargs):
    dst, src = args[0], args[1]
    if not isinstance(src, QuantizedTensor):
        raise TypeError(f"Cannot copy {type(src).__name__} to QuantizedTensor")
    if dst._layout_cls != src._layout_cls:
        raise TypeError(f"Layout mismatch: {dst._layout_cls} vs {src._layout_cls}")
    keep_dtype = dst._params.orig_dtype
    non_blocking = kwargs.get("non_blocking", len(args) >= 3)
    dst._qdata.copy_(src._qdata, non_blocking=non_blocking)
    dst._params.copy_from(src._params, non_blocking=non_blocking)
    dst._params = dataclasses.replace(dst._params, orig_dtype=keep_dtype)
    return dst


def _empty_like(qt, args, kwargs):
    dtype = kwargs.pop("dtype", None)
    device = kwargs.get("device")
    params = qt._params.clone()
    if device is not None:
        params = params.to_device(device)
    if dtype is not None:
        params = dataclasses.replace(params, orig_dtype=dtype)
    return qt._copy_with(qdata=torch.empty_like(qt._qdata, device=device), params=params, clone_params=False)


aten = torch.ops.aten
_GENERIC_HANDLERS: dict[Any, Callable] = {
    aten.detach.default: lambda qt, a, k: qt._copy_with(qdata=qt._qdata.detach()),
    aten.clone.default: lambda qt, a, k: qt._copy_with(qdata=qt._qdata.clone()),
    aten._to_copy.default: lambda qt, a, k: _to(qt, a, k, force_copy=True),
    aten.to.dtype_layout: _to,
    aten.to.dtype: _to,
    aten.contiguous.default: lambda qt, a, k: qt if qt._qdata.is_contiguous()
    else qt._copy_with(qdata=qt._qdata.contiguous()),
    aten.is_contiguous.default: lambda qt, a, k: qt._qdata.is_contiguous(),
    aten.copy_.default: _copy_,
    aten.empty_like.default: _empty_like,
    aten._has_compatible_shallow_copy_type.default: lambda qt, a, k: True,
}

# {aten op: {layout class: handler(qt, args, kwargs)}}
_LAYOUT_HANDLERS: dict[Any, dict[type, Callable]] = {}


def register_layout_op(torch_op: Any, layout_cls: type[QuantizedLayout]):
    """Decorator: handle `torch_op` for QuantizedTensors of `layout_cls` (and subclasses)."""

    def decorator(handler):
        _LAYOUT_HANDLERS.setdefault(torch_op, {})[layout_cls] = handler
        return handler

    return decorator


def slice_to(result: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """Cut a padded matmul result back to [rows, cols]."""
    if result.shape[0] != rows or result.shape[1] != cols:
        return result[:rows, :cols]
    return result
