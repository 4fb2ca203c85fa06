"""Declarative per-function constraints that the registry checks before dispatch.

Same public names and semantics as the reference (comfy_kitchen/constraints.py:30-250):
a backend declares, per function, which dtypes / device types / shapes each keyword
argument may have; `validate_function_call` returns the first violation.

The one addition is `FunctionConstraints.required_arch`: ROCm devices report no CUDA
compute capability that means anything for gfx950 features, so a backend can instead
require the device's `gcnArchName` to start with one of the given prefixes.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from collections.abc import Mapping
from dataclasses import dataclass, field

import torch

__all__ = [
    "DivisibleBy",
    "ExactDims",
    "FunctionConstraints",
    "MinDims",
    "ParamConstraint",
    "ShapeRule",
    "ValidationResult",
    "validate_function_call",
    "validate_param",
]


class ShapeRule(ABC):
    """A predicate on a tensor's shape with a human-readable description."""

    @abstractmethod
    def check(self, tensor: torch.Tensor) -> bool: ...

    @abstractmethod
    def describe(self) -> str: ...


@dataclass(frozen=True)
class DivisibleBy(ShapeRule):
    dim: int
    factor: int

    def check(self, tensor: torch.Tensor) -> bool:
        return tensor.dim() > self.dim and tensor.shape[self.dim] % self.factor == 0

    def describe(self) -> str:
        return f"dim[{self.dim}] divisible by {self.factor}"


@dataclass(frozen=True)
class MinDims(ShapeRule):
    ndim: int

    def check(self, tensor: torch.Tensor) -> bool:
        return tensor.dim() >= self.ndim

    def describe(self) -> str:
        return f"at least {self.ndim}D"


@dataclass(frozen=True)
class ExactDims(ShapeRule):
    ndim: int

    def check(self, tensor: torch.Tensor) -> bool:
        return tensor.dim() == self.ndim

    def describe(self) -> str:
        return f"exactly {self.ndim}D"


@dataclass(frozen=True)
class ParamConstraint:
    """Constraint on one keyword argument.

    dtypes: allowed dtypes (for a tensor, its dtype; for a dtype-valued argument such
        as `output_type`, the value itself).  None accepts anything.
    devices: allowed device types; None inherits the function's default_devices.
    shape_rules: rules that must all hold.
    """

    dtypes: frozenset[torch.dtype] | None = None
    devices: frozenset[str] | None = None
    shape_rules: tuple[ShapeRule, ...] = ()

    def check_dtype(self, value) -> bool:
        if self.dtypes is None:
            return True
        dt = value.dtype if isinstance(value, torch.Tensor) else value
        return dt in self.dtypes

    def check_device(self, tensor: torch.Tensor, default_devices: frozenset[str]) -> bool:
        allowed = self.devices if self.devices is not None else default_devices
        return "*" in allowed or tensor.device.type in allowed

    def check_shape(self, tensor: torch.Tensor) -> bool:
        return all(r.check(tensor) for r in self.shape_rules)


@dataclass(frozen=True)
class FunctionConstraints:
    params: dict[str, ParamConstraint] = field(default_factory=dict)
    default_devices: frozenset[str] = field(default_factory=lambda: frozenset({"cuda", "cpu"}))
    min_compute_capability: tuple[int, int] | None = None
    required_arch: tuple[str, ...] | None = None

    def __hash__(self) -> int:
        return hash((tuple(sorted(self.params.items())), self.default_devices,
                     self.min_compute_capability, self.required_arch))


@dataclass
class ValidationResult:
    success: bool
    failed_param: str | None = None
    failure_reason: str | None = None

    @staticmethod
    def ok() -> ValidationResult:
        return ValidationResult(True)

    @staticmethod
    def fail(param: str, reason: str) -> ValidationResult:
        return ValidationResult(False, param, reason)


def validate_param(name: str, value, constraint: ParamConstraint,
                   default_devices: frozenset[str]) -> ValidationResult:
    """Check one argument; None values (optional tensors) always pass."""
    if value is None:
        return ValidationResult.ok()
    if not constraint.check_dtype(value):
        dt = value.dtype if isinstance(value, torch.Tensor) else value
        return ValidationResult.fail(name, f"dtype {dt} not in {set(constraint.dtypes)}")
    if not isinstance(value, torch.Tensor):
        return ValidationResult.ok()
    if not constraint.check_device(value, default_devices):
        allowed = constraint.devices if constraint.devices is not None else default_devices
        return ValidationResult.fail(name, f"device {value.device.type} not in {set(allowed)}")
    for rule in constraint.shape_rules:
        if not rule.check(value):
            return ValidationResult.fail(name, f"shape {list(value.shape)} fails: {rule.describe()}")
    return ValidationResult.ok()


def validate_function_call(constraints: FunctionConstraints, kwargs: Mapping,
                           compute_capability: tuple[int, int] | None = None,
                           arch: str | None = None) -> ValidationResult:
    """Return the first violated constraint for this call, or ok()."""
    if constraints.min_compute_capability is not None:
        if compute_capability is None:
            return ValidationResult.fail("__hardware__", "compute capability required but not available")
        if tuple(compute_capability) < tuple(constraints.min_compute_capability):
            cur = ".".join(map(str, compute_capability))
            req = ".".join(map(str, constraints.min_compute_capability))
            return ValidationResult.fail("__hardware__", f"compute capability {cur} < required {req}")
    if constraints.required_arch is not None:
        if arch is None or not any(arch.startswith(p) for p in constraints.required_arch):
            return ValidationResult.fail(
                "__hardware__", f"device arch {arch!r} not in {list(constraints.required_arch)}")
    for pname, pcons in constraints.params.items():
        res = validate_param(pname, kwargs.get(pname), pcons, constraints.default_devices)
        if not res.success:
            return res
    return ValidationResult.ok()
