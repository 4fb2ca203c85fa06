"""Backend registry: the plugin boundary the `ck.*` ops dispatch through.

Public surface matches the reference registry (comfy_kitchen/registry.py:20-307):
`register(name, module, {func: FunctionConstraints})`, `mark_unavailable`,
`disable/enable`, `set_priority`, `list_backends`, `get_capable_backend`,
`get_implementation` and the thread-local, nestable `use_backend` context.
Implementations are looked up as `getattr(module, func_name)` and called with the
eager backend's keyword arguments.

In this build one backend is registered, "hip" (hand-written gfx950 kernels behind a
C ABI).  There is deliberately no CPU or eager fallback: a call that the hip backend
cannot take raises NoCapableBackendError naming the reason.
"""
from __future__ import annotations

import logging
import threading
from collections.abc import Callable, Mapping
from contextlib import contextmanager
from typing import Any

import torch

from .constraints import FunctionConstraints, ValidationResult, validate_function_call
from .exceptions import BackendNotFoundError, BackendNotImplementedError, NoCapableBackendError

logger = logging.getLogger("comfy_kitchen.dispatch")

DEFAULT_PRIORITY = ("hip",)


class BackendRegistry:
    def __init__(self):
        self._backends: dict[str, Any] = {}
        self._capabilities: dict[str, set[str]] = {}
        self._constraints: dict[tuple[str, str], FunctionConstraints] = {}
        self._priority: list[str] = list(DEFAULT_PRIORITY)
        self._disabled: set[str] = set()
        self._unavailable: dict[str, str] = {}
        self._lock = threading.Lock()
        self._tls = threading.local()
        self._hw: tuple | None = None

    # ---------------------------------------------------------------- hardware
    def _hardware(self) -> tuple[tuple[int, int] | None, str | None]:
        """(compute capability, gcnArchName) of the current device, cached."""
        if self._hw is None:
            cc, arch = None, None
            if torch.cuda.is_available():
                try:
                    p = torch.cuda.get_device_properties(torch.cuda.current_device())
                    cc = (p.major, p.minor)
                    arch = getattr(p, "gcnArchName", None)
                except Exception:  # pragma: no cover - device query failure
                    pass
            self._hw = (cc, arch)
        return self._hw

    # ------------------------------------------------------------ registration
    def register(self, name: str, module, capabilities: dict[str, FunctionConstraints]):
        with self._lock:
            self._backends[name] = module
            self._capabilities[name] = set(capabilities)
            for fn, cons in capabilities.items():
                self._constraints[(name, fn)] = cons
            self._unavailable.pop(name, None)

    def get_constraints(self, backend_name: str, func_name: str) -> FunctionConstraints | None:
        return self._constraints.get((backend_name, func_name))

    def mark_unavailable(self, name: str, reason: str):
        with self._lock:
            self._unavailable[name] = reason

    def disable(self, backend_name: str):
        with self._lock:
            self._disabled.add(backend_name)

    def enable(self, backend_name: str):
        with self._lock:
            self._disabled.discard(backend_name)

    def set_priority(self, priority_list: list[str]):
        with self._lock:
            self._priority = list(priority_list)

    def is_available(self, backend_name: str) -> bool:
        return backend_name in self._backends and backend_name not in self._disabled

    def list_backends(self) -> dict:
        names = set(self._priority) | set(self._backends) | set(self._unavailable)
        return {
            n: {
                "available": n in self._backends,
                "disabled": n in self._disabled,
                "unavailable_reason": self._unavailable.get(n),
                "capabilities": sorted(self._capabilities.get(n, ())),
            }
            for n in names
        }

    # -------------------------------------------------------------- selection
    def validate_backend_for_call(self, backend_name: str, func_name: str,
                                  kwargs: Mapping[str, Any]) -> ValidationResult:
        if not self.is_available(backend_name):
            return ValidationResult.fail("__backend__", self._unavailable.get(backend_name, "not available"))
        if func_name not in self._capabilities.get(backend_name, ()):
            return ValidationResult.fail("__function__", "not implemented")
        cons = self._constraints.get((backend_name, func_name))
        if cons is None:
            return ValidationResult.ok()
        cc, arch = (None, None)
        if cons.min_compute_capability is not None or cons.required_arch is not None:
            cc, arch = self._hardware()
        return validate_function_call(cons, kwargs, compute_capability=cc, arch=arch)

    def get_capable_backend(self, func_name: str, kwargs: Mapping[str, Any] | None = None) -> str:
        failures: dict[str, str] = {}
        check = bool(kwargs)
        forced = getattr(self._tls, "override", None)
        if forced:
            if not self.is_available(forced):
                failures[forced] = "not available"
            elif func_name not in self._capabilities.get(forced, ()):
                failures[forced] = "not implemented"
            else:
                res = self.validate_backend_for_call(forced, func_name, kwargs) if check else ValidationResult.ok()
                if res.success:
                    logger.debug("Backend %s selected for %s (override)", forced, func_name)
                    return forced
                failures[forced] = f"{res.failed_param}: {res.failure_reason}"
        for name in self._priority:
            if not self.is_available(name) or func_name not in self._capabilities.get(name, ()):
                if name in self._unavailable and name not in failures:
                    failures[name] = f"__backend__: {self._unavailable[name]}"
                continue
            if check:
                res = self.validate_backend_for_call(name, func_name, kwargs)
                if not res.success:
                    failures[name] = f"{res.failed_param}: {res.failure_reason}"
                    continue
            logger.debug("Backend %s selected for %s", name, func_name)
            return name
        raise NoCapableBackendError(func_name, failures)

    def get_implementation(self, func_name: str, backend: str | None = None,
                           kwargs: Mapping[str, Any] | None = None) -> Callable:
        if backend:
            if backend not in self._backends:
                raise BackendNotFoundError(backend, self._unavailable.get(backend, "not registered"))
            if backend in self._disabled:
                raise BackendNotFoundError(backend, "disabled")
            if func_name not in self._capabilities.get(backend, ()):
                raise BackendNotImplementedError(backend, func_name)
            if kwargs:
                res = self.validate_backend_for_call(backend, func_name, kwargs)
                if not res.success:
                    raise NoCapableBackendError(func_name, {backend: f"{res.failed_param}: {res.failure_reason}"})
            return getattr(self._backends[backend], func_name)
        return getattr(self._backends[self.get_capable_backend(func_name, kwargs)], func_name)

    @contextmanager
    def use_backend(self, backend_name: str):
        """Force `backend_name` for calls made by this thread inside the block."""
        if not self.is_available(backend_name):
            if backend_name in self._unavailable:
                raise BackendNotFoundError(backend_name, self._unavailable[backend_name])
            if backend_name in self._disabled:
                raise BackendNotFoundError(backend_name, "disabled")
            raise BackendNotFoundError(backend_name, "not registered")
        outer = getattr(self._tls, "override", None)
        self._tls.override = backend_name
        try:
            yield
        finally:
            self._tls.override = outer


registry = BackendRegistry()
