"""Backend registry: the plugin boundary every `ck.*` op dispatches through.

The public surface -- method names, arguments, return values, exception types and
messages -- is the reference registry's (comfy_kitchen/registry.py:20-307), so backend
modules and callers written for it work unchanged:

    register(name, module, {func: FunctionConstraints})   mark_unavailable(name, reason)
    disable(name) / enable(name)                           set_priority([names])
    is_available(name)                                     list_backends()
    get_constraints(name, func)                            validate_backend_for_call(...)
    get_capable_backend(func, kwargs)                      get_implementation(func, ...)
    use_backend(name)   (context manager, per thread, nestable)

Implementations are `getattr(module, func)` and are called with the eager backend's
keyword arguments.

Design.  Every backend name the registry has heard of owns one `_Slot`: the module
(None until registered), its per-function constraint table, the reason it failed to
load, and an enabled flag.  Choosing a backend walks a candidate sequence -- the names
forced by `use_backend` on this thread, innermost first, then the priority order -- and
asks each slot for its *objection* to the call (None when it can take it).  The first
candidate without an objection wins; the objections collected on the way become the
`NoCapableBackendError` report.

In this build one backend is registered, "hip" (hand-written gfx950 kernels behind a C
ABI).  There is deliberately no CPU or eager fallback: a call the hip backend cannot
take raises NoCapableBackendError naming the reason.
"""
from __future__ import annotations

import logging
import threading
from collections.abc import Callable, Iterator, Mapping
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any

import torch

from .constraints import FunctionConstraints, ValidationResult, validate_function_call
from .exceptions import BackendNotFoundError, BackendNotImplementedError, NoCapableBackendError

logger = logging.getLogger("comfy_kitchen.dispatch")

DEFAULT_PRIORITY = ("hip",)


@dataclass
class _Slot:
    """Everything the registry knows about one backend name."""

    module: Any = None
    table: dict[str, FunctionConstraints] = field(default_factory=dict)
    load_error: str | None = None
    enabled: bool = True

    @property
    def usable(self) -> bool:
        return self.module is not None and self.enabled

    def absence(self) -> str:
        """Why an unusable slot cannot serve (the text BackendNotFoundError carries)."""
        if self.module is None:
            return self.load_error or "not registered"
        return "disabled"


def _device_identity() -> tuple[tuple[int, int] | None, str | None]:
    """(torch's device capability, gcnArchName) of the current GPU; (None, None) without one."""
    if not torch.cuda.is_available():
        return None, None
    try:
        props = torch.cuda.get_device_properties(torch.cuda.current_device())
    except RuntimeError:  # pragma: no cover - a device query failing on a broken driver
        return None, None
    return (props.major, props.minor), getattr(props, "gcnArchName", None)


class BackendRegistry:
    def __init__(self):
        self._slots: dict[str, _Slot] = {}
        self._order: tuple[str, ...] = DEFAULT_PRIORITY
        self._guard = threading.Lock()
        self._local = threading.local()  # .forced: stack of use_backend names
        self._identity: tuple | None = None

    # ------------------------------------------------------------- bookkeeping
    def _slot(self, name: str) -> _Slot:
        """The slot of `name`, created empty on first mention (callers hold the guard)."""
        slot = self._slots.get(name)
        if slot is None:
            slot = self._slots[name] = _Slot()
        return slot

    def _hardware(self) -> tuple[tuple[int, int] | None, str | None]:
        if self._identity is None:
            self._identity = _device_identity()
        return self._identity

    def _forced(self) -> list[str]:
        stack = getattr(self._local, "forced", None)
        if stack is None:
            stack = self._local.forced = []
        return stack

    # ------------------------------------------------------------ registration
    def register(self, name: str, module, capabilities: dict[str, FunctionConstraints]):
        """Make `module` serve the functions named in `capabilities` under their constraints."""
        with self._guard:
            slot = self._slot(name)
            slot.module = module
            slot.table = dict(capabilities)
            slot.load_error = None

    def mark_unavailable(self, name: str, reason: str):
        """Record that backend `name` could not be loaded, and why."""
        with self._guard:
            self._slot(name).load_error = reason

    def disable(self, backend_name: str):
        with self._guard:
            self._slot(backend_name).enabled = False

    def enable(self, backend_name: str):
        with self._guard:
            self._slot(backend_name).enabled = True

    def set_priority(self, priority_list: list[str]):
        with self._guard:
            self._order = tuple(priority_list)

    # ------------------------------------------------------------------ queries
    def get_constraints(self, backend_name: str, func_name: str) -> FunctionConstraints | None:
        slot = self._slots.get(backend_name)
        return None if slot is None else slot.table.get(func_name)

    def is_available(self, backend_name: str) -> bool:
        slot = self._slots.get(backend_name)
        return slot is not None and slot.usable

    def list_backends(self) -> dict:
        """{name: {available, disabled, unavailable_reason, capabilities}} for every name
        that is registered, failed to load, or appears in the priority order."""
        names = dict.fromkeys([*self._order, *self._slots])
        report = {}
        for name in names:
            slot = self._slots.get(name, _Slot())
            report[name] = {
                "available": slot.module is not None,
                "disabled": not slot.enabled,
                "unavailable_reason": slot.load_error if slot.module is None else None,
                "capabilities": sorted(slot.table),
            }
        return report

    # --------------------------------------------------------------- selection
    def validate_backend_for_call(self, backend_name: str, func_name: str,
                                  kwargs: Mapping[str, Any]) -> ValidationResult:
        """Check one backend against one call's arguments, without choosing anything."""
        slot = self._slots.get(backend_name)
        if slot is None or not slot.usable:
            reason = slot.load_error if slot is not None and slot.load_error else "not available"
            return ValidationResult.fail("__backend__", reason)
        rules = slot.table.get(func_name, False)
        if rules is False:
            return ValidationResult.fail("__function__", "not implemented")
        if rules is None:
            return ValidationResult.ok()
        cc, arch = None, None
        if rules.min_compute_capability is not None or rules.required_arch is not None:
            cc, arch = self._hardware()
        return validate_function_call(rules, kwargs, compute_capability=cc, arch=arch)

    def _objection(self, name: str, func_name: str, kwargs: Mapping[str, Any] | None,
                   forced: bool) -> str | None:
        """Why backend `name` would refuse this call, or None if it can take it.

        A backend chosen by priority that is unusable, or lacks the function, is passed
        over silently unless it failed to load (then the load error is reported); a forced
        backend's refusal is always reported."""
        slot = self._slots.get(name)
        if slot is None or not slot.usable:
            if forced:
                return "not available"
            return f"__backend__: {slot.load_error}" if slot is not None and slot.load_error else ""
        if func_name not in slot.table:
            return "not implemented" if forced else ""
        if kwargs:
            verdict = self.validate_backend_for_call(name, func_name, kwargs)
            if not verdict.success:
                return f"{verdict.failed_param}: {verdict.failure_reason}"
        return None

    def _candidates(self) -> Iterator[tuple[str, bool]]:
        forced = self._forced()
        if forced:
            yield forced[-1], True
        yield from ((name, False) for name in self._order)

    def get_capable_backend(self, func_name: str, kwargs: Mapping[str, Any] | None = None) -> str:
        """Name of the first candidate backend able to take the call (empty or None kwargs
        skip the argument checks)."""
        report: dict[str, str] = {}
        for name, forced in self._candidates():
            why = self._objection(name, func_name, kwargs, forced)
            if why is None:
                logger.debug("Backend %s selected for %s%s", name, func_name, " (override)" if forced else "")
                return name
            if why and name not in report:
                report[name] = why
        raise NoCapableBackendError(func_name, report)

    def get_implementation(self, func_name: str, backend: str | None = None,
                           kwargs: Mapping[str, Any] | None = None) -> Callable:
        """The callable serving `func_name`: from `backend` if named, else the selected one."""
        if not backend:
            backend = self.get_capable_backend(func_name, kwargs)
            return getattr(self._slots[backend].module, func_name)
        slot = self._slots.get(backend, _Slot())
        if not slot.usable:
            raise BackendNotFoundError(backend, slot.absence())
        if func_name not in slot.table:
            raise BackendNotImplementedError(backend, func_name)
        if kwargs:
            verdict = self.validate_backend_for_call(backend, func_name, kwargs)
            if not verdict.success:
                raise NoCapableBackendError(func_name, {backend: f"{verdict.failed_param}: {verdict.failure_reason}"})
        return getattr(slot.module, func_name)

    @contextmanager
    def use_backend(self, backend_name: str):
        """Prefer `backend_name` for calls made by this thread inside the block."""
        slot = self._slots.get(backend_name, _Slot())
        if not slot.usable:
            raise BackendNotFoundError(backend_name, slot.absence())
        stack = self._forced()
        stack.append(backend_name)
        try:
            yield
        finally:
            stack.pop()


registry = BackendRegistry()
