"""Errors raised by backend selection.

Mirrors the exception hierarchy of the reference (comfy_kitchen/exceptions.py:1-40)
so callers that catch these types keep working.  Every class derives from
RuntimeError, which the QuantizedTensor layouts catch to fall back to
dequantize-then-compute.
"""


class BackendError(RuntimeError):
    """Base class for every backend-selection failure."""


class BackendNotFoundError(BackendError):
    """The named backend is not registered, failed to load, or is disabled."""

    def __init__(self, backend_name: str, reason: str | None = None):
        self.backend_name = backend_name
        self.reason = reason
        text = f"Backend '{backend_name}' is not available"
        if reason:
            text = f"{text}: {reason}"
        super().__init__(text)


class BackendNotImplementedError(BackendError):
    """The named backend is registered but does not provide the function."""

    def __init__(self, backend_name: str, func_name: str):
        self.backend_name = backend_name
        self.func_name = func_name
        super().__init__(f"Backend '{backend_name}' does not implement '{func_name}'")


class NoCapableBackendError(BackendError):
    """No registered backend accepts the call; `failures` maps backend -> reason."""

    def __init__(self, func_name: str, failures: dict[str, str]):
        self.func_name = func_name
        self.failures = dict(failures)
        if self.failures:
            why = "; ".join(f"{b}: {r}" for b, r in self.failures.items())
            text = f"No backend can handle '{func_name}': {why}"
        else:
            text = f"No backend available for '{func_name}'"
        super().__init__(text)
