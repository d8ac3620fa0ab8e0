"""Backend selection for the MoE ops — the plugin boundary the public op wrappers
call.

The interface is the reference's: ``register(kernel, Backend)`` as a decorator
(src/xkernels/_dispatch.py:90-95), ``dispatch(kernel, *args, backend=..., **kw)``
(:243-247), ``backend_registration_guard`` for optional backends (:74-87), and
the resolution order explicit argument -> ``$XKERNELS_BACKEND`` -> the vendor's
preference list (amd: HIP, TRITON, REFERENCE; :37-41, :162-187).

Every kernel name owns one ``_Entry``: the callables per backend and the
registration errors seen for it. Errors are surfaced, never swallowed: an
explicit request for a backend that failed to register raises ``RuntimeError``
with the recorded cause, and an automatic choice that had to pass over such a
backend warns once. This package registers HIP only; nothing falls back to the
CPU unless a REFERENCE backend was installed (the tests install the oracle).
"""
from __future__ import annotations

import os
import warnings
from collections.abc import Callable, Iterable
from contextlib import contextmanager

from ._backends import Backend, detect_vendor

_PREFERENCE: dict[str, tuple[Backend, ...]] = {
    "amd": (Backend.HIP, Backend.TRITON, Backend.REFERENCE),
    "nvidia": (Backend.CUDA, Backend.TRITON, Backend.REFERENCE),
    "none": (Backend.REFERENCE,),
}


class _Entry:
    """Callables and registration errors of one kernel name."""

    __slots__ = ("impls", "errors", "warned")

    def __init__(self) -> None:
        self.impls: dict[Backend, Callable] = {}
        self.errors: list[tuple[Backend, str, BaseException]] = []  # (backend, source, exc)
        self.warned = False

    def error_for(self, backend: Backend) -> tuple[str, BaseException] | None:
        for b, source, exc in reversed(self.errors):
            if b is backend:
                return source, exc
        return None


_TABLE: dict[str, _Entry] = {}


def _entry(kernel: str) -> _Entry:
    e = _TABLE.get(kernel)
    if e is None:
        e = _TABLE[kernel] = _Entry()
    return e


def _as_backend(value) -> Backend:
    if isinstance(value, Backend):
        return value
    try:
        return Backend(str(value).strip().lower())
    except ValueError:
        raise KeyError(f"unknown backend {value!r}; known: {[b.value for b in Backend]}") from None


def _describe(exc: BaseException) -> str:
    return f"{type(exc).__name__}: {exc}"


# ---------------------------------------------------------------- registry ---

def register(kernel_name: str, backend: Backend) -> Callable[[Callable], Callable]:
    """Decorator: ``fn`` implements ``kernel_name`` on ``backend``."""
    b = _as_backend(backend)

    def bind(fn: Callable) -> Callable:
        _entry(kernel_name).impls[b] = fn
        return fn

    return bind


def unregister(kernel_name: str, backend: Backend) -> None:
    """Removes one binding (tests install temporary backends)."""
    e = _TABLE.get(kernel_name)
    if e is not None:
        e.impls.pop(_as_backend(backend), None)


def forget(kernel_name: str) -> None:
    """Drops every binding and recorded error of ``kernel_name``."""
    _TABLE.pop(kernel_name, None)


def record_backend_failure(kernel_names: str | Iterable[str], backend: Backend,
                           exc: BaseException, *, source: str) -> None:
    """Remembers that ``backend`` could not be registered for these kernels."""
    names = [kernel_names] if isinstance(kernel_names, str) else list(kernel_names)
    for name in names:
        _entry(name).errors.append((_as_backend(backend), source, exc))


@contextmanager
def backend_registration_guard(kernel_names: str | Iterable[str], backend: Backend, *,
                               source: str):
    """Runs a backend's registration; an exception is recorded for the kernels
    (and re-raised when ``XKERNELS_STRICT_BACKENDS`` is set to a true value)."""
    try:
        yield
    except Exception as exc:  # noqa: BLE001 - recorded, surfaced at dispatch time
        record_backend_failure(kernel_names, backend, exc, source=source)
        if os.environ.get("XKERNELS_STRICT_BACKENDS", "").strip().lower() in ("1", "true", "yes", "on"):
            raise


def registered_backends(kernel_name: str) -> list[Backend]:
    e = _TABLE.get(kernel_name)
    return list(e.impls) if e else []


def registered_kernels() -> list[str]:
    return [k for k, e in _TABLE.items() if e.impls]


def backend_diagnostics() -> dict[str, dict[str, object]]:
    """Per kernel: the registered backends and the recorded registration errors."""
    return {
        name: {
            "registered": [b.value for b in e.impls],
            "failures": [{"backend": b.value, "source": src, "type": type(x).__name__,
                          "message": str(x)} for b, src, x in e.errors],
        }
        for name, e in sorted(_TABLE.items())
    }


# --------------------------------------------------------------- selection ---

def _missing(kernel: str, backend: Backend, e: _Entry | None) -> Exception:
    failed = e.error_for(backend) if e else None
    if failed is not None:
        source, exc = failed
        err = RuntimeError(f"backend {backend.name} for '{kernel}' failed to register "
                           f"({source}): {_describe(exc)}")
        err.__cause__ = exc
        return err
    have = [b.name for b in e.impls] if e else []
    return KeyError(f"backend {backend.name} not registered for '{kernel}'; have {have}")


def select_backend(kernel_name: str, backend="auto") -> Backend:
    """The backend a call of ``kernel_name`` runs on."""
    e = _TABLE.get(kernel_name)
    if e is None or not e.impls:
        if e is not None and e.errors:
            b, source, exc = e.errors[-1]
            raise RuntimeError(f"no backend registered for '{kernel_name}': {b.name} "
                               f"({source}) failed with {_describe(exc)}") from exc
        raise KeyError(f"no backends registered for kernel '{kernel_name}'")
    if backend != "auto":
        want = _as_backend(backend)
        if want not in e.impls:
            raise _missing(kernel_name, want, e)
        return want
    env = os.environ.get("XKERNELS_BACKEND", "").strip()
    if env:
        want = _as_backend(env)
        if want not in e.impls:
            raise _missing(kernel_name, want, e)
        return want
    order = _PREFERENCE.get(detect_vendor(), (Backend.REFERENCE,))
    for b in order:
        if b in e.impls:
            return b
    return next(iter(e.impls))


def _warn_if_passed_over(kernel: str, chosen: Backend, args, kwargs) -> None:
    """An automatic choice of REFERENCE for device tensors after a preferred
    backend failed to register is reported once (the call still runs)."""
    e = _TABLE[kernel]
    if chosen is not Backend.REFERENCE or e.warned:
        return
    order = _PREFERENCE.get(detect_vendor(), ())
    skipped = [(b, *e.error_for(b)) for b in order[:order.index(chosen)] if e.error_for(b)] \
        if chosen in order else []
    if not skipped:
        return
    on_device = any(getattr(a, "is_cuda", False) for a in (*args, *kwargs.values()))
    if not on_device:
        return
    e.warned = True
    why = "; ".join(f"{b.value} ({src}): {_describe(x)}" for b, src, x in skipped)
    warnings.warn(f"backend='auto' selected REFERENCE for '{kernel}' on device tensors because "
                  f"a preferred backend failed to register: {why}", RuntimeWarning, stacklevel=3)


def dispatch(kernel_name: str, *args, backend="auto", **kwargs):
    """Runs ``kernel_name`` on the selected backend."""
    chosen = select_backend(kernel_name, backend)
    if backend == "auto" and not os.environ.get("XKERNELS_BACKEND", "").strip():
        _warn_if_passed_over(kernel_name, chosen, args, kwargs)
    return _TABLE[kernel_name].impls[chosen](*args, **kwargs)
