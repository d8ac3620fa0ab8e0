"""Backend registry and selection — the plugin boundary of the MoE ops.

Mirrors the reference's ``xkernels._dispatch`` contract
(src/xkernels/_dispatch.py:19-247): backends self-register with
``@register(kernel, Backend.X)``; ``dispatch(kernel, *args, backend="auto",
**kw)`` resolves explicit argument -> ``$XKERNELS_BACKEND`` -> the per-vendor
auto order (amd: HIP, TRITON, REFERENCE). Optional backends register inside
``backend_registration_guard`` so an import failure is recorded (and re-raised
under ``XKERNELS_STRICT_BACKENDS=1``) instead of breaking the package.

This package registers only the HIP backend. There is no silent CPU fallback:
with no backend able to take a call, ``dispatch`` raises.
"""
from __future__ import annotations

import os
import warnings
from collections.abc import Callable
from contextlib import contextmanager
from dataclasses import dataclass

from ._backends import Backend, detect_vendor

_REGISTRY: dict[str, dict[Backend, Callable]] = {}


@dataclass(frozen=True)
class BackendFailure:
    kernel_name: str
    backend: Backend
    source: str
    exc_type: str
    message: str
    exception: BaseException


_BACKEND_FAILURES: dict[str, list[BackendFailure]] = {}
_FALLBACK_WARNED: set[tuple] = set()

_AUTO_ORDER: dict[str, list[Backend]] = {
    "nvidia": [Backend.CUDA, Backend.TRITON, Backend.REFERENCE],
    "amd": [Backend.HIP, Backend.TRITON, Backend.REFERENCE],
    "none": [Backend.REFERENCE],
}

_TRUE = {"1", "true", "yes", "on"}


def _strict() -> bool:
    return os.environ.get("XKERNELS_STRICT_BACKENDS", "").lower() in _TRUE


def _names(kernel_names) -> tuple[str, ...]:
    return (kernel_names,) if isinstance(kernel_names, str) else tuple(kernel_names)


def record_backend_failure(kernel_names, backend: Backend, exc: BaseException, *, source: str) -> None:
    """Remember why an optional backend did not register (see ``backend_diagnostics``)."""
    for name in _names(kernel_names):
        _BACKEND_FAILURES.setdefault(name, []).append(
            BackendFailure(name, backend, source, type(exc).__name__, str(exc), exc)
        )


@contextmanager
def backend_registration_guard(kernel_names, backend: Backend, *, source: str):
    """Record (strict mode: re-raise) exceptions raised while registering a backend."""
    try:
        yield
    except Exception as exc:  # noqa: BLE001 - any import/registration error is recorded
        record_backend_failure(kernel_names, backend, exc, source=source)
        if _strict():
            raise


def register(kernel_name: str, backend: Backend) -> Callable[[Callable], Callable]:
    def deco(fn: Callable) -> Callable:
        _REGISTRY.setdefault(kernel_name, {})[backend] = fn
        return fn

    return deco


def unregister(kernel_name: str, backend: Backend) -> None:
    """Remove one registration (used by tests that install temporary backends)."""
    _REGISTRY.get(kernel_name, {}).pop(backend, None)


def registered_backends(kernel_name: str) -> list[Backend]:
    return list(_REGISTRY.get(kernel_name, {}))


def registered_kernels() -> list[str]:
    return list(_REGISTRY)


def backend_failures(kernel_name: str | None = None) -> dict[str, list[BackendFailure]]:
    if kernel_name is not None:
        return {kernel_name: list(_BACKEND_FAILURES.get(kernel_name, ()))}
    return {k: list(v) for k, v in _BACKEND_FAILURES.items()}


def backend_diagnostics() -> dict[str, dict[str, object]]:
    """Registered backends and recorded failures for every known kernel."""
    out: dict[str, dict[str, object]] = {}
    for name in sorted(set(_REGISTRY) | set(_BACKEND_FAILURES)):
        out[name] = {
            "registered": [b.value for b in registered_backends(name)],
            "failures": [
                {"backend": f.backend.value, "source": f.source, "type": f.exc_type,
                 "message": f.message}
                for f in _BACKEND_FAILURES.get(name, ())
            ],
        }
    return out


def _coerce(backend) -> Backend:
    return backend if isinstance(backend, Backend) else Backend(str(backend).lower())


def _unregistered(kernel_name: str, backend: Backend, impls: dict) -> Exception:
    for f in reversed(_BACKEND_FAILURES.get(kernel_name, ())):
        if f.backend is backend:
            err = RuntimeError(
                f"backend {backend.name} failed to register for '{kernel_name}' from "
                f"{f.source}: {f.exc_type}: {f.message}"
            )
            err.__cause__ = f.exception
            return err
    return KeyError(
        f"backend {backend.name} not registered for '{kernel_name}'; have {[b.name for b in impls]}"
    )


def _select_backend_with_source(kernel_name: str, backend="auto") -> tuple[Backend, str]:
    if kernel_name not in _REGISTRY or not _REGISTRY[kernel_name]:
        failures = _BACKEND_FAILURES.get(kernel_name)
        if failures:
            f = failures[-1]
            raise RuntimeError(
                f"no backend registered for '{kernel_name}': {f.backend.name} from {f.source} "
                f"failed with {f.exc_type}: {f.message}"
            ) from f.exception
        raise KeyError(f"no backends registered for kernel '{kernel_name}'")
    impls = _REGISTRY[kernel_name]
    if backend != "auto":
        chosen = _coerce(backend)
        if chosen not in impls:
            raise _unregistered(kernel_name, chosen, impls)
        return chosen, "explicit"
    env = os.environ.get("XKERNELS_BACKEND")
    if env:
        chosen = Backend(env.lower())
        if chosen in impls:
            return chosen, "env"
        raise _unregistered(kernel_name, chosen, impls)
    for cand in _AUTO_ORDER.get(detect_vendor(), [Backend.REFERENCE]):
        if cand in impls:
            return cand, "auto"
    return next(iter(impls)), "fallback_any"


def select_backend(kernel_name: str, backend="auto") -> Backend:
    return _select_backend_with_source(kernel_name, backend)[0]


def _has_cuda_tensor(obj) -> bool:
    if getattr(obj, "is_cuda", False):
        return True
    if isinstance(obj, dict):
        return any(_has_cuda_tensor(v) for v in obj.values())
    if isinstance(obj, (list, tuple)):
        return any(_has_cuda_tensor(v) for v in obj)
    return False


def _warn_reference_fallback(kernel_name, backend, chosen, source, args, kwargs) -> None:
    # Same policy as the reference (_dispatch.py:204-240): auto picking REFERENCE
    # for GPU tensors after an optimized backend failed to register is loud.
    if backend != "auto" or chosen is not Backend.REFERENCE or source != "auto":
        return
    if not (_has_cuda_tensor(args) or _has_cuda_tensor(kwargs)):
        return
    failures = [f for f in _BACKEND_FAILURES.get(kernel_name, ()) if f.backend is not Backend.REFERENCE]
    if not failures:
        return
    key = (kernel_name, tuple((f.backend.value, f.source, f.message) for f in failures))
    if key in _FALLBACK_WARNED:
        return
    _FALLBACK_WARNED.add(key)
    summary = "; ".join(f"{f.backend.value} from {f.source}: {f.exc_type}: {f.message}" for f in failures)
    warnings.warn(
        f"backend='auto' selected REFERENCE for '{kernel_name}' on a GPU tensor after "
        f"optimized backend registration failed ({summary})",
        RuntimeWarning,
        stacklevel=3,
    )


def dispatch(kernel_name: str, *args, backend="auto", **kwargs):
    """Run ``kernel_name`` on the selected backend."""
    chosen, source = _select_backend_with_source(kernel_name, backend)
    _warn_reference_fallback(kernel_name, backend, chosen, source, args, kwargs)
    return _REGISTRY[kernel_name][chosen](*args, **kwargs)
