"""Backend registry with the HIP backend registered at import
(as ``src/ollm/backends/__init__.py:22-24`` registers MLX/Metal/ANE)."""
from .base import (Backend, BackendError, BackendSelection, ComputeUnit, InferencePhase,
                   OperationKind, RuntimeCapabilities, get_backend, list_backends,
                   register_backend, select_backend)
from .hip_backend import HipBackend

register_backend(HipBackend())

__all__ = [
    "Backend", "BackendError", "BackendSelection", "ComputeUnit", "HipBackend",
    "InferencePhase", "OperationKind", "RuntimeCapabilities", "get_backend", "list_backends",
    "register_backend", "select_backend",
]
