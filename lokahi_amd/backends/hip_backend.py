"""The "hip" backend: MI355X (gfx950) kernels behind the reference's Backend hook.

Template: ``MLXBackend`` (``src/ollm/backends/mlx_backend.py:15-96``).
Availability is fail-closed like ``MetalBackend`` (``metal_backend.py:74-163``):
the backend is available only if ``libstrata_hip.so`` loads, a context binds to
a gfx950 device, and the library's self-test envelope reports
``dispatch_success`` with ``numerical_max_error`` under its threshold.
"""
from __future__ import annotations

import json
from typing import Any, Optional

from .base import (Backend, BackendError, ComputeUnit, InferencePhase, OperationKind,
                   RuntimeCapabilities)


class HipBackend(Backend):
    name = "hip"

    def __init__(self):
        self._probe: Optional[dict] = None
        self._probe_error: Optional[str] = None

    def probe(self) -> dict:
        """Run (once) and return the self-test evidence envelope."""
        if self._probe is None and self._probe_error is None:
            try:
                import torch
                if not torch.cuda.is_available():
                    raise BackendError("no HIP device is visible")
                from .. import _abi
                ctx = _abi.context(torch.cuda.current_device())
                envelope = json.loads(ctx.selftest())
                if envelope.get("schema_version") != 1 or envelope.get("backend") != "hip":
                    raise BackendError(f"unexpected self-test envelope: {envelope}")
                if not envelope.get("dispatch_success"):
                    raise BackendError(f"self-test failed: {envelope}")
                self._probe = envelope
            except Exception as exc:  # fail closed
                self._probe_error = str(exc)
        if self._probe is None:
            raise BackendError(f"HIP backend unavailable: {self._probe_error}")
        return self._probe

    def is_available(self) -> bool:
        try:
            self.probe()
            return True
        except BackendError:
            return False

    def resolve_device(self, device_request: Optional[str]) -> Any:
        import torch
        if not self.is_available():
            raise BackendError(f"HIP backend is not available: {self._probe_error}")
        if device_request in (None, "", "auto", "gpu"):
            return torch.device("cuda", torch.cuda.current_device())
        req = device_request.lower()
        if req.startswith("gpu:"):
            req = req[4:]
        if req.isdigit() and int(req) < torch.cuda.device_count():
            return torch.device("cuda", int(req))
        raise BackendError(f"Unsupported HIP device specification: {device_request}")

    def move_model_to_device(self, model: Any, device: Any) -> Any:
        to = getattr(model, "to", None)
        return to(device) if callable(to) else model

    def create_kv_cache(self, cache_dir: Optional[str], stats: Optional[Any],
                        config: Optional[Any] = None, model_id: Optional[str] = None,
                        **kwargs):
        if config is None:
            raise BackendError("config is required to create HIP KV cache")
        from ..kvcache import HipKVCache
        return HipKVCache(config, cache_dir, stats, **kwargs)

    def attention_kernel(self):
        from ..ops import attention
        return attention

    def capabilities(self) -> RuntimeCapabilities:
        return RuntimeCapabilities(
            compute_units=(ComputeUnit.GPU,),
            supported_phases=(InferencePhase.PREFILL, InferencePhase.DECODE),
            supported_operations=(OperationKind.EMBEDDING, OperationKind.NORMALIZATION,
                                  OperationKind.LINEAR, OperationKind.ROPE,
                                  OperationKind.ATTENTION, OperationKind.RESIDUAL,
                                  OperationKind.ACTIVATION, OperationKind.LOGITS),
            supported_dtypes=("bfloat16", "float32"),
            supports_external_kv_cache=True,
            supports_quantized_weights=True,
            supports_dynamic_shapes=True,
        )
