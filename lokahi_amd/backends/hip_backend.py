"""The "hip" backend: MI355X (gfx950) kernels behind the reference's Backend hook.

Template: ``MLXBackend`` (``src/ollm/backends/mlx_backend.py:15-96``).
Availability is fail-closed like ``MetalBackend`` (``metal_backend.py:74-163``):
the backend is available only if ``libstrata_hip.so`` loads, a context binds to
a gfx950 device, and the library's self-test envelope reports
``dispatch_success`` with ``numerical_max_error`` under its threshold.

With ``probe_path`` (or ``STRATA_HIP_PROBE``) the evidence comes, as in
``MetalBackend``, from a native executable (``lokahi_amd/_lib/strata-hip-probe``)
run as a child process: one JSON envelope on stdout (schema_version 1,
backend "hip", dispatch_success, device_name, operation, dtype,
numerical_max_error, timing.average_dispatch_wall_time_ms, failure_reason)
and a zero exit status.
"""
from __future__ import annotations

import json
import os
import subprocess
from pathlib import Path
from typing import Any, Optional

from .base import (Backend, BackendError, ComputeUnit, InferencePhase, OperationKind,
                   RuntimeCapabilities)


DEFAULT_PROBE = Path(__file__).resolve().parents[1] / "_lib" / "strata-hip-probe"


class HipBackend(Backend):
    name = "hip"

    def __init__(self, probe_path: Optional[str] = None, timeout_seconds: float = 60.0,
                 maximum_error: float = 1e-4):
        self._probe: Optional[dict] = None
        self._probe_error: Optional[str] = None
        self._probe_path = probe_path or os.environ.get("STRATA_HIP_PROBE")
        self._timeout = timeout_seconds
        self._maximum_error = maximum_error

    def _probe_executable(self) -> dict:
        """Evidence from the native probe (``metal_backend.py:74-163`` contract)."""
        path = Path(self._probe_path).expanduser()
        if not path.is_file() or not os.access(path, os.X_OK):
            raise BackendError("native HIP probe is missing or not executable")
        try:
            done = subprocess.run([str(path)], capture_output=True, check=False, text=True,
                                  timeout=self._timeout)
        except (OSError, subprocess.SubprocessError) as exc:
            raise BackendError(f"native HIP probe failed to execute: {exc}")
        try:
            env = json.loads(done.stdout)
            if not isinstance(env, dict):
                raise ValueError("root JSON value is not an object")
        except (json.JSONDecodeError, ValueError) as exc:
            raise BackendError(f"native HIP probe returned invalid JSON: {exc}")
        if env.get("schema_version") != 1 or env.get("backend") != "hip":
            raise BackendError("native HIP probe returned an unsupported evidence envelope")
        if done.returncode != 0 or env.get("dispatch_success") is not True:
            raise BackendError(env.get("failure_reason")
                               or f"native HIP probe exited with status {done.returncode}")
        err = env.get("numerical_max_error")
        if not isinstance(err, (int, float)) or not 0 <= err <= self._maximum_error:
            raise BackendError("native HIP evidence did not satisfy the capability contract")
        return env

    def probe(self) -> dict:
        """Run (once) and return the self-test evidence envelope."""
        if self._probe is None and self._probe_error is None and self._probe_path:
            try:
                self._probe = self._probe_executable()
            except BackendError as exc:  # fail closed
                self._probe_error = str(exc)
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
