"""Native evidence lane: strata-hip-probe and the backend's executable mode
(the MetalBackend probe contract, src/ollm/backends/metal_backend.py:74-163)."""
import json
import os
import stat
import subprocess

import pytest

from lokahi_amd.backends.hip_backend import DEFAULT_PROBE, HipBackend


def _fake(tmp_path, payload, status=0):
    p = tmp_path / "probe.sh"
    text = payload if isinstance(payload, str) else json.dumps(payload)
    p.write_text(f"#!/bin/sh\ncat <<'EOF'\n{text}\nEOF\nexit {status}\n")
    p.chmod(p.stat().st_mode | stat.S_IEXEC)
    return str(p)


GOOD = {"schema_version": 1, "backend": "hip", "device_name": "x", "operation": "linear_q4_gemv",
        "dtype": "bf16x_q4w_f32y", "dispatch_success": True, "numerical_max_error": 1e-7,
        "timing": {"average_dispatch_wall_time_ms": 0.01}}


def test_probe_executable_is_built():
    assert DEFAULT_PROBE.is_file() and os.access(DEFAULT_PROBE, os.X_OK)


def test_executable_mode_accepts_a_valid_envelope(tmp_path):
    b = HipBackend(probe_path=_fake(tmp_path, GOOD))
    assert b.is_available() and b.probe()["operation"] == "linear_q4_gemv"


@pytest.mark.parametrize("payload,status,reason", [
    ({**GOOD, "dispatch_success": False, "failure_reason": "no device"}, 1, "no device"),
    ({**GOOD, "backend": "metal"}, 0, "unsupported evidence envelope"),
    ({**GOOD, "numerical_max_error": 0.5}, 0, "capability contract"),
    ("not json", 0, "invalid JSON"),
    (GOOD, 3, "status 3"),
])
def test_executable_mode_fails_closed(tmp_path, payload, status, reason):
    b = HipBackend(probe_path=_fake(tmp_path, payload, status))
    assert not b.is_available()
    with pytest.raises(Exception, match=reason):
        b.probe()


def test_missing_probe_fails_closed(tmp_path):
    b = HipBackend(probe_path=str(tmp_path / "nope"))
    assert not b.is_available()


@pytest.mark.gpu
def test_native_probe_reports_dispatch_and_timing(dev):
    done = subprocess.run([str(DEFAULT_PROBE)], capture_output=True, text=True, timeout=120)
    env = json.loads(done.stdout)
    assert done.returncode == 0 and env["schema_version"] == 1 and env["backend"] == "hip"
    assert env["dispatch_success"] is True and 0 <= env["numerical_max_error"] <= 1e-4
    assert env["timing"]["average_dispatch_wall_time_ms"] > 0
    assert "gfx950" in env["device_name"]
    assert HipBackend(probe_path=str(DEFAULT_PROBE)).is_available()
