"""CPU-side checks of the C ABI library and the backend registry."""
import ctypes as C
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "strata_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(strata_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from lokahi_amd import _abi
    if not _abi.lib_path().exists():
        pytest.skip("library not built")
    lib = C.CDLL(str(_abi.lib_path()))
    syms = declared_symbols()
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, f"missing exports: {missing}"
    assert set(syms) == set(_abi.EXPORTED), "ctypes signatures out of sync with the header"
    lib.strata_abi_version.restype = C.c_int
    assert lib.strata_abi_version() == 2


def test_loader_declares_signatures_and_fails_loudly_on_missing_library(tmp_path):
    from lokahi_amd import _abi
    with pytest.raises(OSError):
        _abi.load(tmp_path / "nope.so")


def test_registry_mirrors_reference_behaviour():
    from lokahi_amd.backends import (BackendError, HipBackend, get_backend, list_backends,
                                     register_backend, select_backend)
    from lokahi_amd.backends.base import _route_device
    assert list_backends() == ("hip",)
    assert get_backend("hip").name == "hip"
    assert _route_device(None) == ("hip", None)
    assert _route_device("hip:0") == ("hip", "0")
    assert _route_device("cpu") == ("hip", "cpu")
    # base.py:83-105 semantics: a bare registered name, an empty device part,
    # and an unregistered prefix kept whole as the default backend's request
    assert _route_device("hip") == ("hip", None)
    assert _route_device("hip:") == ("hip", None)
    assert _route_device("cuda:1") == ("hip", "cuda:1")
    with pytest.raises(BackendError):
        register_backend(HipBackend())
    with pytest.raises(BackendError):
        get_backend("unknown")
    with pytest.raises(BackendError):
        _route_device(3)
    if not torch.cuda.is_available():
        # fail closed without a device
        assert not get_backend("hip").is_available()
        with pytest.raises(BackendError):
            select_backend("hip:0")


def test_capabilities_declare_the_hot_path():
    from lokahi_amd.backends import InferencePhase, OperationKind, get_backend
    caps = get_backend("hip").capabilities()
    assert set(caps.supported_phases) == {InferencePhase.PREFILL, InferencePhase.DECODE}
    for op in (OperationKind.LINEAR, OperationKind.ROPE, OperationKind.ATTENTION):
        assert op in caps.supported_operations
    assert caps.supports_quantized_weights and caps.supports_external_kv_cache
    assert set(caps.supported_dtypes) == {"bfloat16", "float32"}
