"""Strata weight packs: aligned, checksummed containers of opaque tensor bytes.

The on-disk layout is the reference's version-1 format
(``src/ollm/storage/weight_pack.py:21-37, 343-388``), kept byte-compatible so
a pack written by either side reads on the other:

* a 128-byte header: ``<8sIIQQQ32s`` = magic ``STRATAPK``, format version 1,
  header size 128, manifest length, data offset, file size, SHA-256 of the
  manifest bytes; the remaining bytes are zero;
* the manifest right after the header: canonical JSON (sorted keys, ``,``/``:``
  separators, UTF-8) of exactly ``{format, version, alignment, data_offset,
  file_size, tensors}``, each tensor exactly ``{name, offset, length,
  sha256}``;
* payloads from ``data_offset`` on, each at the next multiple of
  ``alignment`` (a power of two in [64, 1 MiB]) after the previous one, zero
  padding between, the file ending with the last payload.

Readers validate everything before a tensor is touched (the checks of
``WeightPackManifest.from_dict``/``_validate_layout``/``_read_manifest``,
lines 99-169, 390-431, with the same exception classes and message
substrings), read one tensor with positioned reads and verify its SHA-256
(235-241), or map it read-only (243-259).  Writers go through a temporary file
beside the target, fsync it and ``os.replace`` it (266-314).

Payloads are opaque: shape and dtype come from the model (``TensorRef``,
``src/ollm/core/tensor_ref.py``).  ``WeightPackGroupTensorStore`` loads a
weight group as the reference's store does (``weight_pack_store.py:59-152``:
every reference checked, then every payload verified, before the decoder sees
any); ``device_decoder`` is this build's decoder, which places each verified
payload in device memory as a tensor of the reference's shape and dtype.
``load_pack_llama`` builds the HIP Llama from a pack whose tensor names are
the MLX checkpoint's, and ``pack_mlx_checkpoint`` writes one.  The GEMV and
GEMM kernels read the MLX q4 layout as it is, so no tensor is re-laid out at
load time.
"""
from __future__ import annotations

import hashlib
import json
import mmap
import os
import re
import struct
import tempfile
import threading
import warnings
from dataclasses import dataclass
from functools import reduce
from operator import mul
from pathlib import Path
from typing import Any, Callable, Dict, Iterable, Mapping, Optional, Sequence, Tuple

import numpy as np

FORMAT_NAME = "strata-weight-pack"
FORMAT_VERSION = 1
DEFAULT_ALIGNMENT = 4096

MAGIC = b"STRATAPK"
HEADER_SIZE = 128
HEADER = struct.Struct("<8sIIQQQ32s")
MAX_MANIFEST_BYTES = 64 << 20
MANIFEST_KEYS = frozenset({"format", "version", "alignment", "data_offset", "file_size", "tensors"})
TENSOR_KEYS = frozenset({"name", "offset", "length", "sha256"})
_HEX64 = re.compile(r"[0-9a-f]{64}")


class WeightPackError(RuntimeError):
    """Any weight-pack failure."""


class WeightPackFormatError(WeightPackError):
    """The pack violates the version-1 structure."""


class WeightPackChecksumError(WeightPackError):
    """Bytes on disk differ from the SHA-256 the manifest records."""


def _is_int(v: Any) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def _align(v: int, a: int) -> int:
    return -(-v // a) * a


def _alignment_ok(v: Any) -> bool:
    return _is_int(v) and 64 <= v <= (1 << 20) and (v & (v - 1)) == 0


def _canonical(obj: Mapping[str, Any]) -> bytes:
    return json.dumps(obj, sort_keys=True, separators=(",", ":"), ensure_ascii=False).encode("utf-8")


def _exact_keys(obj: Mapping[str, Any], want: frozenset, what: str) -> None:
    have = set(obj.keys())
    if have != want:
        raise WeightPackFormatError(
            f"{what} keys are invalid; missing={sorted(want - have)}, unknown={sorted(have - want)}")


@dataclass(frozen=True)
class WeightPackTensor:
    """Where one payload lives in the pack and what its bytes hash to."""

    name: str
    offset: int
    length: int
    sha256: str

    @classmethod
    def from_dict(cls, d: Mapping[str, Any]) -> "WeightPackTensor":
        _exact_keys(d, TENSOR_KEYS, "tensor record")
        name, off, n, digest = d["name"], d["offset"], d["length"], d["sha256"]
        if not isinstance(name, str) or not name:
            raise WeightPackFormatError("tensor name must be a non-empty string")
        if not _is_int(off) or off < 0:
            raise WeightPackFormatError(f"tensor {name!r} offset must be non-negative")
        if not _is_int(n) or n <= 0:
            raise WeightPackFormatError(f"tensor {name!r} length must be positive")
        if not isinstance(digest, str) or not _HEX64.fullmatch(digest):
            raise WeightPackFormatError(
                f"tensor {name!r} sha256 must be 64 lowercase hexadecimal characters")
        return cls(name, off, n, digest)

    def to_dict(self) -> Dict[str, Any]:
        return {"name": self.name, "offset": self.offset, "length": self.length,
                "sha256": self.sha256}


@dataclass(frozen=True)
class WeightPackManifest:
    """A validated version-1 manifest (canonical layout enforced)."""

    alignment: int
    data_offset: int
    file_size: int
    tensors: Tuple[WeightPackTensor, ...]

    @classmethod
    def from_dict(cls, d: Mapping[str, Any]) -> "WeightPackManifest":
        _exact_keys(d, MANIFEST_KEYS, "weight-pack manifest")
        if d["format"] != FORMAT_NAME:
            raise WeightPackFormatError("unsupported weight-pack format name")
        if not _is_int(d["version"]) or d["version"] != FORMAT_VERSION:
            raise WeightPackFormatError(f"unsupported weight-pack version {d['version']!r}")
        a, off, size, recs = d["alignment"], d["data_offset"], d["file_size"], d["tensors"]
        if not _alignment_ok(a):
            raise WeightPackFormatError(
                "alignment must be a power of two between 64 and 1048576 bytes")
        if not _is_int(off) or off < HEADER_SIZE:
            raise WeightPackFormatError("data_offset is before the fixed header")
        if off % a:
            raise WeightPackFormatError("data_offset is not aligned")
        if not _is_int(size) or size <= off:
            raise WeightPackFormatError("file_size must extend beyond data_offset")
        if not isinstance(recs, list) or not recs:
            raise WeightPackFormatError("manifest must contain at least one tensor")
        tensors = []
        for r in recs:
            if not isinstance(r, Mapping):
                raise WeightPackFormatError("each tensor record must be an object")
            tensors.append(WeightPackTensor.from_dict(r))
        m = cls(a, off, size, tuple(tensors))
        m.validate_layout()
        return m

    def validate_layout(self) -> None:
        """Unique names; each payload exactly at the aligned end of the
        previous one; the file ends with the last payload."""
        seen = set()
        end, prev = self.data_offset, None
        for t in self.tensors:
            if t.name in seen:
                raise WeightPackFormatError(f"duplicate tensor name {t.name!r}")
            seen.add(t.name)
            if t.offset < end:
                raise WeightPackFormatError(f"tensor {t.name!r} overlaps tensor {prev!r}")
            want = _align(end, self.alignment)
            if t.offset != want:
                raise WeightPackFormatError(
                    f"tensor {t.name!r} has non-canonical offset {t.offset}; expected {want}")
            if t.offset + t.length > self.file_size:
                raise WeightPackFormatError(f"tensor {t.name!r} extends beyond declared file bounds")
            end, prev = t.offset + t.length, t.name
        if end != self.file_size:
            raise WeightPackFormatError("declared file_size must equal the end of the final tensor")

    def to_dict(self) -> Dict[str, Any]:
        return {"format": FORMAT_NAME, "version": FORMAT_VERSION, "alignment": self.alignment,
                "data_offset": self.data_offset, "file_size": self.file_size,
                "tensors": [t.to_dict() for t in self.tensors]}

    def tensor(self, name: str) -> WeightPackTensor:
        for t in self.tensors:
            if t.name == name:
                return t
        raise KeyError(name)


def _parse_json(raw: bytes) -> Any:
    def no_dupes(pairs):
        out = {}
        for k, v in pairs:
            if k in out:
                raise WeightPackFormatError(f"duplicate JSON key {k!r}")
            out[k] = v
        return out
    try:
        return json.loads(raw.decode("utf-8"), object_pairs_hook=no_dupes)
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise WeightPackFormatError(f"manifest JSON is invalid: {e}") from e


def read_manifest(path: Path) -> WeightPackManifest:
    """Header + manifest of the pack at ``path``, fully validated."""
    try:
        size = path.stat().st_size
        with path.open("rb") as f:
            head = f.read(HEADER_SIZE)
            if len(head) != HEADER_SIZE:
                raise WeightPackFormatError("weight-pack header is truncated")
            magic, ver, hsize, mlen, off, fsize, digest = HEADER.unpack_from(head)
            if magic != MAGIC:
                raise WeightPackFormatError("weight-pack magic is invalid")
            if ver != FORMAT_VERSION:
                raise WeightPackFormatError(f"unsupported header version {ver}")
            if hsize != HEADER_SIZE:
                raise WeightPackFormatError("unsupported fixed header size")
            if any(head[HEADER.size:]):
                raise WeightPackFormatError("weight-pack reserved header bytes are nonzero")
            if not 0 < mlen <= MAX_MANIFEST_BYTES:
                raise WeightPackFormatError("manifest length is invalid")
            if HEADER_SIZE + mlen > off:
                raise WeightPackFormatError("manifest extends into tensor payload area")
            if fsize != size:
                raise WeightPackFormatError("declared file size does not match the physical file")
            raw = f.read(mlen)
            if len(raw) != mlen:
                raise WeightPackFormatError("weight-pack manifest is truncated")
    except OSError as e:
        raise WeightPackError(f"failed to read weight pack {path}: {e}") from e
    if hashlib.sha256(raw).digest() != digest:
        raise WeightPackChecksumError("weight-pack manifest checksum mismatch")
    obj = _parse_json(raw)
    if not isinstance(obj, Mapping):
        raise WeightPackFormatError("weight-pack manifest root must be an object")
    if _canonical(obj) != raw:
        raise WeightPackFormatError("weight-pack manifest JSON is not canonical")
    m = WeightPackManifest.from_dict(obj)
    if m.data_offset != off or m.file_size != fsize:
        raise WeightPackFormatError("header and manifest layout fields disagree")
    return m


def _pread_exact(path: Path, offset: int, length: int) -> bytes:
    try:
        fd = os.open(path, os.O_RDONLY)
        try:
            parts, got = [], 0
            while got < length:
                b = os.pread(fd, length - got, offset + got)
                if not b:
                    break
                parts.append(b)
                got += len(b)
        finally:
            os.close(fd)
    except OSError as e:
        raise WeightPackError(f"failed to read tensor range: {e}") from e
    data = b"".join(parts)
    if len(data) != length:
        raise WeightPackFormatError(
            f"tensor range is truncated: expected {length} bytes, read {len(data)}")
    return data


def _check_digest(t: WeightPackTensor, data) -> None:
    if hashlib.sha256(data).hexdigest() != t.sha256:
        raise WeightPackChecksumError(f"tensor {t.name!r} checksum mismatch")


class MappedTensor:
    """Read-only memoryview of one payload; closing it unmaps the file."""

    def __init__(self, f, mm: mmap.mmap, t: WeightPackTensor):
        self._f, self._mm, self.tensor = f, mm, t
        self._view: Optional[memoryview] = memoryview(mm)[t.offset:t.offset + t.length]

    @property
    def view(self) -> memoryview:
        if self._view is None:
            raise WeightPackError("mapped tensor is already closed")
        return self._view

    def close(self) -> None:
        if self._view is not None:
            self._view.release()
            self._view = None
        try:
            self._mm.close()
        finally:
            self._f.close()

    def __enter__(self) -> memoryview:
        return self.view

    def __exit__(self, *exc) -> None:
        self.close()


class WeightPack:
    """A validated, immutable pack on disk."""

    def __init__(self, path):
        self.path = Path(path)
        self.manifest = read_manifest(self.path)
        self._by_name = {t.name: t for t in self.manifest.tensors}

    def __contains__(self, name: str) -> bool:
        return name in self._by_name

    def tensor_info(self, name: str) -> WeightPackTensor:
        t = self._by_name.get(name)
        if t is None:
            raise KeyError(f"weight pack has no tensor {name!r}")
        return t

    def read_tensor(self, name: str, *, verify_checksum: bool = True) -> bytes:
        """Exactly this tensor's bytes (positioned reads of its range only)."""
        t = self.tensor_info(name)
        data = _pread_exact(self.path, t.offset, t.length)
        if verify_checksum:
            _check_digest(t, data)
        return data

    def mmap_tensor(self, name: str, *, verify_checksum: bool = True) -> MappedTensor:
        t = self.tensor_info(name)
        f = self.path.open("rb")
        try:
            mt = MappedTensor(f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ), t)
        except Exception:
            f.close()
            raise
        if verify_checksum:
            try:
                _check_digest(t, mt.view)
            except Exception:
                mt.close()
                raise
        return mt

    def verify_all(self) -> None:
        for t in self.manifest.tensors:
            self.read_tensor(t.name)


def _payloads(items: Iterable[Tuple[str, Any]]) -> Tuple[Tuple[str, bytes], ...]:
    out, names = [], set()
    for item in items:
        if not isinstance(item, tuple) or len(item) != 2:
            raise TypeError("each tensor must be a (name, bytes-like payload) tuple")
        name, payload = item
        if not isinstance(name, str) or not name:
            raise ValueError("tensor names must be non-empty strings")
        if name in names:
            raise ValueError(f"duplicate tensor name {name!r}")
        names.add(name)
        try:
            data = memoryview(payload).tobytes()
        except (TypeError, ValueError) as e:
            raise TypeError(f"tensor {name!r} payload must be bytes-like") from e
        if not data:
            raise ValueError(f"tensor {name!r} payload must not be empty")
        out.append((name, data))
    if not out:
        raise ValueError("at least one tensor payload is required")
    return tuple(out)


def plan_layout(payloads: Sequence[Tuple[str, bytes]],
                alignment: int) -> Tuple[WeightPackManifest, bytes]:
    """Manifest of ``payloads`` packed canonically.  The data offset depends on
    the manifest's own length, so iterate until it is a fixed point."""
    digests = [hashlib.sha256(p).hexdigest() for _, p in payloads]
    off = _align(HEADER_SIZE, alignment)
    for _ in range(16):
        recs, cur = [], off
        for (name, p), h in zip(payloads, digests):
            cur = _align(cur, alignment)
            recs.append(WeightPackTensor(name, cur, len(p), h))
            cur += len(p)
        m = WeightPackManifest(alignment, off, cur, tuple(recs))
        m.validate_layout()
        raw = _canonical(m.to_dict())
        nxt = _align(HEADER_SIZE + len(raw), alignment)
        if nxt == off:
            return m, raw
        off = nxt
    raise WeightPackError("weight-pack manifest layout did not converge")


def header_bytes(m: WeightPackManifest, raw: bytes) -> bytes:
    h = HEADER.pack(MAGIC, FORMAT_VERSION, HEADER_SIZE, len(raw), m.data_offset, m.file_size,
                    hashlib.sha256(raw).digest())
    return h + bytes(HEADER_SIZE - len(h))


def _zeros(f, n: int) -> None:
    if n < 0:
        raise WeightPackError("internal error: attempted to write negative padding")
    while n:
        k = min(n, 1 << 16)
        f.write(bytes(k))
        n -= k


def write_weight_pack(path, tensors: Iterable[Tuple[str, Any]], *,
                      alignment: int = DEFAULT_ALIGNMENT) -> WeightPackManifest:
    """Create or atomically replace the pack at ``path`` from ordered
    ``(name, bytes-like)`` payloads; on any failure an existing pack stays as
    it was and no temporary file is left behind."""
    if not _alignment_ok(alignment):
        raise ValueError("alignment must be a power of two from 64 to 1048576")
    items = _payloads(tensors)
    m, raw = plan_layout(items, alignment)
    target = Path(path)
    target.parent.mkdir(parents=True, exist_ok=True)
    tmp: Optional[Path] = None
    try:
        fd, name = tempfile.mkstemp(prefix=f".{target.name}.", suffix=".tmp", dir=target.parent)
        tmp = Path(name)
        with os.fdopen(fd, "wb") as f:
            f.write(header_bytes(m, raw))
            f.write(raw)
            _zeros(f, m.data_offset - f.tell())
            for t, (_, p) in zip(m.tensors, items):
                _zeros(f, t.offset - f.tell())
                f.write(p)
            if f.tell() != m.file_size:
                raise WeightPackError("internal error: emitted pack length is inconsistent")
            f.flush()
            os.fsync(f.fileno())
        os.replace(tmp, target)
        tmp = None
        try:
            dfd = os.open(target.parent, os.O_RDONLY)
            try:
                os.fsync(dfd)
            finally:
                os.close(dfd)
        except OSError:
            pass  # directory fsync is not supported everywhere; the file itself was synced
        return m
    finally:
        if tmp is not None:
            try:
                tmp.unlink()
            except FileNotFoundError:
                pass


# ------------------------------------------------------------ weight groups
_DTYPE_BITS = {"bool": 8, "int8": 8, "uint8": 8, "int16": 16, "uint16": 16, "float16": 16,
               "bfloat16": 16, "int32": 32, "uint32": 32, "float32": 32, "int64": 64,
               "uint64": 64, "float64": 64, "int4": 4, "uint4": 4}


@dataclass(frozen=True)
class TensorRef:
    """A tensor's logical name, storage key, shape, dtype and byte size, with
    the fields and rules of ``src/ollm/core/tensor_ref.py:29-71``."""

    name: str
    shape: Tuple[int, ...]
    dtype: str
    storage_key: Optional[str] = None
    storage_nbytes: Optional[int] = None

    def __post_init__(self) -> None:
        if not self.name:
            raise ValueError("tensor name must not be empty")
        if any(d <= 0 for d in self.shape):
            raise ValueError("tensor dimensions must be positive")
        if self.storage_nbytes is not None and self.storage_nbytes <= 0:
            raise ValueError("storage_nbytes must be positive")
        if self.storage_nbytes is None and self.normalized_dtype not in _DTYPE_BITS:
            raise ValueError(f"unknown dtype {self.dtype!r}; provide storage_nbytes explicitly")

    @property
    def normalized_dtype(self) -> str:
        return self.dtype.lower().replace("mlx.core.", "").replace("torch.", "")

    @property
    def element_count(self) -> int:
        return reduce(mul, self.shape, 1)

    @property
    def nbytes(self) -> int:
        if self.storage_nbytes is not None:
            return self.storage_nbytes
        return (self.element_count * _DTYPE_BITS[self.normalized_dtype] + 7) // 8

    @property
    def key(self) -> str:
        return self.storage_key or self.name


@dataclass(frozen=True)
class WeightGroup:
    """Tensors that load together (``src/ollm/core/model_spec.py:11-32``)."""

    group_id: str
    order: int
    tensors: Tuple[TensorRef, ...]
    kind: str = "dense_layer"

    def __post_init__(self) -> None:
        if not self.group_id:
            raise ValueError("group_id must not be empty")
        if self.order < 0:
            raise ValueError("group order must be non-negative")
        if not self.tensors:
            raise ValueError("weight groups must contain at least one tensor")
        names = [t.name for t in self.tensors]
        if len(names) != len(set(names)):
            raise ValueError(f"duplicate tensor name in group {self.group_id!r}")

    @property
    def nbytes(self) -> int:
        return sum(t.nbytes for t in self.tensors)


class WeightPackStoreError(RuntimeError):
    """A weight group cannot be served by this pack."""


@dataclass(frozen=True)
class ImmutableWeightBytes:
    """The default decoded value: the verified payload, unchanged."""

    data: bytes

    def __post_init__(self) -> None:
        if not isinstance(self.data, bytes):
            raise TypeError("ImmutableWeightBytes data must be bytes")

    @property
    def nbytes(self) -> int:
        return len(self.data)

    @property
    def view(self) -> memoryview:
        return memoryview(self.data)

    def __bytes__(self) -> bytes:
        return self.data

    def __len__(self) -> int:
        return len(self.data)

    def __getitem__(self, i):
        return self.data[i]


def immutable_bytes_decoder(tensor_ref, payload: bytes) -> ImmutableWeightBytes:
    del tensor_ref
    return ImmutableWeightBytes(payload)


_TORCH_DTYPES = {"bfloat16": "bfloat16", "float16": "float16", "float32": "float32",
                 "int8": "int8", "uint8": "uint8", "int16": "int16", "int32": "int32",
                 "uint32": "uint32", "int64": "int64"}


def device_decoder(device: int = 0) -> Callable[[Any, bytes], Any]:
    """Decoder that returns each payload as a device tensor of the reference's
    shape and dtype on ``cuda:device`` (uint32 stays uint32: the q4 words)."""
    import torch

    dev = torch.device("cuda", device)

    def decode(tensor_ref, payload: bytes):
        dt = _TORCH_DTYPES.get(tensor_ref.normalized_dtype)
        if dt is None:
            raise WeightPackStoreError(
                f"tensor {tensor_ref.key!r}: dtype {tensor_ref.dtype!r} has no device form")
        with warnings.catch_warnings():  # the bytes are copied to the device at once
            warnings.simplefilter("ignore", UserWarning)
            host = torch.frombuffer(payload, dtype=torch.uint8)
        return host.to(dev).view(getattr(torch, dt)).reshape(tuple(tensor_ref.shape))

    return decode


class WeightPackGroupTensorStore:
    """Checksum-verified weight groups from one pack
    (``src/ollm/storage/weight_pack_store.py:59-152``)."""

    def __init__(self, pack, decoder: Optional[Callable[[Any, bytes], Any]] = None):
        if isinstance(pack, WeightPack):
            self.pack = pack
        elif isinstance(pack, (str, os.PathLike)):
            self.pack = WeightPack(pack)
        else:
            raise TypeError("pack must be a WeightPack or filesystem path")
        if decoder is not None and not callable(decoder):
            raise TypeError("decoder must be callable")
        self.decoder = decoder or immutable_bytes_decoder
        self._closed = False
        self._lock = threading.RLock()

    @property
    def closed(self) -> bool:
        with self._lock:
            return self._closed

    def load_group(self, group) -> Mapping[str, Any]:
        """All tensors of ``group``, decoded; nothing is decoded unless every
        reference exists with the right size and every payload verifies."""
        if not hasattr(group, "tensors") or not hasattr(group, "group_id"):
            raise TypeError("group must be a WeightGroup")
        keys = [t.key for t in group.tensors]
        dupes = sorted({k for k in keys if keys.count(k) > 1})
        if dupes:
            raise WeightPackStoreError(
                f"group {group.group_id!r} contains duplicate storage keys: {dupes}")
        with self._lock:
            if self._closed:
                raise WeightPackStoreError("weight-pack store is closed")
            for ref in group.tensors:
                try:
                    rec = self.pack.tensor_info(ref.key)
                except KeyError as e:
                    raise WeightPackStoreError(
                        f"group {group.group_id!r} references missing packed tensor "
                        f"{ref.key!r}") from e
                if rec.length != ref.nbytes:
                    raise WeightPackStoreError(
                        f"packed tensor {ref.key!r} length {rec.length} does not match "
                        f"TensorRef.nbytes {ref.nbytes}")
            payloads = [(ref, self.pack.read_tensor(ref.key)) for ref in group.tensors]
            return {ref.name: self.decoder(ref, p) for ref, p in payloads}

    def close(self) -> None:
        with self._lock:
            self._closed = True

    def __enter__(self) -> "WeightPackGroupTensorStore":
        with self._lock:
            if self._closed:
                raise WeightPackStoreError("weight-pack store is closed")
        return self

    def __exit__(self, *exc) -> None:
        self.close()


# ------------------------------------------------------------ Llama packs
def pack_mlx_checkpoint(model_dir, pack_path, *, alignment: int = DEFAULT_ALIGNMENT) -> WeightPackManifest:
    """Write every tensor of an MLX 4-bit Llama checkpoint directory into one
    pack, under its checkpoint name, in ``checkpoint_names`` order."""
    from .loader import SafeTensorReader, _files, checkpoint_names, config_from_dict

    model_dir = Path(model_dir)
    cfg = config_from_dict(json.loads((model_dir / "config.json").read_text()))
    where: Dict[str, SafeTensorReader] = {}
    for p in _files(model_dir):
        r = SafeTensorReader(p)
        for k in r.keys():
            where[k] = r
    head = "tied"
    if "lm_head.weight" in where:
        head = "q4" if "lm_head.scales" in where else "bf16"
    names = checkpoint_names(cfg, quantized_embed="model.embed_tokens.scales" in where, head=head)
    missing = [n for n in names if n not in where]
    if missing:
        raise KeyError(f"Tensor '{missing[0]}' not found in the checkpoint")
    return write_weight_pack(pack_path, ((n, where[n].get(n).tobytes()) for n in names),
                             alignment=alignment)


class _PackTensors:
    """The loader's tensor-source interface over a pack: payload bytes plus
    the shape and dtype the model expects (a length mismatch is an error)."""

    def __init__(self, pack: WeightPack):
        self.pack = pack

    def __contains__(self, name: str) -> bool:
        return name in self.pack

    def get(self, name: str, dtype: Optional[str] = None, shape=None) -> np.ndarray:
        from .loader import NP_DTYPES

        if name not in self.pack:
            raise KeyError(f"Tensor '{name}' not found in the weight pack")
        np_dt = np.dtype(NP_DTYPES[dtype or "BF16"])
        want = int(np.prod(shape)) * np_dt.itemsize
        rec = self.pack.tensor_info(name)
        if rec.length != want:
            raise ValueError(f"'{name}' holds {rec.length} bytes, expected {want} "
                             f"({dtype} {list(shape)})")
        return np.frombuffer(self.pack.read_tensor(name), dtype=np_dt).reshape(shape)


def load_pack_llama(pack, config, device: int = 0):
    """``HipLlamaForCausalLM`` from a pack holding the MLX checkpoint's tensor
    names; ``config`` is the checkpoint's config (dict, or path to its JSON)."""
    from .loader import build_llama, config_from_dict

    if not isinstance(config, Mapping):
        config = json.loads(Path(config).read_text())
    cfg = config_from_dict(config)
    if not isinstance(pack, WeightPack):
        pack = WeightPack(pack)
    return build_llama(cfg, _PackTensors(pack), device)
