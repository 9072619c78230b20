"""Strata weight-pack format and group store on the CPU.

The cases follow the reference's ``tests/test_weight_pack.py`` and
``tests/test_weight_pack_store.py`` (round trip, atomic replacement, payload
and truncation detection, strict schema, writer argument checks, group-store
ordering guarantees).  ``test_bytes_match_the_format`` pins the layout itself:
the file is compared byte for byte with a header and manifest spelled out by
hand from the version-1 format (``src/ollm/storage/weight_pack.py:21-37,
343-388``), so a wrong field order, key order, separator or alignment fails.
"""
import hashlib
import json
import struct
from unittest import mock

import numpy as np
import pytest

from lokahi_amd import weight_pack as wp


def _rec(name, offset, length, fill=b"x"):
    return {"name": name, "offset": offset, "length": length,
            "sha256": hashlib.sha256(fill * length).hexdigest()}


def _manifest(tensors, *, alignment=64, data_offset=512, file_size=None, **extra):
    if file_size is None:
        file_size = tensors[-1]["offset"] + tensors[-1]["length"]
    d = {"format": wp.FORMAT_NAME, "version": wp.FORMAT_VERSION, "alignment": alignment,
         "data_offset": data_offset, "file_size": file_size, "tensors": tensors}
    d.update(extra)
    return d


def test_bytes_match_the_format(tmp_path):
    path = tmp_path / "one.strata-pack"
    payload = b"xyz"
    wp.write_weight_pack(path, [("a", payload)], alignment=64)
    digest = hashlib.sha256(payload).hexdigest()
    # 128-byte header + this 217-byte manifest end at 345; the next multiple of 64 is 384
    manifest = ('{"alignment":64,"data_offset":384,"file_size":387,'
                '"format":"strata-weight-pack","tensors":[{"length":3,"name":"a",'
                '"offset":384,"sha256":"' + digest + '"}],"version":1}').encode()
    assert len(manifest) == 217
    header = (b"STRATAPK" + (1).to_bytes(4, "little") + (128).to_bytes(4, "little")
              + len(manifest).to_bytes(8, "little") + (384).to_bytes(8, "little")
              + (387).to_bytes(8, "little") + hashlib.sha256(manifest).digest())
    header += bytes(128 - len(header))
    expected = header + manifest + bytes(384 - 128 - len(manifest)) + payload
    assert path.read_bytes() == expected
    # and a hand-made file in that layout reads back
    other = tmp_path / "hand.strata-pack"
    other.write_bytes(expected)
    assert wp.WeightPack(other).read_tensor("a") == payload


def test_round_trip_exact_reads_and_mmap(tmp_path):
    path = tmp_path / "tiny.strata-pack"
    payloads = [("layer.0", b"abc" * 17), ("layer.1", bytes(range(64)))]
    written = wp.write_weight_pack(path, payloads, alignment=256)
    pack = wp.WeightPack(path)
    assert pack.manifest == written
    assert pack.read_tensor("layer.0") == payloads[0][1]
    assert pack.read_tensor("layer.1") == payloads[1][1]
    assert pack.manifest.file_size == path.stat().st_size
    assert all(t.offset % 256 == 0 for t in pack.manifest.tensors)
    with pack.mmap_tensor("layer.1") as view:
        assert bytes(view) == payloads[1][1] and view.readonly
    pack.verify_all()
    with pytest.raises(KeyError, match="no tensor"):
        pack.tensor_info("missing")


def test_layout_is_canonical_for_many_sizes(tmp_path):
    rng = np.random.default_rng(3)
    for align in (64, 4096):
        items = [(f"t{i}", rng.integers(0, 256, int(n), dtype=np.uint8).tobytes())
                 for i, n in enumerate(rng.integers(1, 9000, 7))]
        path = tmp_path / f"p{align}.strata-pack"
        m = wp.write_weight_pack(path, items, alignment=align)
        end = m.data_offset
        for t, (name, data) in zip(m.tensors, items):
            assert t.offset == -(-end // align) * align and t.length == len(data)
            end = t.offset + t.length
        assert end == m.file_size == path.stat().st_size
        raw = path.read_bytes()
        for t, (_, data) in zip(m.tensors, items):
            assert raw[t.offset:t.offset + t.length] == data
        gaps = bytearray(raw[m.data_offset:])
        for t in m.tensors:  # everything outside the payloads is zero padding
            gaps[t.offset - m.data_offset:t.offset - m.data_offset + t.length] = bytes(t.length)
        assert not any(gaps)


def test_failed_replacement_keeps_existing_pack(tmp_path):
    path = tmp_path / "recoverable.strata-pack"
    wp.write_weight_pack(path, [("original", b"preserved")])
    with mock.patch("lokahi_amd.weight_pack.os.replace",
                    side_effect=OSError("simulated atomic replacement failure")):
        with pytest.raises(OSError, match="simulated atomic"):
            wp.write_weight_pack(path, [("replacement", b"not installed")])
    assert wp.WeightPack(path).read_tensor("original") == b"preserved"
    assert [p.name for p in tmp_path.iterdir()] == [path.name]


def test_payload_corruption_is_detected_on_read(tmp_path):
    path = tmp_path / "corrupt.strata-pack"
    wp.write_weight_pack(path, [("weight", b"immutable bytes")], alignment=64)
    t = wp.WeightPack(path).tensor_info("weight")
    with path.open("r+b") as f:
        f.seek(t.offset + 2)
        f.write(b"X")
    pack = wp.WeightPack(path)
    with pytest.raises(wp.WeightPackChecksumError, match="checksum mismatch"):
        pack.read_tensor("weight")
    with pytest.raises(wp.WeightPackChecksumError, match="checksum mismatch"):
        pack.mmap_tensor("weight")
    assert pack.read_tensor("weight", verify_checksum=False)[2:3] == b"X"


def test_manifest_corruption_is_detected(tmp_path):
    path = tmp_path / "m.strata-pack"
    wp.write_weight_pack(path, [("w", b"abcd")], alignment=64)
    raw = bytearray(path.read_bytes())
    raw[130] ^= 1  # inside the manifest
    path.write_bytes(bytes(raw))
    with pytest.raises(wp.WeightPackChecksumError, match="manifest checksum"):
        wp.WeightPack(path)
    raw[130] ^= 1
    raw[0:8] = b"NOTAPACK"
    path.write_bytes(bytes(raw))
    with pytest.raises(wp.WeightPackFormatError, match="magic"):
        wp.WeightPack(path)
    raw[0:8] = b"STRATAPK"
    raw[100] = 1  # reserved header byte
    path.write_bytes(bytes(raw))
    with pytest.raises(wp.WeightPackFormatError, match="reserved"):
        wp.WeightPack(path)


def test_non_canonical_manifest_is_rejected(tmp_path):
    path = tmp_path / "nc.strata-pack"
    m = wp.write_weight_pack(path, [("w", b"abcd")], alignment=64)
    pretty = json.dumps(m.to_dict(), sort_keys=True).encode()  # ", " and ": " separators
    assert 128 + len(pretty) <= m.data_offset  # still fits before the payload
    raw = bytearray(path.read_bytes())
    raw[128:m.data_offset] = pretty + bytes(m.data_offset - 128 - len(pretty))
    struct.pack_into("<Q", raw, 16, len(pretty))
    raw[40:72] = hashlib.sha256(pretty).digest()
    path.write_bytes(bytes(raw))
    with pytest.raises(wp.WeightPackFormatError, match="not canonical"):
        wp.WeightPack(path)


def test_duplicate_overlap_and_bounds_are_rejected():
    ok = hashlib.sha256(b"x" * 64).hexdigest()
    cases = {
        "duplicate": _manifest([_rec("same", 512, 64),
                                {"name": "same", "offset": 576, "length": 64, "sha256": ok}],
                               file_size=640),
        "overlaps": _manifest([_rec("first", 512, 64), _rec("second", 544, 64)], file_size=608),
        "beyond declared file bounds": _manifest([_rec("outside", 512, 64)], file_size=540),
        "non-canonical offset": _manifest([_rec("first", 512, 64), _rec("gap", 640, 64)]),
        "final tensor": _manifest([_rec("short", 512, 64)], file_size=700),
    }
    for message, payload in cases.items():
        with pytest.raises(wp.WeightPackFormatError, match=message):
            wp.WeightPackManifest.from_dict(payload)


def test_manifest_schema_and_version_are_strict():
    t = _rec("weight", 512, 64)
    with pytest.raises(wp.WeightPackFormatError, match="unsupported.*version"):
        wp.WeightPackManifest.from_dict(_manifest([t], version=wp.FORMAT_VERSION + 1))
    with pytest.raises(wp.WeightPackFormatError, match="unsupported.*version"):
        wp.WeightPackManifest.from_dict(_manifest([t], version=True))
    with pytest.raises(wp.WeightPackFormatError, match="unknown=.*extra"):
        wp.WeightPackManifest.from_dict(_manifest([t], extra="not allowed"))
    with pytest.raises(wp.WeightPackFormatError, match="power of two"):
        wp.WeightPackManifest.from_dict(_manifest([t], alignment=96))
    bad = dict(t, sha256="ABC")
    with pytest.raises(wp.WeightPackFormatError, match="hexadecimal"):
        wp.WeightPackManifest.from_dict(_manifest([bad]))


def test_truncated_file_is_rejected_before_tensor_access(tmp_path):
    path = tmp_path / "truncated.strata-pack"
    wp.write_weight_pack(path, [("weight", bytes(range(32)))], alignment=64)
    path.write_bytes(path.read_bytes()[:-1])
    with pytest.raises(wp.WeightPackFormatError, match="physical file"):
        wp.WeightPack(path)


def test_writer_rejects_invalid_alignment_and_payloads(tmp_path):
    path = tmp_path / "invalid.strata-pack"
    with pytest.raises(ValueError, match="power of two"):
        wp.write_weight_pack(path, [("weight", b"x")], alignment=96)
    with pytest.raises(ValueError, match="must not be empty"):
        wp.write_weight_pack(path, [("weight", b"")])
    with pytest.raises(TypeError, match="bytes-like"):
        wp.write_weight_pack(path, [("weight", [1, 2, 3])])
    with pytest.raises(ValueError, match="duplicate tensor"):
        wp.write_weight_pack(path, [("same", b"a"), ("same", b"b")])
    assert not path.exists()


def _group(i, key, *, nbytes=4, name="weight"):
    return wp.WeightGroup(f"layer.{i}", i, (wp.TensorRef(name, (nbytes,), "uint8", key, nbytes),))


def test_store_checks_sizes_and_keys_before_decoding(tmp_path):
    path = tmp_path / "s.strata-pack"
    wp.write_weight_pack(path, [("packed.weight", b"abc"), ("shared", b"abcd")], alignment=64)
    calls = []
    store = wp.WeightPackGroupTensorStore(path, decoder=lambda r, p: calls.append(r) or p)
    with pytest.raises(wp.WeightPackStoreError, match="TensorRef.nbytes"):
        store.load_group(_group(0, "packed.weight", nbytes=4))
    with pytest.raises(wp.WeightPackStoreError, match="missing packed tensor"):
        store.load_group(_group(0, "nope"))
    dup = wp.WeightGroup("d", 0, (wp.TensorRef("first", (4,), "uint8", "shared"),
                                  wp.TensorRef("second", (4,), "uint8", "shared")))
    with pytest.raises(wp.WeightPackStoreError, match="duplicate storage keys"):
        store.load_group(dup)
    assert calls == []
    store.close()


def test_store_checksum_failure_decodes_nothing(tmp_path):
    path = tmp_path / "c.strata-pack"
    wp.write_weight_pack(path, [("good", b"good"), ("bad", b"bad!")], alignment=64)
    rec = wp.WeightPack(path).tensor_info("bad")
    with path.open("r+b") as f:
        f.seek(rec.offset)
        f.write(b"X")
    calls = []
    store = wp.WeightPackGroupTensorStore(path, decoder=lambda r, p: calls.append(r) or p)
    g = wp.WeightGroup("g", 0, (wp.TensorRef("a", (4,), "uint8", "good"),
                                wp.TensorRef("b", (4,), "uint8", "bad")))
    with pytest.raises(wp.WeightPackChecksumError):
        store.load_group(g)
    assert calls == []


def test_store_decoder_gets_exact_bytes_and_close_is_final(tmp_path):
    path = tmp_path / "decoder.strata-pack"
    payload = b"decoder input"
    wp.write_weight_pack(path, [("packed", payload)], alignment=64)
    seen = []

    def decoder(ref, data):
        seen.append((ref.key, isinstance(data, bytes), memoryview(data).readonly,
                     hashlib.sha256(data).hexdigest()))
        return wp.ImmutableWeightBytes(data)

    store = wp.WeightPackGroupTensorStore(path, decoder=decoder)
    group = _group(0, "packed", nbytes=len(payload), name="decoded")
    assert bytes(store.load_group(group)["decoded"]) == payload
    assert seen == [("packed", True, True, hashlib.sha256(payload).hexdigest())]
    with wp.WeightPackGroupTensorStore(path) as s2:  # default decoder: immutable bytes
        v = s2.load_group(group)["decoded"]
        assert isinstance(v, wp.ImmutableWeightBytes) and v.nbytes == len(payload)
    store.close()
    assert store.closed
    with pytest.raises(wp.WeightPackStoreError, match="closed"):
        store.load_group(group)


def test_tensor_ref_sizes():
    assert wp.TensorRef("q", (4096, 512), "uint32").nbytes == 4096 * 512 * 4
    assert wp.TensorRef("s", (3, 5), "torch.bfloat16").nbytes == 30
    assert wp.TensorRef("n", (7,), "int4").nbytes == 4
    with pytest.raises(ValueError, match="unknown dtype"):
        wp.TensorRef("x", (1,), "weird")
    with pytest.raises(ValueError, match="duplicate tensor name"):
        wp.WeightGroup("g", 0, (wp.TensorRef("a", (1,), "uint8"), wp.TensorRef("a", (1,), "uint8")))


def test_mlx_checkpoint_packs_under_its_names(tmp_path):
    from lokahi_amd import loader
    from oracle import llama as oll
    from tests import mlx_checkpoint
    cfg = oll.Config(vocab_size=96, hidden_size=128, intermediate_size=192, num_hidden_layers=2,
                     num_attention_heads=2, num_key_value_heads=1, rms_norm_eps=1e-5,
                     rope_theta=10000.0)
    hw = oll.random_weights(cfg, seed=4, std=0.05)
    mlx_checkpoint.export(tmp_path / "ckpt", cfg, hw, embed="q4", head="bf16")
    m = wp.pack_mlx_checkpoint(tmp_path / "ckpt", tmp_path / "model.strata-pack")
    lcfg = loader.config_from_dict(json.loads((tmp_path / "ckpt" / "config.json").read_text()))
    names = loader.checkpoint_names(lcfg, quantized_embed=True, head="bf16")
    assert [t.name for t in m.tensors] == names
    pack = wp.WeightPack(tmp_path / "model.strata-pack")
    src = loader._Tensors(loader.SafeTensorReader(p) for p in loader._files(tmp_path / "ckpt"))
    pt = wp._PackTensors(pack)
    for n in names:
        a = src.get(n)
        dt = "U32" if a.dtype == np.uint32 else "BF16"
        assert np.array_equal(pt.get(n, dt, a.shape), a)
    with pytest.raises(ValueError, match="expected"):
        pt.get("model.norm.weight", "BF16", (64,))
