"""The global-index file format (host side, no GPU): round trip, and the
errors a damaged or foreign file raises."""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from suffixgpu_amd.persist import (FORMAT_VERSION, MAGIC, IndexFormatError,
                                   read_index_file, write_index_file)


def _sample(tmp_path):
    rng = np.random.default_rng(0)
    arrays = {"corpus": rng.integers(-2, 1000, size=1001).astype(np.int32),
              "sa": rng.permutation(1001).astype(np.int32),
              "delta": np.zeros(0, np.int32),
              "wide": rng.integers(0, 2 ** 40, size=7).astype(np.int64)}
    meta = {"capacity": 4096, "active_doc_lens": [10, 991], "note": "x"}
    path = tmp_path / "idx.sfx"
    write_index_file(path, meta, arrays)
    return path, meta, arrays


def test_round_trip(tmp_path):
    path, meta, arrays = _sample(tmp_path)
    m2, a2 = read_index_file(path)
    assert m2 == meta
    assert set(a2) == set(arrays)
    for k, v in arrays.items():
        assert a2[k].dtype == v.dtype and a2[k].shape == v.shape
        np.testing.assert_array_equal(a2[k], v)


def test_layout_is_aligned_and_versioned(tmp_path):
    path, _, _ = _sample(tmp_path)
    data = path.read_bytes()
    assert data[:8] == MAGIC
    (hlen,) = struct.unpack("<Q", data[8:16])
    header = json.loads(data[16:16 + hlen])
    assert header["format"] == FORMAT_VERSION
    for e in header["arrays"].values():
        assert e["offset"] % 64 == 0 and e["offset"] >= 16 + hlen


def test_damage_is_detected(tmp_path):
    path, _, _ = _sample(tmp_path)
    data = bytearray(path.read_bytes())
    (hlen,) = struct.unpack("<Q", bytes(data[8:16]))
    header = json.loads(bytes(data[16:16 + hlen]))
    off = header["arrays"]["sa"]["offset"]
    data[off + 5] ^= 0x40
    bad = tmp_path / "bad.sfx"
    bad.write_bytes(bytes(data))
    with pytest.raises(IndexFormatError, match="checksum"):
        read_index_file(bad)
    (tmp_path / "foreign.bin").write_bytes(b"PK\x03\x04" + b"\0" * 64)
    with pytest.raises(IndexFormatError, match="not a suffixgpu_amd"):
        read_index_file(tmp_path / "foreign.bin")
    trunc = tmp_path / "trunc.sfx"
    trunc.write_bytes(bytes(path.read_bytes()[:40]))
    with pytest.raises(IndexFormatError):
        read_index_file(trunc)


def test_other_version_is_refused(tmp_path):
    path, _, _ = _sample(tmp_path)
    data = path.read_bytes()
    (hlen,) = struct.unpack("<Q", data[8:16])
    hdr = data[16:16 + hlen].replace(
        b'"format": %d' % FORMAT_VERSION, b'"format": %d' % (FORMAT_VERSION + 1))
    other = tmp_path / "v2.sfx"
    other.write_bytes(data[:16] + hdr + data[16 + hlen:])
    with pytest.raises(IndexFormatError, match="format"):
        read_index_file(other)
