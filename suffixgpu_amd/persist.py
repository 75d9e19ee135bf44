"""On-disk format of a global index (corpus, suffix array, delta, document
lengths), so a drafter can be restarted without re-ingesting its history.

The reference keeps its index in memory only (its README lists
persistence as future work, README.md:212-217); this format is this
library's own.  One file:

    bytes 0..7     magic b"SFXIDX\\x00\\x01" (format version 1)
    bytes 8..15    little-endian u64: length J of the JSON header
    bytes 16..     J bytes of UTF-8 JSON, then zero padding to 64 bytes
    arrays         each array's raw little-endian bytes at the offset the
                   header names, 64-byte aligned

The header holds the index geometry, the host state (active / delta
lengths and document lengths) and, per array, dtype, shape, offset and a
SHA-256 of its bytes, checked on load.  The SA key rows are not stored:
they are a function of corpus and SA and are rebuilt on load.
"""

from __future__ import annotations

import hashlib
import json
import struct
from pathlib import Path

import numpy as np

MAGIC = b"SFXIDX\x00\x01"
FORMAT_VERSION = 1
_ALIGN = 64


class IndexFormatError(ValueError):
    pass


def _pad(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


def write_index_file(path: str | Path, meta: dict,
                     arrays: dict[str, np.ndarray]) -> None:
    """Write ``meta`` (JSON-serialisable) and the named arrays."""
    entries = {}
    blobs = []
    for name, arr in arrays.items():
        a = np.ascontiguousarray(arr)
        if a.dtype.byteorder == ">":
            a = a.astype(a.dtype.newbyteorder("<"))
        raw = a.tobytes()
        entries[name] = {"dtype": a.dtype.str, "shape": list(a.shape),
                         "nbytes": len(raw),
                         "sha256": hashlib.sha256(raw).hexdigest()}
        blobs.append((name, raw))
    # offsets depend on the header length, which depends on the offsets:
    # fix the header size first with placeholder offsets of full width
    for name in entries:
        entries[name]["offset"] = 10 ** 15
    header = {"format": FORMAT_VERSION, "meta": meta, "arrays": entries}
    hlen = len(json.dumps(header, sort_keys=True).encode())
    off = _pad(16 + hlen)
    for name, raw in blobs:
        entries[name]["offset"] = off
        off = _pad(off + len(raw))
    hbytes = json.dumps(header, sort_keys=True).encode()
    hbytes = hbytes + b" " * (hlen - len(hbytes))
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<Q", len(hbytes)))
        f.write(hbytes)
        for name, raw in blobs:
            f.seek(entries[name]["offset"])
            f.write(raw)
        f.truncate(off)


def read_index_file(path: str | Path) -> tuple[dict, dict[str, np.ndarray]]:
    """Inverse of :func:`write_index_file`; raises IndexFormatError on a
    bad magic, version, layout or checksum."""
    data = Path(path).read_bytes()
    if len(data) < 16 or data[:8] != MAGIC:
        raise IndexFormatError(f"{path}: not a suffixgpu_amd index file")
    (hlen,) = struct.unpack("<Q", data[8:16])
    if 16 + hlen > len(data):
        raise IndexFormatError(f"{path}: truncated header")
    try:
        header = json.loads(data[16:16 + hlen].decode())
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise IndexFormatError(f"{path}: bad header ({e})") from e
    if header.get("format") != FORMAT_VERSION:
        raise IndexFormatError(
            f"{path}: format {header.get('format')} (expected "
            f"{FORMAT_VERSION})")
    arrays = {}
    for name, e in header["arrays"].items():
        off, nb = int(e["offset"]), int(e["nbytes"])
        if off < 16 + hlen or off + nb > len(data):
            raise IndexFormatError(f"{path}: array {name} out of bounds")
        raw = data[off:off + nb]
        if hashlib.sha256(raw).hexdigest() != e["sha256"]:
            raise IndexFormatError(f"{path}: checksum mismatch in {name}")
        a = np.frombuffer(raw, dtype=np.dtype(e["dtype"]))
        arrays[name] = a.reshape(e["shape"]).copy()
    return header["meta"], arrays
