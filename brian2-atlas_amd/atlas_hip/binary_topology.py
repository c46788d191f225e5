"""B2CSR001: source-major static CSR files for empirical connectivity.

A Synapses instance may take its edges from such a file (AtlasIR topology kind
``binary_csr``: edge_count, path, sha256, column_count, initializers mapping each
per-edge parameter to a column).  The layout (binary_topology.rs:24-130,
python/brian2_rust/binary_topology.py:1-16):

    b"B2CSR001", then source, target, edge and column counts as little-endian u64;
    offsets u64[sources + 1] (0, non-decreasing, ending at the edge count);
    targets u32[edges]; then the columns, column-major, f64[columns][edges].

Edge e of source s lies at offsets[s] <= e < offsets[s + 1]; the file order is the
edge order.  ``read_csr`` applies the reference's checks (shape bounds, file length,
SHA-256 of the whole file, header against the document, offsets, targets inside
the population, finite values) and returns the edges.
"""
from __future__ import annotations

import hashlib
import struct
from pathlib import Path

import numpy as np

MAGIC = b"B2CSR001"
HEADER = struct.Struct("<8sQQQQ")
MAX_NEURONS = 1_000_000
MAX_EDGES = 100_000_000
MAX_COLUMNS = 128


class BinaryCsrError(ValueError):
    """A B2CSR001 file that does not match its declaration or is malformed."""


def file_sha256(path) -> str:
    digest = hashlib.sha256()
    with Path(path).open("rb") as stream:
        for chunk in iter(lambda: stream.read(1 << 20), b""):
            digest.update(chunk)
    return digest.hexdigest()


def write_csr(path, sources: int, target_count: int, offsets, targets, columns=()) -> str:
    """Write a B2CSR001 file (offsets u64[sources + 1], targets, columns f64[k][edges]) and
    return its SHA-256."""
    offsets = np.asarray(offsets, "<u8")
    targets = np.asarray(targets, "<u4")
    columns = np.asarray(columns, "<f8").reshape(-1, targets.size) if len(columns) else np.zeros((0, targets.size))
    if offsets.size != sources + 1:
        raise BinaryCsrError("offsets need sources + 1 entries")
    with Path(path).open("wb") as stream:
        stream.write(HEADER.pack(MAGIC, sources, target_count, targets.size, columns.shape[0]))
        stream.write(offsets.tobytes())
        stream.write(targets.tobytes())
        stream.write(np.ascontiguousarray(columns, "<f8").tobytes())
    return file_sha256(path)


def read_csr(path, sources: int, targets: int, edges: int, columns: int, sha256: str):
    """The edges of a declared B2CSR001 file (binary_topology.rs:24-130): source and
    target indices (int64, file order) and the columns (f64[columns, edges])."""
    if not (0 < sources <= MAX_NEURONS and 0 < targets <= MAX_NEURONS and 0 < edges <= MAX_EDGES
            and 0 <= columns <= MAX_COLUMNS):
        raise BinaryCsrError("invalid binary CSR shape")
    path = Path(path)
    expected = HEADER.size + (sources + 1) * 8 + edges * (4 + 8 * columns)
    if path.stat().st_size != expected:
        raise BinaryCsrError("binary CSR file length mismatch")
    if file_sha256(path) != str(sha256).lower():
        raise BinaryCsrError("binary CSR checksum mismatch")
    with path.open("rb") as stream:
        magic, *counts = HEADER.unpack(stream.read(HEADER.size))
    if magic != MAGIC or counts != [sources, targets, edges, columns]:
        raise BinaryCsrError("binary CSR header mismatch")
    offsets = np.fromfile(path, "<u8", sources + 1, offset=HEADER.size)
    if offsets[0] != 0:
        raise BinaryCsrError("binary CSR offsets must start at zero")
    if np.any(offsets[1:] < offsets[:-1]) or np.any(offsets > edges):
        raise BinaryCsrError("invalid binary CSR offsets")
    if offsets[-1] != edges:
        raise BinaryCsrError("binary CSR final offset mismatch")
    target = np.fromfile(path, "<u4", edges, offset=HEADER.size + (sources + 1) * 8)
    if np.any(target >= targets):
        raise BinaryCsrError("binary CSR target outside population")
    values = np.fromfile(path, "<f8", edges * columns,
                         offset=HEADER.size + (sources + 1) * 8 + edges * 4).reshape(columns, edges)
    if not np.all(np.isfinite(values)):
        raise BinaryCsrError("nonfinite binary CSR parameter")
    source = np.repeat(np.arange(sources, dtype=np.int64), np.diff(offsets.astype(np.int64)))
    return source, target.astype(np.int64), values
