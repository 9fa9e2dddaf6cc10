"""Brute-force vector search on the GPU, mirroring go-semantica's search/brute
package (builder.go, index.go, storage.go): Builder -> Index ->
search_vector / search_normalized, plus Serializer.

The index lives in HBM (libsemantica_gpu.so, k_search.hip); scores are
bit-identical to the reference's amd64 dot products and the top-k is the
reference's selection, ties included.  `search_batch` runs many queries in
one call.
"""
from __future__ import annotations

import ctypes
from collections import namedtuple

import numpy as np

from . import _lib

# brute.QuantizationMode (search/brute/quant.go:8-15)
QUANTIZE_FLOAT32, QUANTIZE_INT8, QUANTIZE_INT16 = 0, 1, 2

# search.Result (search/search.go:8-11)
Result = namedtuple("Result", "id distance")


def _err(msg: str):
    return _lib.SemanticaError(_lib.SG_ERR_INVALID, msg)


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


class Builder:
    """brute.NewBuilder(WithDimension(dimension), WithQuantization(quantization))
    (builder.go:40-50).  Vectors are collected on the host; build() normalizes,
    quantizes and uploads them on the GPU."""

    def __init__(self, ctx, dimension: int = 0, quantization: int = QUANTIZE_INT8):
        self.ctx = ctx
        self.dimension = dimension
        self.quantization = quantization
        self._ids: list[int] = []
        self._vecs: list[np.ndarray] = []
        self._seen: set[int] = set()
        self._built = False

    def add_vector(self, id: int, vec) -> None:
        """AddVector (builder.go:52-75)."""
        if self._built:
            raise _err("brute: builder already built")
        if id in self._seen:
            raise _err(f"brute: duplicate id {id}")
        v = np.asarray(vec, np.float32).reshape(-1)
        if self.dimension == 0:
            self.dimension = v.size
        if v.size != self.dimension:
            raise _err(f"brute: vector dimension mismatch: got {v.size} want {self.dimension}")
        self._ids.append(int(id))
        self._vecs.append(v.copy())
        self._seen.add(int(id))

    def add_vectors(self, ids, vecs) -> None:
        """AddVector for each (ids[i], vecs[i]) of an [n, dim] array."""
        ids = np.asarray(ids).reshape(-1)
        vecs = np.asarray(vecs, np.float32)
        if vecs.ndim != 2 or vecs.shape[0] != ids.size:
            raise _err("brute: add_vectors needs ids[n] and vecs[n, dim]")
        if self._built:
            raise _err("brute: builder already built")
        if self.dimension == 0:
            self.dimension = vecs.shape[1]
        if vecs.shape[1] != self.dimension:
            raise _err(f"brute: vector dimension mismatch: got {vecs.shape[1]} want {self.dimension}")
        for i in ids.tolist():
            if i in self._seen:
                raise _err(f"brute: duplicate id {i}")
            self._seen.add(i)
        self._ids.extend(int(i) for i in ids.tolist())
        self._vecs.append(np.array(vecs, np.float32, copy=True))

    def build(self) -> "Index":
        """Build (builder.go:78-128)."""
        if self._built:
            raise _err("brute: builder already built")
        if not self._vecs:
            raise _err("brute: no vectors added")
        ids = np.asarray(self._ids, np.int32)
        vecs = np.ascontiguousarray(np.concatenate([v.reshape(-1, self.dimension) for v in self._vecs]), np.float32)
        idx = Index._build(self.ctx, self.dimension, self.quantization, ids, vecs)
        self._built = True
        return idx


class Index:
    """brute.Index (index.go:11-25) held on the GPU."""

    def __init__(self, ctx, handle):
        self.ctx = ctx
        self.lib = _lib.load()
        self.handle = handle
        d, n, q = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        _lib.check(self.lib.sg_index_info(handle, ctypes.byref(d), ctypes.byref(n), ctypes.byref(q)))
        self._dim, self._count, self.quantization = d.value, n.value, q.value

    @classmethod
    def _build(cls, ctx, dim, quantization, ids: np.ndarray, vecs: np.ndarray) -> "Index":
        h = ctypes.c_void_p()
        _lib.check(_lib.load().sg_index_build(ctx.handle, dim, quantization, _ptr(ids), _ptr(vecs), ids.size,
                                              ctypes.byref(h)))
        return cls(ctx, h)

    @classmethod
    def from_device(cls, ctx, ids, d_vectors_ptr: int, dim: int, n: int, quantization: int = QUANTIZE_INT8,
                    ld: int = 0, stream: int = 0) -> "Index":
        """Build from vectors already in HBM (e.g. embeddings left there by
        Model.forward_device): same normalization and quantization as Builder."""
        ids = np.ascontiguousarray(ids, np.int32)
        h = ctypes.c_void_p()
        _lib.check(_lib.load().sg_index_build_device(ctx.handle, dim, quantization, _ptr(ids),
                                                     ctypes.c_void_p(d_vectors_ptr), ld or dim, n,
                                                     ctypes.c_void_p(stream) if stream else None, ctypes.byref(h)))
        return cls(ctx, h)

    def close(self):
        if self.handle:
            self.lib.sg_index_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def dimension(self) -> int:
        """Dimension (index.go:149-150)."""
        return self._dim

    def count(self) -> int:
        """Count (index.go:152-153)."""
        return self._count

    def vector(self, id: int):
        """Vector (index.go:155-172): (dequantized copy, True) or (None, False)."""
        out = np.empty(self._dim, np.float32)
        if self.lib.sg_index_vector(self.handle, int(id), _ptr(out)) != _lib.SG_OK:
            return None, False
        return out, True

    def for_each(self, fn) -> None:
        """ForEach (index.go:174-190): fn(id, dequantized copy) in stored order."""
        raw = Serializer().serialize(self)
        ids = np.frombuffer(raw, np.int32, self._count, 20)
        dt, scale = {QUANTIZE_FLOAT32: (np.float32, None), QUANTIZE_INT8: (np.int8, np.float32(1.0 / 127.0)),
                     QUANTIZE_INT16: (np.int16, np.float32(1.0 / 32767.0))}[self.quantization]
        rows = np.frombuffer(raw, dt, self._count * self._dim, 20 + 4 * self._count).reshape(self._count, self._dim)
        for i, r in zip(ids, rows):  # dequantizeInt8/16 (quant.go:43-55)
            fn(int(i), r.astype(np.float32) * scale if scale is not None else r.copy())

    def search_batch(self, queries, top_k: int, normalized: bool = False):
        """Many queries in one call: (ids [n, k], distances [n, k], n_found [n])
        with k = top_k; rows are SearchVector's (normalized=False) or
        SearchNormalized's results."""
        q = np.ascontiguousarray(queries, np.float32)
        if q.ndim == 1:
            q = q.reshape(1, -1)
        if q.shape[1] != self._dim:
            raise _err(f"brute: query dimension mismatch: got {q.shape[1]} want {self._dim}")
        n = q.shape[0]
        k = max(top_k, 1)
        ids = np.zeros((n, k), np.int32)
        dist = np.zeros((n, k), np.float32)
        found = np.zeros(n, np.int32)
        _lib.check(self.lib.sg_index_search(self.handle, _ptr(q), n, top_k, 0 if normalized else 1, _ptr(ids),
                                            _ptr(dist), _ptr(found), None))
        return ids, dist, found

    def _search(self, vec, top_k: int, normalized: bool):
        if top_k <= 0:
            raise _err("brute: topK must be positive")
        v = np.asarray(vec, np.float32).reshape(-1)
        if v.size != self._dim:
            raise _err(f"brute: query dimension mismatch: got {v.size} want {self._dim}")
        ids, dist, found = self.search_batch(v.reshape(1, -1), top_k, normalized)
        return [Result(int(ids[0, j]), float(dist[0, j])) for j in range(found[0])]

    def search_vector(self, vec, top_k: int):
        """SearchVector (index.go:27-41): the query is L2-normalized first."""
        return self._search(vec, top_k, False)

    def search_normalized(self, vec, top_k: int):
        """SearchNormalized (index.go:43-51): the query is used as given."""
        return self._search(vec, top_k, True)


class Serializer:
    """brute.Serializer (storage.go:29-45)."""

    def serialize(self, index: Index) -> bytes:
        lib = _lib.load()
        size = ctypes.c_size_t()
        _lib.check(lib.sg_index_serialize(index.handle, None, 0, ctypes.byref(size)))
        buf = ctypes.create_string_buffer(size.value)
        _lib.check(lib.sg_index_serialize(index.handle, buf, size.value, ctypes.byref(size)))
        return buf.raw[:size.value]

    def deserialize(self, ctx, data: bytes) -> Index:
        lib = _lib.load()
        data = bytes(data)
        buf = ctypes.create_string_buffer(data, len(data)) if data else None
        h = ctypes.c_void_p()
        _lib.check(lib.sg_index_deserialize(ctx.handle, buf, len(data), ctypes.byref(h)))
        return Index(ctx, h)
