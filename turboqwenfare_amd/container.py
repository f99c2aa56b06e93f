"""Routed-expert superextents of a ``.tqf`` container, through the C ABI.

``ExpertTable`` binds ``tqf_hip_expert_table_*`` / ``tqf_hip_expert_lookup``
(the expert-index half of ``TqfReader``, ``format/tqf/reader.rs:170-247,
312-327``); ``reserve_bytes`` and ``upload`` bind the staging path of
``Qwen36WeightLoader::expert_stored_bytes`` / ``load_expert``
(``model/qwen36/weights.rs:1387-1444``) with ``stage_expert_values``
(``experts/mod.rs:512-545``). The caller supplies the container region (a
``bytes``-like object, e.g. an ``mmap`` of the file); reading the file and
verifying the checksum table's BLAKE3 digests stay on its side.

``encode_index_record`` / ``encode_tile_record`` write the on-disk records
(``format/tqf/records.rs:221-313``): containers for tests and tools.
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass

import numpy as np

from . import _lib

MATRIX_GATE_UP = 0
MATRIX_DOWN = 1
LAYOUT_Q4_K = 2  # TQF_QUANT_PASSTHROUGH_Q4_K
FLAG_TILE_CHECKSUMS = 1
SUPEREXTENT_ALIGNMENT = 4096


class _Index(C.Structure):
    _fields_ = [("layer", C.c_uint8), ("expert", C.c_uint16), ("flags", C.c_uint16),
                ("layout_id", C.c_uint16), ("file_offset", C.c_uint64), ("stored_bytes", C.c_uint32),
                ("tile_first", C.c_uint32), ("tile_count", C.c_uint16), ("checksum_index", C.c_uint32)]


class _Tile(C.Structure):
    _fields_ = [("matrix", C.c_uint8), ("tile_id", C.c_uint16), ("neuron_start", C.c_uint16),
                ("neuron_count", C.c_uint16), ("relative_offset", C.c_uint32), ("stored_bytes", C.c_uint32),
                ("quant_layout_id", C.c_uint16), ("flags", C.c_uint16)]


@dataclass(frozen=True)
class ExpertIndex:
    layer: int
    expert: int
    flags: int
    layout_id: int
    file_offset: int
    stored_bytes: int
    tile_first: int
    tile_count: int
    checksum_index: int


@dataclass(frozen=True)
class ExpertTile:
    matrix: int
    tile_id: int
    neuron_start: int
    neuron_count: int
    relative_offset: int
    stored_bytes: int
    quant_layout_id: int
    flags: int


def encode_index_record(r: ExpertIndex) -> bytes:
    """ExpertIndexRecord::encode (records.rs:247-259), 32 bytes."""
    return struct.pack("<BxHHHQIIHxxI", r.layer, r.expert, r.flags, r.layout_id, r.file_offset,
                       r.stored_bytes, r.tile_first, r.tile_count, r.checksum_index)


def encode_tile_record(t: ExpertTile) -> bytes:
    """ExpertTileRecord::encode (records.rs:286-297), 24 bytes."""
    return struct.pack("<BxHHHIIHH4x", t.matrix, t.tile_id, t.neuron_start, t.neuron_count,
                       t.relative_offset, t.stored_bytes, t.quant_layout_id, t.flags)


class ExpertTable:
    """An opened expert index; ``ctx`` may be None (host-only calls)."""

    def __init__(self, blob: bytes, expert_count: int, file_len: int, checksum_entries: int = 0,
                 ctx=None):
        self.lib = _lib.load()
        self.ctx = ctx
        buf = C.create_string_buffer(bytes(blob), len(blob))
        h = C.c_void_p()
        rc = self.lib.tqf_hip_expert_table_open(ctx, buf, len(blob), expert_count, file_len,
                                                checksum_entries, C.byref(h))
        if rc:
            raise _lib.HipError(rc, self._msg("expert table"))
        self.handle = h

    def _msg(self, what: str) -> str:
        if self.ctx is None:
            return what
        return what + ": " + self.lib.tqf_hip_last_error(self.ctx).decode()

    def counts(self) -> tuple[int, int]:
        e, t = C.c_uint64(), C.c_uint64()
        self.lib.tqf_hip_expert_table_counts(self.handle, C.byref(e), C.byref(t))
        return e.value, t.value

    def lookup(self, layer: int, expert: int) -> tuple[ExpertIndex, list]:
        """TqfReader::expert(layer, expert)."""
        n = C.c_size_t()
        rc = self.lib.tqf_hip_expert_lookup(self.ctx, self.handle, layer, expert, None, None, 0, C.byref(n))
        if rc:
            raise _lib.HipError(rc, self._msg("expert lookup"))
        idx = _Index()
        tiles = (_Tile * max(n.value, 1))()
        rc = self.lib.tqf_hip_expert_lookup(self.ctx, self.handle, layer, expert, C.byref(idx), tiles,
                                            n.value, C.byref(n))
        if rc:
            raise _lib.HipError(rc, self._msg("expert lookup"))
        index = ExpertIndex(*(getattr(idx, f) for f, _ in _Index._fields_))
        return index, [ExpertTile(*(getattr(tiles[i], f) for f, _ in _Tile._fields_)) for i in range(n.value)]

    def reserve_bytes(self, layer: int, expert: int) -> tuple[int, int]:
        """(host staging bytes of the superextent, device bytes of its uploads)."""
        s, d = C.c_uint64(), C.c_uint64()
        rc = self.lib.tqf_hip_expert_reserve_bytes(self.ctx, self.handle, layer, expert, C.byref(s), C.byref(d))
        if rc:
            raise _lib.HipError(rc, self._msg("expert reservation"))
        return s.value, d.value

    def upload(self, be, layer: int, expert: int, container) -> tuple:
        """load_expert + stage_expert_values: three Q4_K weight handles."""
        from .backend import Q4KWeights

        buf = np.frombuffer(container, dtype=np.uint8)
        g, u, d = C.c_void_p(), C.c_void_p(), C.c_void_p()
        rc = self.lib.tqf_hip_expert_upload(be.ctx, self.handle, layer, expert,
                                            buf.ctypes.data_as(C.c_void_p), buf.nbytes, C.byref(g), C.byref(u),
                                            C.byref(d))
        if rc:
            raise _lib.HipError(rc, be.lib.tqf_hip_last_error(be.ctx).decode())
        return (Q4KWeights(g.value, 512, 2048), Q4KWeights(u.value, 512, 2048),
                Q4KWeights(d.value, 2048, 512))

    def close(self) -> None:
        if self.handle:
            self.lib.tqf_hip_expert_table_free(self.ctx, self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
