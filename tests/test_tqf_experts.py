"""The .tqf expert index through the C ABI on the host (no GPU): records
decoded from hand-assembled bytes (tests/tqf_fixture.py, the layouts of
format/tqf/records.rs:221-313), lookups as TqfReader::expert
(reader.rs:312-327), and TqfReader::open's validation (reader.rs:170-247):
records beyond the blob, partial tile records, unknown matrices,
superextents outside the container, tile ranges outside the table,
non-partitioning tile tables and per-tile checksum ranges."""
import numpy as np
import pytest

import tqf_fixture as fx
from turboqwenfare_amd import _lib, container


def parts(seed, g=fx.GATE_BYTES, u=fx.GATE_BYTES, d=fx.DOWN_BYTES):
    rng = np.random.default_rng(seed)
    return tuple(rng.integers(0, 256, n, dtype=np.uint8).tobytes() for n in (g, u, d))


EXPERTS = [dict(layer=0, expert=1, parts=parts(1)),
           dict(layer=3, expert=10, parts=parts(2), width=128),
           dict(layer=39, expert=255, parts=parts(3), width=64, flags=1, checksum_index=7)]


def open_table(blob, count, file_len, checksums=64):
    return container.ExpertTable(blob, count, file_len, checksums)


def test_records_decode_and_look_up():
    data, blob, meta = fx.build(EXPERTS)
    with open_table(blob, len(EXPERTS), len(data)) as t:
        assert t.counts() == (3, sum(len(m[1]) for m in meta))
        for (fields, tiles) in meta:
            idx, got = t.lookup(fields[0], fields[1])
            assert (idx.layer, idx.expert, idx.flags, idx.layout_id, idx.file_offset, idx.stored_bytes,
                    idx.tile_first, idx.tile_count, idx.checksum_index) == fields
            assert [(x.matrix, x.tile_id, x.neuron_start, x.neuron_count, x.relative_offset, x.stored_bytes,
                     x.quant_layout_id, x.flags) for x in got] == tiles
            # the spec's placement: 4096-aligned superextents, tiles inside them
            assert idx.file_offset % 4096 == 0
            assert all(x.relative_offset + x.stored_bytes <= idx.stored_bytes for x in got)
            assert idx.file_offset + idx.stored_bytes <= len(data)
        with pytest.raises(_lib.HipError):
            t.lookup(0, 2)


def test_canonical_tiles_keep_three_matrix_boundaries():
    """format/tqf/tests.rs:131-155: the GateUp tile spans gate + up, the Down
    tile follows; the payload slices are gate, up, down -- here also with
    sizes that are not a Q4_K expert's (17, 19, 23 bytes)."""
    for g, u, d in ((fx.GATE_BYTES, fx.GATE_BYTES, fx.DOWN_BYTES), (17, 19, 23)):
        p = parts(9, g, u, d)
        data, blob, _ = fx.build([dict(layer=0, expert=1, parts=p)])
        with open_table(blob, 1, len(data)) as t:
            idx, tiles = t.lookup(0, 1)
            assert [(x.matrix, x.relative_offset, x.stored_bytes) for x in tiles] == [(0, 0, g + u), (1, g + u, d)]
            ext = data[idx.file_offset:idx.file_offset + idx.stored_bytes]
            assert ext[:g] == p[0] and ext[g:g + u] == p[1] and ext[g + u:] == p[2]


def test_encoders_equal_the_hand_assembled_records():
    idx = container.ExpertIndex(5, 300, 1, 2, 8192, 1769472, 12, 10, 44)
    assert container.encode_index_record(idx) == fx.index_record(5, 300, 1, 2, 8192, 1769472, 12, 10, 44)
    tile = container.ExpertTile(1, 9, 256, 256, 1179648, 294912, 2, 0)
    assert container.encode_tile_record(tile) == fx.tile_record(1, 9, 256, 256, 1179648, 294912, 2, 0)


def test_reservations_are_the_stored_and_device_bytes():
    data, blob, _ = fx.build(EXPERTS[:1])
    with open_table(blob, 1, len(data)) as t:
        stored, device = t.reserve_bytes(0, 1)
    lib = _lib.load()
    assert stored == 3 * 589_824
    assert device == 2 * lib.tqf_hip_q4k_weights_bytes_for(512, 2048) + lib.tqf_hip_q4k_weights_bytes_for(2048, 512)


def corrupt(blob: bytes, offset: int, value: bytes) -> bytes:
    b = bytearray(blob)
    b[offset:offset + len(value)] = value
    return bytes(b)


def test_open_rejects_malformed_tables():
    data, blob, meta = fx.build(EXPERTS)
    n, L = len(EXPERTS), len(data)
    tiles0 = n * 32  # first tile record
    cases = {
        "records beyond the blob": (blob, n + 200, L, 64),
        "a partial tile record": (blob[:-5], n, L, 64),
        "an unknown matrix": (corrupt(blob, tiles0, b"\x02"), n, L, 64),
        "a superextent past the container": (blob, n, meta[-1][0][4] + meta[-1][0][5] - 1, 64),
        "a tile range past the table": (corrupt(blob, 20, fx.le(10_000, 4)), n, L, 64),
        "a gap in the tiles": (corrupt(blob, tiles0 + 24 + 8, fx.le(meta[0][1][1][3] + 16, 4)), n, L, 64),
        "tiles short of the extent": (corrupt(blob, 16, fx.le(meta[0][0][5] + 4096, 4)), n, L + 10**7, 64),
        "per-tile checksums past the table": (blob, n, L, 7 + meta[2][0][7]),
    }
    for name, (b, count, flen, sums) in cases.items():
        with pytest.raises(_lib.HipError):
            open_table(b, count, flen, sums)
        # the unmodified table opens with the same sizes
    with open_table(blob, n, L, 8 + meta[2][0][7]) as t:
        assert t.counts()[0] == n


def test_empty_index_opens():
    with open_table(b"", 0, 0) as t:
        assert t.counts() == (0, 0)
