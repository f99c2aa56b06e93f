"""Hand-assembled .tqf containers for the expert-superextent tests.

The records are written byte by byte from the layouts of
format/tqf/records.rs:221-313 (ExpertIndexRecord::encode, ExpertTileRecord::
encode) -- not through the package's encoder -- so the tests compare the
library's decoding with an independent encoding.  Superextents are placed as
the writer places them (format/tqf/writer.rs:484-485: the next 4096-aligned
offset), with the tile tables of tiling.rs:tile_plan: the canonical layout
(one GateUp tile over gate+up, one Down tile) or neuron-width tiles (gate and
up in rows of `width`, down in columns of 256 or 512)."""
from __future__ import annotations

GATE_BYTES = 512 * 8 * 144   # Q4_K [512 x 2048]
DOWN_BYTES = 2048 * 2 * 144  # Q4_K [2048 x 512]


def le(v: int, n: int) -> bytes:
    return int(v).to_bytes(n, "little")


def index_record(layer, expert, flags, layout_id, file_offset, stored_bytes, tile_first, tile_count,
                 checksum_index) -> bytes:
    b = bytearray(32)
    b[0] = layer
    b[2:4] = le(expert, 2)
    b[4:6] = le(flags, 2)
    b[6:8] = le(layout_id, 2)
    b[8:16] = le(file_offset, 8)
    b[16:20] = le(stored_bytes, 4)
    b[20:24] = le(tile_first, 4)
    b[24:26] = le(tile_count, 2)
    b[28:32] = le(checksum_index, 4)
    return bytes(b)


def tile_record(matrix, tile_id, neuron_start, neuron_count, relative_offset, stored_bytes,
                quant_layout_id, flags=0) -> bytes:
    b = bytearray(24)
    b[0] = matrix
    b[2:4] = le(tile_id, 2)
    b[4:6] = le(neuron_start, 2)
    b[6:8] = le(neuron_count, 2)
    b[8:12] = le(relative_offset, 4)
    b[12:16] = le(stored_bytes, 4)
    b[16:18] = le(quant_layout_id, 2)
    b[18:20] = le(flags, 2)
    return bytes(b)


def tile_plan(gate: int, up: int, down: int, width=None):
    """(matrix, neuron_start, neuron_count, relative_offset, stored_bytes) per
    tile: width None is the canonical two-tile layout; width w tiles gate and
    up by w rows (w * 8 Q4_K blocks of 144 B) and down by max(w, 256) columns."""
    if width is None:
        return [(0, 0, 0, 0, gate + up), (1, 0, 0, gate + up, down)]
    out, off = [], 0
    gt = width * 8 * 144
    for size in (gate, up):
        for i in range(size // gt):
            out.append((0, i * width, width, off, gt))
            off += gt
    dw = max(width, 256)
    dt = 2048 * (dw // 256) * 144
    for i in range(down // dt):
        out.append((1, i * dw, dw, off, dt))
        off += dt
    return out


def build(experts, header_bytes: int = 4096, layout_id: int = 2):
    """experts: dicts with layer, expert, parts (gate, up, down bytes) and
    optional width, flags, checksum_index, layout_id, tile_layout_id.
    Returns (container bytes, expert-index blob, [(index fields, tiles)])."""
    buf = bytearray(header_bytes)
    idx_recs, tile_recs, meta = [], [], []
    for e in experts:
        off = (len(buf) + 4095) // 4096 * 4096
        buf.extend(bytes(off - len(buf)))
        g, u, d = e["parts"]
        buf.extend(g + u + d)
        plan = tile_plan(len(g), len(u), len(d), e.get("width"))
        first = len(tile_recs)
        tiles = []
        for t, (mx, ns, nc, ro, sb) in enumerate(plan):
            fields = (mx, t, ns, nc, ro, sb, e.get("tile_layout_id", layout_id), 0)
            tiles.append(fields)
            tile_recs.append(tile_record(*fields))
        fields = (e["layer"], e["expert"], e.get("flags", 0), e.get("layout_id", layout_id), off,
                  len(g) + len(u) + len(d), first, len(plan), e.get("checksum_index", len(idx_recs)))
        idx_recs.append(index_record(*fields))
        meta.append((fields, tiles))
    blob = b"".join(idx_recs) + b"".join(tile_recs)
    pos = (len(buf) + 63) // 64 * 64
    buf.extend(bytes(pos - len(buf)))
    buf.extend(blob)
    return bytes(buf), blob, meta
