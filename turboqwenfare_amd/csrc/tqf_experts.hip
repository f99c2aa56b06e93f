// tqf_experts.hip -- routed-expert superextents of a .tqf container to the
// device: the expert-index half of TqfReader and the staging of
// Qwen36WeightLoader::load_expert / WholeExpertLfuCache::stage_expert_values
// (host code; the uploads use the Q4_K repack of tqf_api.hip).
//
// The container's expert-index blob (superblock expert_index_offset /
// expert_index_bytes, spec section 124) holds expert_count 32-byte
// ExpertIndexRecords, then 24-byte ExpertTileRecords
// (format/tqf/records.rs:221-313; little endian, padding bytes ignored):
//
//   ExpertIndexRecord  [0] layer u8  [2] expert u16  [4] flags u16
//                      [6] layout_id u16  [8] file_offset u64
//                      [16] stored_bytes u32  [20] tile_first u32
//                      [24] tile_count u16  [28] checksum_index u32
//   ExpertTileRecord   [0] matrix u8 (0 GateUp, 1 Down)  [2] tile_id u16
//                      [4] neuron_start u16  [6] neuron_count u16
//                      [8] relative_offset u32  [12] stored_bytes u32
//                      [16] quant_layout_id u16  [18] flags u16
//
// Opening validates as TqfReader::open does (format/tqf/reader.rs:170-247):
// the index part fits the blob, the tile part is whole records, every
// superextent lies inside the container, every tile range lies inside the
// tile table and exactly partitions its superextent in order
// (partition_is_contiguous, tiling.rs:300-313), and per-tile checksum ranges
// fit the checksum table.  Uploading validates as load_expert does
// (model/qwen36/weights.rs:1404-1428: layout Q4_K passthrough, the canonical
// 3 x 589,824 bytes, Q4_K tiles, classify_partition, tiling.rs:236-283),
// then splits the superextent into payload_parts (weights.rs:552-561) and
// uploads gate, up and down as three Q4_K handles.  The BLAKE3 digests of the
// checksum table are the caller's reader's to verify: this library reads no
// file and computes no digest.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

#include "../../include/tqf_hip.h"
#include "tqf_internal.h"

struct tqf_hip_expert_table {
    std::vector<tqf_hip_expert_index> experts;
    std::vector<tqf_hip_expert_tile> tiles;
};

namespace {

constexpr size_t kIndexRecord = 32;
constexpr size_t kTileRecord = 24;
constexpr uint16_t kFlagTileChecksums = 1;   // EXPERT_INDEX_FLAG_TILE_CHECKSUMS
constexpr uint16_t kLayoutQ4K = 2;           // TQF_QUANT_PASSTHROUGH_Q4_K
constexpr uint32_t kHidden = 2048, kWidth = 512;
constexpr uint32_t kMatrixBytes = kHidden * kWidth / 256 * 144;  // one Q4_K expert matrix: 589,824

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t *p) { return (uint32_t)rd16(p) | ((uint32_t)rd16(p + 2) << 16); }
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

int32_t table_fail(tqf_hip_ctx *ctx, const std::string &msg) {
    if (ctx) ctx->last_error = msg;
    return TQF_HIP_ERR_INVALID;
}

// partition_is_contiguous: ordered, non-empty, exactly covering `total`.
bool contiguous(const tqf_hip_expert_tile *t, size_t n, uint32_t total) {
    uint64_t expected = 0;
    for (size_t i = 0; i < n; ++i) {
        if (t[i].stored_bytes == 0 || t[i].relative_offset != expected) return false;
        expected += t[i].stored_bytes;
        if (expected > 0xFFFFFFFFull) return false;
    }
    return expected == total;
}

// classify_partition: contiguous and every tile inside its matrix's region.
bool matrix_partition(const tqf_hip_expert_tile *t, size_t n, uint32_t gate_up, uint32_t down, std::string &why) {
    const uint64_t total = (uint64_t)gate_up + down;
    if (n == 0) {
        why = "expert extent has no tile records";
        return false;
    }
    uint64_t expected = 0;
    for (size_t i = 0; i < n; ++i) {
        if (t[i].stored_bytes == 0 || t[i].relative_offset != expected) {
            why = "tile " + std::to_string(i) + " is empty or does not start at the next unclaimed byte";
            return false;
        }
        const uint64_t end = (uint64_t)t[i].relative_offset + t[i].stored_bytes;
        const bool inside = t[i].matrix == TQF_HIP_MATRIX_GATE_UP
                                ? end <= gate_up
                                : (t[i].relative_offset >= gate_up && end <= total);
        if (!inside) {
            why = "tile " + std::to_string(i) + " lies outside its matrix region";
            return false;
        }
        expected = end;
    }
    if (expected != total) {
        why = "the tile table does not cover the extent";
        return false;
    }
    return true;
}

const tqf_hip_expert_index *find(const tqf_hip_expert_table *t, uint8_t layer, uint16_t expert) {
    for (const tqf_hip_expert_index &e : t->experts)
        if (e.layer == layer && e.expert == expert) return &e;
    return nullptr;
}

}  // namespace

// The table functions are host-only: ctx (may be NULL) only receives the
// last-error message.
extern "C" int32_t tqf_hip_expert_table_open(tqf_hip_ctx *ctx, const uint8_t *blob, size_t blob_len,
                                             uint64_t expert_count, uint64_t file_len, uint64_t checksum_entries,
                                             tqf_hip_expert_table **out) {
    if (ctx) ctx->last_error.clear();
    if (!out || (!blob && blob_len)) return table_fail(ctx, "null pointer");
    *out = nullptr;
    if (expert_count > blob_len / kIndexRecord) return table_fail(ctx, "expert index: records beyond the blob");
    const size_t index_bytes = (size_t)expert_count * kIndexRecord;
    const size_t tile_bytes = blob_len - index_bytes;
    if (tile_bytes % kTileRecord) return table_fail(ctx, "expert tiles: a partial record");
    tqf_hip_expert_table *t = new tqf_hip_expert_table();
    t->experts.resize((size_t)expert_count);
    for (size_t i = 0; i < (size_t)expert_count; ++i) {
        const uint8_t *p = blob + i * kIndexRecord;
        tqf_hip_expert_index &e = t->experts[i];
        e.layer = p[0];
        e.expert = rd16(p + 2);
        e.flags = rd16(p + 4);
        e.layout_id = rd16(p + 6);
        e.file_offset = rd64(p + 8);
        e.stored_bytes = rd32(p + 16);
        e.tile_first = rd32(p + 20);
        e.tile_count = rd16(p + 24);
        e.checksum_index = rd32(p + 28);
    }
    t->tiles.resize(tile_bytes / kTileRecord);
    for (size_t i = 0; i < t->tiles.size(); ++i) {
        const uint8_t *p = blob + index_bytes + i * kTileRecord;
        tqf_hip_expert_tile &r = t->tiles[i];
        if (p[0] > 1) {
            delete t;
            return table_fail(ctx, "expert tiles: unknown matrix in record " + std::to_string(i));
        }
        r.matrix = p[0];
        r.tile_id = rd16(p + 2);
        r.neuron_start = rd16(p + 4);
        r.neuron_count = rd16(p + 6);
        r.relative_offset = rd32(p + 8);
        r.stored_bytes = rd32(p + 12);
        r.quant_layout_id = rd16(p + 16);
        r.flags = rd16(p + 18);
    }
    for (size_t i = 0; i < t->experts.size(); ++i) {
        const tqf_hip_expert_index &e = t->experts[i];
        std::string why;
        if (e.file_offset > file_len || e.stored_bytes > file_len - e.file_offset)
            why = "expert superextent outside the container";
        else if ((uint64_t)e.tile_first + e.tile_count > t->tiles.size())
            why = "expert tile range outside the tile table";
        else if (!contiguous(t->tiles.data() + e.tile_first, e.tile_count, e.stored_bytes))
            why = "expert tiles do not partition the superextent";
        else if ((e.flags & kFlagTileChecksums) && (uint64_t)e.checksum_index + 1 + e.tile_count > checksum_entries)
            why = "expert per-tile checksum range outside the checksum table";
        if (!why.empty()) {
            delete t;
            return table_fail(ctx, why + " (index record " + std::to_string(i) + ")");
        }
    }
    *out = t;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_expert_table_free(tqf_hip_ctx *ctx, tqf_hip_expert_table *table) {
    (void)ctx;
    delete table;
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_expert_table_counts(const tqf_hip_expert_table *table, uint64_t *experts,
                                               uint64_t *tiles) {
    if (!table) return TQF_HIP_ERR_INVALID;
    if (experts) *experts = table->experts.size();
    if (tiles) *tiles = table->tiles.size();
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_expert_lookup(tqf_hip_ctx *ctx, const tqf_hip_expert_table *table, uint8_t layer,
                                         uint16_t expert, tqf_hip_expert_index *index_out,
                                         tqf_hip_expert_tile *tiles_out, size_t tiles_cap, size_t *n_tiles) {
    if (ctx) ctx->last_error.clear();
    if (!table) return table_fail(ctx, "null pointer");
    const tqf_hip_expert_index *e = find(table, layer, expert);
    if (!e) return table_fail(ctx, "expert not found: layer " + std::to_string(layer) + " expert " +
                                       std::to_string(expert));
    if (index_out) *index_out = *e;
    if (n_tiles) *n_tiles = e->tile_count;
    if (tiles_out) {
        if (tiles_cap < e->tile_count) return table_fail(ctx, "tile buffer too small");
        std::memcpy(tiles_out, table->tiles.data() + e->tile_first, e->tile_count * sizeof(tqf_hip_expert_tile));
    }
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_expert_reserve_bytes(tqf_hip_ctx *ctx, const tqf_hip_expert_table *table, uint8_t layer,
                                                uint16_t expert, uint64_t *stored_bytes, uint64_t *device_bytes) {
    if (ctx) ctx->last_error.clear();
    if (!table) return table_fail(ctx, "null pointer");
    const tqf_hip_expert_index *e = find(table, layer, expert);
    if (!e) return table_fail(ctx, "expert not found: layer " + std::to_string(layer) + " expert " +
                                       std::to_string(expert));
    if (stored_bytes) *stored_bytes = e->stored_bytes;
    if (device_bytes)
        *device_bytes = 2 * tqf_hip_q4k_weights_bytes_for(kWidth, kHidden) + tqf_hip_q4k_weights_bytes_for(kHidden, kWidth);
    return TQF_HIP_OK;
}

extern "C" int32_t tqf_hip_expert_upload(tqf_hip_ctx *ctx, const tqf_hip_expert_table *table, uint8_t layer,
                                         uint16_t expert, const uint8_t *container, size_t container_len,
                                         tqf_hip_weights **gate, tqf_hip_weights **up, tqf_hip_weights **down) {
    if (!ctx) return TQF_HIP_ERR_INVALID;
    ctx->last_error.clear();
    if (!table || !container || !gate || !up || !down) return table_fail(ctx, "null pointer");
    *gate = *up = *down = nullptr;
    const tqf_hip_expert_index *e = find(table, layer, expert);
    if (!e) return table_fail(ctx, "expert not found: layer " + std::to_string(layer) + " expert " +
                                       std::to_string(expert));
    if (e->file_offset > container_len || e->stored_bytes > container_len - e->file_offset)
        return table_fail(ctx, "expert superextent outside the container region");
    const tqf_hip_expert_tile *tiles = table->tiles.data() + e->tile_first;
    bool tiles_q4k = true;
    for (uint32_t i = 0; i < e->tile_count; ++i) tiles_q4k = tiles_q4k && tiles[i].quant_layout_id == kLayoutQ4K;
    std::string why;
    if (e->layout_id != kLayoutQ4K || !tiles_q4k || e->stored_bytes != 3 * kMatrixBytes ||
        !matrix_partition(tiles, e->tile_count, 2 * kMatrixBytes, kMatrixBytes, why))
        return table_fail(ctx, "the expert's tiles are not a valid Qwen3.6 Q4_K partition" +
                                   (why.empty() ? std::string() : ": " + why));
    // payload_parts: gate, up and down, each one whole Q4_K matrix
    const uint8_t *base = container + e->file_offset;
    tqf_hip_weights *w[3] = {nullptr, nullptr, nullptr};
    const uint32_t rows[3] = {kWidth, kWidth, kHidden}, cols[3] = {kHidden, kHidden, kWidth};
    for (int k = 0; k < 3; ++k) {
        const int32_t rc = tqf_hip_q4k_weights_upload(ctx, base + (size_t)k * kMatrixBytes, kMatrixBytes, rows[k],
                                                      cols[k], &w[k]);
        if (rc != TQF_HIP_OK) {
            const std::string msg = ctx->last_error;
            for (int j = 0; j < k; ++j) (void)tqf_hip_weights_free(ctx, w[j]);
            ctx->last_error = msg;
            return rc;
        }
    }
    *gate = w[0];
    *up = w[1];
    *down = w[2];
    return TQF_HIP_OK;
}
