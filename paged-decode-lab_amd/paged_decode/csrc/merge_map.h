// Work and address map of the merge kernels, shared by the device code in
// decode.hip and the host: which (sequence, query head) row and column chunk a
// merge workgroup or wave owns, which states it reads (how many before the
// row's live count is known, which after), at which element offsets, where
// it writes the output, and which kernel variant and grid a launch uses.
// Everything here is plain integer arithmetic, so the same functions compile
// for gfx950 (hipcc) and for the host C++ compiler; tests/address_audit.cpp
// walks every workgroup and lane of a merge launch through them and checks
// each access against the caller's buffers and the launch's LDS.
//
// The merge is the max-corrected combination of reference
// src/paged_decode/csrc/decode.cu:87-108 (serial) and :120-168 (LDS-bounded
// weights), over the states the partition kernels leave (partition_map.h).
#ifndef PAGED_DECODE_MERGE_MAP_H
#define PAGED_DECODE_MERGE_MAP_H

#include "partition_map.h"

namespace pd {

struct MergeParams {
    const float* numerator;  // [B, Hq, parts, D]
    const float* stats;      // [B, Hq, parts, 2]
    float* out;              // [B, Hq, D]
    const int32_t* lengths;  // [B]
    int parts;               // allocated states per row (4 * splits)
    int stride_shift;        // read every (1 << stride_shift)-th state: 0, or log2 of the combined quarters
    int query_heads;
    int split_tokens;
    int reach;               // tokens a row may hold: min(caller's splits * split_tokens, table_width * page_size)
    int first_states;        // states (read units) loaded before the live count arrives: the host's
                             // bound on any row's live states, else the whole row
    int xcd_rows;            // rows per row group of an XCD-grouped partition grid (merge_xcd_row), 0: plain
    int xcd_shift;           // log2 of that grid's head groups per sequence
};

constexpr int kMergeThreads = 256;

// merge_cols_kernel (see decode.hip): column chunks of CH floats, NB numerator
// loads per lane per round, the first kOptimisticRounds of them issued before
// the row's live count arrives.
constexpr int kMergeChunkLocal = 32;  // floats per column chunk, XCD-grouped merge
constexpr int kMergeChunkWide = 64;   // floats per column chunk, otherwise
constexpr int kMergeColBatchShort = 8;
constexpr int kMergeColBatchLong = 32;
constexpr int kOptimisticRounds = 2;

// merge_rows_kernel: one wave per row, NB loads per lane, RPG rows per
// workgroup; used from kMergeRowsMin rows on for rows of more than two rounds.
constexpr int kMergeWaveBatch = 8;
constexpr int kMergeRowsMin = 256;
constexpr int kMergeRowsPerGroup = 4;

// States a merge_rows wave holds at once: NB loads of kWave / (D / 4) states.
constexpr int merge_wave_max_parts(int head_dim, int nb = kMergeWaveBatch) { return nb * (kWave / (head_dim / 4)); }

// States of row b to merge: per_part per partition up to the last one holding
// a token of the sequence (none for an empty sequence), capped at the row's
// states. len_raw is the device length, clamped to reach (decode.cu:42-44).
PD_HD int live_states(int len_raw, int split_tokens, int reach, int per_part, int states) {
    const int len = imax(0, imin(len_raw, reach));
    const int64_t live = (static_cast<int64_t>(len) + split_tokens - 1) / split_tokens;
    return static_cast<int>(lmin(static_cast<int64_t>(per_part) * live, states));
}

// Row of merge_cols workgroup (bx, by): the XCD-grouped row map, or query
// head bx of sequence by.
PD_HD MergeRow merge_cols_row(const MergeParams& mp, uint32_t bx, uint32_t by) {
    if (mp.xcd_rows > 0) return merge_xcd_row(bx, by, mp.xcd_rows, mp.xcd_shift, 1, 0);
    return MergeRow{static_cast<int>(by), static_cast<int64_t>(by) * mp.query_heads + bx};
}

// Row of wave `wave` of merge_rows workgroup (bx, by), rpg rows per workgroup;
// row -1 for a wave past the last query head of a plain grid (it exits).
PD_HD MergeRow merge_rows_row(const MergeParams& mp, uint32_t bx, uint32_t by, int wave, int rpg) {
    if (mp.xcd_rows > 0) return merge_xcd_row(bx, by, mp.xcd_rows, mp.xcd_shift, rpg, wave);
    const int h = static_cast<int>(bx) * rpg + wave;
    if (h >= mp.query_heads) return MergeRow{static_cast<int>(by), -1};
    return MergeRow{static_cast<int>(by), static_cast<int64_t>(by) * mp.query_heads + h};
}

// A row's statistics, in (m, l) pairs: the row's first state, and read unit
// j's offset from it (allocated state j << stride_shift).
PD_HD int64_t merge_stats_base(const MergeParams& mp, int64_t row) { return row * mp.parts; }
PD_HD int merge_stats_offset(const MergeParams& mp, int j) { return j << mp.stride_shift; }

// A row's numerators, in 16-byte columns: column `col` of column chunk
// `chunk` (CH floats) of the row's first state (merge_rows reads whole rows:
// chunk 0, CH = D), and read unit j's offset from it.
PD_HD int64_t merge_numerator_base(const MergeParams& mp, int64_t row, int head_dim, int chunk, int ch, int col) {
    return row * mp.parts * (head_dim / 4) + chunk * (ch / 4) + col;
}
PD_HD int64_t merge_numerator_offset(const MergeParams& mp, int head_dim, int j) {
    return static_cast<int64_t>(j) * ((head_dim / 4) << mp.stride_shift);
}

// Clamped read unit of the numerator loads: state group pg's k-th load of the
// round at `base` (groups of `groups` states per load), kept inside the row.
PD_HD int merge_load_unit(int base, int pg, int k, int groups, int last) {
    return imin(base + pg + k * groups, last);
}

// Loads of a merge_cols round from `base` that still hold states below limit.
PD_HD int merge_cols_rounds(int base, int limit, int nb, int groups) {
    return imin(nb, (limit - base + groups - 1) / groups);
}

// States (read units) a merge loads before a row's live count arrives: the
// host bounds' longest row, else the whole row (host; decode.hip's run_merge).
inline int merge_first_states(int parts, int stride_shift, int split_tokens, int reach, const int32_t* length_bounds,
                              int batch) {
    const int states = parts >> stride_shift;
    if (length_bounds == nullptr) return states;
    int64_t longest = 0;
    for (int b = 0; b < batch; ++b) {
        const int64_t bound = lmin(reach, length_bounds[b] < 0 ? 0 : length_bounds[b]);
        longest = bound > longest ? bound : longest;
    }
    const int64_t live = static_cast<int64_t>(kQuarters >> stride_shift) * ((longest + split_tokens - 1) / split_tokens);
    return static_cast<int>(lmin(states, live));
}

// The launch a merge of these rows uses.
enum MergeKind { kMergeRows = 0, kMergeCols = 1 };

struct MergeLaunch {
    int kind;        // kMergeRows or kMergeCols
    int shared;      // weights formed once (LDS-bounded merge) or recomputed per lane (serial)
    int nb;          // loads per lane per round
    int ch;          // floats per column chunk (merge_cols), head_dim (merge_rows)
    int xcd_rows;    // the row map's rows per row group (0: plain); may be cleared from the params' value
    uint32_t grid_x, grid_y, grid_z;
    int threads;
    int lds_bytes;   // dynamic LDS: one weight per read state (shared merge_cols)
};

// Kernel, variant and grid of a merge (decode.hip's launch_merge). merge_rows
// keeps a row in one wave, loading (states / groups) 16-byte columns per
// lane; with few rows of many states, merge_cols (D / CH workgroups per row)
// finishes sooner. The merge_cols variant of NB = kMergeColBatchLong loads
// per round holds one (serial) or two (shared) workgroups per CU: it pays
// only while the grid fits the device in one round; larger grids take
// 256-state rounds at full occupancy (rows of a plan whose reserved context
// exceeds the live one among them: the variant follows the allocated states).
inline MergeLaunch plan_merge(const MergeParams& mp, int batch, int head_dim, bool shared, int compute_units) {
    MergeLaunch ml{};
    ml.shared = shared;
    const int states = mp.parts >> mp.stride_shift;
    const int64_t rows = static_cast<int64_t>(batch) * mp.query_heads;
    const uint32_t row_groups = mp.xcd_rows > 0 ? static_cast<uint32_t>(rows / mp.xcd_rows / 8) : 0u;
    const int per_round = kWave / (head_dim / 4);
    const int rounds = (states + per_round - 1) / per_round;
    const bool many_rows = rows >= kMergeRowsMin;
    if (states <= merge_wave_max_parts(head_dim) && (many_rows || rounds <= 2)) {
        ml.kind = kMergeRows;
        ml.nb = kMergeWaveBatch;
        ml.ch = head_dim;
        ml.xcd_rows = mp.xcd_rows % kMergeRowsPerGroup == 0 ? mp.xcd_rows : 0;
        if (ml.xcd_rows > 0) {
            ml.grid_x = static_cast<uint32_t>(8 * ml.xcd_rows / kMergeRowsPerGroup);
            ml.grid_y = row_groups;
        } else {
            ml.grid_x = static_cast<uint32_t>((mp.query_heads + kMergeRowsPerGroup - 1) / kMergeRowsPerGroup);
            ml.grid_y = static_cast<uint32_t>(batch);
        }
        ml.grid_z = 1;
        ml.threads = kWave * kMergeRowsPerGroup;
        ml.lds_bytes = 0;
        return ml;
    }
    ml.kind = kMergeCols;
    ml.ch = mp.xcd_rows > 0 ? kMergeChunkLocal : kMergeChunkWide;
    ml.xcd_rows = mp.xcd_rows;
    if (ml.xcd_rows > 0) {
        ml.grid_x = static_cast<uint32_t>(8 * ml.xcd_rows);
        ml.grid_y = row_groups;
    } else {
        ml.grid_x = static_cast<uint32_t>(mp.query_heads);
        ml.grid_y = static_cast<uint32_t>(batch);
    }
    ml.grid_z = static_cast<uint32_t>(head_dim / ml.ch);
    ml.threads = kMergeThreads;
    ml.lds_bytes = shared ? states * static_cast<int>(sizeof(float)) : 0;
    const int groups = kMergeThreads / (ml.ch / 4);
    const int64_t workgroups = static_cast<int64_t>(ml.grid_x) * ml.grid_y * ml.grid_z;
    const bool long_rows = states > kMergeColBatchShort * groups && workgroups <= compute_units;
    ml.nb = long_rows ? kMergeColBatchLong : kMergeColBatchShort;
    return ml;
}

}  // namespace pd

#endif  // PAGED_DECODE_MERGE_MAP_H
