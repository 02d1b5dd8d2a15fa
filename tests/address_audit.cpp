// Host audit of every memory access the partition kernels form -- TEST
// INFRASTRUCTURE, the CPU stand-in for a GPU memory checker.
//
// For each problem below, the launch is planned with the library's own host
// code (partition_map.h: plan_items, plan_mfma / plan_fp32, partial_grid) and
// then every workgroup, wave, lane and load group of the grid is walked with
// the same device-side functions the kernels call (block_coords,
// partition_range, wave_work, speculative_page, window_entry, tile_span,
// tile_live, tile_page_offset, token_offset, numerator_offset, stats_offset),
// following the kernels' loop structure (page-id windows of 64 entries, load
// groups issued two ahead in blocks of two for the matrix-core kernel -- four
// and four with FP8 K/V outside whole rows -- and four ahead in blocks of sixteen for the FP32
// kernel). Every global load is
// checked to lie inside q, k, v, table or lengths (parked loads of dead
// groups inside q), every store inside numerator or stats, every LDS access
// inside the launch's dynamic LDS; every live token is read from the page its
// table entry names; and every live state slot is written exactly once, none
// past a sequence's end. Built with -fsanitize=address,undefined by
// tests/test_address_audit.py; prints one line per problem and exits nonzero
// on the first problem with a failure.
#include <cinttypes>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "partition_map.h"

using namespace pd;

namespace {

struct Problem {
    std::string name;
    int batch, q_heads, kv_heads, head_dim, page_size, width, pages;
    int q_elem, kv_elem;  // bytes: 4 (FP32), 2 (FP16/BF16), 1 (FP8 K/V)
    int split_tokens, splits;
    // The caller's partitions: a full call over coarser partitions keeps them
    // here (split_tokens and splits are then the coarser ones), and no token
    // at or past caller_splits * caller_split_tokens may be read.
    int caller_split_tokens, caller_splits;
    std::vector<int32_t> table, lengths, bounds;  // bounds empty: none
    bool unshared = true, ragged = false;
};

uint64_t g_checks = 0;
int g_failures = 0;
bool g_plant_reach = false;  // --plant-reach: launch params that ignore the caller's partitions (negative control)

// Tokens of a row the caller's partitions cover, clamped to the table.
int reach_of(const Problem& pr) {
    return static_cast<int>(lmin(static_cast<int64_t>(pr.caller_splits) * pr.caller_split_tokens,
                                 static_cast<int64_t>(pr.width) * pr.page_size));
}

#define AUDIT(cond, ...)                                                    \
    do {                                                                    \
        ++g_checks;                                                         \
        if (!(cond)) {                                                      \
            if (g_failures++ < 20) {                                        \
                std::fprintf(stderr, "  FAIL %s:%d: ", __FILE__, __LINE__); \
                std::fprintf(stderr, __VA_ARGS__);                          \
                std::fprintf(stderr, "\n");                                 \
            }                                                               \
        }                                                                   \
    } while (0)

// Sizes of the buffers a caller passes for a problem.
struct Buffers {
    uint64_t q_bytes, kv_bytes, numerator_elems, stats_elems;
    int64_t table_elems;
};

Buffers buffers(const Problem& pr) {
    Buffers b;
    b.q_bytes = static_cast<uint64_t>(pr.batch) * pr.q_heads * pr.head_dim * pr.q_elem;
    b.kv_bytes = static_cast<uint64_t>(pr.pages) * pr.page_size * pr.kv_heads * pr.head_dim * pr.kv_elem;
    const uint64_t states = static_cast<uint64_t>(pr.batch) * pr.q_heads * kQuarters * pr.splits;
    b.numerator_elems = states * pr.head_dim;
    b.stats_elems = states * 2;
    b.table_elems = static_cast<int64_t>(pr.batch) * pr.width;
    return b;
}

PartialParams params(const Problem& pr, int cus, bool mfma, bool rows) {
    PartialParams p{};
    p.row_allowed = rows;
    p.batch = pr.batch;
    p.query_heads = pr.q_heads;
    p.group = pr.q_heads / pr.kv_heads;
    p.page_shift = pr.page_size == 16 ? 4 : 5;
    p.table_width = pr.width;
    p.physical_pages = pr.pages;
    p.splits = pr.splits;
    p.split_tokens = pr.split_tokens;
    p.reach = g_plant_reach ? pr.width * pr.page_size : reach_of(pr);
    p.token_bytes = static_cast<uint32_t>(pr.kv_heads * pr.head_dim * pr.kv_elem);
    p.page_bytes = static_cast<uint64_t>(pr.page_size) * p.token_bytes;
    p.unshared_pages = pr.unshared;
    p.ragged_lengths = pr.ragged;
    plan_items(p, pr.bounds.empty() ? nullptr : pr.bounds.data());
    if (mfma) plan_mfma(p, pr.kv_heads, cus, pr.head_dim, pr.kv_elem);
    else plan_fp32(p, pr.kv_heads, pr.head_dim);
    return p;
}

// Writers of each state slot, to check that every live slot is written once.
// Also the XCD (linear dispatch index % 8) of the workgroups storing each
// row's states: -1 none yet, -2 more than one.
struct Coverage {
    std::vector<uint8_t> writes;
    std::vector<int8_t> row_xcd;
    Coverage(uint64_t states, uint64_t rows) : writes(states, 0), row_xcd(rows, -1) {}
    void store(uint64_t slot, int64_t row, int xcd) {
        AUDIT(slot < writes.size(), "state slot %" PRIu64 " past the workspace", slot);
        if (slot < writes.size() && writes[slot] < 255) ++writes[slot];
        if (row >= 0 && static_cast<uint64_t>(row) < row_xcd.size()) {
            int8_t& x = row_xcd[row];
            x = x == -1 ? static_cast<int8_t>(xcd) : x == xcd ? x : -2;
        }
    }
};

// Writers of each output element of a whole-row launch.
struct OutCoverage {
    std::vector<uint8_t> writes;
    explicit OutCoverage(uint64_t elems) : writes(elems, 0) {}
    void store(int64_t e) {
        AUDIT(e >= 0 && static_cast<uint64_t>(e) < writes.size(), "output element %" PRId64 " past out", e);
        if (e >= 0 && static_cast<uint64_t>(e) < writes.size() && writes[e] < 255) ++writes[e];
    }
};

void check_coverage(const Problem& pr, const Coverage& cov) {
    for (int b = 0; b < pr.batch; ++b) {
        const int len = imax(0, imin(pr.lengths[b], reach_of(pr)));
        const int live_parts = (len + pr.split_tokens - 1) / pr.split_tokens;
        for (int h = 0; h < pr.q_heads; ++h) {
            for (int part = 0; part < kQuarters * pr.splits; ++part) {
                const uint64_t slot = (static_cast<uint64_t>(b) * pr.q_heads + h) * kQuarters * pr.splits + part;
                const int expected = part < kQuarters * live_parts ? 1 : 0;
                AUDIT(cov.writes[slot] == expected, "seq %d head %d state %d written %d times, expected %d", b, h,
                      part, cov.writes[slot], expected);
            }
        }
    }
}

// The merge's side of an XCD-grouped grid (merge_xcd_row), for both merge
// kernels (one row per workgroup, and kMergeRowsPerGroup = 4 rows of one wave
// each): every row is taken exactly once, by a workgroup of its own sequence
// on the XCD whose workgroups stored all of the row's states.
void check_merge_xcd(const Problem& pr, const PartialParams& p, const Coverage& cov) {
    const int group_rows = xcd_row_group_rows(p);
    const int64_t rows = static_cast<int64_t>(pr.batch) * pr.q_heads;
    AUDIT(group_rows > 0 && rows % (8 * group_rows) == 0, "row groups of %d rows over %" PRId64 " rows", group_rows,
          rows);
    if (group_rows <= 0 || rows % (8 * group_rows) != 0) return;
    for (int64_t r = 0; r < rows; ++r) {
        const int len = imax(0, imin(pr.lengths[r / pr.q_heads], pr.width * pr.page_size));
        if (len > 0) AUDIT(cov.row_xcd[r] >= 0, "row %" PRId64 " states stored from XCDs %d", r, cov.row_xcd[r]);
    }
    for (int unit : {1, 4}) {
        if (group_rows % unit != 0) continue;
        const uint32_t gx = static_cast<uint32_t>(8 * group_rows / unit);
        const uint32_t gy = static_cast<uint32_t>(rows / group_rows / 8);
        std::vector<uint8_t> taken(rows, 0);
        for (uint32_t by = 0; by < gy; ++by) {
            for (uint32_t bx = 0; bx < gx; ++bx) {
                const int xcd = static_cast<int>((bx + static_cast<uint64_t>(gx) * by) % 8);
                for (int sub = 0; sub < unit; ++sub) {
                    const MergeRow m = merge_xcd_row(bx, by, group_rows, p.merge_xcd_shift, unit, sub);
                    AUDIT(m.row >= 0 && m.row < rows, "merge row %" PRId64, m.row);
                    if (m.row < 0 || m.row >= rows) continue;
                    AUDIT(m.b == m.row / pr.q_heads, "merge row %" PRId64 " given sequence %d", m.row, m.b);
                    ++taken[m.row];
                    const int stored = cov.row_xcd[m.row];
                    if (stored >= 0)
                        AUDIT(stored == xcd, "merge row %" PRId64 " on XCD %d, states on XCD %d", m.row, xcd, stored);
                }
            }
        }
        for (int64_t r = 0; r < rows; ++r) AUDIT(taken[r] == 1, "merge row %" PRId64 " taken %d times", r, taken[r]);
    }
}

int page_of(const Problem& pr, int b, int window, int slot, const PartialParams& p) {
    const int entry = window_entry(p, window + slot, 0);  // the lane holding slot reads entry window + slot
    return pr.table[static_cast<size_t>(b) * pr.width + entry];
}

// One load group of the matrix-core kernel (a 16-token tile), all 64 lanes.
template <int D>
void mfma_tile(const Problem& pr, const PartialParams& p, const Buffers& buf, const WaveWork& w, int b, int t0,
               int rb, int re, int window, int wave, int waves, int len) {
    const int ES = pr.kv_elem;
    const int VH = D / 16, VW = VH * ES / 4, KR = D * ES / 16, TK = kWave / KR, KL = kTileTokens / TK;
    const int stage_row = mfma_stage_bytes(D, ES) / kTileTokens;
    const TileSpan span = tile_span(p, t0, kTileTokens, rb, re, window);
    AUDIT(span.slot >= 0 && span.slot < kWave, "window slot %d", span.slot);
    const int page = page_of(pr, b, window, span.slot, p);
    const bool ok = tile_live(p, t0, re, page);
    if (ok) {
        // The page id read is the table entry of the tile's logical page, and
        // the tile's live tokens lie on that one page, inside the sequence.
        AUDIT((span.lo >> p.page_shift) == window + span.slot, "tile %d reads window slot %d of window %d", t0,
              span.slot, window);
        AUDIT((span.hi >> p.page_shift) == (span.lo >> p.page_shift), "tile %d straddles a page", t0);
        AUDIT(span.lo >= rb && span.hi < re && span.hi < len, "tile %d span [%d, %d] outside [%d, %d)", t0, span.lo,
              span.hi, rb, re);
    }
    const uint64_t page_off = tile_page_offset(p, ok, page);
    const uint64_t head_off = static_cast<uint64_t>(w.kv_head) * D * ES;
    const uint64_t park = static_cast<uint64_t>(w.q_row) * D * 2;
    for (int lane = 0; lane < kWave; ++lane) {
        const int n = lane % 16, g = lane / 16;
        for (int s = 0; s < KL; ++s) {
            const uint32_t off = token_offset(p, ok, t0 + TK * s + lane / KR, span, static_cast<uint32_t>(lane % KR) * 16u);
            if (ok) AUDIT(head_off + page_off + off + 16 <= buf.kv_bytes, "K load past the cache");
            else AUDIT(park + off + 16 <= buf.q_bytes, "parked K load past q");
            const int lds = wave * kTileTokens * stage_row + (TK * s + lane / KR) * stage_row + (lane % KR) * 16;
            AUDIT(lds >= 0 && lds + (ES == 2 ? 16 : 8) <= waves * mfma_stage_bytes(D, ES), "K stage write");
        }
        for (int s = 0; s < D / 32; ++s) {
            const int lds = wave * kTileTokens * stage_row + k_token_of_row(n) * stage_row + (32 * s + 8 * g) * ES;
            AUDIT(lds + (ES == 2 ? 16 : 8) <= (wave + 1) * mfma_stage_bytes(D, ES), "K stage read outside the wave's tile");
        }
        for (int e = 0; e < 4; ++e) {
            const uint32_t off = token_offset(p, ok, t0 + 4 * e + g, span, static_cast<uint32_t>(n) * VH * ES);
            if (ok) AUDIT(head_off + page_off + off + 4u * VW <= buf.kv_bytes, "V load past the cache");
            else AUDIT(park + off + 4u * VW <= buf.q_bytes, "parked V load past q");
        }
    }
}

// One load group of the FP32 kernel (TPL tokens, NL = 1 load per chunk).
template <int D>
void fp32_group(const Problem& pr, const PartialParams& p, const Buffers& buf, const WaveWork& w, int b, int g0,
                int rb, int re, int window, int len) {
    const int LPT = D / 4, TPL = kWave / LPT;
    const TileSpan span = tile_span(p, g0, TPL, rb, re, window);
    const int page = page_of(pr, b, window, span.slot, p);
    const bool ok = tile_live(p, g0, re, page);
    if (ok) {
        AUDIT((span.lo >> p.page_shift) == window + span.slot, "group %d reads the wrong window slot", g0);
        AUDIT((span.hi >> p.page_shift) == (span.lo >> p.page_shift), "group %d straddles a page", g0);
        AUDIT(span.lo >= rb && span.hi < re && span.hi < len, "group %d span outside the range", g0);
    }
    const uint64_t page_off = tile_page_offset(p, ok, page);
    const uint64_t head_off = static_cast<uint64_t>(w.kv_head) * D * 4;
    const uint64_t park = static_cast<uint64_t>(w.q_row) * D * 4;
    for (int lane = 0; lane < kWave; ++lane) {
        const uint32_t off = token_offset(p, ok, g0 + lane / LPT, span, static_cast<uint32_t>(lane % LPT) * 16u);
        if (ok) AUDIT(head_off + page_off + off + 16 <= buf.kv_bytes, "K/V load past the cache");
        else AUDIT(park + off + 16 <= buf.q_bytes, "parked load past q");
    }
}

// Page-id window loads of all lanes at `window`.
void window_loads(const Problem& pr, const PartialParams& p, const Buffers& buf, int b, int window) {
    for (int lane = 0; lane < kWave; ++lane) {
        const int entry = window_entry(p, window, lane);
        AUDIT(entry >= 0 && entry < pr.width, "window entry %d", entry);
        AUDIT(static_cast<int64_t>(b) * pr.width + entry < buf.table_elems, "table load past the table");
    }
}

template <int D, int GT>
void audit_launch(const Problem& pr, const PartialParams& p, bool mfma, Coverage& cov, OutCoverage& out) {
    constexpr int TPLV = kWave / (D / 4);  // FP32 kernel: token rows per 16-byte load group
    const Buffers buf = buffers(pr);
    const Grid grid = partial_grid(p, pr.kv_heads);
    AUDIT(p.grid_x == grid.x && p.grid_y == grid.y, "kernel-argument grid %ux%u, launch %ux%u", p.grid_x, p.grid_y,
          grid.x, grid.y);
    const int waves = partial_threads(p) / kWave;
    AUDIT(waves >= 1 && waves <= (p.row_mode ? kRowMaxWaves : 8), "workgroup of %d waves", waves);
    if (mfma) AUDIT(mfma_lds_bytes(p, D, pr.kv_elem) <= 160 * 1024, "LDS %d bytes", mfma_lds_bytes(p, D, pr.kv_elem));
    const int align = mfma ? kTileTokens : kWave / (D / 4);
    // Load groups per straight-line block and issued ahead, as the kernels'
    // constants: matrix-core 2 and 2 (FP8 K/V outside whole rows: 4 and 4);
    // FP32 16 and 4, whole-row FP32 launches 4 and 4.
    const bool fp8_deep = mfma && pr.kv_elem == 1 && !p.row_mode;
    const int block = mfma ? (fp8_deep ? 4 : 2) : p.row_mode ? 4 : 16;
    const int ahead = mfma ? (fp8_deep ? 4 : 2) : 4, group_tokens = align;
    const int qw = p.quarters_per_wg;
    for (uint32_t bz = 0; bz < grid.z; ++bz) {
        for (uint32_t by = 0; by < grid.y; ++by) {
            for (uint32_t bx = 0; bx < grid.x; ++bx) {
                const int kind = grid_kind(p);
                const BlockCoords bc =
                    kind == kGridRectTails
                        ? block_coords<kGridRectTails>(bx, by, bz, p.grid_x, p.grid_y, p.xcd_shift, p.xcd_main_rows,
                                                       p.xcd_tail_shift)
                        : block_coords<kGridRect>(bx, by, bz, p.grid_x, p.grid_y, p.xcd_shift, p.xcd_main_rows,
                                                  p.xcd_tail_shift);
                const int xcd = static_cast<int>((bx + static_cast<uint64_t>(grid.x) * (by + static_cast<uint64_t>(grid.y) * bz)) % 8);
                const PartitionRange r = kind == kGridList        ? partition_range<kGridList>(p, bc)
                                         : kind == kGridRectTails ? partition_range<kGridRectTails>(p, bc)
                                                                  : partition_range<kGridRect>(p, bc);
                AUDIT(r.b >= 0 && r.b < pr.batch, "sequence %d", r.b);
                AUDIT(r.first >= 0 && r.count >= 0 && r.first + r.count <= pr.splits && r.count <= p.tail_span &&
                          r.first < pr.splits,
                      "partition range %d + %d", r.first, r.count);
                if (r.b < 0 || r.b >= pr.batch) continue;
                const int b = r.b;
                const int len_raw = pr.lengths[b];
                // Live tokens: the length clamped to the table and to the
                // caller's partitions; every read below is checked against it.
                const int len = imax(0, imin(len_raw, reach_of(pr)));
                const bool rows = p.row_mode != 0;
                const int row_limit = mfma ? kRowMaxWaves : fp32_row_max_waves(GT);
                if (rows) {
                    AUDIT(!p.compact && waves == p.row_waves && waves <= row_limit, "whole-row launch of %d waves",
                          waves);
                    AUDIT(grid.x == 1 && r.first == 0 && r.count == 1 && r.qgroup == 0, "whole-row workgroup item");
                }
                int64_t row_q = -1;
                int row_heads = -1, row_next = 0;
                const int row_end = static_cast<int>(lmin(static_cast<int64_t>(pr.splits) * pr.split_tokens, len));
                for (int wave = 0; wave < waves; ++wave) {
                    const int split = r.first;
                    int window = rows ? (mfma ? row_speculative_page<kTileTokens>(p, wave, waves)
                                              : row_speculative_page<TPLV>(p, wave, waves))
                                      : mfma ? speculative_page<kTileTokens>(p, split, r.count, r.qgroup, wave)
                                             : speculative_page<TPLV>(p, split, r.count, r.qgroup, wave);
                    window_loads(pr, p, buf, b, window);
                    {
                        const WaveWork w =
                            rows ? (mfma ? row_wave_work<GT, kTileTokens>(p, b, bc.heads, wave, waves, len_raw)
                                         : row_wave_work<GT, TPLV>(p, b, bc.heads, wave, waves, len_raw))
                            : mfma ? wave_work<GT, kTileTokens>(p, b, split, r.count, r.qgroup, bc.heads, wave,
                                                                len_raw)
                                   : wave_work<GT, TPLV>(p, b, split, r.count, r.qgroup, bc.heads, wave, len_raw);
                        if (rows) {
                            // Every wave writes its LDS slot (an empty slice
                            // the empty state); the slices tile the row's
                            // tokens [0, min(len, splits * split_tokens)) in
                            // wave order; all waves share the row.
                            if (mfma) {
                                const int lds = mfma_lds_bytes(p, D, pr.kv_elem);
                                const int base = waves * mfma_stage_bytes(D, pr.kv_elem);
                                AUDIT(base + (wave + 1) * combine_slot_bytes(D) <= lds && lds <= 160 * 1024,
                                      "row slot write");
                            } else {
                                AUDIT(waves * row_slot_bytes_fp32(D) <= 160 * 1024, "row slots");
                            }
                            if (row_q < 0) {
                                row_q = w.q_row;
                                row_heads = w.heads_here;
                            }
                            AUDIT(w.q_row == row_q && w.heads_here == row_heads, "waves of one row disagree");
                            if (!w.dead) {
                                AUDIT(w.wb == row_next, "slice %d starts at %d, expected %d", wave, w.wb, row_next);
                                row_next = w.we;
                            }
                            if (wave == waves - 1) AUDIT(row_next == row_end, "slices end at %d of %d", row_next, row_end);
                        }
                        AUDIT(r.count > 0 || w.dead, "an empty grid item is not dead");
                        if (w.dead) {
                            AUDIT(!rows || w.wb == w.we, "dead row wave with tokens");
                            continue;
                        }
                        AUDIT(w.kv_head >= 0 && w.kv_head < pr.kv_heads, "KV head %d", w.kv_head);
                        AUDIT(w.tile >= 0 && w.tile < p.head_tiles, "head tile %d", w.tile);
                        AUDIT(w.q_row >= 0 && w.q_row + w.heads_here <= static_cast<int64_t>(pr.batch) * pr.q_heads,
                              "q row %" PRId64, w.q_row);
                        // A wave's tokens lie in its partitions (a whole-row
                        // wave's: in the row's, [0, splits * split_tokens)).
                        const int64_t first = rows ? 0 : static_cast<int64_t>(split) * pr.split_tokens;
                        const int64_t parts = rows ? pr.splits : r.count;
                        AUDIT(w.wb >= first && w.we <= first + parts * pr.split_tokens && w.wb <= w.we && w.we <= len,
                              "wave range [%d, %d) of partitions %d + %" PRId64, w.wb, w.we, split, parts);
                        // q loads of the tile's live heads.
                        for (int lane = 0; lane < kWave; ++lane) {
                            if (mfma) {
                                const int n = lane % 16, g = lane / 16;
                                if (n < w.heads_here)
                                    for (int s = 0; s < D / 32; ++s)
                                        AUDIT(static_cast<uint64_t>((w.q_row + n) * D + 32 * s + 8 * g) * 2 + 16 <=
                                                  buf.q_bytes, "q load");
                            } else {
                                for (int h = 0; h < w.heads_here; ++h)
                                    AUDIT(static_cast<uint64_t>((w.q_row + h) * D + (lane % (D / 4)) * 4) * 4 + 16 <=
                                              buf.q_bytes, "q load");
                            }
                        }
                        // The kernels' token loop: page-id windows of 64 pages,
                        // load groups issued `ahead` in blocks of `block`.
                        int rb = w.wb, re = w.wb;
                        for (rb = w.wb; rb < w.we; rb = re) {
                            if ((rb >> p.page_shift) != window) {
                                window = rb >> p.page_shift;
                                window_loads(pr, p, buf, b, window);
                            }
                            re = imin(w.we, (window + kWave) << p.page_shift);
                            for (int s0 = rb & ~(group_tokens - 1); s0 < re; s0 += block * group_tokens) {
                                auto issue = [&](int t0) {
                                    if (mfma) mfma_tile<D>(pr, p, buf, w, b, t0, rb, re, window, wave, waves, len);
                                    else fp32_group<D>(pr, p, buf, w, b, t0, rb, re, window, len);
                                };
                                for (int n0 = 0; n0 < ahead; ++n0) issue(s0 + n0 * group_tokens);
                                for (int c = 0; c < block; ++c) {
                                    if (s0 + c * group_tokens >= re) break;
                                    if (c + ahead < block) issue(s0 + (c + ahead) * group_tokens);
                                }
                            }
                        }
                        if (rows) continue;  // no state stores: the fold below writes out
                        // State stores: one state per live head of the tile;
                        // a combining workgroup's later quarters store the empty
                        // state in their own slots.
                        const int part = split * kQuarters + w.quarter;
                        AUDIT(part >= 0 && part < kQuarters * pr.splits, "state %d", part);
                        for (int h = 0; h < w.heads_here; ++h) {
                            const int64_t row = w.q_row + h;
                            AUDIT(numerator_offset(p, row, part, D) + D <= static_cast<int64_t>(buf.numerator_elems),
                                  "numerator store");
                            AUDIT(stats_offset(p, row, part) + 2 <= static_cast<int64_t>(buf.stats_elems), "stats store");
                            cov.store(static_cast<uint64_t>(row) * kQuarters * pr.splits + part, row, xcd);
                            // Empty states of the span's other live partitions.
                            const int extra = extra_live_partitions(p, split, r.count, len_raw);
                            for (int e = 1; e <= extra; ++e) {
                                const int ep = (split + e) * kQuarters + w.quarter;
                                AUDIT(stats_offset(p, row, ep) + 2 <= static_cast<int64_t>(buf.stats_elems),
                                      "empty-state store");
                                cov.store(static_cast<uint64_t>(row) * kQuarters * pr.splits + ep, row, xcd);
                            }
                        }
                        if (mfma && p.combine) {
                            const int qq = wave % qw;
                            const int slot_bytes = combine_slot_bytes(D);
                            const int base = waves * mfma_stage_bytes(D, pr.kv_elem);
                            const int lds = mfma_lds_bytes(p, D, pr.kv_elem);
                            if (qq != 0)
                                AUDIT(base + (wave / qw * (qw - 1) + qq) * slot_bytes <= lds, "combine slot write");
                            else
                                AUDIT(base + (wave / qw * (qw - 1) + qw - 1) * slot_bytes <= lds, "combine slot read");
                        }
                    }
                }
                if (rows) {
                    // The fold. Matrix-core kernel: output element o of the
                    // row's live heads, o < heads_here * D, is column o % 16,
                    // dims (o / 16) % (D / 16) of head o / D, read from lane
                    // 16 (h / 4) + col of each slot. FP32 kernel: element o is
                    // slot word 16 + o.
                    const int vh = D / 16;
                    for (int o = 0; o < row_heads * D; ++o) {
                        if (mfma) {
                            const int col = o % 16, j = (o / 16) % vh, h = o / D;
                            AUDIT(h < GT && 16 * (h / 4) + col < kWave && j < vh, "fold element %d", o);
                            out.store((row_q + h) * D + col * vh + j);
                        } else {
                            AUDIT(16 + o < row_slot_bytes_fp32(D) / 4 && o / D < GT, "fold element %d", o);
                            out.store(row_q * D + o);
                        }
                    }
                }
            }
        }
    }
}

template <int D>
void audit_gt(const Problem& pr, const PartialParams& p, bool mfma, Coverage& cov, OutCoverage& out) {
    switch (p.head_tile) {
        case 1: return audit_launch<D, 1>(pr, p, mfma, cov, out);
        case 2: return audit_launch<D, 2>(pr, p, mfma, cov, out);
        case 4: return audit_launch<D, 4>(pr, p, mfma, cov, out);
        case 8: return audit_launch<D, 8>(pr, p, mfma, cov, out);
        default: return audit_launch<D, 16>(pr, p, mfma, cov, out);
    }
}

// Audits the launch planned for a partition-only call (states), and for a
// full decode call (rows: the planner may choose a whole-row launch).
bool audit(const Problem& pr, bool rows) {
    const int before = g_failures;
    const uint64_t checks_before = g_checks;
    const bool mfma = pr.q_elem == 2;
    const PartialParams p = params(pr, 256, mfma, rows);
    Coverage cov(static_cast<uint64_t>(pr.batch) * pr.q_heads * kQuarters * pr.splits,
                 static_cast<uint64_t>(pr.batch) * pr.q_heads);
    OutCoverage out(static_cast<uint64_t>(pr.batch) * pr.q_heads * pr.head_dim);
    if (pr.head_dim == 64) audit_gt<64>(pr, p, mfma, cov, out);
    else audit_gt<128>(pr, p, mfma, cov, out);
    if (p.row_mode) {
        AUDIT(mfma_lds_bytes(p, pr.head_dim, pr.kv_elem) <= 160 * 1024, "whole-row LDS");
        for (size_t e = 0; e < out.writes.size(); ++e)
            AUDIT(out.writes[e] == 1, "output element %zu written %d times", e, out.writes[e]);
    } else {
        check_coverage(pr, cov);
        if (p.merge_xcd_rows > 0) check_merge_xcd(pr, p, cov);
    }
    const Grid grid = partial_grid(p, pr.kv_heads);
    std::printf("%-44s %s grid %ux%ux%u x %d waves, GT %d, qw %d, %s%s%s, %" PRIu64 " checks: %s\n",
                (pr.name + (rows ? " [call]" : "")).c_str(), mfma ? "mfma" : "fp32", grid.x, grid.y, grid.z,
                partial_threads(p) / kWave, p.head_tile, p.quarters_per_wg,
                p.row_mode ? "whole rows" : p.compact ? "compact" : p.main_splits < p.splits ? "rectangular+tails"
                                                                                              : "rectangular",
                p.combine ? ", combined" : "",
                p.xcd_shift >= 0 ? ", xcd-grouped" : p.merge_xcd_rows > 0 ? ", xcd merge" : "",
                g_checks - checks_before, g_failures == before ? "ok" : "FAILED");
    std::fflush(stdout);
    return g_failures == before;
}

// Deterministic generator for tables and lengths.
struct Lcg {
    uint64_t s;
    uint32_t next() {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        return static_cast<uint32_t>(s >> 33);
    }
    int below(int n) { return static_cast<int>(next() % static_cast<uint32_t>(n)); }
};

// Problem with shuffled pages, `width` logical pages per sequence and the
// given lengths; splits cover `reserve` times the longest sequence.
Problem make(const std::string& name, int batch, int q_heads, int kv_heads, int head_dim, int page_size, int width,
             std::vector<int32_t> lengths, int split_tokens, int q_elem, int kv_elem, uint64_t seed,
             int reserve = 1) {
    Problem pr;
    pr.name = name;
    pr.batch = batch;
    pr.q_heads = q_heads;
    pr.kv_heads = kv_heads;
    pr.head_dim = head_dim;
    pr.page_size = page_size;
    pr.width = width;
    pr.pages = batch * width;
    pr.q_elem = q_elem;
    pr.kv_elem = kv_elem;
    pr.split_tokens = split_tokens;
    pr.caller_split_tokens = split_tokens;
    pr.lengths = lengths;
    int longest = 0;
    for (int v : lengths) longest = imax(longest, v);
    const int capacity = width * page_size;
    const int reserved = imin(capacity, imax(1, longest) * reserve);
    pr.splits = imax(1, (reserved + split_tokens - 1) / split_tokens);
    pr.caller_splits = pr.splits;
    std::vector<int32_t> perm(pr.pages);
    for (int i = 0; i < pr.pages; ++i) perm[i] = i;
    Lcg rng{seed};
    for (int i = pr.pages - 1; i > 0; --i) std::swap(perm[i], perm[rng.below(i + 1)]);
    pr.table.assign(static_cast<size_t>(batch) * width, -1);
    for (int b = 0; b < batch; ++b)
        for (int i = 0; i < width; ++i) pr.table[static_cast<size_t>(b) * width + i] = perm[b * width + i];
    return pr;
}

std::vector<int32_t> uniform(int batch, int len) { return std::vector<int32_t>(batch, len); }

std::vector<int32_t> ragged(int batch, int hi, uint64_t seed) {
    Lcg rng{seed};
    std::vector<int32_t> v(batch);
    for (auto& x : v) x = rng.below(hi + 1);
    v[0] = hi;
    if (batch > 2) v[1] = 0;
    return v;
}

// The same problem with host bounds: exact lengths, half, zero, or none.
std::vector<Problem> with_bounds(const Problem& base) {
    std::vector<Problem> out{base};
    const char* kinds[] = {"exact", "half", "zero"};
    for (int k = 0; k < 3; ++k) {
        Problem pr = base;
        pr.name += std::string(" bounds=") + kinds[k];
        pr.bounds = base.lengths;
        for (auto& x : pr.bounds) x = k == 0 ? x : k == 1 ? x / 2 : 0;
        out.push_back(pr);
    }
    return out;
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "";
    const bool quick = mode == "--quick";
    std::vector<Problem> problems;
    auto add = [&](const Problem& pr, bool bounds = true) {
        if (bounds) for (const auto& x : with_bounds(pr)) problems.push_back(x);
        else problems.push_back(pr);
    };
    // The five measured workloads (FP32 oracle case; Llama-3-8B FP16 and FP8;
    // ragged + shared pages; MQA; long-context MHA over its split sweep).
    add(make("fp32 B2 Hq8/2 D64 L[100,256] split 256", 2, 8, 2, 64, 16, 16, {100, 256}, 256, 4, 4, 1));
    add(make("fp32 B2 Hq8/2 D64 L[100,256] split 32", 2, 8, 2, 64, 16, 16, {100, 256}, 32, 4, 4, 1));
    add(make("llama3-8b B4 L4096 fp16", 4, 32, 8, 128, 16, 256, uniform(4, 4096), 256, 2, 2, 2));
    add(make("llama3-8b B4 L4096 fp8", 4, 32, 8, 128, 16, 256, uniform(4, 4096), 256, 2, 1, 2));
    {
        Problem pr = make("ragged shared B16 T32 split 128", 16, 32, 8, 128, 32, 256, ragged(16, 8192, 3), 128, 2, 2, 3);
        for (int b = 1; b < 16; ++b)  // a 25% shared prefix: the first 64 pages of sequence 0
            for (int i = 0; i < 64; ++i) pr.table[static_cast<size_t>(b) * 256 + i] = pr.table[i];
        pr.unshared = false;
        pr.ragged = true;
        add(pr);
        Problem reserved = make("ragged B16 T32 split 128 reserve x4", 16, 32, 8, 128, 32, 1024, ragged(16, 8192, 3),
                                128, 2, 2, 3, 4);
        add(reserved);
    }
    add(make("mqa B128 Hq16/1 D64 L1024", 128, 16, 1, 64, 16, 64, uniform(128, 1024), 256, 2, 2, 4), false);
    add(make("mqa B64 Hq16/1 D64 ragged split 64", 64, 16, 1, 64, 16, 64, ragged(64, 1024, 41), 64, 2, 2, 41));
    for (int split : {128, 256, 512, 1024})
        add(make("long mha B1 Hq32/32 L32768 split " + std::to_string(split), 1, 32, 32, 128, 16, 2048,
                 uniform(1, 32768), split, 2, 2, 5),
            !quick && split == 128);
    // XCD-grouped grids (plan_xcd) under exact bounds, the shapes of
    // tests/test_gpu_xcd_grid.py: both merge kernels' row maps are walked too.
    add(make("xcd gqa4 B8 Hq32/8 D128 L1024 split 128 fp16", 8, 32, 8, 128, 16, 64, uniform(8, 1024), 128, 2, 2, 71));
    add(make("xcd gqa4 B8 Hq32/8 D128 L1024 split 128 fp8", 8, 32, 8, 128, 16, 64, uniform(8, 1024), 128, 2, 1, 71));
    add(make("xcd mqa B64 Hq16/1 D64 L1024 split 256 fp16", 64, 16, 1, 64, 16, 64, uniform(64, 1024), 256, 2, 2, 73));
    add(make("xcd mha B2 Hq16/16 D128 L2048 split 256 fp16", 2, 16, 16, 128, 16, 128, uniform(2, 2048), 256, 2, 2, 75));
    add(make("xcd fp32 B8 Hq16/8 D64 L1024 split 128", 8, 16, 8, 64, 16, 64, uniform(8, 1024), 128, 4, 4, 77));
    // Eight head groups per sequence: the plain grids (rectangular, with
    // tails, or a work list) already keep a row group on one XCD, and only
    // the merge is XCD-grouped, whatever the lengths.
    add(make("xcd merge ragged mha B16 Hq32/32 D128 split 128", 16, 32, 32, 128, 16, 64, ragged(16, 1024, 83), 128, 2,
             2, 83));
    // Seeded random problems (small sizes), each with every kind of bounds:
    // batch sizes and head layouts that do and do not make the XCD-grouped
    // grids, uniform and ragged lengths, reserved context, both page sizes,
    // head dimensions and element sizes.
    {
        Lcg rng{2026};
        const int kv_choices[] = {1, 2, 4, 8, 16, 32};
        const int group_choices[] = {1, 2, 3, 4, 8, 16};
        const int batch_choices[] = {1, 2, 3, 4, 6, 8, 12, 16};
        const int split_choices[] = {16, 32, 64, 128, 256};
        for (int i = 0; i < (quick ? 8 : 40); ++i) {
            const int kv = kv_choices[rng.below(6)];
            const int group = group_choices[rng.below(6)];
            const int batch = batch_choices[rng.below(8)];
            const int dim = rng.below(2) ? 128 : 64;
            const int page = rng.below(2) ? 32 : 16;
            const int split = split_choices[rng.below(5)];
            const int len = 1 + rng.below(1024);
            const bool uni = rng.below(2) != 0;
            const int reserve = 1 + rng.below(2);
            const int elems = rng.below(3);  // 0: FP16, 1: FP8 K/V, 2: FP32
            const int q_elem = elems == 2 ? 4 : 2, kv_elem = elems == 0 ? 2 : elems == 1 ? 1 : 4;
            const int width = (len * reserve + page - 1) / page;
            const std::string name = "random " + std::to_string(i) + " B" + std::to_string(batch) + " Hq" +
                                     std::to_string(kv * group) + "/" + std::to_string(kv) + " D" +
                                     std::to_string(dim) + " T" + std::to_string(page) + (uni ? " L" : " ragged L") +
                                     std::to_string(len) + " x" + std::to_string(reserve) + " split " +
                                     std::to_string(split) + (elems == 2 ? " fp32" : elems == 1 ? " fp8" : " fp16");
            add(make(name, batch, kv * group, kv, dim, page, width,
                     uni ? uniform(batch, len) : ragged(batch, len, 100 + i), split, q_elem, kv_elem, 100 + i,
                     reserve));
        }
    }
    // Reserved context over uniform lengths: tail rows, partly empty slots.
    add(make("xcd llama3-8b B4 L4096 reserve x4", 4, 32, 8, 128, 16, 1024, uniform(4, 4096), 256, 2, 2, 79, 4));
    add(make("xcd mqa B128 Hq16/1 D64 L1024 reserve x2", 128, 16, 1, 64, 16, 128, uniform(128, 1024), 256, 2, 2, 81,
             2));
    // Device lengths past the caller's partitions (splits * split_tokens <
    // length <= table capacity): a full call over coarser partitions must
    // still read only the first splits * split_tokens tokens. B64, 3
    // partitions of 256 tokens, lengths 1000 in a 1024-token table: the
    // coarse split is 2 x 512, whose second partition would reach token 999.
    {
        Problem pr = make("past reach B64 Hq32/8 D128 splits 3x256 L1000", 64, 32, 8, 128, 16, 64, uniform(64, 1000),
                          256, 2, 2, 19);
        pr.splits = pr.caller_splits = 3;
        add(pr);
        Problem ragged_past = make("past reach B16 Hq8/2 D64 splits 5x64 ragged", 16, 8, 2, 64, 16, 32,
                                   ragged(16, 512, 23), 64, 2, 2, 23);
        ragged_past.splits = ragged_past.caller_splits = 5;
        add(ragged_past);
        Problem fp8_past = make("past reach B32 Hq16/4 D128 fp8 splits 6x128 L900", 32, 16, 4, 128, 32, 32,
                                uniform(32, 900), 128, 2, 1, 29);
        fp8_past.splits = fp8_past.caller_splits = 6;
        add(fp8_past);
    }
    // Edge lengths around page and partition boundaries, both page sizes.
    for (int page : {16, 32}) {
        add(make("edges fp16 page " + std::to_string(page), 8, 8, 2, 128, page, 8,
                 {0, 1, page - 1, page, page + 1, 2 * page - 1, 2 * page + 1, 8 * page}, 33, 2, 2, 7));
        add(make("edges fp32 page " + std::to_string(page), 8, 8, 2, 64, page, 8,
                 {0, 1, page - 1, page, page + 1, 2 * page - 1, 2 * page + 1, 8 * page}, 1, 4, 4, 7));
    }
    // Invalid page ids inside live ranges (parked loads) and lengths beyond
    // the table (clamped).
    {
        Problem pr = make("invalid page ids fp16", 4, 16, 4, 128, 16, 16, {256, 200, 300, 17}, 64, 2, 2, 9);
        pr.table[3] = -1;
        pr.table[16 + 5] = pr.pages;
        pr.table[32 + 0] = 2147483647;
        pr.table[48 + 1] = -2147483647 - 1;
        add(pr);
        Problem f = make("invalid page ids fp32", 4, 16, 4, 64, 16, 16, {256, 200, 300, 17}, 64, 4, 4, 9);
        f.table = pr.table;
        add(f);
        Problem e8 = make("invalid page ids fp8", 4, 16, 4, 64, 16, 16, {256, 200, 300, 17}, 64, 2, 1, 9);
        e8.table = pr.table;
        add(e8);
    }
    // Uncommon head layouts (partial and multiple head tiles, odd workgroups).
    for (auto hk : std::vector<std::pair<int, int>>{{12, 4}, {20, 4}, {48, 2}, {96, 4}, {21, 3}, {35, 5}, {42, 7},
                                                    {66, 11}, {80, 20}, {72, 12}, {24, 1}}) {
        add(make("heads " + std::to_string(hk.first) + "/" + std::to_string(hk.second) + " fp16", 3, hk.first,
                 hk.second, 128, 16, 12, {192, 77, 150}, 64, 2, 2, 11),
            false);
        add(make("heads " + std::to_string(hk.first) + "/" + std::to_string(hk.second) + " fp32", 3, hk.first,
                 hk.second, 64, 16, 12, {192, 77, 150}, 64, 4, 4, 11),
            false);
    }
    // Whole-row launches (a full decode call of at most four partitions per
    // row): ragged lengths with empty rows and partial partitions, GQA and
    // MQA tiles, both head dimensions, FP8 K/V, page 32, a single partition
    // per row, invalid page ids.
    add(make("rows mqa B128 D64 ragged split 256", 128, 16, 1, 64, 16, 64, ragged(128, 1024, 51), 256, 2, 2, 51),
        false);
    add(make("rows B64 Hq32/8 D128 ragged split 192", 64, 32, 8, 128, 16, 32, ragged(64, 512, 53), 192, 2, 2, 53),
        false);
    add(make("rows B64 Hq32/8 D128 fp8 split 192", 64, 32, 8, 128, 32, 16, ragged(64, 512, 55), 192, 2, 1, 55),
        false);
    add(make("rows B2 Hq8/2 D64 L[100,256] split 256", 2, 8, 2, 64, 16, 16, {100, 256}, 256, 2, 2, 57), false);
    add(make("rows B3 Hq20/4 D128 split 512 page 32", 3, 20, 4, 128, 32, 16, {512, 1, 0}, 512, 2, 2, 59), false);
    {
        Problem pr = make("rows invalid page ids B32 Hq16/4 split 64", 32, 16, 4, 64, 16, 16, ragged(32, 256, 61), 64,
                          2, 2, 61);
        pr.table[3] = -1;
        pr.table[16 + 5] = pr.pages;
        pr.table[32 + 0] = 2147483647;
        add(pr, false);
    }
    if (!quick) {
        // A 1M-token context in a 65536-wide table (16384 states per row).
        add(make("1M context W65536 fp16", 1, 8, 2, 128, 16, 65536, uniform(1, 1 << 20), 256, 2, 2, 13), false);
        // Live pages above 4 GiB of cache (64-bit page offsets).
        Problem big = make("pages above 4 GiB", 2, 32, 8, 128, 16, 64, {1024, 700}, 128, 2, 2, 17);
        big.pages = 163840;  // 5 GiB per K/V tensor at 32 KB per page
        for (int i = 0; i < 128; ++i) big.table[i] = 163840 - 1 - i;
        add(big);
    }
    if (mode == "--plant-reach") {
        // Negative control: the same problems with launch params that clamp
        // lengths to the table only. The walk must report reads past the
        // caller's partitions.
        g_plant_reach = true;
        std::vector<Problem> planted;
        for (const auto& pr : problems)
            if (pr.name.rfind("past reach", 0) == 0) planted.push_back(pr);
        problems = planted;
    }
    int failed = 0;
    for (const auto& pr : problems) {
        failed += audit(pr, false) ? 0 : 1;
        // The plan for a full decode call, when it is a whole-row launch.
        if (params(pr, 256, pr.q_elem == 2, true).row_mode) failed += audit(pr, true) ? 0 : 1;
        // A full call over coarser partitions: fewer of them, covering at
        // least the caller's, their states inside the caller's workspace
        // (the audited buffers are those of the coarser split, a prefix).
        const KernelSplit ks = full_call_split(pr.q_elem == 4, pr.kv_elem, pr.batch, pr.q_heads, pr.kv_heads,
                                               pr.head_dim, pr.page_size, pr.width, pr.splits, pr.split_tokens,
                                               pr.bounds.empty() ? nullptr : pr.bounds.data(), 256);
        if (ks.splits != pr.splits || ks.split_tokens != pr.split_tokens) {
            AUDIT(ks.splits < pr.splits && ks.split_tokens % pr.split_tokens == 0 &&
                      static_cast<int64_t>(ks.splits) * ks.split_tokens >=
                          static_cast<int64_t>(pr.splits) * pr.split_tokens,
                  "coarse split %d x %d for %d x %d", ks.splits, ks.split_tokens, pr.splits, pr.split_tokens);
            Problem coarse = pr;
            coarse.name += " coarse x" + std::to_string(ks.split_tokens / pr.split_tokens);
            coarse.splits = ks.splits;
            coarse.split_tokens = ks.split_tokens;
            failed += audit(coarse, true) ? 0 : 1;
        }
    }
    std::printf("%zu problems, %" PRIu64 " checks, %d failures\n", problems.size(), g_checks, g_failures);
    return failed == 0 ? 0 : 1;
}
