// Address map of the cache-metadata kernels, shared by the device code in
// decode.hip and the host: where the paged KV-cache append reads its page ids
// and which cache rows it writes, and which CSR entries the device CSR -> page
// table conversion reads and writes. Plain integer arithmetic (host and
// gfx950); tests/address_audit.cpp walks every workgroup and lane of both
// kernels through these functions and checks each access against the
// caller's buffers.
//
// The append writes where the decode reads: token t of sequence b at page
// table[b, t / T], slot t % T (reference docs/DESIGN.md:10-13). The CSR form is
// the one reference src/paged_decode/competitors.py:8-18 builds from a table.
#ifndef PAGED_DECODE_CACHE_MAP_H
#define PAGED_DECODE_CACHE_MAP_H

#include "partition_map.h"

namespace pd {

struct AppendParams {
    const char* k_new;
    const char* v_new;
    const int32_t* table;
    const int32_t* positions;  // explicit variant: first position per sequence
    int32_t* lengths;          // advance variant: positions in, advanced lengths out
    char* k_cache;
    char* v_cache;
    int tokens;
    int table_width;
    int page_shift;
    int physical_pages;
    int64_t capacity;          // positions [0, capacity) may be written: the table's, or less (advance variant)
    uint32_t row_bytes;        // kv_heads * head_dim * element size
};

// Table entry (within sequence b's row) holding the page of logical position
// pos, or -1 if pos is outside [0, capacity); capacity never exceeds the
// table's width * page_size.
PD_HD int64_t append_table_entry(const AppendParams& a, int64_t pos) {
    if (pos < 0 || pos >= a.capacity) return -1;
    return pos >> a.page_shift;
}

// Physical cache row of logical position pos on page `page`, or -1 if the
// page id is outside [0, physical_pages).
PD_HD int64_t append_cache_row(const AppendParams& a, int page, int64_t pos) {
    if (static_cast<uint32_t>(page) >= static_cast<uint32_t>(a.physical_pages)) return -1;
    return (static_cast<int64_t>(page) << a.page_shift) + (pos & ((1 << a.page_shift) - 1));
}

// Row of the new-token tensors [B, tokens, Hkv, D] holding token j of sequence b.
PD_HD int64_t append_source_row(const AppendParams& a, int b, int j) {
    return static_cast<int64_t>(b) * a.tokens + j;
}

// Byte offset of 16-byte chunk c of token row `row` (new tokens or cache).
PD_HD int64_t append_chunk_offset(const AppendParams& a, int64_t row, uint32_t c) {
    return row * a.row_bytes + static_cast<int64_t>(c) * 16;
}

struct CsrParams {
    const int32_t* indptr;
    const int32_t* indices;
    const int32_t* last_page_len;
    int32_t* table;
    int32_t* lengths;
    int32_t* overflow;  // may be null
    int64_t indices_count;  // entries of indices: no page list reaches past it
    int table_width;
    int page_size;
    int max_context;
};

// Row b of the conversion, from its indptr pair and last-page length: the
// page ids it copies (live, from indices[begin] on), its length, and whether
// it fits (else the row is written empty and the overflow flag raised).
struct CsrRow {
    int64_t begin, live, length;
    bool fits;
};

PD_HD CsrRow csr_row(const CsrParams& c, int64_t begin, int64_t end, int last_page_len) {
    CsrRow r;
    const int64_t n = end - begin;
    const int last = n > 0 ? last_page_len : 0;
    r.begin = begin;
    r.length = n > 0 ? (n - 1) * c.page_size + last : 0;
    r.fits = n >= 0 && n <= c.table_width && begin >= 0 && end <= c.indices_count &&
             (n == 0 || (last >= 1 && last <= c.page_size)) && r.length <= c.max_context;
    r.live = r.fits ? n : 0;
    return r;
}

}  // namespace pd

#endif  // PAGED_DECODE_CACHE_MAP_H
