// air_hip_kv.hpp -- device view of the paged fp32 KV pool (internal).
//
// Page p of the pool holds [layer][K, V][page_tokens][kv_width] floats; a
// sequence is named by its page table (int32 page indices, max_pages per
// row).  The pool is either one allocation (page p at pool + p pages) or a
// table of separately allocated chunks of 2^chunk_shift pages each (page p
// in chunk p >> chunk_shift), so a pool can grow without moving the pages it
// already holds.  Slots whose table entry is outside [0, pool_pages), or in
// a chunk not allocated yet, read as absent.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace air_hip {

struct KvGeometry {
    float* pool;                  // contiguous pool, or null when chunks is set
    std::uint32_t page_tokens;
    std::uint32_t kv_width;       // kv_heads * head_dim
    std::uint32_t layers;
    std::uint32_t max_pages;      // page-table row length
    std::uint32_t pool_pages;     // page ids accepted: [0, pool_pages)
    float* const* chunks;         // pool_pages >> chunk_shift chunk bases (null: not allocated)
    std::uint32_t chunk_shift;
};

__device__ __forceinline__ std::uint64_t page_floats(const KvGeometry& g) {
    return static_cast<std::uint64_t>(g.layers) * 2u * g.page_tokens * g.kv_width;
}

// First float of page `page`, or null when the pool holds no such page.
__device__ __forceinline__ float* kv_page(const KvGeometry& g, std::int32_t page) {
    if (page < 0 || static_cast<std::uint32_t>(page) >= g.pool_pages) return nullptr;
    const std::uint32_t p = static_cast<std::uint32_t>(page);
    if (g.chunks == nullptr) return g.pool + static_cast<std::uint64_t>(p) * page_floats(g);
    float* const base = g.chunks[p >> g.chunk_shift];
    if (base == nullptr) return nullptr;
    return base + static_cast<std::uint64_t>(p & ((1u << g.chunk_shift) - 1u)) * page_floats(g);
}

// K and V of (layer, token) of a row's sequence; null when the page table
// does not name a page of the pool (the caller skips the token).
__device__ __forceinline__ float* kv_slot(const KvGeometry& g, const std::int32_t* table, std::uint32_t layer,
                                          std::uint64_t token, bool value) {
    const std::uint64_t slot = token / g.page_tokens;
    if (slot >= g.max_pages) return nullptr;
    float* const page = kv_page(g, table[slot]);
    if (page == nullptr) return nullptr;
    return page + ((static_cast<std::uint64_t>(layer) * 2u + (value ? 1u : 0u)) * g.page_tokens +
                   token % g.page_tokens) *
                      g.kv_width;
}

} // namespace air_hip
