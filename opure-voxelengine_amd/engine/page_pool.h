// ============================================================================
//  page_pool.h -- the free list of a paged KV pool's pages.
//
//  The reference sizes one contiguous cache per layer up front
//  (ModelConfig::KvCacheWords, src/engine/Opure_Graph.h:81-84) and its only way
//  to give positions back is EvictOldestKV (src/engine/Opure_VoxelEngine.cpp:
//  721-763), a memmove that never reaches the KV buffer.  Here sequences own
//  16-token pages of a shared pool through their page-table rows: a sequence
//  takes pages as it grows (GrowSeq, before a verify step writes positions
//  ctx..ctx+K), and opure_kv_rollback hands back the ids of the pages wholly
//  past the accepted length, which go straight to Release.
//
//  Host-only bookkeeping, no device calls; not thread-safe (the engine's
//  caller serialises, as for every other engine call).
// ============================================================================
#pragma once

#include <cstdint>
#include <vector>

namespace opure::engine {

class PagePool {
public:
    explicit PagePool(uint32_t nPages);

    [[nodiscard]] uint32_t Capacity() const { return static_cast<uint32_t>(inUse_.size()); }
    [[nodiscard]] uint32_t Available() const { return static_cast<uint32_t>(free_.size()); }

    // n pages into ids[0..n), all or none: Error(OPURE_E_CAPACITY) when fewer
    // than n are free.  A fresh pool hands out 0, 1, 2, ...; a released page
    // is handed out again before any page that was never used (last in,
    // first out).
    void Alloc(uint32_t n, int32_t* ids);

    // Returns pages to the pool.  Entries < 0 (the -1 padding of the
    // rollback's freed lists) are skipped.  An id past the pool, one not
    // handed out, or one listed twice is Error(OPURE_E_INVALID), and then
    // nothing is released.
    void Release(const int32_t* ids, uint32_t n);

    // Makes entries [0, ceil(tokens / pageSize)) of one sequence's page-table
    // row valid, taking a page for each entry < 0; all or none
    // (Error(OPURE_E_CAPACITY) when the row or the pool is too short).
    // Returns the number of pages taken.
    uint32_t GrowSeq(int32_t* row, uint32_t maxPages, uint32_t tokens, uint32_t pageSize);

private:
    std::vector<int32_t> free_;    // stack: the next page handed out is free_.back()
    std::vector<uint8_t> inUse_;   // 1 while a page is handed out
};

}  // namespace opure::engine
