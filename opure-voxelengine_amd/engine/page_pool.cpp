// ============================================================================
//  page_pool.cpp -- PagePool: the free list of a paged KV pool.
// ============================================================================
#include "page_pool.h"

#include <string>

#include "opure_hip.h"
#include "voxel_engine.h"

namespace opure::engine {

PagePool::PagePool(uint32_t nPages) : inUse_(nPages, 0)
{
    if (nPages == 0 || nPages > 0x7FFFFFFFu) throw Error(OPURE_E_INVALID, "PagePool: page count out of range");
    free_.reserve(nPages);
    for (uint32_t i = nPages; i-- > 0;) free_.push_back(static_cast<int32_t>(i));
}

void PagePool::Alloc(uint32_t n, int32_t* ids)
{
    if (n && !ids) throw Error(OPURE_E_INVALID, "PagePool::Alloc: null id array");
    if (n > free_.size())
        throw Error(OPURE_E_CAPACITY, "PagePool::Alloc: " + std::to_string(n) + " pages asked, " +
                                          std::to_string(free_.size()) + " free");
    for (uint32_t i = 0; i < n; ++i)
    {
        const int32_t id = free_.back();
        free_.pop_back();
        inUse_[static_cast<uint32_t>(id)] = 1;
        ids[i] = id;
    }
}

void PagePool::Release(const int32_t* ids, uint32_t n)
{
    if (n && !ids) throw Error(OPURE_E_INVALID, "PagePool::Release: null id array");
    // validate the whole list first (marking with 2), then commit
    uint32_t i = 0;
    for (; i < n; ++i)
    {
        const int32_t id = ids[i];
        if (id < 0) continue;
        if (static_cast<uint32_t>(id) >= inUse_.size() || inUse_[static_cast<uint32_t>(id)] != 1) break;
        inUse_[static_cast<uint32_t>(id)] = 2;
    }
    if (i < n)
    {
        const int32_t bad = ids[i];
        for (uint32_t j = 0; j < i; ++j)
            if (ids[j] >= 0) inUse_[static_cast<uint32_t>(ids[j])] = 1;
        throw Error(OPURE_E_INVALID, "PagePool::Release: page " + std::to_string(bad) +
                                         (static_cast<uint32_t>(bad) >= inUse_.size() ? " is past the pool"
                                                                                      : " is not in use (or listed twice)"));
    }
    for (uint32_t j = 0; j < n; ++j)
    {
        if (ids[j] < 0) continue;
        inUse_[static_cast<uint32_t>(ids[j])] = 0;
        free_.push_back(ids[j]);
    }
}

uint32_t PagePool::GrowSeq(int32_t* row, uint32_t maxPages, uint32_t tokens, uint32_t pageSize)
{
    if (!row || pageSize == 0) throw Error(OPURE_E_INVALID, "PagePool::GrowSeq: bad argument");
    const uint64_t need = (static_cast<uint64_t>(tokens) + pageSize - 1u) / pageSize;
    if (need > maxPages)
        throw Error(OPURE_E_CAPACITY, "PagePool::GrowSeq: " + std::to_string(tokens) + " tokens need " +
                                          std::to_string(need) + " pages, the row holds " + std::to_string(maxPages));
    uint32_t missing = 0;
    for (uint32_t i = 0; i < need; ++i) missing += row[i] < 0 ? 1u : 0u;
    std::vector<int32_t> got(missing);
    Alloc(missing, got.data());
    for (uint32_t i = 0, k = 0; i < need; ++i)
        if (row[i] < 0) row[i] = got[k++];
    return missing;
}

}  // namespace opure::engine
