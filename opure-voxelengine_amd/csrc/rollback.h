// ============================================================================
//  rollback.h -- the KV rollback of one sequence after acceptance, run by one
//  workgroup: shared by the acceptance kernels (accept.hip) and the LM head's
//  in-launch greedy acceptance (gemv_kernel.h).
// ============================================================================
#pragma once
#include "internal.h"

namespace opure_hip {

using opure_dev_math::kv_elem;

// What a sequence's rollback reads before it can decide anything: its
// context length and the page-table entries of positions ctx .. ctx + K (at
// most two pages, K + 1 <= 16).  Loaded together, early, by one thread.
struct RollbackPre {
    uint32_t ctx;
    int32_t pte[2];           // entries ctx/16 and ctx/16 + 1 (-1 past the table)
};

__device__ __forceinline__ RollbackPre rollback_pre(const RollbackParams& p, uint32_t b)
{
    RollbackPre r;
    r.ctx = static_cast<uint32_t>(p.seq_len[b]);
    const int32_t* pt = p.page_table + static_cast<uint64_t>(b) * p.max_pages;
    const uint32_t q0 = r.ctx / OPURE_PAGE_SIZE;
    r.pte[0] = q0 < p.max_pages ? pt[q0] : -1;
    r.pte[1] = q0 + 1u < p.max_pages ? pt[q0 + 1u] : -1;
    return r;
}

// Rollback of sequence b, run by one workgroup: poison the rolled-back slots,
// then release the pages wholly past the new length.  `pre` (from
// rollback_pre, shared by the workgroup) holds everything read before the
// writes, so the rollback costs no further round trip to memory.
__device__ inline void rollback_seq(const RollbackParams& p, uint32_t b, uint32_t acc, const RollbackPre& pre)
{
    int32_t* pt = p.page_table + static_cast<uint64_t>(b) * p.max_pages;
    const uint32_t ctx = pre.ctx, q0 = ctx / OPURE_PAGE_SIZE;
    if (acc > p.K) acc = p.K;
    const uint32_t old_end = ctx + p.K + 1u, nl = ctx + acc + 1u;
    // positions nl .. old_end - 1 lie in pages q0 and q0 + 1
    auto entry = [&](uint32_t q) { return pre.pte[q - q0]; };
    if (p.poison)
    {
        const uint32_t per_pos = p.n_layers * 2u * p.n_kv * p.hd;
        for (uint32_t pos = nl; pos < old_end; ++pos)
        {
            if (pos / OPURE_PAGE_SIZE >= p.max_pages) break;
            const int32_t page = entry(pos / OPURE_PAGE_SIZE);
            if (page < 0 || static_cast<uint32_t>(page) >= p.n_pages) continue;
            for (uint32_t e = threadIdx.x; e < per_pos; e += blockDim.x)
            {
                const uint32_t d = e % p.hd, rest = e / p.hd;
                const uint32_t h = rest % p.n_kv, rest2 = rest / p.n_kv;
                const uint32_t s = rest2 % 2u, L = rest2 / 2u;
                const uint64_t idx = kv_elem(L, p.n_pages, static_cast<uint32_t>(page), s, p.n_kv, h, p.hd,
                                             pos % OPURE_PAGE_SIZE, d);
                if (p.afmt == OPURE_A_F32) static_cast<uint32_t*>(p.pool)[idx] = p.poison_bits;
                else static_cast<uint16_t*>(p.pool)[idx] = static_cast<uint16_t>(p.poison_bits);
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0)
    {
        p.new_len[b] = static_cast<int32_t>(nl);
        int32_t nf = 0;
        if (p.freed)
        {
            const uint32_t first_free = (nl + OPURE_PAGE_SIZE - 1u) / OPURE_PAGE_SIZE;
            const uint32_t last_used = (old_end - 1u) / OPURE_PAGE_SIZE;
            for (uint32_t q = first_free; q <= last_used && q < p.max_pages; ++q)
            {
                if (entry(q) < 0) continue;
                if (static_cast<uint32_t>(nf) < p.freed_stride) p.freed[static_cast<uint64_t>(b) * p.freed_stride + nf] = entry(q);
                pt[q] = -1;
                ++nf;
            }
        }
        if (p.n_freed) p.n_freed[b] = nf;
    }
}

}  // namespace opure_hip
