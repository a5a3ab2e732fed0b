// ============================================================================
//  attention.hip -- paged decode attention for the K+1 verify rows.
//
//  Replaces AttentionMain{hd} (shaders/Opure_FlashAttention_Decode.usf:58-179),
//  which ran one workgroup per query head serially over every position, and
//  the never-dispatched SpeculativeVerifyMain{hd} (Opure_SpeculativeDecode.usf).
//
//  Split-K ("flash-decoding") over fixed chunks of the paged cache: one
//  workgroup per (KV head, chunk, sequence) scores all query rows of that KV
//  head's GQA group against the chunk (query head h reads KV head
//  h / (n_heads / n_kv_heads), Opure_FlashAttention_Decode.usf:71-72), keeps a
//  per-chunk (max, sum, unnormalised output), and a combine kernel merges
//  chunks 0..last(row) in order.  Chunk boundaries sit at fixed positions, so
//  each row's output depends only on its own position: verifying K+1 rows
//  gives bitwise the same rows as K+1 single-row decodes.  Row j of sequence b
//  is at position seq_len[b] + j and sees positions 0 .. seq_len[b] + j.
//  Scores are scaled by attn_scale (1.0 = the reference, which has no
//  1/sqrt(head_dim): Opure_FlashAttention_Decode.usf:91-104).
//
//  fp16/bf16 caches with head_dim 64 or 128 run on matrix cores
//  (k_attn_mfma): S^T = K Q^T and O^T = V^T P^T with v_mfma_f32_16x16x32, K
//  tokens assigned to MFMA rows so that the score tile a lane holds is already
//  its P^T operand, and V read as V^T tiles straight from the channel-major V
//  planes of the pool.  P^T enters as a sum of 16-bit operands: fp16 hi + lo
//  (22 significant bits), bf16 hi + mid + lo (the fp32 probability to within
//  2^-25 relative, where one bf16 operand would give 8 bits).  A bf16 model
//  rounds the attention output to 8 bits next, and any difference from the
//  exactly summed softmax moves some of those roundings.  fp32 caches and other
//  head sizes use VALU kernels.
// ============================================================================
#include "internal.h"

using namespace opure_dev_math;

namespace {

typedef uint32_t u4v __attribute__((ext_vector_type(4)));

struct AttnParams {
    const void* q;
    void* out;
    const void* pool;
    const int32_t* page_table;
    const int32_t* seq_len;
    float* part_acc;     // [B][nkv][npart][Gq][hd]
    float* part_ml;      // [B][nkv][npart][Gq][2]
    uint32_t n_heads, n_kv, hd, rows, n_pages, max_pages, layer, nch, chunk, afmt;
    uint32_t npart;      // partials a (sequence, KV head): one a chunk, or one a group of cpp chunks
    uint32_t cpp;        // chunks a partial
    float scale;
    uint32_t qoff;       // matrix-core path: first query row of this launch
    uint32_t zt;         // matrix-core path: row blocks of 16 * NT rows along blockIdx.z (b = z / zt)
    uint32_t* err;       // opure_dev::err: a row past max_ctx sets ERR_POSITION
};

// zero the elements n.. of a 16-byte piece of consecutive tokens (stale slots
// past the cache may hold anything, even NaN poison, and meet p = 0)
template <int AF>
__device__ __forceinline__ u4v mask_tail(u4v v, uint32_t n)
{
    constexpr uint32_t PER = AF == OPURE_A_F32 ? 1u : 2u;     // elements per dword
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i)
    {
        if (PER == 1u) { if (i >= n) v[i] = 0u; }
        else
        {
            if (2u * i >= n) v[i] = 0u;
            else if (2u * i + 1u >= n) v[i] &= 0x0000FFFFu;
        }
    }
    return v;
}

// wave-wide reductions with a fixed butterfly order (deterministic)
__device__ __forceinline__ float wave_max(float v)
{
    return wave_max64(v);
}
__device__ __forceinline__ float wave_sum(float v)
{
    return wave_sum64(v);
}

__global__ __launch_bounds__(256) void k_attn_chunk_generic(AttnParams p)
{
    extern __shared__ __align__(16) float sm[];
    const uint32_t kh = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
    const uint32_t group = p.n_heads / p.n_kv, R = p.rows, Gq = group * R, hd = p.hd, CH = p.chunk;
    const uint32_t ctx = static_cast<uint32_t>(p.seq_len[b]);
    const uint32_t total = ctx + R;
    const uint32_t t0 = c * CH;
    if (t0 >= total) return;                       // no row reaches this chunk
    const uint32_t kvs = hd + 1;                   // padded row stride (bank spread)
    float* qs = sm;                                // [Gq][hd]
    float* S = qs + Gq * hd;                       // [Gq][CH]
    float* T = S + Gq * CH;                        // [CH][hd+1]  K, then V
    const int32_t* pt = p.page_table + static_cast<uint64_t>(b) * p.max_pages;

    for (uint32_t e = threadIdx.x; e < Gq * hd; e += 256u)
    {
        const uint32_t qi = e / hd, d = e - qi * hd;
        const uint32_t j = qi / group, head = kh * group + (qi - j * group);
        qs[e] = load_act_rt(p.q, (static_cast<uint64_t>(b * R + j) * p.n_heads + head) * hd + d, p.afmt);
    }
    auto stage = [&](uint32_t kvsel) {
        for (uint32_t e = threadIdx.x; e < CH * hd; e += 256u)
        {
            const uint32_t tl = e / hd, d = e - tl * hd, pos = t0 + tl;
            float v = 0.0f;
            if (pos < total)
            {
                // a missing page or a length past the table reads as NaN, never out of bounds
                const int32_t page = pos / OPURE_PAGE_SIZE < p.max_pages ? pt[pos / OPURE_PAGE_SIZE] : -1;
                if (page < 0 || static_cast<uint32_t>(page) >= p.n_pages) { T[tl * kvs + d] = __builtin_nanf(""); continue; }
                v = load_act_rt(p.pool, kv_elem(p.layer, p.n_pages, static_cast<uint32_t>(page), kvsel, p.n_kv, kh, hd,
                                                pos % OPURE_PAGE_SIZE, d),
                                p.afmt);
            }
            T[tl * kvs + d] = v;
        }
    };
    stage(0u);
    __syncthreads();

    for (uint32_t e = threadIdx.x; e < Gq * CH; e += 256u)
    {
        const uint32_t qi = e / CH, tl = e - qi * CH;
        const uint32_t j = qi / group;
        float sc = -__builtin_huge_valf();
        if (t0 + tl <= ctx + j)
        {
            const float* qr = qs + qi * hd;
            const float* kr = T + tl * kvs;
            float acc = 0.0f;
            for (uint32_t d = 0; d < hd; ++d) acc = __fmaf_rn(qr[d], kr[d], acc);
            sc = __fmul_rn(acc, p.scale);
        }
        S[e] = sc;
    }
    __syncthreads();

    // per-row softmax over the chunk: one wave per row, CH <= 64 lanes
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint64_t pbase = ((static_cast<uint64_t>(b) * p.n_kv + kh) * p.npart + c) * Gq;
    for (uint32_t qi = wave; qi < Gq; qi += 4u)
    {
        const float s = lane < CH ? S[qi * CH + lane] : -__builtin_huge_valf();
        const float mx = wave_max(s);
        const float e = (s == -__builtin_huge_valf()) ? 0.0f : expf_ref(__fsub_rn(s, mx));
        const float l = wave_sum(e);
        if (lane < CH) S[qi * CH + lane] = e;
        if (lane == 0)
        {
            p.part_ml[(pbase + qi) * 2u] = mx;
            p.part_ml[(pbase + qi) * 2u + 1u] = l;
        }
    }
    __syncthreads();
    stage(1u);
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < Gq * hd; e += 256u)
    {
        const uint32_t qi = e / hd, d = e - qi * hd;
        const float* pr = S + qi * CH;
        float acc = 0.0f;
        for (uint32_t tl = 0; tl < CH; ++tl) acc = __fmaf_rn(pr[tl], T[tl * kvs + d], acc);
        p.part_acc[(pbase + qi) * hd + d] = acc;
    }
}

// Fast path for head_dim <= 128 and 64-token chunks.  The chunk's K and V
// slices of this KV head are staged once in LDS with 128-bit loads; each wave
// then keeps one K row per lane (lane = token) and one or two V columns per
// lane (lane = channel) in registers and walks its share of the query rows:
// scores = K row . q (q broadcast from LDS), a wave-wide softmax over the 64
// tokens, and out[d] = sum_t p_t V[t][d] with p broadcast from LDS.  The
// sequence length, Q and the page-table entries of the workgroup's chunks load
// in one round trip.
// ALL: one workgroup takes every chunk of its (KV head, sequence) in turn (a
// launch of at most ATTN_ALL_CHUNKS chunks), keeps the chunks' partials in LDS
// and merges them with k_attn_combine's operations in its order, so the result
// has the combine's bits and no combine launch follows.
constexpr uint32_t ATTN_ALL_CHUNKS = 4;

template <int HD>
constexpr uint32_t attn_all_lds(uint32_t gq)
{
    return ATTN_ALL_CHUNKS * gq * (HD + 2u) * 4u;
}

// threads of the fast path's workgroup: head_dim 64 runs 8 waves (a row pair
// a wave covers 16 query rows at once), 128 runs 4 (its registers)
template <int HD>
constexpr uint32_t attn_fast_threads()
{
    return HD == 64 ? 512u : 256u;
}

template <int HD, int AF, bool ALL>
__global__ __launch_bounds__(attn_fast_threads<HD>()) void k_attn_chunk(AttnParams p)
{
    constexpr uint32_t NT = attn_fast_threads<HD>(), NWV = NT / 64u, RB = 2;   // RB: rows a wave scores together
    constexpr uint32_t CH = 64, EB = AF == OPURE_A_F32 ? 4u : 2u, PPC = CH / OPURE_PAGE_SIZE;
    constexpr uint32_t ROWB = HD * EB + 16u;              // padded LDS row (bank spread)
    constexpr uint32_t DPL = (HD + 63u) / 64u;             // V channels per lane
    constexpr uint32_t VROWB = CH * EB + 16u;              // padded LDS V column (channel-major)
    constexpr uint32_t NE = ALL ? ATTN_ALL_CHUNKS * PPC : PPC;   // page-table entries staged
    __shared__ __align__(16) uint8_t kt[CH * ROWB];
    __shared__ __align__(16) uint8_t vt[HD * VROWB];
    __shared__ __align__(16) float pbuf[NWV][RB][CH];
    __shared__ int32_t spg[NE];                            // the chunks' page-table entries (-1 past the table)
    __shared__ float wsh[NWV][ATTN_ALL_CHUNKS];            // ALL: a row's chunk weights
    extern __shared__ __align__(16) float qs[];            // [Gq][HD], then (ALL) the chunks' partials

    const uint32_t kh = blockIdx.x, b = blockIdx.z;
    const uint32_t group = p.n_heads / p.n_kv, R = p.rows, Gq = group * R;
    const uint32_t c_first = ALL ? 0u : blockIdx.y, c_end = ALL ? p.nch : blockIdx.y + 1u;
    const int32_t* pt = p.page_table + static_cast<uint64_t>(b) * p.max_pages;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    float* pm = qs + Gq * HD;                              // ALL: [chunk][Gq] maxima
    float* pl = pm + ATTN_ALL_CHUNKS * Gq;                 //      [chunk][Gq] sums
    float* pa = pl + ATTN_ALL_CHUNKS * Gq;                 //      [chunk][Gq][HD] outputs

    // every load issued before any is waited for: the sequence length, the
    // page entries, QU of Q's elements a thread (a row j's group of heads is
    // contiguous in Q), then the stores to LDS
    const int32_t seq = p.seq_len[b];
    constexpr uint32_t QU = 8;
    const uint32_t GH = group * HD;
    float qv[QU];
    auto q_load = [&](uint32_t e0) {
#pragma unroll
        for (uint32_t u = 0; u < QU; ++u)
        {
            const uint32_t e = e0 + threadIdx.x + NT * u, j = e / GH;
            qv[u] = e < Gq * HD ? load_act_rt(p.q, (static_cast<uint64_t>(b * R + j) * p.n_heads + kh * group) * HD + (e - j * GH), AF)
                                : 0.0f;
        }
    };
    auto q_store = [&](uint32_t e0) {
#pragma unroll
        for (uint32_t u = 0; u < QU; ++u)
        {
            const uint32_t e = e0 + threadIdx.x + NT * u;
            if (e < Gq * HD) qs[e] = qv[u];
        }
    };
    q_load(0u);
    int32_t pte = -1;
    if (threadIdx.x < NE && c_first * PPC + threadIdx.x < p.max_pages) pte = pt[c_first * PPC + threadIdx.x];
    q_store(0u);
    for (uint32_t e0 = NT * QU; e0 < Gq * HD; e0 += NT * QU)   // more than NT * QU elements: a block at a time
    {
        q_load(e0);
        q_store(e0);
    }
    if (threadIdx.x < NE) spg[threadIdx.x] = pte;
    // keeps the loads above issued before the exit below
    asm volatile("" ::: "memory");
    const uint32_t ctx = static_cast<uint32_t>(seq);
    const uint32_t total = ctx + R;
    if (c_first * CH >= total) return;                    // no row reaches this chunk
    __syncthreads();                                      // Q and the page entries staged
    // stage K rows (token-major) and V columns (channel-major, as stored):
    // 16-byte pieces; a page's 16 tokens of this head are contiguous in both planes
    constexpr uint32_t KP = HD * EB / 16u;                 // pieces per K row
    constexpr uint32_t VP = CH * EB / 16u;                 // pieces per V column of the chunk
    constexpr uint32_t TPP = 16u / EB;                     // tokens per V piece
    constexpr uint32_t NPC = (CH * KP + HD * VP) / NT;     // pieces a thread stages a chunk
    static_assert((CH * KP) % NT == 0 && (HD * VP) % NT == 0, "K and V pieces split evenly over the threads");
    const uint32_t nan = AF == OPURE_A_F32 ? 0x7FC00000u : (AF == OPURE_A_F16 ? 0x7E007E00u : 0x7FC07FC0u);
    u4v buf[NPC];
    uint32_t tail = 0u;                                    // pieces whose slots past the cache read 0
    auto piece = [&](uint32_t k, bool& isk, uint32_t& row, uint32_t& pc) {
        const uint32_t e = threadIdx.x + NT * k;
        isk = e < CH * KP;
        const uint32_t r = isk ? e : e - CH * KP;
        row = isk ? r / KP : r / VP;                       // token or channel
        pc = isk ? r - row * KP : r - row * VP;
    };
    auto load = [&](uint32_t c) {
        const uint32_t t0 = c * CH;
        tail = 0u;
#pragma unroll
        for (uint32_t k = 0; k < NPC; ++k)
        {
            bool isk;
            uint32_t row, pc;
            piece(k, isk, row, pc);
            const uint32_t pos = isk ? t0 + row : t0 + pc * TPP;
            u4v val = {0u, 0u, 0u, 0u};
            if (pos < total)
            {
                const int32_t page = spg[pos / OPURE_PAGE_SIZE - c_first * PPC];
                if (page >= 0 && static_cast<uint32_t>(page) < p.n_pages)
                {
                    const uint64_t idx = isk ? kv_elem(p.layer, p.n_pages, static_cast<uint32_t>(page), 0u, p.n_kv, kh, HD,
                                                       pos % OPURE_PAGE_SIZE, pc * (16u / EB))
                                             : kv_elem(p.layer, p.n_pages, static_cast<uint32_t>(page), 1u, p.n_kv, kh, HD,
                                                       pos % OPURE_PAGE_SIZE, row);
                    val = *reinterpret_cast<const u4v*>(static_cast<const uint8_t*>(p.pool) + idx * EB);
                    if (!isk && pos + TPP > total) tail |= 1u << k;   // masked when stored: no wait here
                }
                else
                {
                    // a missing page or a length past the table reads as NaN, never out of bounds
                    val = {nan, nan, nan, nan};
                }
            }
            buf[k] = val;
        }
    };
    auto put = [&](uint32_t c) {
#pragma unroll
        for (uint32_t k = 0; k < NPC; ++k)
        {
            bool isk;
            uint32_t row, pc;
            piece(k, isk, row, pc);
            u4v val = buf[k];
            if (tail & (1u << k)) val = mask_tail<AF>(val, total - (c * CH + pc * TPP));   // slots past the cache read 0
            if (isk) *reinterpret_cast<u4v*>(kt + row * ROWB + pc * 16u) = val;
            else *reinterpret_cast<u4v*>(vt + row * VROWB + pc * 16u) = val;
        }
    };
    for (uint32_t c = c_first; c < c_end; ++c)
    {
        const uint32_t t0 = c * CH;
        if (t0 >= total) break;                           // whole workgroup: past the sequence
        load(c);
        if (c != c_first) __syncthreads();                // the chunk before's buffers read
        put(c);
        __syncthreads();

        // this lane's K row (token t0 + lane) and V channels (lane, lane + 64)
        float kr[HD];
#pragma unroll
        for (uint32_t d = 0; d < HD; ++d)
        {
            if constexpr (AF == OPURE_A_F32) kr[d] = reinterpret_cast<const float*>(kt + lane * ROWB)[d];
            else kr[d] = AF == OPURE_A_F16 ? f16_to_f32(reinterpret_cast<const uint16_t*>(kt + lane * ROWB)[d])
                                           : bf16_to_f32(reinterpret_cast<const uint16_t*>(kt + lane * ROWB)[d]);
        }
        float vc[DPL][CH];
#pragma unroll
        for (uint32_t i = 0; i < DPL; ++i)
        {
            const uint32_t d = lane + 64u * i;
#pragma unroll
            for (uint32_t t = 0; t < CH; ++t)
                vc[i][t] = d < HD ? load_act_rt(vt + d * VROWB, t, AF) : 0.0f;
        }
        const uint64_t pbase = ((static_cast<uint64_t>(b) * p.n_kv + kh) * p.npart + c) * Gq;
        const uint32_t pos = t0 + lane;
        // rows q0 and q0 + NWV together: two independent chains of the same
        // per-row operations (a missing second row scores row q0 again, unstored)
        for (uint32_t q0 = wave; q0 < Gq; q0 += NWV * RB)
        {
            uint32_t qi[RB];
            bool has[RB];
            float acc[RB], mx[RB], l[RB];
#pragma unroll
            for (uint32_t r = 0; r < RB; ++r)
            {
                has[r] = q0 + NWV * r < Gq;
                qi[r] = has[r] ? q0 + NWV * r : q0;
                acc[r] = 0.0f;
            }
#pragma unroll
            for (uint32_t d = 0; d < HD; ++d)
#pragma unroll
                for (uint32_t r = 0; r < RB; ++r) acc[r] = __fmaf_rn(qs[qi[r] * HD + d], kr[d], acc[r]);
#pragma unroll
            for (uint32_t r = 0; r < RB; ++r)
            {
                const uint32_t j = qi[r] / group;
                const float sc = pos <= ctx + j ? __fmul_rn(acc[r], p.scale) : -__builtin_huge_valf();
                mx[r] = wave_max(sc);
                const float e = sc == -__builtin_huge_valf() ? 0.0f : expf_ref(__fsub_rn(sc, mx[r]));
                l[r] = wave_sum(e);
                pbuf[wave][r][lane] = e;
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
            for (uint32_t i = 0; i < DPL; ++i)
            {
                float o[RB];
#pragma unroll
                for (uint32_t r = 0; r < RB; ++r) o[r] = 0.0f;
#pragma unroll
                for (uint32_t t = 0; t < CH; ++t)
#pragma unroll
                    for (uint32_t r = 0; r < RB; ++r) o[r] = __fmaf_rn(pbuf[wave][r][t], vc[i][t], o[r]);
                const uint32_t d = lane + 64u * i;
#pragma unroll
                for (uint32_t r = 0; r < RB; ++r)
                    if (has[r] && d < HD)
                    {
                        if constexpr (ALL) pa[(c * Gq + qi[r]) * HD + d] = o[r];
                        else p.part_acc[(pbase + qi[r]) * HD + d] = o[r];
                    }
            }
            if (lane == 0)
#pragma unroll
                for (uint32_t r = 0; r < RB; ++r)
                    if (has[r])
                    {
                        if constexpr (ALL)
                        {
                            pm[c * Gq + qi[r]] = mx[r];
                            pl[c * Gq + qi[r]] = l[r];
                        }
                        else
                        {
                            p.part_ml[(pbase + qi[r]) * 2u] = mx[r];
                            p.part_ml[(pbase + qi[r]) * 2u + 1u] = l[r];
                        }
                    }
            __builtin_amdgcn_wave_barrier();
        }
    }
    if constexpr (ALL)
    {
        // ---- the merge of each row's chunks 0..last, as k_attn_combine does:
        //      lanes over chunks for the maximum, the weights and the
        //      denominator, then channels d = lane + 64 i over the chunks in order
        __syncthreads();
        const uint32_t nc = p.nch;
        for (uint32_t qi = wave; qi < Gq; qi += NWV)
        {
            const uint32_t j = qi / group, head = kh * group + (qi - j * group);
            uint32_t last = (ctx + j) / p.chunk;
            if (last >= nc)
            {
                last = nc - 1u;
                if (lane == 0u && p.err) p.err[ERR_POSITION] = 1u;
            }
            const uint32_t c0 = min(lane, nc - 1u);
            const float m0 = pm[c0 * Gq + qi], l0 = pl[c0 * Gq + qi];
            float mx = -__builtin_huge_valf();
            if (lane <= last) mx = fmaxf(mx, m0);
            mx = wave_max64(mx);
            float den = 0.0f;
            if (lane <= last)
            {
                const float w = m0 == -__builtin_huge_valf() ? 0.0f : expf_ref(__fsub_rn(m0, mx));
                wsh[wave][lane] = w;
                den = __fmaf_rn(w, l0, den);
            }
            den = wave_sum64(den);
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            const float dd = den > 0.0f ? den : 1.0f;
#pragma unroll
            for (uint32_t i = 0; i < DPL; ++i)
            {
                const uint32_t d = lane + 64u * i;
                float num = 0.0f;
#pragma unroll
                for (uint32_t c = 0; c < ATTN_ALL_CHUNKS; ++c)
                {
                    const bool in = c <= last;
                    const float w = wsh[wave][in ? c : 0u];
                    const float v = pa[(min(c, nc - 1u) * Gq + qi) * HD + min(d, HD - 1u)];
                    num = in ? __fmaf_rn(w, v, num) : num;
                }
                if (d < HD)
                    store_act_rt(p.out, (static_cast<uint64_t>(b * R + j) * p.n_heads + head) * HD + d,
                                 __fdiv_rn(num, dd), p.afmt);
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// Head_dim 64 over at most ATTN_SPLIT_CHUNKS chunks of 64 tokens (a short
// context): a workgroup per (KV head, pair of query rows, sequence) with a
// wave per chunk, so a batch of one sequence still spreads over many CUs.  A
// wave loads its chunk's K rows (lane = token) and V columns (lane = channel)
// straight into registers, all at once (a missing page's lanes read page 0
// and are replaced when used), scores the pair of rows with the chunk
// kernel's per-row operations and leaves the chunk's (max, sum, output) in
// LDS; the waves then merge each row's chunks with k_attn_combine's
// operations in its order.  A row has the bits of k_attn_chunk + combine.
constexpr uint32_t ATTN_SPLIT_CHUNKS = 8;

template <int AF>
__global__ __launch_bounds__(64 * ATTN_SPLIT_CHUNKS) void k_attn_split(AttnParams p)
{
    constexpr uint32_t HD = 64, CH = 64, RB = 2, NW = ATTN_SPLIT_CHUNKS, PPC = CH / OPURE_PAGE_SIZE;
    constexpr uint32_t EB = AF == OPURE_A_F32 ? 4u : 2u, EPP = 16u / EB;   // elements a 16-byte piece
    __shared__ __align__(16) float qsm[NW][RB][HD];       // each wave's copy of the pair's Q rows
    __shared__ __align__(16) float pbuf[NW][RB][CH];
    __shared__ __align__(16) float pa[NW][RB][HD];        // the chunks' outputs
    __shared__ float pm[NW][RB], pl[NW][RB];               // the chunks' maxima and sums
    __shared__ float wsh[RB][NW];                          // a row's chunk weights

    const uint32_t kh = blockIdx.x, b = blockIdx.z;
    const uint32_t group = p.n_heads / p.n_kv, R = p.rows, Gq = group * R;
    const uint32_t c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;   // wave = chunk
    const uint32_t nw = blockDim.x >> 6, q0 = blockIdx.y * RB;
    const int32_t* pt = p.page_table + static_cast<uint64_t>(b) * p.max_pages;

    // round trip 1: the sequence length, the pair's Q rows, the chunk's page entries
    const int32_t seq = p.seq_len[b];
    bool has[RB];
    uint32_t qi[RB], jr[RB];
    float qv[RB];
#pragma unroll
    for (uint32_t r = 0; r < RB; ++r)
    {
        has[r] = q0 + r < Gq;
        qi[r] = has[r] ? q0 + r : q0;
        jr[r] = qi[r] / group;
        const uint32_t head = kh * group + (qi[r] - jr[r] * group);
        qv[r] = load_act_rt(p.q, (static_cast<uint64_t>(b * R + jr[r]) * p.n_heads + head) * HD + lane, AF);
    }
    const uint32_t pi = c * PPC + (lane & (PPC - 1u));
    const int32_t pe = pi < p.max_pages ? pt[pi] : -1;
    asm volatile("" ::: "memory");                         // every load above issued before the entries are read
    const uint32_t ctx = static_cast<uint32_t>(seq), total = ctx + R, t0 = c * CH;
    int32_t pg[PPC];
#pragma unroll
    for (uint32_t i = 0; i < PPC; ++i) pg[i] = __builtin_amdgcn_readlane(pe, i);
#pragma unroll
    for (uint32_t r = 0; r < RB; ++r) qsm[c][r][lane] = qv[r];

    if (t0 < total)   // wave-uniform: the chunk holds positions of the sequence
    {
        // round trip 2: K row of token t0 + lane, V column of channel `lane`
        auto ok = [&](int32_t pg_) { return pg_ >= 0 && static_cast<uint32_t>(pg_) < p.n_pages; };
        auto safe = [&](int32_t pg_) { return ok(pg_) ? static_cast<uint32_t>(pg_) : 0u; };
        const uint32_t pos = t0 + lane, sl = lane / OPURE_PAGE_SIZE;
        const int32_t kpg = sl == 0u ? pg[0] : sl == 1u ? pg[1] : sl == 2u ? pg[2] : pg[3];
        const u4v* kp = reinterpret_cast<const u4v*>(static_cast<const uint8_t*>(p.pool) +
                                                     kv_elem(p.layer, p.n_pages, safe(kpg), 0u, p.n_kv, kh, HD,
                                                             pos % OPURE_PAGE_SIZE, 0u) * EB);
        u4v kw[HD / EPP], vw[PPC][OPURE_PAGE_SIZE / EPP];
#pragma unroll
        for (uint32_t k = 0; k < HD / EPP; ++k) kw[k] = kp[k];
#pragma unroll
        for (uint32_t i = 0; i < PPC; ++i)
        {
            const u4v* vp = reinterpret_cast<const u4v*>(static_cast<const uint8_t*>(p.pool) +
                                                         kv_elem(p.layer, p.n_pages, safe(pg[i]), 1u, p.n_kv, kh, HD, 0u,
                                                                 lane) * EB);
#pragma unroll
            for (uint32_t k = 0; k < OPURE_PAGE_SIZE / EPP; ++k) vw[i][k] = vp[k];
        }
        // the fills: a position past the cache reads 0, a missing page (or an
        // entry past the table) NaN, a V piece reaching past the cache keeps
        // its slots before the end
        const uint32_t nan = AF == OPURE_A_F32 ? 0x7FC00000u : (AF == OPURE_A_F16 ? 0x7E007E00u : 0x7FC07FC0u);
        const u4v zero = {0u, 0u, 0u, 0u}, nanv = {nan, nan, nan, nan};
#pragma unroll
        for (uint32_t k = 0; k < HD / EPP; ++k) kw[k] = pos < total ? (ok(kpg) ? kw[k] : nanv) : zero;
#pragma unroll
        for (uint32_t i = 0; i < PPC; ++i)
#pragma unroll
            for (uint32_t k = 0; k < OPURE_PAGE_SIZE / EPP; ++k)
            {
                const uint32_t pp = t0 + i * OPURE_PAGE_SIZE + k * EPP;
                u4v v = ok(pg[i]) ? (pp + EPP > total ? mask_tail<AF>(vw[i][k], total - pp) : vw[i][k]) : nanv;
                vw[i][k] = pp < total ? v : zero;
            }
        float kr[HD], vc[CH];
#pragma unroll
        for (uint32_t d = 0; d < HD; ++d)
        {
            const uint32_t w = kw[d / EPP][(d % EPP) * EB / 4u];
            if constexpr (AF == OPURE_A_F32) kr[d] = __uint_as_float(w);
            else
            {
                const uint16_t h = static_cast<uint16_t>(d % 2u ? w >> 16 : w & 0xFFFFu);
                kr[d] = AF == OPURE_A_F16 ? f16_to_f32(h) : bf16_to_f32(h);
            }
        }
#pragma unroll
        for (uint32_t t = 0; t < CH; ++t)
        {
            const uint32_t i = t / OPURE_PAGE_SIZE, s = t % OPURE_PAGE_SIZE;
            const uint32_t w = vw[i][s / EPP][(s % EPP) * EB / 4u];
            if constexpr (AF == OPURE_A_F32) vc[t] = __uint_as_float(w);
            else
            {
                const uint16_t h = static_cast<uint16_t>(s % 2u ? w >> 16 : w & 0xFFFFu);
                vc[t] = AF == OPURE_A_F16 ? f16_to_f32(h) : bf16_to_f32(h);
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        float acc[RB], mx[RB], l[RB];
#pragma unroll
        for (uint32_t r = 0; r < RB; ++r) acc[r] = 0.0f;
#pragma unroll
        for (uint32_t d = 0; d < HD; ++d)
#pragma unroll
            for (uint32_t r = 0; r < RB; ++r) acc[r] = __fmaf_rn(qsm[c][r][d], kr[d], acc[r]);
#pragma unroll
        for (uint32_t r = 0; r < RB; ++r)
        {
            const float sc = pos <= ctx + jr[r] ? __fmul_rn(acc[r], p.scale) : -__builtin_huge_valf();
            mx[r] = wave_max(sc);
            const float e = sc == -__builtin_huge_valf() ? 0.0f : expf_ref(__fsub_rn(sc, mx[r]));
            l[r] = wave_sum(e);
            pbuf[c][r][lane] = e;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        float o[RB];
#pragma unroll
        for (uint32_t r = 0; r < RB; ++r) o[r] = 0.0f;
#pragma unroll
        for (uint32_t t = 0; t < CH; ++t)
#pragma unroll
            for (uint32_t r = 0; r < RB; ++r) o[r] = __fmaf_rn(pbuf[c][r][t], vc[t], o[r]);
#pragma unroll
        for (uint32_t r = 0; r < RB; ++r)
        {
            pa[c][r][lane] = o[r];
            if (lane == 0u)
            {
                pm[c][r] = mx[r];
                pl[c][r] = l[r];
            }
        }
    }
    __syncthreads();

    // the merge of each row's chunks 0..last, as k_attn_combine does: lanes
    // over chunks for the maximum, the weights and the denominator, then
    // channel `lane` over the chunks in order
    for (uint32_t r = c; r < RB; r += nw)
    {
        if (!has[r]) continue;
        uint32_t last = (ctx + jr[r]) / p.chunk;
        if (last >= p.nch)
        {
            last = p.nch - 1u;
            if (lane == 0u && p.err) p.err[ERR_POSITION] = 1u;
        }
        const uint32_t c0 = min(lane, NW - 1u);
        const float m0 = pm[c0][r], l0 = pl[c0][r];
        float mx = -__builtin_huge_valf();
        if (lane <= last) mx = fmaxf(mx, m0);
        mx = wave_max64(mx);
        float den = 0.0f;
        if (lane <= last)
        {
            const float w = m0 == -__builtin_huge_valf() ? 0.0f : expf_ref(__fsub_rn(m0, mx));
            wsh[r][lane] = w;
            den = __fmaf_rn(w, l0, den);
        }
        den = wave_sum64(den);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        const float dd = den > 0.0f ? den : 1.0f;
        float num = 0.0f;
#pragma unroll
        for (uint32_t cc = 0; cc < NW; ++cc)
        {
            const bool in = cc <= last;
            num = in ? __fmaf_rn(wsh[r][in ? cc : 0u], pa[in ? cc : 0u][r][lane], num) : num;
        }
        const uint32_t head = kh * group + (qi[r] - jr[r] * group);
        store_act_rt(p.out, (static_cast<uint64_t>(b * R + jr[r]) * p.n_heads + head) * HD + lane, __fdiv_rn(num, dd),
                     p.afmt);
    }
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

template <int AF>
__device__ __forceinline__ f4_t mfma32(u4v a, u4v b, f4_t c)
{
    if constexpr (AF == OPURE_A_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c, 0,
                                                      0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                       0, 0, 0);
}

template <int AF>
__device__ __forceinline__ float unpack_lo(uint32_t v)
{
    return AF == OPURE_A_F16 ? f16_to_f32(static_cast<uint16_t>(v)) : bf16_to_f32(static_cast<uint16_t>(v));
}

template <int AF>
__device__ __forceinline__ float unpack_hi(uint32_t v)
{
    return AF == OPURE_A_F16 ? f16_to_f32(static_cast<uint16_t>(v >> 16)) : bf16_to_f32(static_cast<uint16_t>(v >> 16));
}

template <int AF>
__device__ __forceinline__ uint32_t pack_pair(float a, float b)
{
    if constexpr (AF == OPURE_A_F16) return f32_to_f16(a) | (static_cast<uint32_t>(f32_to_f16(b)) << 16);
    else return f32_to_bf16(a) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// Matrix-core flash-decoding for fp16/bf16 caches, head_dim HD in {64, 128}.
// One workgroup of NWV waves per (KV head, chunk of NWV*32*KK tokens,
// sequence); wave w scores tokens [t0 + 32*KK*w, +32*KK) against query rows
// qoff .. qoff+16*NT-1 of the KV head's Gq = group*rows rows:
//   S^T = K Q^T   A = K, lane l = (r, g): token tb + 8(r/4) + r%4 (+4 in the
//                 second tile), channels 32s + 8g..;  B = Q^T, column = query row
//   so the score tile a lane holds -- query row r, tokens tb + 8g .. 8g+7 --
//   is exactly its B operand of
//   O^T = V^T P^T A = V^T tile (channel r, tokens tb + 8g..8g+7: 16 contiguous
//                 bytes of a channel-major V plane)
// All K and V loads are issued before the first MFMA (in the folded kernel
// unconditionally, so the scores and the softmax run while V lands).  The
// waves' (max, sum, output) go to LDS; then the (channel tile, query tile) pieces of the merge
// are shared out over the waves, each merging in wave order, and the chunk's
// partial is written for the combine kernel.
// exp(x) for x <= 0 as 2^(x log2 e) on the transcendental unit (v_exp_f32,
// about 1 ulp).  x log2 e is carried as t + dt: t = fl(x L), dt = the fma
// residual of that product plus x (log2 e - L), so 2^(t + dt) = 2^t (1 + dt ln 2)
// to within dt^2 -- without dt the rounding of t alone (up to 2^-24 |t|, 14x the
// ulp of the result at x = -10) would dominate the error of every probability.
// The ~15-instruction exp of the oracle was the kernel's largest VALU cost.
__device__ __forceinline__ float exp_hw(float x)
{
    constexpr float L = 1.44269502162933349609375f;          // log2 e rounded to fp32
    constexpr float L_LO = 1.92596299e-8f;                       // log2 e - L
    constexpr float LN2 = 0.693147182464599609375f;
    const float t = __fmul_rn(x, L);
    const float dt = __fmaf_rn(x, L_LO, __fmaf_rn(x, L, -t));
    const float e = __builtin_amdgcn_exp2f(t);
    return __fmaf_rn(e, __fmul_rn(dt, LN2), e);
}

template <int HD, int NT, int NWV>
constexpr uint32_t attn_mfma_lds()
{
    return NWV * (HD / 16u) * NT * 64u * 16u + NWV * NT * 16u * 2u * 4u;
}

// Chunks that one workgroup of the folded head_dim-64 launch (a grid of many
// sequences) merges into one partial, so that it writes a quarter of the
// partials and the combine reads a quarter.  The combine merges the chunk
// partials of the other head_dim-64 launches in groups of as many chunks, with
// the same operations, so a row's bits do not depend on the launch that scored it.
constexpr uint32_t ATTN_GROUP = 4;

// One step of the in-order merge of a group's chunks: the running state
// (m, l, acc) and the next chunk (mc, lc, ac) become
// (max(m, mc), sa l + sb lc, sa acc + sb ac) with sa = exp(m - max) and
// sb = exp(mc - max) on the transcendental unit (exp_hw: the running merge is
// a chain of these, and the kernel and the combine both take them from here),
// a side whose maximum is -inf weighing 0.
__device__ __forceinline__ void merge_scales(float m, float mc, float& mn, float& sa, float& sb)
{
    mn = fmaxf(m, mc);
    sa = m == -__builtin_huge_valf() ? 0.0f : exp_hw(__fsub_rn(m, mn));
    sb = mc == -__builtin_huge_valf() ? 0.0f : exp_hw(__fsub_rn(mc, mn));
}
__device__ __forceinline__ float merge_val(float sa, float a, float sb, float c)
{
    return __fmaf_rn(sb, c, __fmul_rn(sa, a));
}

// ZS: blockIdx.z holds (sequence, block of 16 * NT query rows) as b * zt + block
// CL: a workgroup takes the ATTN_GROUP chunks from ATTN_GROUP * blockIdx.y and
//     writes their merge as partial blockIdx.y
template <int HD, int AF, int NT, int KK, int NWV, bool ZS, bool CL = false>
__global__ __launch_bounds__(NWV * 64) __attribute__((amdgpu_waves_per_eu(CL ? 4 : 1))) void k_attn_mfma(AttnParams p)
{
    constexpr uint32_t KS = HD / 32u, DT = HD / 16u, EB = 2u, TPW = 32u * KK, OWN = DT * NT / NWV;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    f4_t (*cacc)[DT][NT][64] = reinterpret_cast<f4_t (*)[DT][NT][64]>(lds_raw);
    float (*cml)[NT][16][2] = reinterpret_cast<float (*)[NT][16][2]>(lds_raw + NWV * DT * NT * 64u * 16u);
    const uint32_t kh = blockIdx.x, b = ZS ? blockIdx.z / p.zt : blockIdx.z;
    const uint32_t qoff = ZS ? (blockIdx.z - b * p.zt) * 16u * NT : p.qoff;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, g = lane >> 4, r = lane & 15u;
    const uint32_t group = p.n_heads / p.n_kv, R = p.rows, Gq = group * R;
    const int32_t* pt = p.page_table + static_cast<uint64_t>(b) * p.max_pages;
    const uint8_t* pool = static_cast<const uint8_t*>(p.pool);
    const uint32_t nan2 = AF == OPURE_A_F16 ? 0x7E007E00u : 0x7FC07FC0u;
    // chunks c_first .. c_end - 1 of this workgroup
    const uint32_t c_first = CL ? blockIdx.y * ATTN_GROUP : blockIdx.y;
    const uint32_t c_end = CL ? min(c_first + ATTN_GROUP, p.nch) : c_first + 1u;

    // ---- the sequence length, the page-table entries of the first chunk's
    //      tokens and Q^T in one round trip: none of them depends on another,
    //      and the entries are loaded unconditionally (index clamped to the
    //      table) and checked only when used, so no load waits behind another
    const int32_t seq = p.seq_len[b];
    auto raw_entry = [&](uint32_t tok) { return pt[min(tok / OPURE_PAGE_SIZE, p.max_pages - 1u)]; };
    auto load_entries = [&](uint32_t c, int32_t (&ek)[KK][2], int32_t (&ev)[KK]) {
        const uint32_t tw = c * NWV * TPW + TPW * wave;
#pragma unroll
        for (uint32_t kk = 0; kk < KK; ++kk)
        {
            const uint32_t tb = tw + 32u * kk;
#pragma unroll
            for (uint32_t T = 0; T < 2; ++T) ek[kk][T] = raw_entry(tb + 8u * (r >> 2) + (r & 3u) + 4u * T);
            ev[kk] = raw_entry(tb + 8u * g);
        }
    };
    int32_t pgk[KK][2], pgv[KK];
    load_entries(c_first, pgk, pgv);
    // the entry of `tok` as page_of gives it, from its raw load
    auto checked = [&](uint32_t tok, int32_t pg) -> int32_t {
        return tok / OPURE_PAGE_SIZE < p.max_pages && pg >= 0 && static_cast<uint32_t>(pg) < p.n_pages ? pg : -1;
    };
    u4v qop[NT][KS];
    uint32_t qj[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
    {
        const uint32_t qi = min(qoff + 16u * n + r, Gq - 1u);
        const uint32_t j = qi / group, head = kh * group + (qi - j * group);
        qj[n] = j;
        const uint8_t* qrow = static_cast<const uint8_t*>(p.q) + ((static_cast<uint64_t>(b * R + j) * p.n_heads + head) * HD) * EB;
#pragma unroll
        for (uint32_t s = 0; s < KS; ++s) qop[n][s] = *reinterpret_cast<const u4v*>(qrow + (32u * s + 8u * g) * EB);
    }
    // keeps the loads above issued before the exit below (the compiler would
    // otherwise test the length first and make them wait for it)
    asm volatile("" ::: "memory");
    const uint32_t ctx = static_cast<uint32_t>(seq);
    const uint32_t total = ctx + R;
    if (c_first * NWV * TPW >= total) return;             // whole workgroup: no row reaches its chunks
    uint32_t lim[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) lim[n] = ctx + qj[n];
    // the merge's share of wave w: row block w % NT, channel tiles w / NT,
    // w / NT + NWV / NT, ...; the row's last chunk (the folded merge takes
    // chunks up to it) and the merged state of the chunks so far
    static_assert(NWV % NT == 0 && (DT * NT) % NWV == 0, "whole channel tiles of one row block a wave");
    const uint32_t n_own = wave % NT, qi_own = qoff + 16u * n_own + r;
    const uint32_t last_own = (ctx + min(qi_own, Gq - 1u) / group) / p.chunk;
    float sm = 0.0f, sl = 0.0f;
    f4_t sacc[OWN];

    for (uint32_t c = c_first; c < c_end; ++c)
    {
        const uint32_t t0 = c * NWV * TPW;
        const uint32_t tw = t0 + TPW * wave;
        if (t0 >= total) break;                           // whole workgroup: past the sequence
        const bool active = tw < total;

        // ---- then K (both score tiles of each k-step) and V^T.  In the folded
        //      kernel (a grid of many workgroups) every load is unconditional -- a
        //      lane without a valid page reads page 0 and takes its fill when the
        //      operand is used -- so the loads are one straight run and the scores
        //      and softmax wait only for K while V lands (C5 3.294 -> 3.252 ms).
        //      Elsewhere each load sits under its page test and the first product
        //      waits for all of them: at one workgroup a CU (C3, C4) that measured
        //      faster, 2-10 us a step ------------------------------------------
        u4v kop[KK][2][KS], vop[KK][DT];
        bool kok[KK][2], vok[KK];
        uint32_t kfill[KK][2], vfill[KK], vlen[KK];
#pragma unroll
        for (uint32_t kk = 0; kk < KK; ++kk)
        {
            const uint32_t tb = tw + 32u * kk;
#pragma unroll
            for (uint32_t T = 0; T < 2; ++T)
            {
                const uint32_t tok = tb + 8u * (r >> 2) + (r & 3u) + 4u * T;
                const int32_t pg = active && tok < total ? checked(tok, pgk[kk][T]) : -1;
                const uint32_t f = active && tok < total ? nan2 : 0u;
                if constexpr (CL)
                {
                    kfill[kk][T] = f;
                    kok[kk][T] = pg >= 0;
                    const uint32_t pgc = pg >= 0 ? static_cast<uint32_t>(pg) : 0u;
#pragma unroll
                    for (uint32_t s = 0; s < KS; ++s)
                        kop[kk][T][s] = *reinterpret_cast<const u4v*>(
                            pool + kv_elem(p.layer, p.n_pages, pgc, 0u, p.n_kv, kh, HD, tok % OPURE_PAGE_SIZE, 32u * s + 8u * g) * EB);
                }
                else
                {
#pragma unroll
                    for (uint32_t s = 0; s < KS; ++s)
                        kop[kk][T][s] = pg >= 0 ? *reinterpret_cast<const u4v*>(
                                                      pool + kv_elem(p.layer, p.n_pages, static_cast<uint32_t>(pg), 0u, p.n_kv, kh,
                                                                     HD, tok % OPURE_PAGE_SIZE, 32u * s + 8u * g) * EB)
                                                : u4v{f, f, f, f};
                }
            }
            const uint32_t tok = tb + 8u * g;             // 8 tokens of one page
            const int32_t pg = active && tok < total ? checked(tok, pgv[kk]) : -1;
            const uint32_t f = active && tok < total ? nan2 : 0u;
            if constexpr (CL)
            {
                vfill[kk] = f;
                vok[kk] = pg >= 0;
                vlen[kk] = tok < total ? total - tok : 0u;
                const uint32_t pgc = pg >= 0 ? static_cast<uint32_t>(pg) : 0u;
#pragma unroll
                for (uint32_t dt = 0; dt < DT; ++dt)
                    vop[kk][dt] = *reinterpret_cast<const u4v*>(
                        pool + kv_elem(p.layer, p.n_pages, pgc, 1u, p.n_kv, kh, HD, tok % OPURE_PAGE_SIZE, 16u * dt + r) * EB);
            }
            else
            {
#pragma unroll
                for (uint32_t dt = 0; dt < DT; ++dt)
                {
                    if (pg >= 0)
                    {
                        vop[kk][dt] = *reinterpret_cast<const u4v*>(pool + kv_elem(p.layer, p.n_pages, static_cast<uint32_t>(pg), 1u,
                                                                                   p.n_kv, kh, HD, tok % OPURE_PAGE_SIZE,
                                                                                   16u * dt + r) * EB);
                        if (tok + 8u > total) vop[kk][dt] = mask_tail<AF>(vop[kk][dt], total - tok);   // stale slots read 0
                    }
                    else
                    {
                        vop[kk][dt] = u4v{f, f, f, f};
                    }
                }
            }
        }
        // the folded kernel's operands as used: the fill where the page is
        // missing, and V's slots past the cache read 0
        auto fix_k = [&](uint32_t kk) {
            if constexpr (CL)
#pragma unroll
                for (uint32_t T = 0; T < 2; ++T)
#pragma unroll
                    for (uint32_t s = 0; s < KS; ++s)
                    {
                        const uint32_t f = kfill[kk][T];
                        kop[kk][T][s] = kok[kk][T] ? kop[kk][T][s] : u4v{f, f, f, f};
                    }
        };
        auto fix_v = [&](uint32_t kk) {
            if constexpr (CL)
            {
                const uint32_t f = vfill[kk];
#pragma unroll
                for (uint32_t dt = 0; dt < DT; ++dt) vop[kk][dt] = vok[kk] ? vop[kk][dt] : u4v{f, f, f, f};
                if (vok[kk] && vlen[kk] < 8u)
#pragma unroll
                    for (uint32_t dt = 0; dt < DT; ++dt) vop[kk][dt] = mask_tail<AF>(vop[kk][dt], vlen[kk]);
            }
        };
        // the next chunk's page-table entries (clamped, as the first's) land
        // while this chunk computes
        int32_t npk[KK][2], npv[KK];
        if constexpr (CL) load_entries(c + 1u, npk, npv);
        // every K and V load is issued before the first product
        if constexpr (CL) __builtin_amdgcn_sched_barrier(0);

        // ---- scores, masked past each row's position --------------------------
        float sc[KK][2][NT][4];
#pragma unroll
        for (uint32_t kk = 0; kk < KK; ++kk)
        {
            const uint32_t tb = tw + 32u * kk;
            fix_k(kk);
#pragma unroll
            for (uint32_t T = 0; T < 2; ++T)
#pragma unroll
                for (int n = 0; n < NT; ++n)
                {
                    f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (uint32_t s = 0; s < KS; ++s) acc = mfma32<AF>(kop[kk][T][s], qop[n][s], acc);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                    {
                        const uint32_t tok = tb + 8u * g + 4u * T + i;
                        sc[kk][T][n][i] = active && tok <= lim[n] ? __fmul_rn(acc[i], p.scale) : -__builtin_huge_valf();
                    }
                }
        }

        // ---- softmax statistics of each query row over this wave's tokens -----
        // P^T = hi + lo (fp16) or hi + mid + lo (bf16), every part in the 16-bit format
        constexpr bool P3 = AF == OPURE_A_BF16;
        float mrow[NT], lrow[NT];
        u4v pop[KK][NT], plo[KK][NT], plo2[KK][NT];
#pragma unroll
        for (int n = 0; n < NT; ++n)
        {
            float mx = -__builtin_huge_valf();
#pragma unroll
            for (uint32_t kk = 0; kk < KK; ++kk)
#pragma unroll
                for (uint32_t T = 0; T < 2; ++T)
#pragma unroll
                    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[kk][T][n][i]);
            mx = max_xor32(max_xor16(mx));
            float sum = 0.0f;
#pragma unroll
            for (uint32_t kk = 0; kk < KK; ++kk)
            {
                float e[8];
#pragma unroll
                for (uint32_t T = 0; T < 2; ++T)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                    {
                        const float v = sc[kk][T][n][i];
                        e[4 * T + i] = v == -__builtin_huge_valf() ? 0.0f : exp_hw(__fsub_rn(v, mx));
                        sum += e[4 * T + i];
                    }
                pop[kk][n] = u4v{pack_pair<AF>(e[0], e[1]), pack_pair<AF>(e[2], e[3]), pack_pair<AF>(e[4], e[5]),
                                 pack_pair<AF>(e[6], e[7])};
                float lo[8];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    const uint32_t pr = pop[kk][n][i];
                    lo[2 * i] = __fsub_rn(e[2 * i], unpack_lo<AF>(pr));
                    lo[2 * i + 1] = __fsub_rn(e[2 * i + 1], unpack_hi<AF>(pr));
                }
                plo[kk][n] = u4v{pack_pair<AF>(lo[0], lo[1]), pack_pair<AF>(lo[2], lo[3]), pack_pair<AF>(lo[4], lo[5]),
                                 pack_pair<AF>(lo[6], lo[7])};
                if constexpr (P3)
                {
                    // the remainders are exact in fp32: e - hi and (e - hi) - mid
                    float lo2[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                    {
                        const uint32_t pr = plo[kk][n][i];
                        lo2[2 * i] = __fsub_rn(lo[2 * i], unpack_lo<AF>(pr));
                        lo2[2 * i + 1] = __fsub_rn(lo[2 * i + 1], unpack_hi<AF>(pr));
                    }
                    plo2[kk][n] = u4v{pack_pair<AF>(lo2[0], lo2[1]), pack_pair<AF>(lo2[2], lo2[3]),
                                      pack_pair<AF>(lo2[4], lo2[5]), pack_pair<AF>(lo2[6], lo2[7])};
                }
            }
            sum = add_xor32(add_xor16(sum));
            mrow[n] = mx;
            lrow[n] = sum;
        }

        // ---- O^T = V^T P^T ------------------------------------------------------
#pragma unroll
        for (uint32_t kk = 0; kk < KK; ++kk) fix_v(kk);
        f4_t o[DT][NT];
#pragma unroll
        for (uint32_t dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int n = 0; n < NT; ++n)
            {
                o[dt][n] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (uint32_t kk = 0; kk < KK; ++kk)
                {
                    if constexpr (P3) o[dt][n] = mfma32<AF>(vop[kk][dt], plo2[kk][n], o[dt][n]);
                    o[dt][n] = mfma32<AF>(vop[kk][dt], plo[kk][n], o[dt][n]);
                    o[dt][n] = mfma32<AF>(vop[kk][dt], pop[kk][n], o[dt][n]);
                }
            }

        // ---- merge the waves in wave order: m = max, weights exp(m_w - m) -------
#pragma unroll
        for (uint32_t dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int n = 0; n < NT; ++n) cacc[wave][dt][n][lane] = o[dt][n];
        if (g == 0)
        {
#pragma unroll
            for (int n = 0; n < NT; ++n)
            {
                cml[wave][n][r][0] = mrow[n];
                cml[wave][n][r][1] = lrow[n];
            }
        }
        __syncthreads();
        // the chunk's (max, sum, output) of this wave's share: the block's
        // weights once, then every tile's loads in one round
        float mw[NWV], lw[NWV];
#pragma unroll
        for (int w = 0; w < NWV; ++w)
        {
            mw[w] = cml[w][n_own][r][0];
            lw[w] = cml[w][n_own][r][1];
        }
        float M = mw[0];
#pragma unroll
        for (int w = 1; w < NWV; ++w) M = fmaxf(M, mw[w]);
        float ew[NWV];
#pragma unroll
        for (int w = 0; w < NWV; ++w)
            ew[w] = mw[w] == -__builtin_huge_valf() ? 0.0f : expf_ref_nonpos(__fsub_rn(mw[w], M));
        float L = __fmul_rn(ew[0], lw[0]);
#pragma unroll
        for (int w = 1; w < NWV; ++w) L = __fmaf_rn(ew[w], lw[w], L);
        f4_t a[OWN];
#pragma unroll
        for (uint32_t j = 0; j < OWN; ++j)
        {
            const uint32_t dt = wave / NT + (NWV / NT) * j;
            a[j] = cacc[0][dt][n_own][lane] * ew[0];
#pragma unroll
            for (int w = 1; w < NWV; ++w)
            {
                const f4_t v = cacc[w][dt][n_own][lane];
#pragma unroll
                for (int i = 0; i < 4; ++i) a[j][i] = __fmaf_rn(ew[w], v[i], a[j][i]);
            }
        }
        if constexpr (!CL)
        {
            // the chunk's partial
            const uint64_t pbase = ((static_cast<uint64_t>(b) * p.n_kv + kh) * p.npart + c) * Gq;
            if (qi_own < Gq)
            {
                if (wave < NT && g == 0)
                {
                    p.part_ml[(pbase + qi_own) * 2u] = M;
                    p.part_ml[(pbase + qi_own) * 2u + 1u] = L;
                }
#pragma unroll
                for (uint32_t j = 0; j < OWN; ++j)
                    *reinterpret_cast<f4_t*>(p.part_acc + (pbase + qi_own) * HD + 16u * (wave / NT + (NWV / NT) * j) +
                                             4u * g) = a[j];
            }
        }
        else
        {
            // merged, in chunk order, with the group's chunks so far that the
            // row sees (chunks past the row's last are left out, as the combine
            // leaves them out)
            if (c == c_first)
            {
                sm = M;
                sl = L;
#pragma unroll
                for (uint32_t j = 0; j < OWN; ++j) sacc[j] = a[j];
            }
            else if (c <= last_own)
            {
                float mn, sa, sb;
                merge_scales(sm, M, mn, sa, sb);
                sm = mn;
                sl = merge_val(sa, sl, sb, L);
#pragma unroll
                for (uint32_t j = 0; j < OWN; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) sacc[j][i] = merge_val(sa, sacc[j][i], sb, a[j][i]);
            }
#pragma unroll
            for (uint32_t kk = 0; kk < KK; ++kk)
            {
                pgk[kk][0] = npk[kk][0];
                pgk[kk][1] = npk[kk][1];
                pgv[kk] = npv[kk];
            }
            // the next chunk writes the merge buffers again
            if (c + 1u < c_end) __syncthreads();
        }
    }
    if constexpr (CL)
    {
        // the group's partial
        const uint64_t pbase = ((static_cast<uint64_t>(b) * p.n_kv + kh) * p.npart + blockIdx.y) * Gq;
        if (qi_own < Gq)
        {
            if (wave < NT && g == 0)
            {
                p.part_ml[(pbase + qi_own) * 2u] = sm;
                p.part_ml[(pbase + qi_own) * 2u + 1u] = sl;
            }
#pragma unroll
            for (uint32_t j = 0; j < OWN; ++j)
                *reinterpret_cast<f4_t*>(p.part_acc + (pbase + qi_own) * HD + 16u * (wave / NT + (NWV / NT) * j) + 4u * g) =
                    sacc[j];
        }
    }
}

// One wave per (row, query head): merge that row's items 0..last in order.
// An item is a partial, or (GRP > 1) a group of GRP chunk partials merged in
// chunk order by merge_scales/merge_val, as the folded attention kernel merges
// its chunks into one partial -- so a row's bits are the same whichever
// launch scored it.  Lanes first take items (max, then weights and the
// denominator with a fixed butterfly), then channels d = lane + 64 i
// (i < DPL), summing the items' outputs in order.  The first CB partials'
// outputs are loaded together with the statistics, so a context of up to CB
// partials costs one round trip (CB 20 where a launch has at most 20
// partials: fewer loads of the clamped last one).
template <int DPL, int GRP, uint32_t CB = 32u>
__global__ __launch_bounds__(64) void k_attn_combine(AttnParams p)
{
    static_assert(CB % GRP == 0, "whole groups preloaded");
    constexpr uint32_t NI = 1024u / GRP, NS = GRP > 1 ? 1024u : 1u, NG = GRP > 1 ? NI : 1u;
    __shared__ float wsh[NI];                              // the items' weights
    __shared__ float gsc[2][NS];                           // GRP > 1: each chunk's merge scales (state, chunk)
    __shared__ float gml[2][NG];                           // GRP > 1: each group's (max, sum)
    const uint32_t head = blockIdx.x, rr = blockIdx.y;    // rr = b * R + j
    const uint32_t R = p.rows, b = rr / R, j = rr - b * R;
    const uint32_t group = p.n_heads / p.n_kv, kh = head / group, qi = j * group + (head - kh * group);
    const uint32_t Gq = group * R, hd = p.hd, lane = threadIdx.x;
    const int32_t seq = p.seq_len[b];
    const uint64_t base = (static_cast<uint64_t>(b) * p.n_kv + kh) * p.npart;
    // partials are clamped to the launch's last, not the row's: these loads do
    // not wait for the sequence length, and partials past the row's last are
    // loaded but never used
    auto acc_at = [&](uint32_t c, int i) {
        const uint32_t d = min(lane + 64u * i, hd - 1u);
        return p.part_acc[((base + min(c, p.npart - 1u)) * Gq + qi) * hd + d];
    };
    auto ml_at = [&](uint32_t c, uint32_t k) { return p.part_ml[((base + min(c, p.npart - 1u)) * Gq + qi) * 2u + k]; };
    // the statistics of item `lane`'s partials and the first CB partials'
    // outputs, in one round trip
    float m0[GRP], l0[GRP];
#pragma unroll
    for (uint32_t k = 0; k < GRP; ++k)
    {
        m0[k] = ml_at(lane * GRP + k, 0u);
        l0[k] = ml_at(lane * GRP + k, 1u);
    }
    float v[CB][DPL];
#pragma unroll
    for (uint32_t c = 0; c < CB; ++c)
#pragma unroll
        for (int i = 0; i < DPL; ++i) v[c][i] = acc_at(c, i);
    uint32_t last = (static_cast<uint32_t>(seq) + j) / p.chunk;
    if (last >= p.nch)
    {
        // a position beyond the launch's max_ctx: clamped (never read past the
        // partials) and reported, since the row's output is then wrong
        last = p.nch - 1u;
        if (lane == 0u && p.err) p.err[ERR_POSITION] = 1u;
    }
    const uint32_t lastp = last / p.cpp, lasti = lastp / GRP;   // the row's last partial, last item
    // item i's (max, sum): the partial's, or its group's merge
    auto item = [&](uint32_t i, float& m, float& l) {
        m = i == lane ? m0[0] : ml_at(i * GRP, 0u);
        l = i == lane ? l0[0] : ml_at(i * GRP, 1u);
        if constexpr (GRP > 1)
        {
            float mc[GRP], lc[GRP];
#pragma unroll
            for (uint32_t k = 1; k < GRP; ++k)
            {
                mc[k] = i == lane ? m0[k] : ml_at(i * GRP + k, 0u);
                lc[k] = i == lane ? l0[k] : ml_at(i * GRP + k, 1u);
            }
            // without branches, so the steps' exponentials (which wait only
            // for the running maximum) overlap; a chunk past the row's last
            // leaves the state as it is
#pragma unroll
            for (uint32_t k = 1; k < GRP; ++k)
            {
                const bool in = i * GRP + k <= lastp;
                float mn, sa, sb;
                merge_scales(m, mc[k], mn, sa, sb);
                const float ln = merge_val(sa, l, sb, lc[k]);
                m = in ? mn : m;
                l = in ? ln : l;
                gsc[0][i * GRP + k] = sa;
                gsc[1][i * GRP + k] = sb;
            }
            gml[0][i] = m;
            gml[1][i] = l;
        }
    };
    float mx = -__builtin_huge_valf(), mf = 0.0f, lf = 0.0f;  // (GRP > 1) item `lane`'s merge
    for (uint32_t i = lane; i <= lasti; i += 64u)
    {
        float m, l;
        if constexpr (GRP > 1)
        {
            item(i, m, l);
            if (i == lane)
            {
                mf = m;
                lf = l;
            }
        }
        else m = i == lane ? m0[0] : ml_at(i, 0u);
        mx = fmaxf(mx, m);
    }
    mx = wave_max64(mx);
    float den = 0.0f;
    for (uint32_t i = lane; i <= lasti; i += 64u)
    {
        float m, l;
        if constexpr (GRP > 1)
        {
            m = i == lane ? mf : gml[0][i];               // this lane's own entries
            l = i == lane ? lf : gml[1][i];
        }
        else item(i, m, l);
        const float w = m == -__builtin_huge_valf() ? 0.0f : expf_ref(__fsub_rn(m, mx));
        wsh[i] = w;
        den = __fmaf_rn(w, l, den);
    }
    den = wave_sum64(den);
    __syncthreads();
    const float dd = den > 0.0f ? den : 1.0f;
    float num[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) num[i] = 0.0f;
    // item s's output, channel i, from its partials' outputs x(c, i)
    auto item_acc = [&](uint32_t s, int i, auto&& x) {
        float a = x(s * GRP, i);
        if constexpr (GRP > 1)
#pragma unroll
            for (uint32_t k = 1; k < GRP; ++k)
            {
                const uint32_t c = s * GRP + k;
                const float an = merge_val(gsc[0][c], a, gsc[1][c], x(c, i));
                a = c <= lastp ? an : a;
            }
        return a;
    };
    auto pre = [&](uint32_t c, int i) { return v[c][i]; };
#pragma unroll
    for (uint32_t s = 0; s < CB / GRP; ++s)
    {
        const bool in = s <= lasti;                  // past the last item: skipped, not added as zero
        const float w = wsh[in ? s : 0u];
#pragma unroll
        for (int i = 0; i < DPL; ++i) num[i] = in ? __fmaf_rn(w, item_acc(s, i, pre), num[i]) : num[i];
    }
    for (uint32_t s = CB / GRP; s <= lasti; ++s)
    {
        const float w = wsh[s];
#pragma unroll
        for (int i = 0; i < DPL; ++i) num[i] = __fmaf_rn(w, item_acc(s, i, acc_at), num[i]);
    }
#pragma unroll
    for (int i = 0; i < DPL; ++i)
    {
        const uint32_t d = lane + 64u * i;
        if (d < hd) store_act_rt(p.out, (static_cast<uint64_t>(rr) * p.n_heads + head) * hd + d, __fdiv_rn(num[i], dd), p.afmt);
    }
}

template <int HD, int AF, int NT, int KK, int NWV, bool ZS = false, bool CL = false>
int launch_mfma(opure_dev* dev, dim3 grid, const AttnParams& p)
{
    constexpr uint32_t lds = attn_mfma_lds<HD, NT, NWV>();
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_mfma<HD, AF, NT, KK, NWV, ZS, CL>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        configured = true;
    }
    OPURE_LAUNCH(dev, (k_attn_mfma<HD, AF, NT, KK, NWV, ZS, CL>), grid, dim3(NWV * 64), lds, p);
    OPURE_LAUNCH_CHECK("k_attn_mfma");
    return OPURE_OK;
}

template <int HD, int AF, bool ALL>
int launch_fast(opure_dev* dev, dim3 grid, uint32_t lds, const AttnParams& p)
{
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_chunk<HD, AF, ALL>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024));
        configured = true;
    }
    OPURE_LAUNCH(dev, (k_attn_chunk<HD, AF, ALL>), grid, dim3(attn_fast_threads<HD>()), lds, p);
    OPURE_LAUNCH_CHECK("k_attn_chunk");
    return OPURE_OK;
}

}  // namespace

namespace opure_hip {

// Chunk length of the kernel that runs a shape: 256 for the matrix-core path
// (fp16/bf16, head_dim 64/128, <= 64 query rows per KV head), 64 for the VALU
// fast path, 32 for the generic kernel.
static bool use_mfma(uint32_t hd, uint32_t afmt, uint32_t)
{
    return (hd == 64u || hd == 128u) && afmt != OPURE_A_F32;
}

// Chunk length of the kernel that runs a shape: matrix-core path 128 tokens
// (head_dim 64) or 256 (head_dim 128), VALU fast path 64, generic kernel 32.
// It depends on the head size and format only, so a row's chunks never
// depend on how many rows are scored with it.
uint32_t attn_chunk(uint32_t hd, uint32_t afmt, uint32_t gq)
{
    if (use_mfma(hd, afmt, gq)) return hd == 64u ? 128u : 256u;
    return hd <= 128u ? 64u : 32u;
}

uint64_t attn_partial_bytes(uint32_t batch, uint32_t n_kv, uint32_t group, uint32_t rows, uint32_t hd, uint32_t afmt,
                            uint32_t max_ctx)
{
    const uint32_t ch = attn_chunk(hd, afmt, group * rows);
    const uint32_t nch = (max_ctx + ch - 1u) / ch;
    const uint64_t q = static_cast<uint64_t>(batch) * n_kv * nch * group * rows;
    return align_up(q * hd * 4u, 256) + align_up(q * 2u * 4u, 256);
}

int attn_validate(const opure_model* m, const opure_kv* kv, uint32_t batch, uint32_t rows, uint32_t max_ctx)
{
    OPURE_REQUIRE(m && kv && kv->pool && kv->page_table, OPURE_E_INVALID, "attention: null model or cache");
    OPURE_REQUIRE(m->n_kv_heads >= 1 && m->n_heads % m->n_kv_heads == 0, OPURE_E_INVALID,
                  "attention: n_heads %% n_kv_heads != 0");
    OPURE_REQUIRE(m->head_dim >= 16 && m->head_dim <= 256 && m->head_dim % 16 == 0, OPURE_E_UNSUPPORTED,
                  "attention: head_dim %u not in 16..256 step 16", m->head_dim);
    OPURE_REQUIRE(kv->page_size == OPURE_PAGE_SIZE, OPURE_E_UNSUPPORTED, "attention: page_size must be %d",
                  OPURE_PAGE_SIZE);
    // the folded kernel reads page 0 for a missing page entry (and masks it), so the pool holds one page at least
    OPURE_REQUIRE(kv->n_pages >= 1 && kv->max_pages_per_seq >= 1, OPURE_E_INVALID, "attention: the cache has no pages");
    OPURE_REQUIRE(batch >= 1 && rows >= 1 && rows <= OPURE_MAX_ROWS && batch * rows <= OPURE_MAX_BATCH_ROWS,
                  OPURE_E_CAPACITY, "attention: %u rows per sequence x batch %u beyond %d / %d", rows, batch,
                  OPURE_MAX_ROWS, OPURE_MAX_BATCH_ROWS);
    OPURE_REQUIRE(max_ctx >= rows && max_ctx <= kv->max_pages_per_seq * OPURE_PAGE_SIZE, OPURE_E_CAPACITY,
                  "attention: max_ctx %u beyond the page-table capacity %u", max_ctx,
                  kv->max_pages_per_seq * OPURE_PAGE_SIZE);
    OPURE_REQUIRE(m->afmt <= OPURE_A_BF16, OPURE_E_INVALID, "attention: bad activation format");
    const uint32_t group = m->n_heads / m->n_kv_heads, CH = attn_chunk(m->head_dim, m->afmt, group * rows);
    OPURE_REQUIRE((max_ctx + CH - 1u) / CH <= 1024u, OPURE_E_CAPACITY, "attention: max_ctx %u has more than 1024 chunks",
                  max_ctx);
    if (!use_mfma(m->head_dim, m->afmt, group * rows))
    {
        // VALU kernels hold the query rows (and, generic, the scores and K/V) in LDS
        const uint64_t eb = act_bytes(m->afmt), hd = m->head_dim;
        const uint64_t lds = CH == 64u ? static_cast<uint64_t>(group) * rows * hd * 4u + 64u * (hd * eb + 16u) +
                                             hd * (64u * eb + 16u) + 1024u
                                       : (static_cast<uint64_t>(group) * rows * m->head_dim +
                                          static_cast<uint64_t>(group) * rows * CH +
                                          static_cast<uint64_t>(CH) * (m->head_dim + 1)) * 4u;
        OPURE_REQUIRE(lds <= 160u * 1024u, OPURE_E_CAPACITY, "attention: %u query rows per KV head exceed LDS",
                      group * rows);
    }
    return OPURE_OK;
}

int attn_launch(opure_dev* dev, const opure_model* m, const opure_kv* kv, uint32_t layer, uint32_t batch,
                uint32_t rows, const int32_t* seq_len, uint32_t max_ctx, const void* q, void* out, float* part)
{
    AttnParams p{};
    p.q = q;
    p.out = out;
    p.pool = kv->pool;
    p.page_table = kv->page_table;
    p.seq_len = seq_len;
    p.n_heads = m->n_heads;
    p.n_kv = m->n_kv_heads;
    p.hd = m->head_dim;
    p.rows = rows;
    p.n_pages = kv->n_pages;
    p.max_pages = kv->max_pages_per_seq;
    p.layer = layer;
    const uint32_t group = m->n_heads / m->n_kv_heads, Gq = group * rows;
    p.chunk = attn_chunk(m->head_dim, m->afmt, Gq);
    p.nch = (max_ctx + p.chunk - 1u) / p.chunk;
    p.afmt = m->afmt;
    p.scale = m->attn_scale;
    p.err = dev->err;
    const uint64_t q_elems = static_cast<uint64_t>(batch) * p.n_kv * p.nch * Gq;
    p.part_acc = part;
    p.part_ml = part + align_up(q_elems * p.hd * 4u, 256) / 4u;
    const dim3 grid(p.n_kv, p.nch, batch);
    const uint32_t hd = p.hd;
    p.zt = 1u;
    p.npart = p.nch;
    p.cpp = 1u;
    // head_dim 64 on matrix cores: the combine merges groups of ATTN_GROUP
    // chunks as the folded kernel does (1 item = 1 group), unless the folded
    // kernel wrote the groups' partials itself
    uint32_t grp = use_mfma(hd, p.afmt, Gq) && hd == 64u ? ATTN_GROUP : 1u;
    if (use_mfma(hd, p.afmt, Gq))
    {
        // head_dim 64 on a grid of few workgroups (the 1B shape at batch 1:
        // 136 -> 272 workgroups): one 16-row block of query rows a
        // workgroup, every block in one launch, so the chip fills; otherwise
        // launches of up to 2 blocks a workgroup (at head_dim 128 the split
        // grid measured slower).  Rows are independent in the kernel: each
        // row's result is the same either way.
        const uint32_t blocks = (Gq + 15u) / 16u, n_cu = dev->n_cu > 0 ? static_cast<uint32_t>(dev->n_cu) : 256u;
        if (hd == 64u && blocks >= 2u && static_cast<uint64_t>(p.n_kv) * p.nch * batch * blocks <= 2ull * n_cu &&
            batch * blocks <= 65535u)
        {
            AttnParams pq = p;
            pq.qoff = 0u;
            pq.zt = blocks;
            const dim3 g(p.n_kv, p.nch, batch * blocks);
            int rc;
            if (p.afmt == OPURE_A_F16) rc = launch_mfma<64, OPURE_A_F16, 1, 1, 4, true>(dev, g, pq);
            else rc = launch_mfma<64, OPURE_A_BF16, 1, 1, 4, true>(dev, g, pq);
            if (rc) return rc;
        }
        else
        {
            // a grid of many workgroups (a batch of ragged sequences) folded to
            // ATTN_GROUP chunks a workgroup, merged into one partial: a quarter
            // of the partials written and read, a chunk's page-table entries
            // loaded while the chunk before computes, a chunk past a
            // sequence's end costs no round trip of its own
            const bool fold = hd == 64u && static_cast<uint64_t>(p.n_kv) * p.nch * batch > 8ull * n_cu;
            const dim3 fgrid(p.n_kv, (p.nch + ATTN_GROUP - 1u) / ATTN_GROUP, batch);
            if (fold)
            {
                p.npart = fgrid.y;
                p.cpp = ATTN_GROUP;
                grp = 1u;
            }
            for (uint32_t q0 = 0; q0 < Gq; q0 += 32u)
            {
                AttnParams pq = p;
                pq.qoff = q0;
                const bool one = Gq - q0 <= 16u;
                int rc;
                // head_dim 64: 4 waves x 32 tokens; 128: 4 waves x 64 tokens (two
                // k-steps a wave)
                if (fold && p.afmt == OPURE_A_F16)
                    rc = one ? launch_mfma<64, OPURE_A_F16, 1, 1, 4, false, true>(dev, fgrid, pq)
                             : launch_mfma<64, OPURE_A_F16, 2, 1, 4, false, true>(dev, fgrid, pq);
                else if (fold)
                    rc = one ? launch_mfma<64, OPURE_A_BF16, 1, 1, 4, false, true>(dev, fgrid, pq)
                             : launch_mfma<64, OPURE_A_BF16, 2, 1, 4, false, true>(dev, fgrid, pq);
                else if (hd == 64u && p.afmt == OPURE_A_F16)
                    rc = one ? launch_mfma<64, OPURE_A_F16, 1, 1, 4>(dev, grid, pq) : launch_mfma<64, OPURE_A_F16, 2, 1, 4>(dev, grid, pq);
                else if (hd == 64u)
                    rc = one ? launch_mfma<64, OPURE_A_BF16, 1, 1, 4>(dev, grid, pq) : launch_mfma<64, OPURE_A_BF16, 2, 1, 4>(dev, grid, pq);
                else if (p.afmt == OPURE_A_F16)
                    rc = one ? launch_mfma<128, OPURE_A_F16, 1, 2, 4>(dev, grid, pq) : launch_mfma<128, OPURE_A_F16, 2, 2, 4>(dev, grid, pq);
                else
                    rc = one ? launch_mfma<128, OPURE_A_BF16, 1, 2, 4>(dev, grid, pq) : launch_mfma<128, OPURE_A_BF16, 2, 2, 4>(dev, grid, pq);
                if (rc) return rc;
            }
        }
    }
    else if (p.chunk == 64u && hd == 64u && p.nch <= ATTN_SPLIT_CHUNKS)
    {
        // a short context at head_dim 64: a workgroup a pair of query rows, a
        // wave a chunk, merged in the workgroup (no combine launch)
        const dim3 g(p.n_kv, (Gq + 1u) / 2u, batch), blk(64u * p.nch);
        if (p.afmt == OPURE_A_F32) OPURE_LAUNCH(dev, k_attn_split<OPURE_A_F32>, g, blk, 0, p);
        else if (p.afmt == OPURE_A_F16) OPURE_LAUNCH(dev, k_attn_split<OPURE_A_F16>, g, blk, 0, p);
        else OPURE_LAUNCH(dev, k_attn_split<OPURE_A_BF16>, g, blk, 0, p);
        OPURE_LAUNCH_CHECK("k_attn_split");
        return OPURE_OK;
    }
    else if (p.chunk == 64u && (hd == 64u || hd == 128u))
    {
        // head_dim 128 over at most ATTN_ALL_CHUNKS chunks: one workgroup a (KV
        // head, sequence) takes them all and merges them itself (no combine launch)
        const uint64_t all_lds = static_cast<uint64_t>(Gq) * hd * 4u + attn_all_lds<128>(Gq);
        const bool all = hd == 128u && p.nch <= ATTN_ALL_CHUNKS && all_lds <= 48u * 1024u;
        const uint32_t lds = all ? static_cast<uint32_t>(all_lds) : Gq * hd * 4u;
        const dim3 g = all ? dim3(p.n_kv, 1u, batch) : grid;
        int rc;
        if (hd == 64u && p.afmt == OPURE_A_F32) rc = launch_fast<64, OPURE_A_F32, false>(dev, g, lds, p);
        else if (hd == 64u && p.afmt == OPURE_A_F16) rc = launch_fast<64, OPURE_A_F16, false>(dev, g, lds, p);
        else if (hd == 64u) rc = launch_fast<64, OPURE_A_BF16, false>(dev, g, lds, p);
        else if (p.afmt == OPURE_A_F32)
            rc = all ? launch_fast<128, OPURE_A_F32, true>(dev, g, lds, p) : launch_fast<128, OPURE_A_F32, false>(dev, g, lds, p);
        else if (p.afmt == OPURE_A_F16)
            rc = all ? launch_fast<128, OPURE_A_F16, true>(dev, g, lds, p) : launch_fast<128, OPURE_A_F16, false>(dev, g, lds, p);
        else
            rc = all ? launch_fast<128, OPURE_A_BF16, true>(dev, g, lds, p) : launch_fast<128, OPURE_A_BF16, false>(dev, g, lds, p);
        if (rc) return rc;
        if (all) return OPURE_OK;
    }
    else
    {
        const uint32_t lds = (Gq * hd + Gq * p.chunk + p.chunk * (hd + 1u)) * 4u;
        static bool configured = false;
        if (!configured)
        {
            OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_chunk_generic),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
            configured = true;
        }
        OPURE_LAUNCH(dev, k_attn_chunk_generic, grid, dim3(256), lds, p);
        OPURE_LAUNCH_CHECK("k_attn_chunk_generic");
    }
    const dim3 cgrid(p.n_heads, batch * rows);
    const bool few = p.npart <= 20u;
    if (grp > 1u && few) OPURE_LAUNCH(dev, (k_attn_combine<1, ATTN_GROUP, 20u>), cgrid, dim3(64), 0, p);
    else if (grp > 1u) OPURE_LAUNCH(dev, (k_attn_combine<1, ATTN_GROUP>), cgrid, dim3(64), 0, p);
    else
        switch ((p.hd + 63u) / 64u)
        {
        case 1:
            if (few) OPURE_LAUNCH(dev, (k_attn_combine<1, 1, 20u>), cgrid, dim3(64), 0, p);
            else OPURE_LAUNCH(dev, (k_attn_combine<1, 1>), cgrid, dim3(64), 0, p);
            break;
        case 2: OPURE_LAUNCH(dev, (k_attn_combine<2, 1>), cgrid, dim3(64), 0, p); break;
        case 3: OPURE_LAUNCH(dev, (k_attn_combine<3, 1>), cgrid, dim3(64), 0, p); break;
        default: OPURE_LAUNCH(dev, (k_attn_combine<4, 1>), cgrid, dim3(64), 0, p); break;
        }
    OPURE_LAUNCH_CHECK("k_attn_combine");
    return OPURE_OK;
}

}  // namespace opure_hip

using namespace opure_hip;

extern "C" int opure_attn_decode_paged(opure_dev* dev, const opure_attn_args* a)
{
    OPURE_REQUIRE(dev && a && a->model && a->kv && a->q && a->out && a->seq_len, OPURE_E_INVALID,
                  "opure_attn_decode_paged: null argument");
    int rc = attn_validate(a->model, a->kv, a->batch, a->rows, a->max_ctx);
    if (rc) return rc;
    OPURE_REQUIRE(a->layer * static_cast<uint64_t>(1) < a->model->n_layers, OPURE_E_INVALID, "attention: layer %u",
                  a->layer);
    const uint32_t group = a->model->n_heads / a->model->n_kv_heads;
    rc = ensure_workspace(dev, attn_partial_bytes(a->batch, a->model->n_kv_heads, group, a->rows, a->model->head_dim,
                                                  a->model->afmt, a->max_ctx));
    if (rc) return rc;
    return attn_launch(dev, a->model, a->kv, a->layer, a->batch, a->rows, a->seq_len, a->max_ctx, a->q, a->out,
                       static_cast<float*>(dev->ws));
}
