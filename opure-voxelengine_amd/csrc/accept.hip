// ============================================================================
//  accept.hip -- the acceptance stage and KV rollback of speculative decoding.
//
//  The reference has no acceptance rule, no RNG and no rollback: its only
//  relative is ArgMaxMain (shaders/Opure_ArgMax.usf:33-86, one workgroup over
//  the vocabulary) and speculativeAcceptance is hard-wired to -1
//  (src/engine/Opure_Metrics.cpp:65-68).  Built here from Leviathan et al.
//  2023 / Chen et al. 2023:
//
//  greedy     argmax per row (NaN as -inf, ties -> lowest index), accept the
//             longest prefix of drafts equal to the argmax, emit the argmax of
//             the first mismatching row (or of row K: the bonus token).
//  rejection  for row j: accept x_j iff u_j * q_j(x_j) < p_j(x_j), with
//             u_j = Philox(seed; pos_base[b]+j, b, 1) >> 8 scaled by 2^-24.
//             After the first rejection at row n, draw from max(0, p_n - q_n)
//             normalised; after K accepts, draw the bonus from p_K; both by
//             inverse CDF with U = Philox(seed; pos_base[b]+n, b, 2).
//
//  Softmax at temperature tau in exact fixed point, so every parallel order
//  gives the same bits as the CPU oracle:
//      l_v = logit_v / tau,  m = max_v l_v,  e_v = expf_ref(l_v - m)
//      E_v = floor(e_v * 2^32 + 1/2) (u64),  S = sum_v E_v (u64, exact)
//      accept iff (u * e_q(x)) * S_p < e_p(x) * S_q        (double)
//      p_v = (float)(e_v * (2^32 / S)) , r_v = max(0, p_v - q_v), R_v = fixed(r_v)
//      draw: smallest v whose inclusive prefix of W exceeds floor(U * sum W / 2^32)
//
//  One kernel does the whole rejection stage: a workgroup per (row, sequence)
//  computes its row's statistics and accept bit, and the last workgroup of a
//  sequence to finish (atomic counter, reset afterwards) draws the final token.
// ============================================================================
#include "internal.h"

using namespace opure_dev_math;

namespace {

constexpr uint32_t NT = 256;

__device__ __forceinline__ uint64_t to_fixed(float v)
{
    return v > 0.0f ? static_cast<uint64_t>(__dadd_rn(__dmul_rn(static_cast<double>(v), 4294967296.0), 0.5)) : 0ull;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o)
{
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), o);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), o);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// block reductions over 256 threads (4 waves), fixed order
__device__ float block_max(float v, float* red)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    __syncthreads();
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ uint64_t block_sum_u64(uint64_t v, uint64_t* red)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor_u64(v, o);
    __syncthreads();
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// exclusive prefix over the 256 per-thread values (Hillis-Steele in LDS)
__device__ uint64_t block_exclusive_scan_u64(uint64_t v, uint64_t* buf)
{
    __syncthreads();
    buf[threadIdx.x] = v;
    __syncthreads();
    for (uint32_t o = 1; o < NT; o <<= 1)
    {
        const uint64_t add = threadIdx.x >= o ? buf[threadIdx.x - o] : 0ull;
        __syncthreads();
        buf[threadIdx.x] += add;
        __syncthreads();
    }
    return buf[threadIdx.x] - v;
}

struct Stat { float m; uint64_t S; };

__device__ Stat row_stats(const float* row, uint32_t V, float tau, float* fred, uint64_t* ured)
{
    float mx = -__builtin_huge_valf();
    for (uint32_t v = threadIdx.x; v < V; v += NT) mx = fmaxf(mx, __fdiv_rn(row[v], tau));
    mx = block_max(mx, fred);
    uint64_t s = 0;
    for (uint32_t v = threadIdx.x; v < V; v += NT) s += to_fixed(expf_ref(__fsub_rn(__fdiv_rn(row[v], tau), mx)));
    s = block_sum_u64(s, ured);
    return {mx, s};
}

__device__ __forceinline__ float e_of(const float* row, uint32_t v, float tau, float m)
{
    return expf_ref(__fsub_rn(__fdiv_rn(row[v], tau), m));
}

// Inverse-CDF draw over per-element weights w(v) (recomputed deterministically):
// each thread owns a contiguous segment; the scan of segment sums finds the
// segment containing the threshold, whose owner walks it.
template <class WFn>
__device__ int32_t draw(uint32_t V, uint32_t U, WFn wfn, uint64_t* ured, uint64_t* scan, int32_t* s_tok)
{
    const uint32_t seg = (V + NT - 1u) / NT;
    const uint32_t v0 = threadIdx.x * seg, v1 = min(V, v0 + seg);
    uint64_t mine = 0;
    for (uint32_t v = v0; v < v1; ++v) mine += wfn(v);
    const uint64_t total = block_sum_u64(mine, ured);
    const uint64_t excl = block_exclusive_scan_u64(mine, scan);
    const uint64_t hi = __umul64hi(static_cast<uint64_t>(U), total);
    const uint64_t lo = static_cast<uint64_t>(U) * total;
    const uint64_t t = (hi << 32) | (lo >> 32);
    if (threadIdx.x == 0) *s_tok = static_cast<int32_t>(V - 1u);
    __syncthreads();
    if (mine > 0 && excl <= t && t < excl + mine)
    {
        uint64_t pre = excl;
        for (uint32_t v = v0; v < v1; ++v)
        {
            pre += wfn(v);
            if (pre > t) { *s_tok = static_cast<int32_t>(v); break; }
        }
    }
    __syncthreads();
    return *s_tok;
}

__device__ __forceinline__ float uniform24(uint32_t u) { return static_cast<float>(u >> 8) * (1.0f / 16777216.0f); }

// ---------------------------------------------------------------------------
struct ArgmaxParams {
    const float* logits;
    uint32_t rows, V, chunk, parts;
    float* am_val;       // [parts][rows]
    int32_t* am_idx;
};

__global__ __launch_bounds__(256) void k_argmax_partial(ArgmaxParams p)
{
    __shared__ float sv[4];
    __shared__ int32_t si[4];
    const uint32_t part = blockIdx.x, r = blockIdx.y;
    const float* row = p.logits + static_cast<uint64_t>(r) * p.V;
    const uint32_t v0 = part * p.chunk, v1 = min(p.V, v0 + p.chunk);
    float bv = -__builtin_huge_valf();
    int32_t bi = 0x7FFFFFFF;
    for (uint32_t v = v0 + threadIdx.x; v < v1; v += NT)
    {
        const float c = row[v] != row[v] ? -__builtin_huge_valf() : row[v];
        if (c > bv || (c == bv && static_cast<int32_t>(v) < bi)) { bv = c; bi = static_cast<int32_t>(v); }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
    {
        const float ov = __shfl_xor(bv, o);
        const int32_t oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if ((threadIdx.x & 63u) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0)
    {
        bv = sv[0]; bi = si[0];
        for (int w = 1; w < 4; ++w)
            if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) { bv = sv[w]; bi = si[w]; }
        p.am_val[static_cast<uint64_t>(part) * p.rows + r] = bv;
        p.am_idx[static_cast<uint64_t>(part) * p.rows + r] = bi;
    }
}

struct RollbackParams {
    void* pool;
    int32_t* page_table;
    uint32_t max_pages, n_pages, n_layers, n_kv, hd, afmt, K;
    const int32_t* seq_len;
    const int32_t* accepted;
    int32_t* new_len;
    int32_t* freed;
    uint32_t freed_stride;
    int32_t* n_freed;
    uint32_t poison, poison_bits;
};

// Rollback of sequence b, run by one workgroup: poison the rolled-back slots,
// then release the pages wholly past the new length.
__device__ void rollback_seq(const RollbackParams& p, uint32_t b, uint32_t acc)
{
    int32_t* pt = p.page_table + static_cast<uint64_t>(b) * p.max_pages;
    const uint32_t ctx = static_cast<uint32_t>(p.seq_len[b]);
    if (acc > p.K) acc = p.K;
    const uint32_t old_end = ctx + p.K + 1u, nl = ctx + acc + 1u;
    if (p.poison)
    {
        const uint32_t per_pos = p.n_layers * 2u * p.n_kv * p.hd;
        for (uint32_t pos = nl; pos < old_end; ++pos)
        {
            if (pos / OPURE_PAGE_SIZE >= p.max_pages) break;
            const int32_t page = pt[pos / OPURE_PAGE_SIZE];
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
                if (pt[q] < 0) continue;
                if (static_cast<uint32_t>(nf) < p.freed_stride) p.freed[static_cast<uint64_t>(b) * p.freed_stride + nf] = pt[q];
                pt[q] = -1;
                ++nf;
            }
        }
        if (p.n_freed) p.n_freed[b] = nf;
    }
}

__global__ __launch_bounds__(256) void k_rollback(RollbackParams p)
{
    rollback_seq(p, blockIdx.x, static_cast<uint32_t>(p.accepted[blockIdx.x]));
}

struct GreedyParams {
    const float* am_val;
    const int32_t* am_idx;
    uint32_t parts, rows_total, K;
    const int32_t* drafts;
    uint32_t drafts_stride;
    int32_t* out_tokens;
    int32_t* accepted;
    uint32_t rollback;          // 1: run the rollback of this sequence in the same workgroup
    RollbackParams rb;
};

// One workgroup of GNT threads per sequence.  Each thread scans its share of
// the LM head's per-tile partials for 8 rows at a time, four partials' loads
// in flight together, then each row is reduced across the workgroup.  The
// winner (greater value, then lower index) is a total order, so the result
// does not depend on the reduction order.
constexpr uint32_t GNT = 1024;

__global__ __launch_bounds__(GNT) void k_accept_greedy(GreedyParams p)
{
    constexpr uint32_t RB = 8, UP = 4, NWV = GNT / 64u;
    __shared__ float sv[NWV][RB];
    __shared__ int32_t si[NWV][RB];
    __shared__ int32_t am[64];
    __shared__ uint32_t s_n;
    const uint32_t b = blockIdx.x, R = p.K + 1u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    for (uint32_t r0 = 0; r0 < R; r0 += RB)
    {
        const uint32_t nr = min(RB, R - r0);
        float bv[RB];
        int32_t bi[RB];
#pragma unroll
        for (uint32_t i = 0; i < RB; ++i) { bv[i] = -__builtin_huge_valf(); bi[i] = 0x7FFFFFFF; }
        for (uint32_t part = threadIdx.x; part < p.parts; part += GNT * UP)
        {
            float v[UP][RB];
            int32_t x[UP][RB];
#pragma unroll
            for (uint32_t u = 0; u < UP; ++u)
            {
                const uint32_t pp = part + u * GNT;
                const uint64_t base = static_cast<uint64_t>(pp) * p.rows_total + b * R + r0;
#pragma unroll
                for (uint32_t i = 0; i < RB; ++i)
                {
                    const bool on = pp < p.parts && i < nr;
                    v[u][i] = on ? p.am_val[base + i] : -__builtin_huge_valf();
                    x[u][i] = on ? p.am_idx[base + i] : 0x7FFFFFFF;
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < UP; ++u)
#pragma unroll
                for (uint32_t i = 0; i < RB; ++i)
                    if (v[u][i] > bv[i] || (v[u][i] == bv[i] && x[u][i] < bi[i])) { bv[i] = v[u][i]; bi[i] = x[u][i]; }
        }
#pragma unroll
        for (uint32_t i = 0; i < RB; ++i)
        {
#pragma unroll
            for (int o = 32; o > 0; o >>= 1)
            {
                const float ov = __shfl_xor(bv[i], o);
                const int32_t oi = __shfl_xor(bi[i], o);
                if (ov > bv[i] || (ov == bv[i] && oi < bi[i])) { bv[i] = ov; bi[i] = oi; }
            }
        }
        if (lane == 0)
        {
#pragma unroll
            for (uint32_t i = 0; i < RB; ++i) { sv[wave][i] = bv[i]; si[wave][i] = bi[i]; }
        }
        __syncthreads();
        if (threadIdx.x < nr)
        {
            const uint32_t i = threadIdx.x;
            float v = sv[0][i];
            int32_t x = si[0][i];
            for (uint32_t w = 1; w < NWV; ++w)
                if (sv[w][i] > v || (sv[w][i] == v && si[w][i] < x)) { v = sv[w][i]; x = si[w][i]; }
            am[r0 + i] = x == 0x7FFFFFFF ? 0 : x;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0)
    {
        uint32_t n = 0;
        while (n < p.K && am[n] == p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + n]) ++n;
        for (uint32_t j = 0; j < R; ++j)
            p.out_tokens[b * R + j] = j < n ? p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + j] : (j == n ? am[n] : -1);
        p.accepted[b] = static_cast<int32_t>(n);
        s_n = n;
    }
    __syncthreads();
    if (p.rollback) rollback_seq(p.rb, b, s_n);
}

// ---------------------------------------------------------------------------
struct RejRow { float mp, mq; uint64_t Sp, Sq; uint32_t accept, pad; };

struct RejectParams {
    const float* target;      // [B][K+1][V]
    const float* draft;       // [B][K][V]
    const int32_t* drafts;
    uint32_t drafts_stride;
    uint32_t K, V;
    float tau;
    uint64_t seed;
    const uint32_t* pos_base;
    int32_t* out_tokens;
    int32_t* accepted;
    float* dist;
    RejRow* ws;               // [B][K+1]
    uint32_t* counters;       // [B]
    const int32_t* seq_len;   // optional new_seq_len = seq_len + n + 1
    int32_t* new_seq_len;
};

__global__ __launch_bounds__(256) void k_accept_rejection(RejectParams p)
{
    __shared__ float fred[4];
    __shared__ uint64_t ured[4];
    __shared__ uint64_t scan[NT];
    __shared__ int32_t s_tok;
    __shared__ uint32_t s_last;
    const uint32_t j = blockIdx.x, b = blockIdx.y, K = p.K, V = p.V;
    const float tau = p.tau;
    const uint32_t pb = p.pos_base ? p.pos_base[b] : 0u;
    const float* trow = p.target + (static_cast<uint64_t>(b) * (K + 1u) + j) * V;
    const Stat P = row_stats(trow, V, tau, fred, ured);
    RejRow rr{P.m, 0.0f, P.S, 0ull, 0u, 0u};
    if (j < K)
    {
        const float* qrow = p.draft + (static_cast<uint64_t>(b) * K + j) * V;
        const Stat Q = row_stats(qrow, V, tau, fred, ured);
        rr.mq = Q.m;
        rr.Sq = Q.S;
        const int32_t x = p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + j];
        if (x >= 0 && static_cast<uint32_t>(x) < V)
        {
            const float ep = e_of(trow, static_cast<uint32_t>(x), tau, P.m);
            const float eq = e_of(qrow, static_cast<uint32_t>(x), tau, Q.m);
            const float u = uniform24(philox_u32(p.seed, pb + j, b, 1u));
            const double lhs = __dmul_rn(__dmul_rn(static_cast<double>(u), static_cast<double>(eq)), static_cast<double>(P.S));
            const double rhs = __dmul_rn(static_cast<double>(ep), static_cast<double>(Q.S));
            rr.accept = lhs < rhs ? 1u : 0u;
        }
    }
    if (threadIdx.x == 0) p.ws[static_cast<uint64_t>(b) * (K + 1u) + j] = rr;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicAdd(&p.counters[b], 1u) == K ? 1u : 0u;
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    // ---- last workgroup of sequence b: find n, draw the final token --------
    const RejRow* rows = p.ws + static_cast<uint64_t>(b) * (K + 1u);
    uint32_t n = K;
    for (uint32_t i = 0; i < K; ++i)
        if (!__builtin_nontemporal_load(&rows[i].accept)) { n = i; break; }
    const uint32_t U = philox_u32(p.seed, pb + n, b, 2u);
    float* dist = p.dist ? p.dist + static_cast<uint64_t>(b) * V : nullptr;
    const float* tn = p.target + (static_cast<uint64_t>(b) * (K + 1u) + n) * V;
    const float mp = __builtin_nontemporal_load(&rows[n].mp);
    const uint64_t Sp = __builtin_nontemporal_load(&rows[n].Sp);
    const double invP = __ddiv_rn(4294967296.0, static_cast<double>(Sp));
    int32_t tok;
    if (n < K)
    {
        const float* qn = p.draft + (static_cast<uint64_t>(b) * K + n) * V;
        const float mq = __builtin_nontemporal_load(&rows[n].mq);
        const uint64_t Sq = __builtin_nontemporal_load(&rows[n].Sq);
        const double invQ = __ddiv_rn(4294967296.0, static_cast<double>(Sq));
        auto rfn = [&](uint32_t v) -> float {
            const float pf = static_cast<float>(__dmul_rn(static_cast<double>(e_of(tn, v, tau, mp)), invP));
            const float qf = static_cast<float>(__dmul_rn(static_cast<double>(e_of(qn, v, tau, mq)), invQ));
            const float d = __fsub_rn(pf, qf);
            return d > 0.0f ? d : 0.0f;
        };
        uint64_t mine = 0;
        for (uint32_t v = threadIdx.x; v < V; v += NT) mine += to_fixed(rfn(v));
        const uint64_t Rs = block_sum_u64(mine, ured);
        if (Rs > 0)
        {
            tok = draw(V, U, [&](uint32_t v) { return to_fixed(rfn(v)); }, ured, scan, &s_tok);
            if (dist)
            {
                const double invR = __ddiv_rn(4294967296.0, static_cast<double>(Rs));
                for (uint32_t v = threadIdx.x; v < V; v += NT)
                    dist[v] = static_cast<float>(__dmul_rn(static_cast<double>(rfn(v)), invR));
            }
        }
        else
        {
            tok = draw(V, U, [&](uint32_t v) { return to_fixed(e_of(tn, v, tau, mp)); }, ured, scan, &s_tok);
            if (dist)
                for (uint32_t v = threadIdx.x; v < V; v += NT)
                    dist[v] = static_cast<float>(__dmul_rn(static_cast<double>(e_of(tn, v, tau, mp)), invP));
        }
    }
    else
    {
        tok = draw(V, U, [&](uint32_t v) { return to_fixed(e_of(tn, v, tau, mp)); }, ured, scan, &s_tok);
        if (dist)
            for (uint32_t v = threadIdx.x; v < V; v += NT)
                dist[v] = static_cast<float>(__dmul_rn(static_cast<double>(e_of(tn, v, tau, mp)), invP));
    }
    if (threadIdx.x == 0)
    {
        for (uint32_t i = 0; i <= K; ++i)
            p.out_tokens[b * (K + 1u) + i] =
                i < n ? p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + i] : (i == n ? tok : -1);
        p.accepted[b] = static_cast<int32_t>(n);
        if (p.new_seq_len) p.new_seq_len[b] = p.seq_len[b] + static_cast<int32_t>(n) + 1;
        p.counters[b] = 0u;
    }
}

// ---------------------------------------------------------------------------
struct SampleParams {
    const float* logits;
    uint32_t V;
    float tau;
    uint64_t seed;
    const uint32_t* pos;
    const uint32_t* seq;
    uint32_t stream;
    int32_t* out;
};

__global__ __launch_bounds__(256) void k_sample(SampleParams p)
{
    __shared__ float fred[4];
    __shared__ uint64_t ured[4];
    __shared__ uint64_t scan[NT];
    __shared__ int32_t s_tok;
    const uint32_t r = blockIdx.x;
    const float* row = p.logits + static_cast<uint64_t>(r) * p.V;
    const Stat st = row_stats(row, p.V, p.tau, fred, ured);
    const uint32_t U = philox_u32(p.seed, p.pos[r], p.seq[r], p.stream);
    const int32_t tok = draw(p.V, U, [&](uint32_t v) { return to_fixed(e_of(row, v, p.tau, st.m)); }, ured, scan, &s_tok);
    if (threadIdx.x == 0) p.out[r] = tok;
}

__global__ void k_philox(uint64_t seed, const uint32_t* pos, const uint32_t* seq, uint32_t stream, uint32_t n, uint32_t* out)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = philox_u32(seed, pos[i], seq[i], stream);
}

}  // namespace

namespace opure_hip {

uint32_t argmax_parts(uint32_t V) { return (V + 4095u) / 4096u; }

uint64_t accept_ws_bytes(uint32_t batch, uint32_t k, uint32_t vocab, uint32_t mode)
{
    if (mode == OPURE_ACCEPT_REJECTION) return align_up(static_cast<uint64_t>(batch) * (k + 1u) * sizeof(RejRow), 256);
    return 2u * align_up(static_cast<uint64_t>(argmax_parts(vocab)) * batch * (k + 1u) * 4u, 256);
}

int accept_validate(const opure_accept_args* a, bool rejection)
{
    OPURE_REQUIRE(a && a->target_logits && a->drafts && a->out_tokens && a->accepted, OPURE_E_INVALID,
                  "accept: null argument");
    OPURE_REQUIRE(a->batch >= 1 && a->vocab >= 1 && a->k + 1u <= 64u, OPURE_E_INVALID,
                  "accept: bad shape (batch %u, k %u, vocab %u)", a->batch, a->k, a->vocab);
    OPURE_REQUIRE(a->drafts_stride >= a->k, OPURE_E_INVALID, "accept: drafts_stride < k");
    if (rejection)
    {
        OPURE_REQUIRE(a->draft_logits || a->k == 0, OPURE_E_INVALID, "accept: rejection needs draft logits");
        OPURE_REQUIRE(a->temperature > 0.0f && a->temperature == a->temperature, OPURE_E_INVALID,
                      "accept: temperature must be > 0");
    }
    return OPURE_OK;
}

static RollbackParams rollback_params(const opure_rollback_args* a)
{
    const opure_model* m = a->model;
    RollbackParams r;
    r.pool = a->kv->pool;
    r.page_table = a->kv->page_table;
    r.max_pages = a->kv->max_pages_per_seq;
    r.n_pages = a->kv->n_pages;
    r.n_layers = m->n_layers;
    r.n_kv = m->n_kv_heads;
    r.hd = m->head_dim;
    r.afmt = m->afmt;
    r.K = a->k;
    r.seq_len = a->seq_len;
    r.accepted = a->accepted;
    r.new_len = a->new_seq_len;
    r.freed = a->freed;
    r.freed_stride = a->freed_stride;
    r.n_freed = a->n_freed;
    r.poison = a->poison;
    r.poison_bits = a->poison_bits;
    return r;
}

int greedy_from_partials(opure_dev* dev, const float* am_val, const int32_t* am_idx, uint32_t parts, uint32_t batch,
                         uint32_t K, const int32_t* drafts, uint32_t stride, int32_t* out_tokens, int32_t* accepted,
                         const opure_rollback_args* rb)
{
    GreedyParams g;
    g.am_val = am_val;
    g.am_idx = am_idx;
    g.parts = parts;
    g.rows_total = batch * (K + 1u);
    g.K = K;
    g.drafts = drafts;
    g.drafts_stride = stride;
    g.out_tokens = out_tokens;
    g.accepted = accepted;
    g.rollback = rb ? 1u : 0u;
    if (rb) g.rb = rollback_params(rb);
    hipLaunchKernelGGL(k_accept_greedy, dim3(batch), dim3(GNT), 0, dev->stream, g);
    OPURE_LAUNCH_CHECK("k_accept_greedy");
    return OPURE_OK;
}

int accept_greedy_launch(opure_dev* dev, const opure_accept_args* a, void* ws)
{
    const uint32_t rows = a->batch * (a->k + 1u), parts = argmax_parts(a->vocab);
    ArgmaxParams ap;
    ap.logits = a->target_logits;
    ap.rows = rows;
    ap.V = a->vocab;
    ap.chunk = 4096u;
    ap.parts = parts;
    ap.am_val = static_cast<float*>(ws);
    ap.am_idx = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + align_up(static_cast<uint64_t>(parts) * rows * 4u, 256));
    hipLaunchKernelGGL(k_argmax_partial, dim3(parts, rows), dim3(NT), 0, dev->stream, ap);
    OPURE_LAUNCH_CHECK("k_argmax_partial");
    return greedy_from_partials(dev, ap.am_val, ap.am_idx, parts, a->batch, a->k, a->drafts, a->drafts_stride,
                                a->out_tokens, a->accepted, nullptr);
}

int accept_rejection_launch(opure_dev* dev, const opure_accept_args* a, void* ws, uint32_t* counters,
                            const int32_t* seq_len, int32_t* new_seq_len)
{
    RejectParams r;
    r.target = a->target_logits;
    r.draft = a->draft_logits;
    r.drafts = a->drafts;
    r.drafts_stride = a->drafts_stride;
    r.K = a->k;
    r.V = a->vocab;
    r.tau = a->temperature;
    r.seed = a->seed;
    r.pos_base = a->pos_base;
    r.out_tokens = a->out_tokens;
    r.accepted = a->accepted;
    r.dist = a->dist_out;
    r.ws = static_cast<RejRow*>(ws);
    r.counters = counters;
    r.seq_len = seq_len;
    r.new_seq_len = new_seq_len;
    hipLaunchKernelGGL(k_accept_rejection, dim3(a->k + 1u, a->batch), dim3(NT), 0, dev->stream, r);
    OPURE_LAUNCH_CHECK("k_accept_rejection");
    return OPURE_OK;
}

int rollback_launch(opure_dev* dev, const opure_rollback_args* a)
{
    const RollbackParams r = rollback_params(a);
    hipLaunchKernelGGL(k_rollback, dim3(a->batch), dim3(NT), 0, dev->stream, r);
    OPURE_LAUNCH_CHECK("k_rollback");
    return OPURE_OK;
}

int rollback_validate(const opure_rollback_args* a)
{
    OPURE_REQUIRE(a && a->model && a->kv && a->kv->pool && a->kv->page_table && a->seq_len && a->accepted &&
                      a->new_seq_len, OPURE_E_INVALID, "rollback: null argument");
    OPURE_REQUIRE(a->batch >= 1 && a->kv->page_size == OPURE_PAGE_SIZE, OPURE_E_INVALID, "rollback: bad shape");
    OPURE_REQUIRE(!a->freed || a->freed_stride >= 1, OPURE_E_INVALID, "rollback: freed_stride must be >= 1");
    return OPURE_OK;
}

}  // namespace opure_hip

using namespace opure_hip;

extern "C" {

int opure_accept_greedy(opure_dev* dev, const opure_accept_args* a)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_accept_greedy: null device");
    int rc = accept_validate(a, false);
    if (rc) return rc;
    rc = ensure_workspace(dev, accept_ws_bytes(a->batch, a->k, a->vocab, OPURE_ACCEPT_GREEDY), 0);
    if (rc) return rc;
    return accept_greedy_launch(dev, a, dev->ws);
}

int opure_accept_rejection(opure_dev* dev, const opure_accept_args* a)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_accept_rejection: null device");
    int rc = accept_validate(a, true);
    if (rc) return rc;
    rc = ensure_workspace(dev, accept_ws_bytes(a->batch, a->k, a->vocab, OPURE_ACCEPT_REJECTION), a->batch);
    if (rc) return rc;
    return accept_rejection_launch(dev, a, dev->ws, dev->counters, nullptr, nullptr);
}

int opure_sample_rows(opure_dev* dev, const opure_sample_args* a)
{
    OPURE_REQUIRE(dev && a && a->logits && a->pos && a->seq && a->out && a->rows >= 1 && a->vocab >= 1, OPURE_E_INVALID,
                  "opure_sample_rows: bad argument");
    OPURE_REQUIRE(a->temperature > 0.0f, OPURE_E_INVALID, "opure_sample_rows: temperature must be > 0");
    SampleParams s{a->logits, a->vocab, a->temperature, a->seed, a->pos, a->seq, a->stream, a->out};
    hipLaunchKernelGGL(k_sample, dim3(a->rows), dim3(NT), 0, dev->stream, s);
    OPURE_LAUNCH_CHECK("k_sample");
    return OPURE_OK;
}

int opure_philox_uniform(opure_dev* dev, uint64_t seed, const uint32_t* pos, const uint32_t* seq, uint32_t stream,
                         uint32_t n, uint32_t* out)
{
    OPURE_REQUIRE(dev && pos && seq && out, OPURE_E_INVALID, "opure_philox_uniform: null argument");
    if (!n) return OPURE_OK;
    hipLaunchKernelGGL(k_philox, dim3((n + 255u) / 256u), dim3(256), 0, dev->stream, seed, pos, seq, stream, n, out);
    OPURE_LAUNCH_CHECK("k_philox");
    return OPURE_OK;
}

int opure_kv_rollback(opure_dev* dev, const opure_rollback_args* a)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_kv_rollback: null device");
    int rc = rollback_validate(a);
    if (rc) return rc;
    return rollback_launch(dev, a);
}

}  // extern "C"
