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
//  The rejection stage runs as three launches (row statistics, per-slice draw
//  weights, per-slice draw), described at k_rej_rowstat.
// ============================================================================
#include "internal.h"
#include "rollback.h"

using namespace opure_dev_math;
using opure_hip::RollbackParams;
using opure_hip::RollbackPre;
using opure_hip::rollback_pre;
using opure_hip::rollback_seq;

namespace {

constexpr uint32_t NT = 256;

// the same value as a double, for sums of probabilities: for a float v in
// [0, 2^20) the fma v * 2^32 + 1/2 is exact in double, so its floor is
// fixed(v); with v <= 1 every term is at most 2^32 and sums of fewer than 2^20
// terms stay exact integers.  NaN and v <= 0 give 0.
__device__ __forceinline__ double fixed_d(float v)
{
    const double d = __builtin_floor(__fma_rn(static_cast<double>(v), 4294967296.0, 0.5));
    return d > 0.0 ? d : 0.0;
}

__device__ __forceinline__ uint64_t fixed_sum_u64(double s) { return static_cast<uint64_t>(s); }

// floor(v * 2^32 + 1/2) for v in [0, 2^31) (0 for v <= 0 and NaN), from the
// float's fields: v * 2^32 = m * 2^(e - 118) exactly, rounded half up
__device__ __forceinline__ uint64_t to_fixed(float v)
{
    if (!(v > 0.0f)) return 0ull;
    const uint32_t b = f_bits(v);
    const int32_t sh = static_cast<int32_t>(b >> 23) - 118;
    const uint64_t m = (b & 0x7FFFFFu) | 0x800000u;
    if (sh >= 0) return m << sh;
    const uint32_t rs = static_cast<uint32_t>(-sh);
    return rs >= 25u ? 0ull : (m + (1ull << (rs - 1u))) >> rs;
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
    v = wave_max64(v);
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

__global__ __launch_bounds__(256) void k_rollback(RollbackParams p)
{
    __shared__ RollbackPre pre;
    __shared__ uint32_t acc;
    if (threadIdx.x == 0)
    {
        pre = rollback_pre(p, blockIdx.x);
        acc = static_cast<uint32_t>(p.accepted[blockIdx.x]);
    }
    __syncthreads();
    rollback_seq(p, blockIdx.x, acc, pre);
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
// does not depend on the reduction order.  256 threads: the LM head leaves
// one partial per CU and row, and 1024 threads only lengthened the
// workgroup's reductions (C3 9.3 -> 8.1 us, C4 11.0 -> 9.7 us; 64 and 128
// threads measured the same as 256).
constexpr uint32_t GNT = 256;

__global__ __launch_bounds__(GNT) void k_accept_greedy(GreedyParams p)
{
    constexpr uint32_t RB = 8, UP = 4, NWV = GNT / 64u;
    __shared__ float sv[NWV][RB];
    __shared__ int32_t si[NWV][RB];
    __shared__ int32_t am[64];
    __shared__ int32_t sdraft[OPURE_MAX_ROWS];
    __shared__ RollbackPre pre;
    __shared__ uint32_t s_n;
    const uint32_t b = blockIdx.x, R = p.K + 1u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    // the drafts and the rollback's reads, in flight with the partials below
    if (threadIdx.x < p.K) sdraft[threadIdx.x] = p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + threadIdx.x];
    if (p.rollback && threadIdx.x == 64u) pre = rollback_pre(p.rb, b);
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
        while (n < p.K && am[n] == sdraft[n]) ++n;
        s_n = n;
    }
    __syncthreads();
    const uint32_t n = s_n;
    if (threadIdx.x < R) p.out_tokens[b * R + threadIdx.x] = threadIdx.x < n ? sdraft[threadIdx.x] : (threadIdx.x == n ? am[n] : -1);
    if (threadIdx.x == 0) p.accepted[b] = static_cast<int32_t>(n);
    if (p.rollback) rollback_seq(p.rb, b, n, pre);
}

// ---------------------------------------------------------------------------
// Rejection sampling in three launches, all rows and slices in parallel:
//   k_rej_rowstat  one 1024-thread workgroup per logit row (K+1 target rows
//                  and K draft rows of each sequence): m = max l, S = sum of
//                  fixed(e_v), and e(x) of the row's draft token; rows too
//                  long to hold in registers take the same statistics from
//                  their slices instead (k_rej_smax, k_rej_ssum, k_rej_rowfin)
//   k_rej_slice    per (slice, sequence): n from the accept tests, then the
//                  draw weights of row n for the slice (residual max(0,p-q),
//                  or p_K after K accepts) into a [B][V] buffer, and the
//                  slice's exact sums of fixed(residual) and fixed(p)
//   k_rej_draw     per (slice, sequence): the inverse-CDF threshold against
//                  the slices' exact prefix; the slice holding it finds the
//                  token, every slice writes its part of the distribution
// Every sum is an exact u64 sum of fixed-point weights, so the parallel
// decomposition gives the bits of the sequential definition above.
struct RowStat { float m, ex; uint64_t S; };
struct SlicePart { uint64_t R, P; };

constexpr uint32_t RNT = 1024;                 // k_rej_rowstat threads
constexpr uint32_t RVEC = 12;                  // float4s of logits held per thread by k_rej_rowstat
constexpr uint32_t SLICE = 4096;               // elements per slice of k_rej_slice / k_rej_draw

struct RejectParams {
    const float* target;      // [B][K+1][V]
    const float* draft;       // [B][K][V]
    const int32_t* drafts;
    uint32_t drafts_stride;
    uint32_t K, V, slices;
    uint32_t phase;           // k_rej_rowstat rows: 0 all, 1 position 0's two, 2 the rest (see k_rej_rowstat)
    float tau;
    uint64_t seed;
    const uint32_t* pos_base;
    int32_t* out_tokens;
    int32_t* accepted;
    float* dist;              // [B][V] or null
    RowStat* stats;           // [B][2K+1]: target rows 0..K, then draft rows
    float* smax;              // [B][2K+1][slices] slice maxima        } rows too long for
    uint64_t* ssum;           // [B][2K+1][slices] slice sums of fixed } registers
    float* sex;               // [B][2K+1] e(x) of the row's draft token }
    SlicePart* parts;         // [B][slices]
    float* wbuf;              // [B][V] draw weights of row n
    const int32_t* seq_len;   // optional new_seq_len = seq_len + n + 1
    int32_t* new_seq_len;
    // the one-launch sampler (k_rej_fused): the sequences' launch counts and
    // their slices' published values [REJ_SYNC_SEQS][REJ_MAX_SLICES][6], the
    // bound on a wait (sleeps) and the error word it sets past it
    uint32_t* epoch;
    uint64_t* slots;
    uint32_t wait_limit;
    uint32_t* err;
};

template <uint32_t NTH>
__device__ float block_max_n(float v, float* red)
{
    v = wave_max64(v);
    __syncthreads();
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (uint32_t w = 1; w < NTH / 64u; ++w) r = fmaxf(r, red[w]);
    return r;
}

template <uint32_t NTH>
__device__ uint64_t block_sum_u64_n(uint64_t v, uint64_t* red)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor_u64(v, o);
    __syncthreads();
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t r = 0;
#pragma unroll
    for (uint32_t w = 0; w < NTH / 64u; ++w) r += red[w];
    return r;
}

// logit / tau; DIV is false exactly when tau == 1 (x / 1 == x)
template <bool DIV>
__device__ __forceinline__ float scaled_logit(float x, float tau) { return DIV ? __fdiv_rn(x, tau) : x; }

// logit row r of sequence b: target rows 0..K, draft rows K+1..2K
__device__ __forceinline__ const float* rej_row(const RejectParams& p, uint32_t b, uint32_t r)
{
    return r <= p.K ? p.target + (static_cast<uint64_t>(b) * (p.K + 1u) + r) * p.V
                    : p.draft + (static_cast<uint64_t>(b) * p.K + (r - p.K - 1u)) * p.V;
}

// The accept test of draft j of sequence b (draft token x, target row
// statistics P, draft row statistics Q): u * q(x) < p(x), the rule accept =
// min(1, p/q), as exact products of the row sums
__device__ __forceinline__ bool rej_accepts(const RejectParams& p, uint32_t b, uint32_t pb, uint32_t j, int32_t x,
                                            const RowStat& P, const RowStat& Q)
{
    if (x < 0 || static_cast<uint32_t>(x) >= p.V) return false;
    const float u = uniform24(philox_u32(p.seed, pb + j, b, 1u));
    const double lhs = __dmul_rn(__dmul_rn(static_cast<double>(u), static_cast<double>(Q.ex)), static_cast<double>(P.S));
    const double rhs = __dmul_rn(static_cast<double>(P.ex), static_cast<double>(Q.S));
    return lhs < rhs;
}

// row of blockIdx i in a phase: 0 every row, 1 position 0's target and draft
// rows, 2 the other rows (target 1..K, draft 1..K-1)
__device__ __forceinline__ uint32_t rej_phase_row(const RejectParams& p, uint32_t i)
{
    return p.phase == 0u ? i : p.phase == 1u ? (i == 0u ? 0u : p.K + 1u) : (i < p.K ? i + 1u : i + 2u);
}

// The row is read once, as float4s held in registers (V % 4 == 0,
// V <= 4 * RNT * RVEC, 16-byte aligned rows; longer rows go through the
// slices below).
// Rows by p.phase: 0 every row (blockIdx.x = row); 1 the target and draft
// rows of position 0 (blockIdx.x 0, 1); 2 the other rows (target 1..K, draft
// 1..K-1), where a sequence whose first draft was rejected needs none of them
// -- the stages after this read only the rows up to the first rejection -- so
// its workgroups test draft 0 from phase 1's statistics and leave.
template <bool DIV>
__global__ __launch_bounds__(RNT) void k_rej_rowstat(RejectParams p)
{
    typedef float f4v __attribute__((ext_vector_type(4)));
    __shared__ float fred[RNT / 64];
    __shared__ uint64_t ured[RNT / 64];
    const uint32_t b = blockIdx.y, V = p.V, K = p.K;
    const uint32_t r = rej_phase_row(p, blockIdx.x);
    if (p.phase == 2u)
    {
        const RowStat* st = p.stats + static_cast<uint64_t>(b) * (2u * K + 1u);
        const uint32_t pb = p.pos_base ? p.pos_base[b] : 0u;
        if (!rej_accepts(p, b, pb, 0u, p.drafts[static_cast<uint64_t>(b) * p.drafts_stride], st[0], st[K + 1u])) return;
    }
    const float tau = p.tau;
    const float* row = rej_row(p, b, r);
    float mx = -__builtin_huge_valf();
    f4v vals[RVEC];
    const uint32_t nv = V / 4u;
    const f4v* row4 = reinterpret_cast<const f4v*>(row);
#pragma unroll
    for (uint32_t i = 0; i < RVEC; ++i)
    {
        const uint32_t q = threadIdx.x + i * RNT;
        vals[i] = q < nv ? row4[q] : f4v{-__builtin_huge_valf(), -__builtin_huge_valf(), -__builtin_huge_valf(),
                                         -__builtin_huge_valf()};
#pragma unroll
        for (int e = 0; e < 4; ++e)
        {
            vals[i][e] = scaled_logit<DIV>(vals[i][e], tau);
            mx = fmaxf(mx, vals[i][e]);
        }
    }
    mx = block_max_n<RNT>(mx, fred);
    // padding lanes hold -inf: exp gives 0, fixed 0
    double sd = 0.0;
#pragma unroll
    for (uint32_t i = 0; i < RVEC; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) sd += fixed_d(expf_ref_nonpos(__fsub_rn(vals[i][e], mx)));
    const uint64_t s = block_sum_u64_n<RNT>(fixed_sum_u64(sd), ured);
    if (threadIdx.x == 0)
    {
        float ex = 0.0f;
        const uint32_t j = r <= K ? r : r - K - 1u;
        if (r != K)
        {
            const int32_t x = p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + j];
            if (x >= 0 && static_cast<uint32_t>(x) < V) ex = expf_ref(__fsub_rn(scaled_logit<DIV>(row[x], tau), mx));
        }
        p.stats[static_cast<uint64_t>(b) * (2u * K + 1u) + r] = RowStat{mx, ex, s};
    }
}

// ---- statistics of rows too long for registers, from their slices ----------
// k_rej_smax writes each SLICE-logit slice's maximum; k_rej_ssum takes the
// row maximum from the slice maxima and writes the slice's exact sum of
// fixed(e) and, in the slice holding the row's draft token (slice 0 when the
// row has none), e(x); k_rej_rowfin puts each row's RowStat together: the
// maximum of the slice maxima and the u64 sum of the slice sums.  A maximum
// and an integer sum do not depend on the order of their terms, so the
// RowStat has the bits of k_rej_rowstat's one-workgroup reduction, while a
// row is spread over `slices` workgroups.  Rows by p.phase as in
// k_rej_rowstat (blockIdx.y); in phase 2 a sequence whose first draft was
// rejected reads no rows.

// RowStat of row r of sequence b from its slices, by one wave (lanes over the
// slices; slices <= 64)
__device__ RowStat rej_stat_from_slices(const RejectParams& p, uint32_t b, uint32_t r, uint32_t lane)
{
    const uint64_t rb = static_cast<uint64_t>(b) * (2u * p.K + 1u) + r;
    float m = -__builtin_huge_valf();
    uint64_t s = 0;
    if (lane < p.slices)
    {
        m = p.smax[rb * p.slices + lane];
        s = p.ssum[rb * p.slices + lane];
    }
    const float ex = p.sex[rb];
    m = wave_max64(m);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += shfl_xor_u64(s, o);
    return RowStat{m, ex, s};
}

// phase 2: whether sequence b's first draft was accepted, from the slices of
// rows 0 and K + 1 (wave 0 decides, the workgroup reads the answer)
__device__ bool rej_first_accepted_sliced(const RejectParams& p, uint32_t b, uint32_t* flag)
{
    if (threadIdx.x < 64u)
    {
        const uint32_t lane = threadIdx.x, pb = p.pos_base ? p.pos_base[b] : 0u;
        const int32_t x = p.drafts[static_cast<uint64_t>(b) * p.drafts_stride];
        const RowStat P = rej_stat_from_slices(p, b, 0u, lane);
        const RowStat Q = rej_stat_from_slices(p, b, p.K + 1u, lane);
        if (lane == 0u) *flag = rej_accepts(p, b, pb, 0u, x, P, Q) ? 1u : 0u;
    }
    __syncthreads();
    return *flag != 0u;
}

template <bool DIV>
__global__ __launch_bounds__(NT) void k_rej_smax(RejectParams p)
{
    __shared__ float fred[NT / 64];
    __shared__ uint32_t go;
    constexpr uint32_t PER = SLICE / NT;
    const uint32_t sl = blockIdx.x, b = blockIdx.z, r = rej_phase_row(p, blockIdx.y), V = p.V;
    if (p.phase == 2u && !rej_first_accepted_sliced(p, b, &go)) return;
    const float* row = rej_row(p, b, r);
    const uint32_t v0 = sl * SLICE;
    float x[PER];
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i) x[i] = row[min(v0 + i * NT + threadIdx.x, V - 1u)];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i)
        if (v0 + i * NT + threadIdx.x < V) mx = fmaxf(mx, scaled_logit<DIV>(x[i], p.tau));
    mx = block_max_n<NT>(mx, fred);
    if (threadIdx.x == 0u) p.smax[(static_cast<uint64_t>(b) * (2u * p.K + 1u) + r) * p.slices + sl] = mx;
}

template <bool DIV>
__global__ __launch_bounds__(NT) void k_rej_ssum(RejectParams p)
{
    __shared__ float fred[NT / 64];
    __shared__ uint64_t ured[NT / 64];
    __shared__ uint32_t go;
    constexpr uint32_t PER = SLICE / NT;
    const uint32_t sl = blockIdx.x, b = blockIdx.z, r = rej_phase_row(p, blockIdx.y), V = p.V, K = p.K;
    if (p.phase == 2u && !rej_first_accepted_sliced(p, b, &go)) return;
    const float tau = p.tau;
    const float* row = rej_row(p, b, r);
    const uint64_t rb = static_cast<uint64_t>(b) * (2u * K + 1u) + r;
    const uint32_t v0 = sl * SLICE;
    // the slice's logits and the row's slice maxima in one round
    float x[PER];
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i) x[i] = row[min(v0 + i * NT + threadIdx.x, V - 1u)];
    const float ms = threadIdx.x < p.slices ? p.smax[rb * p.slices + threadIdx.x] : -__builtin_huge_valf();
    const float m = block_max_n<NT>(ms, fred);
    double sd = 0.0;
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i)
        if (v0 + i * NT + threadIdx.x < V) sd += fixed_d(expf_ref_nonpos(__fsub_rn(scaled_logit<DIV>(x[i], tau), m)));
    const uint64_t s = block_sum_u64_n<NT>(fixed_sum_u64(sd), ured);
    if (threadIdx.x == 0u)
    {
        p.ssum[rb * p.slices + sl] = s;
        const int32_t xt = r != K ? p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + (r <= K ? r : r - K - 1u)] : -1;
        const bool valid = xt >= 0 && static_cast<uint32_t>(xt) < V;
        if (valid ? static_cast<uint32_t>(xt) / SLICE == sl : sl == 0u)
            p.sex[rb] = valid ? expf_ref(__fsub_rn(scaled_logit<DIV>(row[xt], tau), m)) : 0.0f;
    }
}

// one wave per row: the RowStat of every row of the sequences (rows a phase
// skipped come out of stale slices and are never read)
__global__ __launch_bounds__(NT) void k_rej_rowfin(RejectParams p)
{
    const uint32_t b = blockIdx.y, nrow = 2u * p.K + 1u, r = blockIdx.x * (NT / 64u) + (threadIdx.x >> 6);
    if (r >= nrow) return;                              // whole wave
    const RowStat st = rej_stat_from_slices(p, b, r, threadIdx.x & 63u);
    if ((threadIdx.x & 63u) == 0u) p.stats[static_cast<uint64_t>(b) * nrow + r] = st;
}

constexpr uint32_t REJ_MAX_K = 63;              // drafts per sequence (k + 1 <= 64)
constexpr uint32_t REJ_MAX_SLICES = 64;         // vocab <= 64 * SLICE

// Sequence b's row statistics, drafts and slice sums, staged in LDS by one
// round of loads of the whole workgroup.
struct SeqShared {
    RowStat st[2 * REJ_MAX_K + 1];
    int32_t dr[REJ_MAX_K];
    SlicePart parts[REJ_MAX_SLICES];
};

__device__ __forceinline__ void rej_stage(const RejectParams& p, uint32_t b, bool with_parts, SeqShared& sh)
{
    const uint32_t K = p.K, nrow = 2u * K + 1u;
    for (uint32_t i = threadIdx.x; i < nrow; i += NT) sh.st[i] = p.stats[static_cast<uint64_t>(b) * nrow + i];
    for (uint32_t i = threadIdx.x; i < K; i += NT) sh.dr[i] = p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + i];
    if (with_parts)
        for (uint32_t i = threadIdx.x; i < p.slices; i += NT) sh.parts[i] = p.parts[static_cast<uint64_t>(b) * p.slices + i];
}

// n = index of the first rejected draft of sequence b (K if all are
// accepted), from the staged statistics
__device__ uint32_t rej_first_reject(const RejectParams& p, uint32_t b, uint32_t pb, const SeqShared& sh)
{
    for (uint32_t j = 0; j < p.K; ++j)
        if (!rej_accepts(p, b, pb, j, sh.dr[j], sh.st[j], sh.st[p.K + 1u + j])) return j;
    return p.K;
}

template <bool DIV>
__global__ __launch_bounds__(NT) void k_rej_slice(RejectParams p)
{
    __shared__ uint64_t ured[NT / 64];
    __shared__ SeqShared sh;
    const uint32_t sl = blockIdx.x, b = blockIdx.y, K = p.K, V = p.V;
    const float tau = p.tau;
    const uint32_t pb = p.pos_base ? p.pos_base[b] : 0u;
    rej_stage(p, b, false, sh);
    __syncthreads();
    const uint32_t n = rej_first_reject(p, b, pb, sh);
    const RowStat* st = sh.st;
    const float* tn = rej_row(p, b, n);
    const RowStat P = st[n];
    const double invP = __ddiv_rn(4294967296.0, static_cast<double>(P.S));
    float* w = p.wbuf + static_cast<uint64_t>(b) * V;
    const uint32_t v0 = sl * SLICE;
    constexpr uint32_t PER = SLICE / NT;
    // every load of the slice is issued before the first use
    float tl[PER], ql[PER];
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i)
    {
        const uint32_t v = min(v0 + i * NT + threadIdx.x, V - 1u);
        tl[i] = tn[v];
    }
    double rs = 0.0, ps = 0.0;
    if (n < K)
    {
        const float* qn = rej_row(p, b, K + 1u + n);
        const RowStat Q = st[K + 1u + n];
        const double invQ = __ddiv_rn(4294967296.0, static_cast<double>(Q.S));
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i) ql[i] = qn[min(v0 + i * NT + threadIdx.x, V - 1u)];
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i)
        {
            const uint32_t v = v0 + i * NT + threadIdx.x;
            if (v >= V) continue;
            const float ep = expf_ref_nonpos(__fsub_rn(scaled_logit<DIV>(tl[i], tau), P.m));
            const float eq = expf_ref_nonpos(__fsub_rn(scaled_logit<DIV>(ql[i], tau), Q.m));
            const float pf = static_cast<float>(__dmul_rn(static_cast<double>(ep), invP));
            const float qf = static_cast<float>(__dmul_rn(static_cast<double>(eq), invQ));
            const float d = __fsub_rn(pf, qf);
            const float r = d > 0.0f ? d : 0.0f;
            w[v] = r;
            rs += fixed_d(r);
            ps += fixed_d(ep);
        }
    }
    else
    {
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i)
        {
            const uint32_t v = v0 + i * NT + threadIdx.x;
            if (v >= V) continue;
            const float ep = expf_ref_nonpos(__fsub_rn(scaled_logit<DIV>(tl[i], tau), P.m));
            w[v] = ep;
            ps += fixed_d(ep);
        }
    }
    const uint64_t rsum = block_sum_u64_n<NT>(fixed_sum_u64(rs), ured);
    const uint64_t psum = block_sum_u64_n<NT>(fixed_sum_u64(ps), ured);
    if (threadIdx.x == 0) p.parts[static_cast<uint64_t>(b) * p.slices + sl] = SlicePart{rsum, psum};
}

// inclusive prefix of one u64 per thread over the 256 threads
__device__ uint64_t block_inclusive_scan_u64(uint64_t v, uint64_t* wsum)
{
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1)
    {
        const uint32_t lo = __shfl_up(static_cast<uint32_t>(v), o);
        const uint32_t hi = __shfl_up(static_cast<uint32_t>(v >> 32), o);
        if (lane >= static_cast<uint32_t>(o)) v += (static_cast<uint64_t>(hi) << 32) | lo;
    }
    __syncthreads();
    if (lane == 63u) wsum[wave] = v;
    __syncthreads();
    for (uint32_t w = 0; w < wave; ++w) v += wsum[w];
    return v;
}

constexpr uint32_t PER = SLICE / NT;             // elements of a slice per thread

// exclusive prefix of one u64 per thread over the 256 threads
__device__ uint64_t block_exclusive_scan_u64_fast(uint64_t v, uint64_t* wsum)
{
    const uint64_t inc = block_inclusive_scan_u64(v, wsum);
    return inc - v;
}

// The draw of sequence b within one slice.  Thread t holds the weights of the
// contiguous elements v0 + PER*t .. +PER-1 (wl), so one scan of the threads'
// sums locates the thread whose run holds the threshold, and that thread
// walks its run in order.  W(v) = fixed(wl).
__device__ __forceinline__ void rej_draw_slice(const RejectParams& p, uint32_t b, uint32_t n, uint32_t v0, uint32_t v1,
                                               uint64_t total, uint64_t excl, uint64_t mine, uint64_t t,
                                               const float (&wl)[PER], uint64_t* wsum, int32_t* s_tok, float* stage)
{
    const uint32_t K = p.K, V = p.V;
    bool finder = mine > 0 && excl <= t && t < excl + mine;
    int32_t tok = static_cast<int32_t>(V - 1u);
    const uint32_t vt = v0 + PER * threadIdx.x;
    if (finder)
    {
        uint64_t run = 0;
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i) run += vt + i < v1 ? to_fixed(wl[i]) : 0ull;
        if (threadIdx.x == 0) *s_tok = -1;
        uint64_t pre = excl + block_exclusive_scan_u64_fast(run, wsum);
        if (run > 0 && pre <= t && t < pre + run)
        {
#pragma unroll
            for (uint32_t i = 0; i < PER; ++i)
            {
                const uint64_t wv = vt + i < v1 ? to_fixed(wl[i]) : 0ull;
                pre += wv;
                if (pre > t) { *s_tok = static_cast<int32_t>(vt + i); break; }
            }
        }
        __syncthreads();
        if (*s_tok >= 0) tok = *s_tok;
    }
    if (total == 0 && blockIdx.x == 0) finder = true;          // no mass anywhere: the last id, as defined
    if (p.dist)
    {
        // normalised through LDS, so each store instruction writes 1 KB of
        // consecutive elements
        typedef float f4v __attribute__((ext_vector_type(4)));
        const double inv = __ddiv_rn(4294967296.0, static_cast<double>(total));
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i)
            stage[PER * threadIdx.x + i] = static_cast<float>(__dmul_rn(static_cast<double>(wl[i]), inv));
        __syncthreads();
        float* d = p.dist + static_cast<uint64_t>(b) * V;
        if (v1 - v0 == SLICE && (V & 3u) == 0)
        {
#pragma unroll
            for (uint32_t j = 0; j < PER / 4u; ++j)
            {
                const uint32_t e = 4u * (threadIdx.x + NT * j);
                *reinterpret_cast<f4v*>(d + v0 + e) = *reinterpret_cast<const f4v*>(stage + e);
            }
        }
        else
        {
            for (uint32_t e = threadIdx.x; e < v1 - v0; e += NT) d[v0 + e] = stage[e];
        }
    }
    if (finder && threadIdx.x == 0)
    {
        for (uint32_t i = 0; i <= K; ++i)
            p.out_tokens[b * (K + 1u) + i] =
                i < n ? p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + i] : (i == n ? tok : -1);
        p.accepted[b] = static_cast<int32_t>(n);
        if (p.new_seq_len) p.new_seq_len[b] = p.seq_len[b] + static_cast<int32_t>(n) + 1;
    }
}

template <bool DIV>
__global__ __launch_bounds__(NT) void k_rej_draw(RejectParams p)
{
    __shared__ uint64_t wsum[NT / 64];
    __shared__ int32_t s_tok;
    __shared__ SeqShared sh;
    __shared__ __align__(16) float stage[SLICE];
    const uint32_t sl = blockIdx.x, b = blockIdx.y, K = p.K, V = p.V;
    const float tau = p.tau;
    const uint32_t pb = p.pos_base ? p.pos_base[b] : 0u;
    const uint32_t v0 = sl * SLICE, v1 = min(V, v0 + SLICE);
    // the stored draw weights of the slice (used unless the residual is empty),
    // loaded together with the staged statistics
    typedef float f4v __attribute__((ext_vector_type(4)));
    float wl[PER];
    const float* w = p.wbuf + static_cast<uint64_t>(b) * V;
    const uint32_t vt = v0 + PER * threadIdx.x;
    if (vt + PER <= V && (V & 3u) == 0)
    {
        const f4v* w4 = reinterpret_cast<const f4v*>(w + vt);
#pragma unroll
        for (uint32_t i = 0; i < PER / 4u; ++i)
        {
            const f4v q = w4[i];
            wl[4 * i] = q[0]; wl[4 * i + 1] = q[1]; wl[4 * i + 2] = q[2]; wl[4 * i + 3] = q[3];
        }
    }
    else
    {
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i) wl[i] = w[min(vt + i, V - 1u)];
    }
    rej_stage(p, b, true, sh);
    __syncthreads();
    const uint32_t n = rej_first_reject(p, b, pb, sh);
    const RowStat P = sh.st[n];
    const SlicePart* parts = sh.parts;
    uint64_t Rt = 0, Pt = 0, Rx = 0, Px = 0;
    for (uint32_t s = 0; s < p.slices; ++s)
    {
        const SlicePart q = parts[s];
        Rt += q.R;
        Pt += q.P;
        if (s < sl) { Rx += q.R; Px += q.P; }
    }
    const uint32_t U = philox_u32(p.seed, pb + n, b, 2u);
    auto threshold = [&](uint64_t total) {
        const uint64_t hi = __umul64hi(static_cast<uint64_t>(U), total);
        const uint64_t lo = static_cast<uint64_t>(U) * total;
        return (hi << 32) | (lo >> 32);
    };
    if (n < K && Rt == 0)
    {
        // the residual has no mass: draw from p_n, recomputed from its logits
        const float* tn = rej_row(p, b, n);
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i)
        {
            const uint32_t v = v0 + PER * threadIdx.x + i;
            wl[i] = v < v1 ? expf_ref_nonpos(__fsub_rn(scaled_logit<DIV>(tn[v], tau), P.m)) : 0.0f;
        }
        rej_draw_slice(p, b, n, v0, v1, Pt, Px, parts[sl].P, threshold(Pt), wl, wsum, &s_tok, stage);
    }
    else
    {
        // the stored weights: the residual of row n, or p_K after K accepts
        const bool resid = n < K;
        const uint64_t total = resid ? Rt : Pt;
        rej_draw_slice(p, b, n, v0, v1, total, resid ? Rx : Px, resid ? parts[sl].R : parts[sl].P, threshold(total), wl,
                       wsum, &s_tok, stage);
    }
}

// ---- the whole rejection step in one launch ---------------------------------
// Grid (slices, B), NT threads.  Workgroup (sl, b) holds slice sl (elements
// v0 + i NT + t) of the rows sequence b needs, in registers: target row j and
// draft row K + 1 + j for j = 0, 1, ... up to the first rejected draft n, or
// the bonus row K after K accepts; then it forms the slice's draw weights
// (the residual of row n, or p_K) and draws.  The slices of a sequence hand
// each other their slice maxima, slice sums and draw-weight sums through
// per-sequence slots in device memory: each value is published with one
// 64-bit store at the coherence point that carries a tag (the sequence's
// launch count and the round), and a slice waits for a round by polling the
// sequence's slots, one lane a slice, until every tag matches -- the values
// arrive with the wait.  A wait is bounded: past the device's wait limit
// ERR_WAIT is set and the launch's outputs are invalid.  Workgroups are
// dispatched in order, each die in order, so a sequence's slices are resident
// or finished before any slice of a later sequence starts: a wait never
// depends on a workgroup that cannot run.  Every value comes from the
// operations of k_rej_rowstat, k_rej_slice and k_rej_draw, and a maximum or an
// integer sum does not depend on how its terms are shared out, so the bits are
// theirs.
enum { SLOT_MT = 0, SLOT_MQ = 1, SLOT_ST = 2, SLOT_SQ = 3, SLOT_PR = 4, SLOT_PP = 5, SLOT_N = 6 };

// a slot word: a maximum as (tag << 32) | float bits, a sum (a slice's sum of
// at most SLICE fixed-point terms < 2^44) as (tag << 48) | sum
__device__ __forceinline__ uint64_t slot_f32(uint32_t tag, float v) { return (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v); }
__device__ __forceinline__ uint64_t slot_u64(uint32_t tag, uint64_t v) { return (static_cast<uint64_t>(tag) << 48) | v; }
__device__ __forceinline__ void slot_put(uint64_t* a, uint64_t v)
{
    __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0: waits until every slice of the sequence has published slots ka and
// kb with `tag` (in bits `shift` up), and leaves slice `lane`'s two words in
// wa, wb (lanes >= slices: 0)
__device__ void rej_gather(const RejectParams& p, const uint64_t* seq_slots, uint32_t ka, uint32_t kb, uint32_t tag,
                           uint32_t shift, uint64_t& wa, uint64_t& wb)
{
    const uint32_t lane = threadIdx.x;
    const bool mine = lane < p.slices;
    wa = wb = 0;
    for (uint32_t n = 0;; ++n)
    {
        bool ok = true;
        if (mine)
        {
            wa = __hip_atomic_load(const_cast<uint64_t*>(seq_slots) + lane * SLOT_N + ka, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wb = __hip_atomic_load(const_cast<uint64_t*>(seq_slots) + lane * SLOT_N + kb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = (wa >> shift) == tag && (wb >> shift) == tag;
        }
        if (__all(ok)) break;
        if (n >= p.wait_limit)
        {
            if (lane == 0u) p.err[ERR_WAIT] = 1u;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// block max / exact u64 sum of two values a thread, one barrier pair
__device__ __forceinline__ void block_max2(float& a, float& c, float (*red)[2])
{
    a = wave_max64(a);
    c = wave_max64(c);
    __syncthreads();
    if ((threadIdx.x & 63u) == 0u)
    {
        red[threadIdx.x >> 6][0] = a;
        red[threadIdx.x >> 6][1] = c;
    }
    __syncthreads();
    a = red[0][0];
    c = red[0][1];
#pragma unroll
    for (uint32_t w = 1; w < NT / 64u; ++w)
    {
        a = fmaxf(a, red[w][0]);
        c = fmaxf(c, red[w][1]);
    }
}
__device__ __forceinline__ void block_sum2_u64(uint64_t& a, uint64_t& c, uint64_t (*red)[2])
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
    {
        a += shfl_xor_u64(a, o);
        c += shfl_xor_u64(c, o);
    }
    __syncthreads();
    if ((threadIdx.x & 63u) == 0u)
    {
        red[threadIdx.x >> 6][0] = a;
        red[threadIdx.x >> 6][1] = c;
    }
    __syncthreads();
    a = 0;
    c = 0;
#pragma unroll
    for (uint32_t w = 0; w < NT / 64u; ++w)
    {
        a += red[w][0];
        c += red[w][1];
    }
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor_u64(v, o);
    return v;
}

template <bool DIV>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void k_rej_fused(RejectParams p)
{
    __shared__ float fred2[NT / 64][2];
    __shared__ uint64_t ured2[NT / 64][2];
    __shared__ uint64_t wsum[NT / 64];
    __shared__ int32_t s_tok;
    __shared__ uint32_t s_epoch;
    __shared__ float bmax[2];
    __shared__ uint64_t bsum[2], bpart[4];
    // et: the slice's e = exp(x - max) of target row j, then (row n) the draw
    // weights of p; eq: the same for draft row K + 1 + j, then the residual.
    // Each thread keeps to its own elements (i NT + t) until the draw.
    __shared__ __align__(16) float et[SLICE];
    __shared__ __align__(16) float eq[SLICE];
    float* stage = et;
    const uint32_t sl = blockIdx.x, b = blockIdx.y, K = p.K, V = p.V, S = p.slices, t = threadIdx.x;
    const float tau = p.tau;
    const uint32_t pb = p.pos_base ? p.pos_base[b] : 0u;
    const uint32_t v0 = sl * SLICE, v1 = min(V, v0 + SLICE);
    uint64_t* seq_slots = p.slots + static_cast<uint64_t>(b) * REJ_MAX_SLICES * SLOT_N;
    uint64_t* my_slots = seq_slots + sl * SLOT_N;
    if (t == 0u) s_epoch = __hip_atomic_load(p.epoch + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    auto inside = [&](uint32_t i) { return v0 + i * NT + t < V; };
    auto load = [&](const float* row, float (&x)[PER]) {
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i) x[i] = row[min(v0 + i * NT + t, V - 1u)];
    };
    uint32_t round = 0, j = 0;
    float tl[PER], ql[PER];
    RowStat P{}, Q{};
    __syncthreads();
    const uint32_t ep = (s_epoch & 0xFFu) << 8;           // a round's tag: (launch count mod 256, round)
    for (;; ++j)
    {
        // ---- statistics of target row j and draft row K + 1 + j --------------
        const bool hq = j < K;
        const float* tr = rej_row(p, b, j);
        const float* qr = hq ? rej_row(p, b, K + 1u + j) : tr;
        load(tr, tl);
        if (hq) load(qr, ql);
        const int32_t x = hq ? p.drafts[static_cast<uint64_t>(b) * p.drafts_stride + j] : -1;
        const bool xv = x >= 0 && static_cast<uint32_t>(x) < V;
        const float xt = xv ? tr[x] : 0.0f, xq = xv ? qr[x] : 0.0f;
        float mt = -__builtin_huge_valf(), mq = -__builtin_huge_valf();
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i)
            if (inside(i))
            {
                mt = fmaxf(mt, scaled_logit<DIV>(tl[i], tau));
                if (hq) mq = fmaxf(mq, scaled_logit<DIV>(ql[i], tau));
            }
        block_max2(mt, mq, fred2);
        const uint32_t tag_m = ep | ++round;
        if (t == 0u)
        {
            slot_put(my_slots + SLOT_MT, slot_f32(tag_m, mt));
            slot_put(my_slots + SLOT_MQ, slot_f32(tag_m, mq));
        }
        if (t < 64u)
        {
            uint64_t wa, wb;
            rej_gather(p, seq_slots, SLOT_MT, SLOT_MQ, tag_m, 32u, wa, wb);
            const float a = wave_max64(t < S ? __uint_as_float(static_cast<uint32_t>(wa)) : -__builtin_huge_valf());
            const float c = wave_max64(t < S ? __uint_as_float(static_cast<uint32_t>(wb)) : -__builtin_huge_valf());
            if (t == 0u)
            {
                bmax[0] = a;
                bmax[1] = c;
            }
        }
        __syncthreads();
        const float Mt = bmax[0], Mq = bmax[1];
        double st = 0.0, sq = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i)
        {
            const float e = inside(i) ? expf_ref_nonpos(__fsub_rn(scaled_logit<DIV>(tl[i], tau), Mt)) : 0.0f;
            et[i * NT + t] = e;
            st += fixed_d(e);
            if (hq)
            {
                const float f = inside(i) ? expf_ref_nonpos(__fsub_rn(scaled_logit<DIV>(ql[i], tau), Mq)) : 0.0f;
                eq[i * NT + t] = f;
                sq += fixed_d(f);
            }
        }
        uint64_t St = fixed_sum_u64(st), Sq = fixed_sum_u64(sq);
        block_sum2_u64(St, Sq, ured2);
        const uint32_t tag_s = ep | ++round;
        if (t == 0u)
        {
            slot_put(my_slots + SLOT_ST, slot_u64(tag_s, St));
            slot_put(my_slots + SLOT_SQ, slot_u64(tag_s, Sq));
        }
        if (t < 64u)
        {
            uint64_t wa, wb;
            rej_gather(p, seq_slots, SLOT_ST, SLOT_SQ, tag_s, 48u, wa, wb);
            const uint64_t lo48 = (1ull << 48) - 1ull;
            const uint64_t a = wave_sum_u64(t < S ? wa & lo48 : 0ull), c = wave_sum_u64(t < S ? wb & lo48 : 0ull);
            if (t == 0u)
            {
                bsum[0] = a;
                bsum[1] = c;
            }
        }
        __syncthreads();
        P = RowStat{Mt, xv ? expf_ref(__fsub_rn(scaled_logit<DIV>(xt, tau), Mt)) : 0.0f, bsum[0]};
        if (!hq) break;                                   // all K accepted: the bonus row's statistics
        Q = RowStat{Mq, xv ? expf_ref(__fsub_rn(scaled_logit<DIV>(xq, tau), Mq)) : 0.0f, bsum[1]};
        if (!rej_accepts(p, b, pb, j, x, P, Q)) break;
    }
    const uint32_t n = j;

    // ---- the slice's draw weights: the residual of row n (into eq), or p_K ----
    const double invP = __ddiv_rn(4294967296.0, static_cast<double>(P.S));
    double rs = 0.0, ps = 0.0;
    if (n < K)
    {
        const double invQ = __ddiv_rn(4294967296.0, static_cast<double>(Q.S));
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i)
        {
            const float ep = et[i * NT + t];
            const float pf = static_cast<float>(__dmul_rn(static_cast<double>(ep), invP));
            const float qf = static_cast<float>(__dmul_rn(static_cast<double>(eq[i * NT + t]), invQ));
            const float d = __fsub_rn(pf, qf);
            const float wi = inside(i) && d > 0.0f ? d : 0.0f;
            eq[i * NT + t] = wi;
            rs += fixed_d(wi);
            ps += fixed_d(ep);
        }
    }
    else
    {
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i) ps += fixed_d(et[i * NT + t]);
    }
    uint64_t Rs = fixed_sum_u64(rs), Ps = fixed_sum_u64(ps);
    block_sum2_u64(Rs, Ps, ured2);
    const uint32_t tag_p = ep | ++round;
    if (t == 0u)
    {
        slot_put(my_slots + SLOT_PR, slot_u64(tag_p, Rs));
        slot_put(my_slots + SLOT_PP, slot_u64(tag_p, Ps));
    }
    if (t < 64u)
    {
        uint64_t wa, wb;
        rej_gather(p, seq_slots, SLOT_PR, SLOT_PP, tag_p, 48u, wa, wb);
        const uint64_t lo48 = (1ull << 48) - 1ull, ra = t < S ? wa & lo48 : 0ull, pa = t < S ? wb & lo48 : 0ull;
        const uint64_t r_all = wave_sum_u64(ra), p_all = wave_sum_u64(pa);
        const uint64_t r_x = wave_sum_u64(t < sl ? ra : 0ull), p_x = wave_sum_u64(t < sl ? pa : 0ull);
        if (t == 0u)
        {
            bpart[0] = r_all;
            bpart[1] = p_all;
            bpart[2] = r_x;
            bpart[3] = p_x;
        }
    }
    __syncthreads();
    const uint64_t Rt = bpart[0], Pt = bpart[1], Rx = bpart[2], Px = bpart[3];
    // every slice has read this launch's count: slice 0 moves it on for the next
    if (sl == 0u && t == 0u) __hip_atomic_store(p.epoch + b, s_epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- the draw -----------------------------------------------------------------
    const uint32_t U = philox_u32(p.seed, pb + n, b, 2u);
    auto threshold = [&](uint64_t total) {
        const uint64_t hi = __umul64hi(static_cast<uint64_t>(U), total);
        const uint64_t lo = static_cast<uint64_t>(U) * total;
        return (hi << 32) | (lo >> 32);
    };
    const bool from_p = n < K && Rt == 0;                 // the residual has no mass: draw from p_n
    // each thread's contiguous run of the slice, as rej_draw_slice walks it:
    // the residual, or p (p_K after K accepts, p_n when the residual is empty)
    const float* wsrc = n < K && !from_p ? eq : et;
    __syncthreads();
    float wl[PER];
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i) wl[i] = wsrc[PER * t + i];
    __syncthreads();
    if (from_p) rej_draw_slice(p, b, n, v0, v1, Pt, Px, Ps, threshold(Pt), wl, wsum, &s_tok, stage);
    else
    {
        const bool resid = n < K;
        const uint64_t total = resid ? Rt : Pt;
        rej_draw_slice(p, b, n, v0, v1, total, resid ? Rx : Px, resid ? Rs : Ps, threshold(total), wl, wsum, &s_tok,
                       stage);
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

uint32_t rej_slices(uint32_t V) { return (V + SLICE - 1u) / SLICE; }

// slice maxima, slice sums and e(x) of the rows read by slices
static uint64_t rej_slice_stat_bytes(uint32_t batch, uint32_t k, uint32_t vocab)
{
    const uint64_t rows = static_cast<uint64_t>(batch) * (2u * k + 1u), sl = rej_slices(vocab);
    return align_up(rows * sl * 4u, 256) + align_up(rows * sl * 8u, 256) + align_up(rows * 4u, 256);
}

uint64_t accept_ws_bytes(uint32_t batch, uint32_t k, uint32_t vocab, uint32_t mode)
{
    if (mode == OPURE_ACCEPT_REJECTION)
        return align_up(static_cast<uint64_t>(batch) * (2u * k + 1u) * sizeof(RowStat), 256) +
               align_up(static_cast<uint64_t>(batch) * rej_slices(vocab) * sizeof(SlicePart), 256) +
               align_up(static_cast<uint64_t>(batch) * vocab * 4u, 256) + rej_slice_stat_bytes(batch, k, vocab);
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
        OPURE_REQUIRE(rej_slices(a->vocab) <= REJ_MAX_SLICES, OPURE_E_CAPACITY,
                      "accept: rejection sampling supports vocab <= %u", REJ_MAX_SLICES * SLICE);
    }
    return OPURE_OK;
}

RollbackParams rollback_params(const opure_rollback_args* a)
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
    OPURE_LAUNCH(dev, k_accept_greedy, dim3(batch), dim3(GNT), 0, g);
    OPURE_LAUNCH_CHECK("k_accept_greedy");
    return OPURE_OK;
}

int argmax_partials_launch(opure_dev* dev, const float* logits, uint32_t rows, uint32_t V, float* am_val,
                           int32_t* am_idx)
{
    ArgmaxParams ap;
    ap.logits = logits;
    ap.rows = rows;
    ap.V = V;
    ap.chunk = 4096u;
    ap.parts = argmax_parts(V);
    ap.am_val = am_val;
    ap.am_idx = am_idx;
    OPURE_LAUNCH(dev, k_argmax_partial, dim3(ap.parts, rows), dim3(NT), 0, ap);
    OPURE_LAUNCH_CHECK("k_argmax_partial");
    return OPURE_OK;
}

int accept_greedy_launch(opure_dev* dev, const opure_accept_args* a, void* ws)
{
    const uint32_t rows = a->batch * (a->k + 1u), parts = argmax_parts(a->vocab);
    float* am_val = static_cast<float*>(ws);
    int32_t* am_idx = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + align_up(static_cast<uint64_t>(parts) * rows * 4u, 256));
    const int rc = argmax_partials_launch(dev, a->target_logits, rows, a->vocab, am_val, am_idx);
    if (rc) return rc;
    return greedy_from_partials(dev, am_val, am_idx, parts, a->batch, a->k, a->drafts, a->drafts_stride,
                                a->out_tokens, a->accepted, nullptr);
}

int accept_rejection_launch(opure_dev* dev, const opure_accept_args* a, void* ws, const int32_t* seq_len,
                            int32_t* new_seq_len)
{
    const uint32_t B = a->batch, K = a->k, V = a->vocab;
    RejectParams r;
    r.target = a->target_logits;
    r.draft = a->draft_logits;
    r.drafts = a->drafts;
    r.drafts_stride = a->drafts_stride;
    r.K = K;
    r.V = V;
    r.slices = rej_slices(V);
    r.tau = a->temperature;
    r.seed = a->seed;
    r.pos_base = a->pos_base;
    r.out_tokens = a->out_tokens;
    r.accepted = a->accepted;
    r.dist = a->dist_out;
    char* w = static_cast<char*>(ws);
    r.stats = reinterpret_cast<RowStat*>(w);
    w += align_up(static_cast<uint64_t>(B) * (2u * K + 1u) * sizeof(RowStat), 256);
    r.parts = reinterpret_cast<SlicePart*>(w);
    w += align_up(static_cast<uint64_t>(B) * r.slices * sizeof(SlicePart), 256);
    r.wbuf = reinterpret_cast<float*>(w);
    w += align_up(static_cast<uint64_t>(B) * V * 4u, 256);
    const uint64_t nrow = static_cast<uint64_t>(B) * (2u * K + 1u);
    r.smax = reinterpret_cast<float*>(w);
    w += align_up(nrow * r.slices * 4u, 256);
    r.ssum = reinterpret_cast<uint64_t*>(w);
    w += align_up(nrow * r.slices * 8u, 256);
    r.sex = reinterpret_cast<float*>(w);
    r.epoch = static_cast<uint32_t*>(dev->rej_sync);
    r.slots = reinterpret_cast<uint64_t*>(static_cast<char*>(dev->rej_sync) + REJ_SYNC_SEQS * sizeof(uint32_t));
    r.wait_limit = dev->wait_limit;
    r.err = dev->err;
    r.seq_len = seq_len;
    r.new_seq_len = new_seq_len;
    const dim3 slices(r.slices, B);
    if (dev->rej_sync && dev->err && B <= REJ_SYNC_SEQS && dev->rej_mode == OPURE_REJ_ONE_LAUNCH)
    {
        // one launch: every slice of every sequence (see k_rej_fused)
        if (r.tau != 1.0f) OPURE_LAUNCH(dev, k_rej_fused<true>, slices, dim3(NT), 0, r);
        else OPURE_LAUNCH(dev, k_rej_fused<false>, slices, dim3(NT), 0, r);
        OPURE_LAUNCH_CHECK("k_rej_fused");
        return OPURE_OK;
    }
    const bool aligned = ((reinterpret_cast<uintptr_t>(a->target_logits) | reinterpret_cast<uintptr_t>(a->draft_logits)) & 15u) == 0;
    const bool reg = V % 4u == 0 && V <= 4u * RNT * RVEC && aligned, div = r.tau != 1.0f;
    // Position 0's two rows first, then the other rows only for sequences
    // whose first draft was accepted.  Rows held in registers take one
    // workgroup each; longer rows (the 128k vocabulary) are spread over their
    // slices, so the first phase still fills the chip.
    const bool split = K > 0u;
    for (uint32_t phase : {1u, 2u})
    {
        r.phase = split ? phase : 0u;
        const uint32_t nr = !split ? 2u * K + 1u : (phase == 1u ? 2u : 2u * K - 1u);
        if (reg)
        {
            if (div) OPURE_LAUNCH(dev, (k_rej_rowstat<true>), dim3(nr, B), dim3(RNT), 0, r);
            else OPURE_LAUNCH(dev, (k_rej_rowstat<false>), dim3(nr, B), dim3(RNT), 0, r);
            OPURE_LAUNCH_CHECK("k_rej_rowstat");
        }
        else
        {
            const dim3 g(r.slices, nr, B);
            if (div) OPURE_LAUNCH(dev, k_rej_smax<true>, g, dim3(NT), 0, r);
            else OPURE_LAUNCH(dev, k_rej_smax<false>, g, dim3(NT), 0, r);
            OPURE_LAUNCH_CHECK("k_rej_smax");
            if (div) OPURE_LAUNCH(dev, k_rej_ssum<true>, g, dim3(NT), 0, r);
            else OPURE_LAUNCH(dev, k_rej_ssum<false>, g, dim3(NT), 0, r);
            OPURE_LAUNCH_CHECK("k_rej_ssum");
        }
        if (!split) break;
    }
    if (!reg)
    {
        OPURE_LAUNCH(dev, k_rej_rowfin, dim3((2u * K + 1u + NT / 64u - 1u) / (NT / 64u), B), dim3(NT), 0, r);
        OPURE_LAUNCH_CHECK("k_rej_rowfin");
    }
    if (div) OPURE_LAUNCH(dev, k_rej_slice<true>, slices, dim3(NT), 0, r);
    else OPURE_LAUNCH(dev, k_rej_slice<false>, slices, dim3(NT), 0, r);
    OPURE_LAUNCH_CHECK("k_rej_slice");
    if (div) OPURE_LAUNCH(dev, k_rej_draw<true>, slices, dim3(NT), 0, r);
    else OPURE_LAUNCH(dev, k_rej_draw<false>, slices, dim3(NT), 0, r);
    OPURE_LAUNCH_CHECK("k_rej_draw");
    return OPURE_OK;
}

int rollback_launch(opure_dev* dev, const opure_rollback_args* a)
{
    const RollbackParams r = rollback_params(a);
    OPURE_LAUNCH(dev, k_rollback, dim3(a->batch), dim3(NT), 0, r);
    OPURE_LAUNCH_CHECK("k_rollback");
    return OPURE_OK;
}

int rollback_validate(const opure_rollback_args* a)
{
    OPURE_REQUIRE(a && a->model && a->kv && a->kv->pool && a->kv->page_table && a->seq_len && a->accepted &&
                      a->new_seq_len, OPURE_E_INVALID, "rollback: null argument");
    OPURE_REQUIRE(a->batch >= 1 && a->kv->page_size == OPURE_PAGE_SIZE, OPURE_E_INVALID, "rollback: bad shape");
    OPURE_REQUIRE(a->kv->n_pages >= 1 && a->kv->max_pages_per_seq >= 1, OPURE_E_INVALID, "rollback: the cache has no pages");
    // a rollback follows a verify step of k + 1 <= OPURE_MAX_ROWS rows, so its
    // positions lie in two pages at most
    OPURE_REQUIRE(a->k + 1u <= OPURE_MAX_ROWS, OPURE_E_CAPACITY, "rollback: k = %u drafts, more than a verify step holds",
                  a->k);
    // the K positions past seq_len hold at most ceil(K / page) page starts: the
    // most pages one rollback can release into a sequence's freed row
    const uint32_t most = a->k == 0u ? 1u : (a->k + OPURE_PAGE_SIZE - 1u) / OPURE_PAGE_SIZE;
    OPURE_REQUIRE(!a->freed || a->freed_stride >= most, OPURE_E_INVALID,
                  "rollback: freed_stride %u < %u, the most pages a rollback of %u drafts can release",
                  a->freed_stride, most, a->k);
    return OPURE_OK;
}

}  // namespace opure_hip

// Device scratch of opure_accept_rejection_noalloc: one copy per GPU, held for
// the life of the process.  Host code never passes this name to a kernel (on
// the host it is only a stand-in for the symbol); it uses the device address
// that hipGetSymbolAddress returns, looked up once per device.
static __device__ __align__(256) uint8_t scratch[OPURE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr uint64_t NOALLOC_SCRATCH_BYTES = OPURE_NOALLOC_SCRATCH_BYTES;

int noalloc_scratch(opure_dev* dev, void** out)
{
    if (!dev->noalloc_scratch)
    {
        OPURE_HIP_TRY(hipSetDevice(dev->ordinal));
        void* ptr = nullptr;
        OPURE_HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        OPURE_REQUIRE(ptr, OPURE_E_HIP, "opure_accept_rejection_noalloc: no device address for the scratch array");
        dev->noalloc_scratch = ptr;
    }
    *out = dev->noalloc_scratch;
    return OPURE_OK;
}

}  // namespace

using namespace opure_hip;

extern "C" {

int opure_accept_greedy(opure_dev* dev, const opure_accept_args* a)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_accept_greedy: null device");
    int rc = accept_validate(a, false);
    if (rc) return rc;
    rc = ensure_workspace(dev, accept_ws_bytes(a->batch, a->k, a->vocab, OPURE_ACCEPT_GREEDY));
    if (rc) return rc;
    return accept_greedy_launch(dev, a, dev->ws);
}

int opure_accept_rejection(opure_dev* dev, const opure_accept_args* a)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_accept_rejection: null device");
    int rc = accept_validate(a, true);
    if (rc) return rc;
    rc = ensure_workspace(dev, accept_ws_bytes(a->batch, a->k, a->vocab, OPURE_ACCEPT_REJECTION));
    if (rc) return rc;
    return accept_rejection_launch(dev, a, dev->ws, nullptr, nullptr);
}

int opure_accept_rejection_noalloc(opure_dev* dev, const opure_accept_args* a)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_accept_rejection_noalloc: null device");
    int rc = accept_validate(a, true);
    if (rc) return rc;
    const uint64_t need = accept_ws_bytes(a->batch, a->k, a->vocab, OPURE_ACCEPT_REJECTION);
    OPURE_REQUIRE(need <= NOALLOC_SCRATCH_BYTES, OPURE_E_CAPACITY,
                  "opure_accept_rejection_noalloc: batch %u x vocab %u needs %llu bytes of scratch, beyond the "
                  "%llu-byte device array",
                  a->batch, a->vocab, static_cast<unsigned long long>(need),
                  static_cast<unsigned long long>(NOALLOC_SCRATCH_BYTES));
    void* ws = nullptr;
    if ((rc = noalloc_scratch(dev, &ws))) return rc;
    // every scratch word the kernels read was written earlier in the same call
    return accept_rejection_launch(dev, a, ws, nullptr, nullptr);
}

int opure_sample_rows(opure_dev* dev, const opure_sample_args* a)
{
    OPURE_REQUIRE(dev && a && a->logits && a->pos && a->seq && a->out && a->rows >= 1 && a->vocab >= 1, OPURE_E_INVALID,
                  "opure_sample_rows: bad argument");
    OPURE_REQUIRE(a->temperature > 0.0f, OPURE_E_INVALID, "opure_sample_rows: temperature must be > 0");
    SampleParams s{a->logits, a->vocab, a->temperature, a->seed, a->pos, a->seq, a->stream, a->out};
    OPURE_LAUNCH(dev, k_sample, dim3(a->rows), dim3(NT), 0, s);
    OPURE_LAUNCH_CHECK("k_sample");
    return OPURE_OK;
}

int opure_philox_uniform(opure_dev* dev, uint64_t seed, const uint32_t* pos, const uint32_t* seq, uint32_t stream,
                         uint32_t n, uint32_t* out)
{
    OPURE_REQUIRE(dev && pos && seq && out, OPURE_E_INVALID, "opure_philox_uniform: null argument");
    if (!n) return OPURE_OK;
    OPURE_LAUNCH(dev, k_philox, dim3((n + 255u) / 256u), dim3(256), 0, seed, pos, seq, stream, n, out);
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
