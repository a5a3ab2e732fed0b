// ============================================================================
//  gemm_wide.h -- the GEMV for more than 16 activation rows (a batch of
//  sequences times K+1 rows, up to 256): a thin GEMM on the matrix cores.
//
//  The same tiled weights and the same MFMA operand mapping as the K+1-row
//  kernel (gemv_kernel.h): y^T = W X^T in 16 x 16 tiles, A = 16 weight rows
//  x 32 k, B = 32 k x 16 columns of X.
//
//  Work split.  A workgroup owns 8 consecutive 16-row weight tiles (a row
//  group), up to 8 16-column tiles of X (a column group) and one range of K
//  blocks (a split; shapes with few row groups split K so the CUs fill).  A
//  set of 4 waves covers the row group: wave w multiplies tiles 2w, 2w + 1 by
//  all of the group's column tiles, so it keeps 16 accumulator tiles, loads
//  each weight byte once and reads each B fragment once per block for two
//  MFMAs.  Weights go straight from HBM into registers: every wave loads its
//  own two tiles' 16 bytes a lane per block, in static register slots DW
//  blocks ahead.  X goes through LDS: per block the set loads its column
//  group's fragments into registers DX blocks ahead and writes them into a
//  two-stage ring laid out fragment by fragment, 16 bytes a lane.  One barrier
//  per block separates a stage's writes from its reads and the reads of two
//  blocks back from the next writes.  The int8 kernel runs two such sets on
//  alternate K blocks (KH = 2, two waves a SIMD) and adds them at the end.
//
//  The budget per block of a workgroup is L2 -> CU traffic (8 KB of weights
//  and 16 KB of X at 128 columns), which is why a wave owns whole weight
//  tiles (no two waves load the same weights) and X loads cover whole
//  128-byte lines.
//
//  With one split the epilogue runs here; with several, each split writes
//  its raw accumulators and k_wide_reduce adds the splits in split order and
//  runs the epilogue (k_wide_reduce_norm for a residual that feeds an
//  rmsnorm: it also writes the normalised rows).  The split count depends on
//  the weight shape only, and each (row, column) sums its blocks in a fixed
//  order (each wave set's blocks in order, then the sets added), so a row's
//  result does not depend on how many rows share the call, and runs are
//  reproducible.
// ============================================================================
#pragma once

#include "gemv_kernel.h"

namespace opure_gemv {

constexpr uint32_t WIDE_WR = 4, WIDE_WC = 1;     // wave grid of a K half: wave rows x wave columns
constexpr uint32_t WIDE_TA = 2;                  // weight tiles per wave
constexpr uint32_t WIDE_TB = 8;                  // column tiles per wave
constexpr uint32_t WIDE_RT = WIDE_WR * WIDE_TA;  // weight tiles per workgroup
constexpr uint32_t WIDE_CG = WIDE_WC * WIDE_TB;  // column tiles per workgroup at most
constexpr uint32_t WIDE_MAX_M = 256;  // rows of X

// register slots of the software pipeline: DW weight blocks and DX X blocks
// in flight; the K loop is unrolled by U = lcm(DW, DX), an even number, so
// slots and LDS stages are compile-time.  KH = 2 runs two sets of 4 waves on
// alternate K blocks (two waves a SIMD: one issues MFMAs while the other
// waits); the uint4 kernel's registers leave room for one.
template <int WF> struct WideDepth;
template <> struct WideDepth<OPURE_W_I8PC>   { static constexpr uint32_t DW = 4, DX = 2, U = 4, KH = 2; };
template <> struct WideDepth<OPURE_W_I4G128> { static constexpr uint32_t DW = 2, DX = 1, U = 2, KH = 1; };

struct WParams {
    KParams p;        // shape, pointers, epilogue
    uint32_t mt;      // 16-column tiles of X
    uint32_t nrg;     // row groups (WIDE_RT tiles each)
    uint32_t ncg;     // column groups
    uint32_t cgs;     // column tiles per group (<= WIDE_CG)
    uint32_t splits;  // K splits
    uint32_t bps;     // blocks per split, a multiple of WideDepth::U
    uint32_t part_rows;  // splits > 1: 0 = accumulators [split][tile][mt][64] lanes, 1 = [split][M][out] rows
    f4_t* part;       // splits > 1: the splits' accumulators
};

// Workgroup -> (split, row group, column group).  Workgroups are dispatched
// to the 8 XCDs round robin; the remap gives each XCD a contiguous range of
// the work list, so the column groups of one row group (the same weights)
// run on one XCD and share its L2.
__device__ __forceinline__ void wide_coords(const WParams& wp, uint32_t& split, uint32_t& rg, uint32_t& cg)
{
    const uint32_t G = gridDim.x, i = blockIdx.x;
    const uint32_t xcd = i & 7u, j = i >> 3, q = G >> 3, r = G & 7u;
    const uint32_t L = xcd < r ? xcd * (q + 1u) + j : r * (q + 1u) + (xcd - r) * q + j;
    cg = L % wp.ncg;
    const uint32_t rest = L / wp.ncg;
    rg = rest % wp.nrg;
    split = rest / wp.nrg;
}

template <int WF, int AF, int EPI>
__global__ __launch_bounds__(256 * WideDepth<WF>::KH) void k_gemm_wide(WParams wp)
{
    static_assert(WF == OPURE_W_I8PC || WF == OPURE_W_I4G128, "the wide GEMV reads quantised weights");
    constexpr uint32_t KB = Fmt<WF>::KB;
    constexpr uint32_t NMF = KB / 32u;             // MFMAs (16-byte B fragments) per block per tile pair
    constexpr uint32_t CH = KB / 8u;               // 16-byte X chunks per row per block
    constexpr uint32_t XR = WIDE_CG * 16u * CH / 256u;  // X chunks a thread stages per block
    constexpr uint32_t STAGE = WIDE_CG * NMF * 64u;     // u4_t per LDS stage
    constexpr uint32_t DW = WideDepth<WF>::DW, DX = WideDepth<WF>::DX, U = WideDepth<WF>::U;
    constexpr uint32_t KH = WideDepth<WF>::KH;
    constexpr uint32_t TA = WIDE_TA, TB = WIDE_TB;
    static_assert(WIDE_WR * WIDE_WC == 4 && TA % 2 == 0, "a K half is 4 waves");
    static_assert(KH == 1 || 2u * STAGE * 2u >= 2u * 4u * (TA / 2u) * TB * 64u, "the halves' exchange reuses the X stages");
    __shared__ u4_t xl[KH * 2 * STAGE];
    const KParams& p = wp.p;
    const uint32_t tid = threadIdx.x & 255u, lane = tid & 63u, g4 = lane >> 4, r16 = lane & 15u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t kh = wave >> 2, w4 = wave & 3u;            // K half, wave within the half
    const uint32_t wr = w4 / WIDE_WC, wc = w4 % WIDE_WC;
    const uint32_t nblk = p.nblk, G = p.in / 128u;
    uint32_t split, rg, cg;
    wide_coords(wp, split, rg, cg);
    const uint32_t ct0 = cg * wp.cgs;
    const uint32_t cn = min(wp.cgs, wp.mt - ct0);            // column tiles of this group
    const uint32_t tb = cn > wc ? (cn - wc + WIDE_WC - 1u) / WIDE_WC : 0u;  // of this wave: local wc, wc + WC, ...
    const uint32_t tile0 = rg * WIDE_RT + wr * TA;
    const uint32_t b_begin = split * wp.bps, b_end = min(nblk, b_begin + wp.bps);
    u4_t* xh = xl + kh * 2u * STAGE;                          // this half's two stages

    // X chunk u of this thread: row rr of local column tile ctl, 16-byte chunk c of the block (a
    // wave's load covers 8 rows x 128 contiguous bytes).  In LDS, chunk c of row rr sits at row
    // slot rr ^ c of its fragment: the 8 chunks of a row land in 8 bank groups, and a fragment
    // read (lane (g4, r16) takes chunk NMF g4 + q of row r16) still reads 16 distinct slots.
    uint64_t xrow[XR];
    uint32_t xdst[XR];
    bool xzero[XR];
#pragma unroll
    for (uint32_t u = 0; u < XR; ++u)
    {
        const uint32_t e = u * 256u + tid;
        const uint32_t c = e % CH, rr = (e / CH) & 15u, ctl = e / (16u * CH);
        const uint32_t m = 16u * (ct0 + ctl) + rr;
        xzero[u] = ctl >= cn || m >= p.M;
        xrow[u] = (static_cast<uint64_t>(min(m, p.M - 1u)) * p.in + 8u * c) * 2u;
        xdst[u] = (ctl * NMF + c % NMF) * 64u + (c / NMF) * 16u + (rr ^ (c & 15u));
    }
    auto xload = [&](u4_t (&v)[XR], uint32_t b) {
        const uint64_t k0 = static_cast<uint64_t>(min(b, nblk - 1u)) * KB * 2u;
#pragma unroll
        for (uint32_t u = 0; u < XR; ++u) v[u] = *reinterpret_cast<const u4_t*>(p.x + xrow[u] + k0);
    };
    auto xstore = [&](const u4_t (&v)[XR], uint32_t st) {
#pragma unroll
        for (uint32_t u = 0; u < XR; ++u) xh[st * STAGE + xdst[u]] = xzero[u] ? u4_t{0u, 0u, 0u, 0u} : v[u];
    };

    // this wave's weight tiles (clamped for loads; the epilogue skips tiles past the end)
    const uint8_t* wbase[TA];
    const uint32_t* sbase[TA];
#pragma unroll
    for (uint32_t a = 0; a < TA; ++a)
    {
        const uint32_t lt = min(tile0 + a, p.tiles - 1u);
        wbase[a] = p.w + (static_cast<uint64_t>(lt) * nblk << 10) + (lane << 4);
        sbase[a] = static_cast<const uint32_t*>(p.sc) + static_cast<uint64_t>(lt) * G * 16u + 4u * g4;
    }
    auto wload = [&](u4_t (&w)[TA], u4_t (&s)[TA], uint32_t b) {
        const uint32_t bc = min(b, nblk - 1u);
#pragma unroll
        for (uint32_t a = 0; a < TA; ++a)
        {
            w[a] = *reinterpret_cast<const u4_t*>(wbase[a] + (static_cast<uint64_t>(bc) << 10));
            if constexpr (WF == OPURE_W_I4G128) s[a] = *reinterpret_cast<const u4_t*>(sbase[a] + bc * 16u);
        }
    };

    f4_t acc[TA][TB];
#pragma unroll
    for (uint32_t a = 0; a < TA; ++a)
#pragma unroll
        for (uint32_t j = 0; j < TB; ++j) acc[a][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // one block: B fragments from LDS stage st, A decoded from the weight registers
    auto compute = [&](const u4_t (&w)[TA], const u4_t (&s)[TA], uint32_t st) {
        const u4_t* xb = xh + st * STAGE;
        f4_t bacc[TA][TB];
        float xpart[TB];
        if constexpr (WF == OPURE_W_I4G128)
        {
#pragma unroll
            for (uint32_t a = 0; a < TA; ++a)
#pragma unroll
                for (uint32_t j = 0; j < TB; ++j) bacc[a][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t j = 0; j < TB; ++j) xpart[j] = 0.0f;
        }
#pragma unroll
        for (uint32_t q = 0; q < NMF; ++q)
        {
            u4_t bf[TB];
#pragma unroll
            for (uint32_t j = 0; j < TB; ++j)
                bf[j] = xb[(min(wc + WIDE_WC * j, WIDE_CG - 1u) * NMF + q) * 64u + g4 * 16u + (r16 ^ ((NMF * g4 + q) & 15u))];
            if constexpr (WF == OPURE_W_I4G128)
            {
#pragma unroll
                for (uint32_t j = 0; j < TB; ++j) xpart[j] += unit_sum<AF>(bf[j][0], bf[j][1], bf[j][2], bf[j][3]);
            }
#pragma unroll
            for (uint32_t a = 0; a < TA; ++a)
            {
                u4_t af;
                if constexpr (WF == OPURE_W_I8PC)
                {
                    uint32_t o[4];
                    u8x4_to_f16(w[a][2u * q], o[0], o[1]);
                    u8x4_to_f16(w[a][2u * q + 1u], o[2], o[3]);
                    af = u4_t{o[0], o[1], o[2], o[3]};
                }
                else
                {
                    uint32_t o[4];
                    u4x8_pairs<AF>(w[a][q], o);
                    af = u4_t{o[0], o[1], o[2], o[3]};
                }
                // every wave runs all TB column slots (a slot past the group reads a
                // clamped fragment and is never stored): no branches between MFMAs
#pragma unroll
                for (uint32_t j = 0; j < TB; ++j)
                {
                    if constexpr (WF == OPURE_W_I8PC)
                        acc[a][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af),
                                                                           __builtin_bit_cast(half8_t, bf[j]), acc[a][j], 0, 0, 0);
                    else if constexpr (AF == OPURE_A_F16)
                        bacc[a][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af),
                                                                            __builtin_bit_cast(half8_t, bf[j]), bacc[a][j], 0, 0, 0);
                    else
                        bacc[a][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af),
                                                                             __builtin_bit_cast(bf16x8_t, bf[j]), bacc[a][j], 0, 0, 0);
                }
            }
        }
        if constexpr (WF == OPURE_W_I4G128)
        {
            // acc += (s / MUL) * (bacc - (OFF + MUL z) * xs), xs = the block's sum of X for this column (see U4)
#pragma unroll
            for (uint32_t j = 0; j < TB; ++j)
            {
                const float xs = add_xor32(add_xor16(xpart[j]));
#pragma unroll
                for (uint32_t a = 0; a < TA; ++a)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                    {
                        float sc, zo;
                        u4_group<AF>(s[a][i], sc, zo);
                        acc[a][j][i] = __fmaf_rn(sc, __fmaf_rn(-zo, xs, bacc[a][j][i]), acc[a][j][i]);
                    }
            }
        }
    };

    // int8 with one split: the row scales of the tiles this wave finishes, loaded
    // now rather than after the K loop (a round trip off the epilogue)
    constexpr uint32_t FT = KH == 1 ? TA : TA / 2u;      // tiles a wave finishes
    f4_t scl[FT];
    if constexpr (WF == OPURE_W_I8PC)
    {
#pragma unroll
        for (uint32_t h = 0; h < FT; ++h)
        {
            const uint32_t t = min(tile0 + (KH == 1 ? h : kh * FT + h), p.tiles - 1u);
#pragma unroll
            for (int i = 0; i < 4; ++i) scl[h][i] = f16_to_f32(static_cast<const uint16_t*>(p.sc)[t * 16u + 4u * g4 + i]);
        }
    }

    // Half kh takes blocks b_begin + kh, + kh + KH, ...; a step moves both
    // halves one block on, with one barrier for the whole workgroup.
    const uint32_t steps = (b_end - b_begin + KH - 1u) / KH;
    const uint32_t bh = b_begin + kh;
    u4_t xr[DX][XR];
    u4_t wv[DW][TA], sv[DW][TA];
#pragma unroll
    for (uint32_t d = 0; d < DX; ++d) xload(xr[d], bh + KH * d);
#pragma unroll
    for (uint32_t d = 0; d < DW; ++d) wload(wv[d], sv[d], bh + KH * d);
    for (uint32_t i0 = 0; i0 < steps; i0 += U)
    {
#pragma unroll
        for (uint32_t s = 0; s < U; ++s)
        {
            const uint32_t b = bh + KH * (i0 + s);
            xstore(xr[s % DX], s & 1u);
            xload(xr[s % DX], b + KH * DX);
            __syncthreads();
            if (b < b_end) compute(wv[s % DW], sv[s % DW], s & 1u);
            wload(wv[s % DW], sv[s % DW], b + KH * DW);
        }
    }

    // a: the tile within the wave's TA, h: its index among the FT it finishes
    auto finish = [&](uint32_t a, uint32_t h, uint32_t j, const f4_t& tot) {
        const uint32_t tile = tile0 + a;
        if (tile >= p.tiles || j >= tb) return;
        const uint32_t ct = ct0 + wc + WIDE_WC * j;
        if (wp.splits == 1u)
        {
            float bv = 0.0f;
            int32_t bi = 0;
            epilogue<WF, EPI>(p, tile, 16u * ct + r16, g4, tot, bv, bi, WF == OPURE_W_I8PC ? &scl[h] : nullptr);
        }
        else if (wp.part_rows)
        {
            const uint32_t m = 16u * ct + r16;
            if (m < p.M)
                *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(wp.part) +
                                         (static_cast<uint64_t>(split) * p.M + m) * p.out + 16u * tile + 4u * g4) = tot;
        }
        else
        {
            wp.part[((static_cast<uint64_t>(split) * p.tiles + tile) * wp.mt + ct) * 64u + lane] = tot;
        }
    };
    if constexpr (KH == 1)
    {
#pragma unroll
        for (uint32_t a = 0; a < TA; ++a)
#pragma unroll
            for (uint32_t j = 0; j < TB; ++j) finish(a, a, j, acc[a][j]);
    }
    else
    {
        // the halves add through LDS (the X stages are free): half 0 finishes
        // the first TA/2 tiles of its wave, half 1 the others; each sum is
        // (even blocks) + (odd blocks)
        constexpr uint32_t HT = TA / 2u;
        __syncthreads();
        u4_t* ex = xl + ((1u - kh) * 4u + w4) * (HT * TB * 64u);  // the other half's inbox for this wave
#pragma unroll
        for (uint32_t h = 0; h < HT; ++h)
#pragma unroll
            for (uint32_t j = 0; j < TB; ++j)
                ex[(h * TB + j) * 64u + lane] = __builtin_bit_cast(u4_t, kh == 0 ? acc[HT + h][j] : acc[h][j]);
        __syncthreads();
        const u4_t* in = xl + (kh * 4u + w4) * (HT * TB * 64u);
        const uint32_t keep = kh == 0 ? 0u : HT;
#pragma unroll
        for (uint32_t h = 0; h < HT; ++h)
#pragma unroll
            for (uint32_t j = 0; j < TB; ++j)
            {
                const f4_t other = __builtin_bit_cast(f4_t, in[(h * TB + j) * 64u + lane]);
                const f4_t mine = kh == 0 ? acc[h][j] : acc[HT + h][j];
                const f4_t even = kh == 0 ? mine : other, odd = kh == 0 ? other : mine;
                finish(keep + h, h, j, even + odd);
            }
    }
}

// the K splits of one (tile, column tile) added in split order, then the epilogue
template <int WF, int EPI>
__global__ __launch_bounds__(256) void k_wide_reduce(WParams wp)
{
    const KParams& p = wp.p;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t id = blockIdx.x * 4u + wave;
    if (id >= p.tiles * wp.mt) return;
    const uint32_t tile = id / wp.mt, ct = id - tile * wp.mt;
    f4_t tot = wp.part[(static_cast<uint64_t>(tile) * wp.mt + ct) * 64u + lane];
    for (uint32_t s = 1; s < wp.splits; ++s)
        tot += wp.part[((static_cast<uint64_t>(s) * p.tiles + tile) * wp.mt + ct) * 64u + lane];
    float bv = 0.0f;
    int32_t bi = 0;
    epilogue<WF, EPI>(p, tile, 16u * ct + (lane & 15u), lane >> 4, tot, bv, bi);
}

// The residual GEMV's splits added (row-major accumulators) with the next
// consumer's rmsnorm fused in: one workgroup per row m.  Per 4 outputs
// (o = 4u .. 4u + 3: tile u / 4, lane group u % 4) the same operations as the
// residual epilogue after k_wide_reduce -- splits added in split order, the
// int8 scale, y += v, the 4-output fma chain of squares and the tile's sum
// (g0 + g1) + (g2 + g3) -- then inv_rms from the tile sums in inv_rms_wave's
// order and round(y * inv * gain) as k_rmsnorm_rows, so y, ss_out and the
// normalised rows equal the separate passes' bit for bit.
constexpr uint32_t RN_THREADS = 256, RN_SPLITS = 8;   // the plan splits K at most 8 ways
template <int WF, int AF, int UNITS>
__global__ __launch_bounds__(RN_THREADS) void k_wide_reduce_norm(WParams wp, const float* gain, void* xn)
{
    const KParams& p = wp.p;
    const uint32_t m = blockIdx.x, tid = threadIdx.x, lane = tid & 63u;
    const uint32_t units = p.out / 4u;
    __shared__ float ss_t[RN_THREADS * UNITS / 4u];
    __shared__ float inv_s;
    float* y = static_cast<float*>(p.y) + static_cast<uint64_t>(m) * p.out;
    const float* part = reinterpret_cast<const float*>(wp.part);
    // every split's accumulators and the residual in one round trip
    f4_t ps[UNITS][RN_SPLITS], y0[UNITS];
#pragma unroll
    for (uint32_t j = 0; j < UNITS; ++j)
    {
        const uint32_t uc = min(tid + RN_THREADS * j, units - 1u);
#pragma unroll
        for (uint32_t s = 0; s < RN_SPLITS; ++s)
            ps[j][s] = *reinterpret_cast<const f4_t*>(part + (static_cast<uint64_t>(min(s, wp.splits - 1u)) * p.M + m) * p.out +
                                                      4u * uc);
        y0[j] = *reinterpret_cast<const f4_t*>(y + 4u * uc);
    }
    f4_t nv[UNITS];
#pragma unroll
    for (uint32_t j = 0; j < UNITS; ++j)
    {
        const uint32_t u = tid + RN_THREADS * j;
        const bool live = u < units;
        const uint32_t uc = live ? u : 0u;
        f4_t tot = ps[j][0];
#pragma unroll
        for (uint32_t s = 1; s < RN_SPLITS; ++s)
            if (s < wp.splits) tot += ps[j][s];
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            float v = tot[i];
            if constexpr (WF == OPURE_W_I8PC) v = __fmul_rn(v, f16_to_f32(static_cast<const uint16_t*>(p.sc)[4u * uc + i]));
            nv[j][i] = __fadd_rn(y0[j][i], v);
            sq = __fmaf_rn(nv[j][i], nv[j][i], sq);
        }
        if (live) *reinterpret_cast<f4_t*>(y + 4u * uc) = nv[j];
        // the tile's 4 lane groups are 4 consecutive threads
        const float a = __fadd_rn(sq, __shfl_xor(sq, 1));
        const float t = __fadd_rn(a, __shfl_xor(a, 2));
        if (live && (u & 3u) == 0u)
        {
            ss_t[u >> 2] = t;
            if (p.ss_out) p.ss_out[static_cast<uint64_t>(u >> 2) * p.M + m] = t;
        }
    }
    __syncthreads();
    if (tid < 64u)
    {
        float ssum = 0.0f;
        for (uint32_t t = lane; t < p.tiles; t += 64u) ssum += ss_t[t];
        KParams q = p;
        q.in = p.out;                 // the rms is over this GEMV's outputs
        const float inv = inv_rms_finish(q, ssum);
        if (tid == 0) inv_s = inv;
    }
    __syncthreads();
    const float inv = inv_s;
    uint8_t* dst = static_cast<uint8_t*>(xn) + static_cast<uint64_t>(m) * p.out * 2u;
#pragma unroll
    for (uint32_t j = 0; j < UNITS; ++j)
    {
        const uint32_t u = tid + RN_THREADS * j;
        if (u >= units) continue;
        const f4_t g = *reinterpret_cast<const f4_t*>(gain + 4u * u);
        float r[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = __fmul_rn(__fmul_rn(nv[j][i], inv), g[i]);
        *reinterpret_cast<u2_t*>(dst + 8u * u) = u2_t{pack2<AF>(r[0], r[1]), pack2<AF>(r[2], r[3])};
    }
}

// outputs up to 2048 (2 units of 4 a thread) or 4096 (4)
template <int WF, int AF>
int launch_wide_reduce_norm(opure_dev* dev, const WParams& wp, const float* gain, void* xn)
{
    if (wp.p.out <= 8u * RN_THREADS)
        OPURE_LAUNCH(dev, (k_wide_reduce_norm<WF, AF, 2>), dim3(wp.p.M), dim3(RN_THREADS), 0, wp, gain, xn);
    else
        OPURE_LAUNCH(dev, (k_wide_reduce_norm<WF, AF, 4>), dim3(wp.p.M), dim3(RN_THREADS), 0, wp, gain, xn);
    OPURE_LAUNCH_CHECK("k_wide_reduce_norm");
    return OPURE_OK;
}

template <int WF, int AF, int EPI>
int launch_wide_epi_only(opure_dev* dev, const WParams& wp)
{
    OPURE_LAUNCH(dev, (k_gemm_wide<WF, AF, EPI>), dim3(wp.nrg * wp.ncg * wp.splits), dim3(256 * WideDepth<WF>::KH), 0, wp);
    OPURE_LAUNCH_CHECK("k_gemm_wide");
    return OPURE_OK;
}

template <int WF, int AF, int EPI>
int launch_wide_epi(opure_dev* dev, const WParams& wp, uint32_t lds)
{
    (void)lds;
    const int rc0 = launch_wide_epi_only<WF, AF, EPI>(dev, wp);
    if (rc0) return rc0;
    if (wp.splits > 1u)
    {
        const uint32_t n = wp.p.tiles * wp.mt;
        OPURE_LAUNCH(dev, (k_wide_reduce<WF, EPI>), dim3((n + 3u) / 4u), dim3(256), 0, wp);
        OPURE_LAUNCH_CHECK("k_wide_reduce");
    }
    return OPURE_OK;
}

// every epilogue but the per-workgroup argmax partials (wide callers store
// fp32 logits and take the argmax over them); a residual with K splits and a
// fused rmsnorm (gain != null) adds its splits in k_wide_reduce_norm
template <int WF, int AF>
int launch_wide_format(opure_dev* dev, uint32_t epi, const WParams& wp, uint32_t lds, const float* gain = nullptr,
                       void* xn = nullptr)
{
    if (gain && epi == opure_hip::EPI_RESIDUAL && wp.splits > 1u)
    {
        const int rc = launch_wide_epi_only<WF, AF, opure_hip::EPI_RESIDUAL>(dev, wp);
        return rc ? rc : launch_wide_reduce_norm<WF, AF>(dev, wp, gain, xn);
    }
    using namespace opure_hip;
    switch (epi)
    {
    case EPI_STORE: return launch_wide_epi<WF, AF, EPI_STORE>(dev, wp, lds);
    case EPI_RESIDUAL: return launch_wide_epi<WF, AF, EPI_RESIDUAL>(dev, wp, lds);
    case EPI_SWIGLU: return launch_wide_epi<WF, AF, EPI_SWIGLU>(dev, wp, lds);
    case EPI_QKV: return launch_wide_epi<WF, AF, EPI_QKV>(dev, wp, lds);
    }
    return set_error(OPURE_E_INVALID, "gemv: epilogue %u is not built for more than %d rows", epi, OPURE_MAX_ROWS);
}

}  // namespace opure_gemv
