// ============================================================================
//  gemm_wide.h -- the GEMV for more than 16 activation rows (a batch of
//  sequences times K+1 rows, up to 256): a thin GEMM on the matrix cores.
//
//  The same tiled weights and the same MFMA operand mapping as the K+1-row
//  kernel (gemv_kernel.h): y^T = W X^T in 16 x 16 tiles, A = 16 weight rows
//  x 32 k, B = 32 k x 16 columns of X.  What changes is the reuse: a weight
//  block is decoded once into LDS and multiplied against every 16-column
//  tile of X, so the weights are still read from HBM exactly once.
//
//  Work split.  A workgroup of 4 waves owns 4 consecutive 16-row tiles and
//  one range of K blocks (a split; shapes with few tiles split K so every CU
//  gets work).  X is staged into LDS one chunk of K at a time (16-bit
//  activations; a fused rmsnorm runs as a pre-pass).  Per weight block each
//  wave loads and decodes the block of "its" tile into an LDS double buffer,
//  then multiplies all 4 tiles by its column tiles (wave w: w, w+4, w+8,
//  w+12), accumulating in registers.  With one split the epilogue runs here;
//  with several, each split writes its raw accumulators and k_wide_reduce
//  adds the splits in split order and runs the epilogue.  Sums have a fixed
//  order set by the shape, so results are reproducible.
// ============================================================================
#pragma once

#include "gemv_kernel.h"

namespace opure_gemv {

constexpr uint32_t WIDE_TO = 4;       // tiles per workgroup (one per wave for loading)
constexpr uint32_t WIDE_CTW = 4;      // column tiles per wave
constexpr uint32_t WIDE_MAX_M = 256;  // rows of X

struct WParams {
    KParams p;        // shape, pointers, epilogue (x_stride: LDS bytes per staged X row)
    uint32_t mt;      // 16-column tiles of X
    uint32_t ckb;     // weight blocks per staged chunk of X
    uint32_t splits;  // K splits (gridDim.y)
    uint32_t bps;     // blocks per split
    uint32_t off_a;   // LDS: decoded A double buffer [2][TO][AW/4][64] x 16 bytes
    uint32_t off_s;   // LDS: uint4 scale double buffer [2][TO][16] u32
    f4_t* part;       // splits > 1: accumulators [split][tile][mt][64]
};

// Stage rows 0..16*mt-1 of X, k in [k0, k0 + kn), into LDS rows of x_stride
// bytes (rows >= M are zero); uint4 also writes each 128-k group's sum to
// xsum[row * ckb + group].
template <int WF, int AF>
__device__ __forceinline__ void stage_wide_x(const WParams& wp, uint8_t* lds, uint32_t k0, uint32_t kn, float* xsum)
{
    constexpr uint32_t KU = 8;
    const KParams& p = wp.p;
    const uint32_t n8 = kn / 8u, rows = 16u * wp.mt;
    const uint32_t total = rows * n8;
    const uint32_t lane = threadIdx.x & 63u;
    for (uint32_t base = 0; base < total; base += 256u * KU)
    {
        u4_t v[KU];
#pragma unroll
        for (uint32_t u = 0; u < KU; ++u)
        {
            const uint32_t idx = min(base + u * 256u + threadIdx.x, total - 1u);
            const uint32_t m = idx / n8, j = idx - m * n8;
            const uint32_t mc = min(m, p.M - 1u);
            v[u] = *reinterpret_cast<const u4_t*>(p.x + (static_cast<uint64_t>(mc) * p.in + k0 + 8u * j) * 2u);
        }
#pragma unroll
        for (uint32_t u = 0; u < KU; ++u)
        {
            const uint32_t idx = base + u * 256u + threadIdx.x;
            if (idx >= total) continue;
            const uint32_t m = idx / n8, j = idx - m * n8;
            const u4_t val = m < p.M ? v[u] : u4_t{0u, 0u, 0u, 0u};
            *reinterpret_cast<u4_t*>(lds + static_cast<uint64_t>(m) * p.x_stride + 16u * j) = val;
            if constexpr (WF == OPURE_W_I4G128)
            {
                // the 16 units of a group sit in 16 aligned lanes (n8 and 256 are multiples of 16)
                const float s = row16_sum(unit_sum<AF>(val[0], val[1], val[2], val[3]));
                if ((lane & 15u) == 0) xsum[m * wp.ckb + j / 16u] = s;
            }
        }
    }
}

template <int WF, int AF, int EPI>
__global__ __launch_bounds__(256) void k_gemm_wide(WParams wp)
{
    static_assert(WF == OPURE_W_I8PC || WF == OPURE_W_I4G128, "the wide GEMV reads quantised weights");
    constexpr uint32_t KB = Fmt<WF>::KB;
    constexpr uint32_t NMF = KB / 32u;          // MFMAs per block per tile pair
    constexpr uint32_t AQ = NMF;                // 16-byte A fragments per lane per block
    constexpr uint32_t TO = WIDE_TO, CTW = WIDE_CTW;
    extern __shared__ __align__(16) uint8_t lds[];
    const KParams& p = wp.p;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, g4 = lane >> 4, r16 = lane & 15u;
    const uint32_t mt = wp.mt, nblk = p.nblk, G = p.in / 128u;
    const uint32_t tile0 = blockIdx.x * TO;
    const uint32_t ltile = min(tile0 + wave, p.tiles - 1u);
    const uint32_t b_begin = blockIdx.y * wp.bps, b_end = min(nblk, b_begin + wp.bps);
    u4_t* abuf = reinterpret_cast<u4_t*>(lds + wp.off_a);
    uint32_t* sbuf = reinterpret_cast<uint32_t*>(lds + wp.off_s);
    float* xsum = reinterpret_cast<float*>(lds + p.off_xsum);

    f4_t acc[TO][CTW];
#pragma unroll
    for (uint32_t t = 0; t < TO; ++t)
#pragma unroll
        for (uint32_t j = 0; j < CTW; ++j) acc[t][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    auto wload = [&](uint32_t b, u4_t& w, u4_t& s) {
        const uint32_t bc = min(b, nblk - 1u);
        w = __builtin_nontemporal_load(
            reinterpret_cast<const u4_t*>(p.w + ((static_cast<uint64_t>(ltile) * nblk + bc) << 10) + (lane << 4)));
        if constexpr (WF == OPURE_W_I4G128)
            s = *reinterpret_cast<const u4_t*>(static_cast<const uint32_t*>(p.sc) +
                                               (static_cast<uint64_t>(ltile) * G + bc) * 16u + 4u * g4);
    };
    u4_t w0, s0{}, w1, s1{};
    wload(b_begin, w0, s0);
    wload(b_begin + 1u, w1, s1);
    uint32_t par = 0;
    for (uint32_t c0 = b_begin; c0 < b_end; c0 += wp.ckb)
    {
        const uint32_t cb = min(wp.ckb, b_end - c0);
        __syncthreads();                                   // the previous chunk is no longer read
        stage_wide_x<WF, AF>(wp, lds, c0 * KB, cb * KB, xsum);
        __syncthreads();
        for (uint32_t bb = 0; bb < cb; ++bb)
        {
            // this wave's tile: decode the block into A[par]
            uint32_t a[4 * AQ];
            if constexpr (WF == OPURE_W_I8PC)
            {
#pragma unroll
                for (int j = 0; j < 4; ++j) u8x4_to_f16(w0[j], a[2 * j], a[2 * j + 1]);
            }
            else
            {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                {
                    uint32_t o[4];
                    u4x8_pairs<AF>(w0[j], o);
#pragma unroll
                    for (int e = 0; e < 4; ++e) a[4 * j + e] = o[e];
                }
            }
#pragma unroll
            for (uint32_t q = 0; q < AQ; ++q)
                abuf[((par * TO + wave) * AQ + q) * 64u + lane] = u4_t{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
            if constexpr (WF == OPURE_W_I4G128)
                if (r16 == 0) *reinterpret_cast<u4_t*>(sbuf + (par * TO + wave) * 16u + 4u * g4) = s0;
            w0 = w1;
            s0 = s1;
            wload(c0 + bb + 2u, w1, s1);
            __syncthreads();
            // all TO tiles times this wave's column tiles
#pragma unroll
            for (uint32_t t = 0; t < TO; ++t)
            {
                u4_t af[AQ];
#pragma unroll
                for (uint32_t q = 0; q < AQ; ++q) af[q] = abuf[((par * TO + t) * AQ + q) * 64u + lane];
                u4_t sz{};
                if constexpr (WF == OPURE_W_I4G128) sz = *reinterpret_cast<const u4_t*>(sbuf + (par * TO + t) * 16u + 4u * g4);
#pragma unroll
                for (uint32_t j = 0; j < CTW; ++j)
                {
                    const uint32_t ct = wave + 4u * j;
                    if (ct >= mt) continue;
                    const uint32_t m = 16u * ct + r16;
                    const uint8_t* xr = lds + static_cast<uint64_t>(m) * p.x_stride + (bb * KB + (KB / 4u) * g4) * 2u;
                    if constexpr (WF == OPURE_W_I8PC)
                    {
                        const half8_t b1 = __builtin_bit_cast(half8_t, *reinterpret_cast<const u4_t*>(xr));
                        const half8_t b2 = __builtin_bit_cast(half8_t, *reinterpret_cast<const u4_t*>(xr + 16));
                        acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af[0]), b1,
                                                                           acc[t][j], 0, 0, 0);
                        acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af[1]), b2,
                                                                           acc[t][j], 0, 0, 0);
                    }
                    else
                    {
                        f4_t bacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (uint32_t q = 0; q < 4; ++q)
                        {
                            const u4_t bx = *reinterpret_cast<const u4_t*>(xr + 16u * q);
                            if constexpr (AF == OPURE_A_F16)
                                bacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, af[q]),
                                                                              __builtin_bit_cast(half8_t, bx), bacc, 0, 0, 0);
                            else
                                bacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af[q]),
                                                                               __builtin_bit_cast(bf16x8_t, bx), bacc, 0, 0, 0);
                        }
                        // acc += (s / MUL) * (bacc - (OFF + MUL z) * xs)   (see U4)
                        const float xs = xsum[m * wp.ckb + bb];
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                        {
                            float sc, zo;
                            u4_group<AF>(sz[i], sc, zo);
                            acc[t][j][i] = __fmaf_rn(sc, __fmaf_rn(-zo, xs, bacc[i]), acc[t][j][i]);
                        }
                    }
                }
            }
            par ^= 1u;
        }
    }
#pragma unroll
    for (uint32_t t = 0; t < TO; ++t)
    {
        const uint32_t tile = tile0 + t;
        if (tile >= p.tiles) continue;
#pragma unroll
        for (uint32_t j = 0; j < CTW; ++j)
        {
            const uint32_t ct = wave + 4u * j;
            if (ct >= mt) continue;
            if (wp.splits == 1u)
            {
                float bv = 0.0f;
                int32_t bi = 0;
                epilogue<WF, EPI>(p, tile, 16u * ct + r16, g4, acc[t][j], bv, bi);
            }
            else
            {
                wp.part[((static_cast<uint64_t>(blockIdx.y) * p.tiles + tile) * mt + ct) * 64u + lane] = acc[t][j];
            }
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

template <int WF, int AF, int EPI>
int launch_wide_epi(opure_dev* dev, const WParams& wp, uint32_t lds)
{
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_wide<WF, AF, EPI>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 159 * 1024));
        configured = true;
    }
    const uint32_t groups = (wp.p.tiles + WIDE_TO - 1u) / WIDE_TO;
    OPURE_LAUNCH(dev, (k_gemm_wide<WF, AF, EPI>), dim3(groups, wp.splits), dim3(256), lds, wp);
    OPURE_LAUNCH_CHECK("k_gemm_wide");
    if (wp.splits > 1u)
    {
        const uint32_t n = wp.p.tiles * wp.mt;
        OPURE_LAUNCH(dev, (k_wide_reduce<WF, EPI>), dim3((n + 3u) / 4u), dim3(256), 0, wp);
        OPURE_LAUNCH_CHECK("k_wide_reduce");
    }
    return OPURE_OK;
}

// every epilogue but the per-workgroup argmax partials (wide callers store
// fp32 logits and take the argmax over them)
template <int WF, int AF>
int launch_wide_format(opure_dev* dev, uint32_t epi, const WParams& wp, uint32_t lds)
{
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
