// ============================================================================
//  gemv.hip -- batched GEMV for the verify step on gfx950 matrix cores.
//
//  Replaces GEMVMain / GEMVQuantMain (shaders/Opure_GEMV.usf:40-89,
//  shaders/Opure_GEMV_Quant.usf:39-95), which read the whole weight matrix
//  once per activation row.  Here every weight byte is read once for all
//  M <= 16 rows (the K+1 draft positions of one or more sequences).
//
//  Mapping.  y^T[o][m] = sum_k W[o][k] X[m][k] is one 16 x 16 MFMA output
//  tile per 16 weight rows: A = 16 weight rows x 32 k, B = 32 k x 16 rows of X
//  (M padded to 16 with zeros).  One workgroup owns T tiles; its NW waves
//  take interleaved 64-byte blocks of every row (so together they stream
//  contiguous 64*NW-byte runs), each wave reusing one X fragment for all T
//  tiles, and the waves are combined through LDS in wave order.  Lane l loads
//  16 contiguous weight bytes of row (l % 16) per block with a 128-bit load,
//  and its X fragment straight from L2.  A consumer of the fp32 residual
//  (qkv, gate/up, LM head) applies the RMSNorm while loading X, from the
//  per-tile sums of squares the residual's producer wrote, so no separate
//  normalisation pass runs.  Weights are widened in registers:
//    f32   -> v_mfma_f32_16x16x4_f32, 4 MFMAs per 16-byte load
//    int8  -> fp16 via the 1024+u exponent trick (exact), 2 x 16x16x32 f16
//    uint4 -> fp16/bf16 via the same trick, 4 x 16x16x32 per 128-k group,
//             the group's scale/zero applied to the fresh group accumulator
//  No workgroup talks to another (a device-scope fence on a multi-XCD part
//  writes back and invalidates L2, which cost 10-20x in a split-K version), so
//  results are bitwise reproducible and independent of M.
// ============================================================================
#include "internal.h"

#include <algorithm>

using namespace opure_dev_math;

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

struct KParams {
    const uint8_t* w;
    const void* scale;
    const void* zero;
    uint32_t out, in;
    const uint8_t* x;
    uint32_t M;
    void* y;
    uint32_t yfmt;
    uint32_t tiles;
    const float* gain;        // NORM: rmsnorm gain [in]; x is then the fp32 residual
    float eps;
    const float* ss_in;       // NORM: producer's per-tile sums of squares [ss_tiles][M]
    uint32_t ss_tiles;
    float* ss_out;            // RESIDUAL: this kernel's per-tile sums of squares [tiles][M]
    // dynamic LDS layout: X stage rows of x_stride bytes at 0 (STAGED), group
    // sums [M][x_groups] at off_xsum, uint4 scale/zero at off_sz; the wave
    // reduction reuses offset 0 after the K loop
    uint32_t x_stride, x_groups, seg_passes, off_xsum, off_sz;
    opure_hip::QkvEpilogue qkv;
    opure_hip::LogitsEpilogue lg;
};

template <int WF> struct WTraits;
// k elements per 64-byte block of one weight row
template <> struct WTraits<OPURE_W_F32>    { static constexpr uint32_t KB = 16; };
template <> struct WTraits<OPURE_W_I8PC>   { static constexpr uint32_t KB = 64; };
template <> struct WTraits<OPURE_W_I4G128> { static constexpr uint32_t KB = 128; };

__device__ __forceinline__ uint32_t weight_row(uint32_t epi, uint32_t tile, uint32_t r, uint32_t out)
{
    if (epi == opure_hip::EPI_SWIGLU) return (r & 1u) ? (out >> 1) + 8u * tile + (r >> 1) : 8u * tile + (r >> 1);
    return 16u * tile + r;
}

__device__ __forceinline__ half8_t as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    u4_t v = {a, b, c, d};
    return __builtin_bit_cast(half8_t, v);
}

__device__ __forceinline__ bf16x8_t as_bf8(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    u4_t v = {a, b, c, d};
    return __builtin_bit_cast(bf16x8_t, v);
}

// int8 x4 -> two f16 pairs holding the exact integers (1024 + (q + 128)) - 1152
__device__ __forceinline__ void i8x4_to_f16(uint32_t d, uint32_t& lo, uint32_t& hi)
{
    const uint32_t u = d ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const half2_t bias = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, a) + bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, b) + bias);
}

// ---- uint4 slot order --------------------------------------------------------
// In a weight dword the nibble at bits 4j holds element e_j, e = {1,0,3,2,5,4,
// 7,6} (element 2i is the high nibble of byte i).  Pairs (nibble j, nibble
// j+4) are cut with one shift and one and-or each, so the 8 MFMA k-slots of a
// dword hold elements [1 5 | 0 4 | 3 7 | 2 6]; the X operand is permuted the
// same way.  fp16 MAGIC 0x6400 = 1024 (subtracted exactly afterwards); bf16
// 0x4300 = 128 (folded into the zero point).
template <int AF>
__device__ __forceinline__ void u4_slot_pairs(uint32_t d, uint32_t (&o)[4])
{
    constexpr uint32_t MAGIC = AF == OPURE_A_F16 ? 0x64646464u : 0x43434343u;
    const uint32_t lo = d & 0x0F0F0F0Fu;            // bytes: e1 e3 e5 e7
    const uint32_t hi = (d >> 4) & 0x0F0F0F0Fu;     // bytes: e0 e2 e4 e6
    o[0] = __builtin_amdgcn_perm(MAGIC, lo, 0x04020400u);   // (e1, e5)
    o[1] = __builtin_amdgcn_perm(MAGIC, hi, 0x04020400u);   // (e0, e4)
    o[2] = __builtin_amdgcn_perm(MAGIC, lo, 0x04030401u);   // (e3, e7)
    o[3] = __builtin_amdgcn_perm(MAGIC, hi, 0x04030401u);   // (e2, e6)
    if constexpr (AF == OPURE_A_F16)
    {
        const half2_t bias = {static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, o[j]) + bias);
    }
}

// natural pairs D0=(e0,e1) .. D3=(e6,e7) of 8 activations -> slot pairs
// (e1,e5) (e0,e4) (e3,e7) (e2,e6)
__device__ __forceinline__ void x_slot_order(const uint32_t (&d)[4], uint32_t (&o)[4])
{
    o[0] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);
    o[1] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);
    o[2] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);
    o[3] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);
}

// sum of 8 rounded activations (the unit of the group sums): four packed
// dot products with (1, 1), accumulated in element order
template <int AF>
__device__ __forceinline__ float unit_sum(const uint32_t (&d)[4])
{
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
    {
        if constexpr (AF == OPURE_A_F16)
            s = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, d[j]), __builtin_bit_cast(half2_t, 0x3C003C00u), s, false);
        else
            s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, d[j]), __builtin_bit_cast(bf16x2_t, 0x3F803F80u), s,
                                                false);
    }
    return s;
}

template <int AF>
__device__ __forceinline__ uint32_t pack2(float a, float b)
{
    if constexpr (AF == OPURE_A_F16)
        return f32_to_f16(a) | (static_cast<uint32_t>(f32_to_f16(b)) << 16);
    else
        return f32_to_bf16(a) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// 8 consecutive activations of row m from k, as fp32 bits (AF f32) or 4
// natural 16-bit pairs; with NORM rmsnorm'd from the fp32 residual:
// round(x * inv * g) (Opure_RMSNorm.usf:44-78).
template <int AF, bool NORM>
__device__ __forceinline__ void load8(const KParams& p, uint32_t m, uint32_t k, float inv, uint32_t (&o)[8])
{
    if constexpr (!NORM)
    {
        if constexpr (AF == OPURE_A_F32)
        {
            const u4_t* src = reinterpret_cast<const u4_t*>(p.x + (static_cast<uint64_t>(m) * p.in + k) * 4u);
            const u4_t a = src[0], b = src[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) { o[e] = a[e]; o[4 + e] = b[e]; }
        }
        else
        {
            const u4_t a = *reinterpret_cast<const u4_t*>(p.x + (static_cast<uint64_t>(m) * p.in + k) * 2u);
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = a[e];
        }
    }
    else
    {
        const f4_t* xr = reinterpret_cast<const f4_t*>(reinterpret_cast<const float*>(p.x) + static_cast<uint64_t>(m) * p.in + k);
        const f4_t* gr = reinterpret_cast<const f4_t*>(p.gain + k);
        const f4_t x0 = xr[0], x1 = xr[1], g0 = gr[0], g1 = gr[1];
        float y[8];
#pragma unroll
        for (int e = 0; e < 4; ++e)
        {
            y[e] = __fmul_rn(__fmul_rn(x0[e], inv), g0[e]);
            y[4 + e] = __fmul_rn(__fmul_rn(x1[e], inv), g1[e]);
        }
        if constexpr (AF == OPURE_A_F32)
        {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = __float_as_uint(y[e]);
        }
        else
        {
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = pack2<AF>(y[2 * j], y[2 * j + 1]);
        }
    }
}

// X fragment of one weight block for lane (m, g4) read straight from global
// memory: f32 4 values (k = kb+4g4..), int8 16 (k = kb+16g4..), uint4 32
// (k = kb+32g4.., in slot order, plus the partial group sum of its 4 units).
template <int WF> struct Frag { static constexpr uint32_t N = WF == OPURE_W_F32 ? 4u : (WF == OPURE_W_I8PC ? 8u : 16u); };

template <int WF, int AF, bool NORM>
__device__ __forceinline__ void frag_global(const KParams& p, uint32_t m, float inv, uint32_t kb, uint32_t g4,
                                            uint32_t (&xd)[Frag<WF>::N], float& xs)
{
    if constexpr (WF == OPURE_W_F32)
    {
        if constexpr (!NORM)
        {
            const u4_t a = *reinterpret_cast<const u4_t*>(p.x + (static_cast<uint64_t>(m) * p.in + kb + 4u * g4) * 4u);
#pragma unroll
            for (int e = 0; e < 4; ++e) xd[e] = a[e];
        }
        else
        {
            const float* xr = reinterpret_cast<const float*>(p.x) + static_cast<uint64_t>(m) * p.in + kb + 4u * g4;
            const f4_t xv = *reinterpret_cast<const f4_t*>(xr);
            const f4_t gv = *reinterpret_cast<const f4_t*>(p.gain + kb + 4u * g4);
#pragma unroll
            for (int e = 0; e < 4; ++e) xd[e] = __float_as_uint(__fmul_rn(__fmul_rn(xv[e], inv), gv[e]));
        }
    }
    else if constexpr (WF == OPURE_W_I8PC)
    {
#pragma unroll
        for (int h = 0; h < 2; ++h)
        {
            uint32_t o[8];
            load8<AF, NORM>(p, m, kb + 16u * g4 + 8u * h, inv, o);
#pragma unroll
            for (int j = 0; j < 4; ++j) xd[4 * h + j] = o[j];
        }
    }
    else
    {
        float u[4];
#pragma unroll
        for (int h = 0; h < 4; ++h)
        {
            uint32_t o[8];
            load8<AF, NORM>(p, m, kb + 32u * g4 + 8u * h, inv, o);
            const uint32_t d[4] = {o[0], o[1], o[2], o[3]};
            u[h] = unit_sum<AF>(d);
            uint32_t sl[4];
            x_slot_order(d, sl);
#pragma unroll
            for (int j = 0; j < 4; ++j) xd[4 * h + j] = sl[j];
        }
        xs = (u[0] + u[1]) + (u[2] + u[3]);
    }
}

// Stage X[:, k0 .. k0+len) of rows 0..M-1 into LDS rows of `stride` bytes
// (uint4: slot order, and each 128-k group's sum into xsum[m][g]).  Every
// thread of the workgroup takes 8-value units; the 16 units of a group sit in
// 16 aligned lanes of one wave, so the group sum is a fixed butterfly.
template <int WF, int AF, bool NORM, int NTH>
__device__ __forceinline__ void stage_x(const KParams& p, uint32_t k0, uint32_t len, uint8_t* lds, float* xsum,
                                        float inv_lane)
{
    constexpr uint32_t EB = AF == OPURE_A_F32 ? 4u : 2u;
    const uint32_t n8 = len / 8u;
    const uint32_t lane = threadIdx.x & 63u;
    for (uint32_t m = 0; m < p.M; ++m)
    {
        float inv = 1.0f;
        if constexpr (NORM) inv = __shfl(inv_lane, static_cast<int>(m), 64);     // whole wave active here
        uint8_t* row = lds + static_cast<uint64_t>(m) * p.x_stride;
        for (uint32_t j = threadIdx.x; j < n8; j += NTH)
        {
            uint32_t o[8];
            load8<AF, NORM>(p, m, k0 + 8u * j, inv, o);
            uint8_t* dst = row + 8u * j * EB;
            if constexpr (AF == OPURE_A_F32)
            {
                reinterpret_cast<u4_t*>(dst)[0] = u4_t{o[0], o[1], o[2], o[3]};
                reinterpret_cast<u4_t*>(dst)[1] = u4_t{o[4], o[5], o[6], o[7]};
            }
            else if constexpr (WF == OPURE_W_I4G128)
            {
                // n8 and NTH are multiples of 16: a group's 16 lanes are all active
                const uint32_t d[4] = {o[0], o[1], o[2], o[3]};
                float u = unit_sum<AF>(d);
                uint32_t sl[4];
                x_slot_order(d, sl);
                *reinterpret_cast<u4_t*>(dst) = u4_t{sl[0], sl[1], sl[2], sl[3]};
                u += __shfl_xor(u, 1);
                u += __shfl_xor(u, 2);
                u += __shfl_xor(u, 4);
                u += __shfl_xor(u, 8);
                if ((lane & 15u) == 0) xsum[m * p.x_groups + j / 16u] = u;
            }
            else
            {
                *reinterpret_cast<u4_t*>(dst) = u4_t{o[0], o[1], o[2], o[3]};
            }
        }
    }
}

// One workgroup owns T 16-row tiles; its NW waves take interleaved 64-byte
// blocks of K, every wave streaming all T tiles of its blocks so one X
// fragment feeds T MFMA tiles.  STAGED kernels stage X (normalised, slot
// ordered) in LDS segment by segment; the others read fragments from global
// memory.  Both give bit-identical results.  The waves' partial tiles are
// combined through LDS in wave order.
template <int WF, int AF, int EPI, int NW, int T, bool NORM, bool STAGED>
__global__ __launch_bounds__(NW * 64) void k_gemv(KParams p)
{
    using W = WTraits<WF>;
    constexpr uint32_t N = Frag<WF>::N;
    constexpr uint32_t EB = AF == OPURE_A_F32 ? 4u : 2u;
    constexpr uint32_t VALS = WF == OPURE_W_F32 ? 4u : (WF == OPURE_W_I8PC ? 16u : 32u);   // per lane per block
    // 64-byte blocks per pass, within the 128 VGPRs a 1024-thread workgroup allows
    constexpr uint32_t U = WF == OPURE_W_I4G128 ? ((T >= 4 || (NORM && NW == 16)) ? 2u : 4u)
                                                : ((T >= 4 || (NORM && NW == 16)) ? 4u : 8u);
    constexpr uint32_t PB = U * NW;                  // blocks per pass
    extern __shared__ __align__(16) uint8_t lds[];
    f4_t* red = reinterpret_cast<f4_t*>(lds);                              // [NW][T][64] after the K loop
    float* szs = reinterpret_cast<float*>(lds + p.off_sz);                 // uint4: scale [T][G][16 rows]
    float* szc = szs + T * (p.in / 128u) * 16u;                            // uint4: scale * zero' [T][G][16 rows]
    float* xsum = reinterpret_cast<float*>(lds + p.off_xsum);              // STAGED uint4: [M][groups per segment]

    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t g4 = lane >> 4, r16 = lane & 15u;
    const uint32_t tile0 = blockIdx.x * T;
    const uint32_t M = p.M;
    const uint32_t G = p.in / 128u;

    constexpr uint32_t WBITS = WF == OPURE_W_F32 ? 32u : (WF == OPURE_W_I8PC ? 8u : 4u);
    const uint64_t w_row_bytes = static_cast<uint64_t>(p.in) * WBITS / 8u;
    const uint8_t* wp[T];
#pragma unroll
    for (int t = 0; t < T; ++t)
    {
        const uint32_t tt = tile0 + t < p.tiles ? tile0 + t : tile0;
        wp[t] = p.w + weight_row(EPI, tt, r16, p.out) * w_row_bytes + 16u * g4;
    }
    const uint32_t nblk = p.in / W::KB;
    const uint32_t npass = (nblk + PB - 1u) / PB;
    // two register buffers: the next pass's weights stream in while this pass computes
    // (unconditional loads, clamped to the last block, so the compiler can wait
    // for one buffer while the other is still in flight)
    u4_t wa[T][U], wb[T][U];
    auto load_w = [&](u4_t (&wv)[T][U], uint32_t b0) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (uint32_t u = 0; u < U; ++u)
            {
                const uint32_t bb = min(b0 + u * NW, nblk - 1u);
                wv[t][u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(wp[t] + bb * 64u));
            }
    };
    load_w(wa, wave);     // the first pass's weights are in flight during the prologue
    if (npass > 1u) load_w(wb, PB + wave);

    if constexpr (WF == OPURE_W_I4G128)
    {
        // per tile, group and row: the scale and scale * zero' (zero' = zero, +128 for bf16)
#pragma unroll
        for (int t = 0; t < T; ++t)
        {
            for (uint32_t e = threadIdx.x; e < 16u * G; e += NW * 64u)
            {
                const uint32_t r = e & 15u, g = e >> 4;
                float sc = 0.0f, c = 0.0f;
                if (tile0 + t < p.tiles)
                {
                    const uint64_t gi = static_cast<uint64_t>(weight_row(EPI, tile0 + t, r, p.out)) * G + g;
                    sc = bf16_to_f32(static_cast<const uint16_t*>(p.scale)[gi]);
                    float z = bf16_to_f32(static_cast<const uint16_t*>(p.zero)[gi]);
                    if constexpr (AF == OPURE_A_BF16) z += 128.0f;
                    c = __fmul_rn(sc, z);
                }
                szs[(t * G + g) * 16u + r] = sc;
                szc[(t * G + g) * 16u + r] = c;
            }
        }
        if constexpr (!STAGED) __syncthreads();
    }

    // rms of column m from the producer's per-tile sums of squares (fixed order);
    // lane l ends up with inv of column l % 16
    const uint32_t m = r16;
    const uint32_t mc = m < M ? m : M - 1u;      // columns >= M compute on a copy of column M-1, never stored
    float inv = 1.0f;
    if constexpr (NORM)
    {
        float ssum = 0.0f;
#pragma unroll 8
        for (uint32_t t = g4; t < p.ss_tiles; t += 4u) ssum += p.ss_in[static_cast<uint64_t>(t) * M + mc];
        ssum += __shfl_xor(ssum, 16);
        ssum += __shfl_xor(ssum, 32);
        inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ssum, static_cast<float>(p.in)), p.eps)));
    }

    f4_t acc[T], zac[T];      // uint4: sum s * (q+off) x and sum s * zero' * x, subtracted at the end
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = zac[t] = {0.0f, 0.0f, 0.0f, 0.0f};

    uint32_t seg_blk0 = 0;
    auto run_pass = [&](const u4_t (&wv)[T][U], uint32_t ps) {
        const uint32_t b0 = ps * PB + wave;
        if constexpr (STAGED)
        {
            if (ps % p.seg_passes == 0)
            {
                if (ps) __syncthreads();            // the previous segment's fragments are consumed
                seg_blk0 = ps * PB;
                const uint32_t k0 = seg_blk0 * W::KB;
                const uint32_t len = min(p.seg_passes * PB * W::KB, p.in - k0);
                stage_x<WF, AF, NORM, NW * 64>(p, k0, len, lds, xsum, inv);
                __syncthreads();
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u)
        {
            const uint32_t blk = b0 + u * NW;
            if (blk >= nblk) break;
            uint32_t xd[N];
            float xs = 0.0f;
            if constexpr (STAGED)
            {
                const uint8_t* src = lds + static_cast<uint64_t>(mc) * p.x_stride + ((blk - seg_blk0) * W::KB + VALS * g4) * EB;
#pragma unroll
                for (uint32_t i = 0; i < N / 4u; ++i)
                {
                    const u4_t v = reinterpret_cast<const u4_t*>(src)[i];
                    xd[4 * i] = v[0]; xd[4 * i + 1] = v[1]; xd[4 * i + 2] = v[2]; xd[4 * i + 3] = v[3];
                }
                if constexpr (WF == OPURE_W_I4G128) xs = xsum[mc * p.x_groups + (blk - seg_blk0)];
            }
            else
            {
                frag_global<WF, AF, NORM>(p, mc, inv, blk * W::KB, g4, xd, xs);
                if constexpr (WF == OPURE_W_I4G128)
                {
                    xs += __shfl_xor(xs, 16);
                    xs += __shfl_xor(xs, 32);
                }
            }
            if constexpr (WF == OPURE_W_F32)
            {
#pragma unroll
                for (int t = 0; t < T; ++t)
                {
                    if (tile0 + t >= p.tiles) break;
                    const f4_t wf = __builtin_bit_cast(f4_t, wv[t][u]);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wf[q], __uint_as_float(xd[q]), acc[t], 0, 0, 0);
                }
            }
            else if constexpr (WF == OPURE_W_I8PC)
            {
                const half8_t b1 = as_half8(xd[0], xd[1], xd[2], xd[3]);
                const half8_t b2 = as_half8(xd[4], xd[5], xd[6], xd[7]);
#pragma unroll
                for (int t = 0; t < T; ++t)
                {
                    if (tile0 + t >= p.tiles) break;
                    uint32_t a[8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) i8x4_to_f16(wv[t][u][j], a[2 * j], a[2 * j + 1]);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(a[0], a[1], a[2], a[3]), b1, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(a[4], a[5], a[6], a[7]), b2, acc[t], 0, 0, 0);
                }
            }
            else
            {
                // one 128-k quantisation group per block: per tile a fresh
                // accumulator, then the group's scale and zero point
                const uint32_t g = blk;
#pragma unroll
                for (int t = 0; t < T; ++t)
                {
                    if (tile0 + t >= p.tiles) break;
                    f4_t bacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                    {
                        uint32_t a[4];
                        u4_slot_pairs<AF>(wv[t][u][j], a);
                        if constexpr (AF == OPURE_A_F16)
                            bacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                as_half8(a[0], a[1], a[2], a[3]),
                                as_half8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]), bacc, 0, 0, 0);
                        else
                            bacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                as_bf8(a[0], a[1], a[2], a[3]),
                                as_bf8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]), bacc, 0, 0, 0);
                    }
                    const uint32_t e = (t * G + g) * 16u + 4u * g4;
                    const f4_t sc = *reinterpret_cast<const f4_t*>(szs + e);
                    const f4_t c = *reinterpret_cast<const f4_t*>(szc + e);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                    {
                        acc[t][i] = __fmaf_rn(sc[i], bacc[i], acc[t][i]);
                        zac[t][i] = __fmaf_rn(c[i], xs, zac[t][i]);
                    }
                }
            }
        }
    };
    // software pipeline over passes: pass ps computes while ps+1 is in flight.
    // Loads are issued only for passes that exist, on straight-line paths, so
    // every wait covers exactly the buffer being consumed.
    uint32_t ps = 0;
    while (npass - ps >= 4u)
    {
        run_pass(wa, ps);
        load_w(wa, (ps + 2u) * PB + wave);
        run_pass(wb, ps + 1u);
        load_w(wb, (ps + 3u) * PB + wave);
        ps += 2u;
    }
    const uint32_t rest = npass - ps;
    if (rest == 3u)
    {
        run_pass(wa, ps);
        load_w(wa, (ps + 2u) * PB + wave);
        run_pass(wb, ps + 1u);
        run_pass(wa, ps + 2u);
    }
    else if (rest == 2u)
    {
        run_pass(wa, ps);
        run_pass(wb, ps + 1u);
    }
    else
    {
        run_pass(wa, ps);
    }

    // ---- combine the waves' K slices in wave order; wave t finishes tile t --
    __syncthreads();                                // LDS X stage is dead from here
#pragma unroll
    for (int t = 0; t < T; ++t)
    {
        if constexpr (WF == OPURE_W_I4G128) acc[t] -= zac[t];
        red[(wave * T + t) * 64u + lane] = acc[t];
    }
    __syncthreads();
    if (wave >= static_cast<uint32_t>(T)) return;
    const uint32_t tile = tile0 + wave;
    if (tile >= p.tiles) return;
    f4_t tot = red[wave * 64u + lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) tot += red[(w * T + wave) * 64u + lane];

    // ---- epilogue: lane holds D rows 4*g4 + i for column m = r16 -----------
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        v[i] = tot[i];
        if constexpr (WF == OPURE_W_I8PC)
            v[i] = __fmul_rn(v[i], f16_to_f32(static_cast<const uint16_t*>(p.scale)[weight_row(EPI, tile, 4u * g4 + i, p.out)]));
    }
    if constexpr (EPI == opure_hip::EPI_LOGITS)
    {
        // logits, then the best (value, lowest index) of this tile for column m
        float bv = -__builtin_huge_valf();
        int32_t bi = 0x7FFFFFFF;
        if (m < M)
        {
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const uint32_t o = 16u * tile + 4u * g4 + i;
                static_cast<float*>(p.y)[static_cast<uint64_t>(m) * p.out + o] = v[i];
                const float c = v[i] != v[i] ? -__builtin_huge_valf() : v[i];
                if (c > bv || (c == bv && static_cast<int32_t>(o) < bi)) { bv = c; bi = static_cast<int32_t>(o); }
            }
        }
#pragma unroll
        for (int off = 16; off <= 32; off <<= 1)
        {
            const float ov = __shfl_xor(bv, off);
            const int32_t oi = __shfl_xor(bi, off);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (m < M && g4 == 0)
        {
            p.lg.am_val[static_cast<uint64_t>(tile) * M + m] = bv;
            p.lg.am_idx[static_cast<uint64_t>(tile) * M + m] = bi;
        }
        return;
    }
    if constexpr (EPI == opure_hip::EPI_RESIDUAL)
    {
        // x += y, and this tile's sum of squares of the new x for the next rmsnorm
        float sq = 0.0f;
        if (m < M)
        {
            float* y = static_cast<float*>(p.y) + static_cast<uint64_t>(m) * p.out + 16u * tile + 4u * g4;
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const float nv = __fadd_rn(y[i], v[i]);
                y[i] = nv;
                sq = __fmaf_rn(nv, nv, sq);
            }
        }
        sq += __shfl_xor(sq, 16);
        sq += __shfl_xor(sq, 32);
        if (p.ss_out && m < M && g4 == 0) p.ss_out[static_cast<uint64_t>(tile) * M + m] = sq;
        return;
    }
    if (m >= M) return;
    if constexpr (EPI == opure_hip::EPI_STORE)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            store_act_rt(p.y, static_cast<uint64_t>(m) * p.out + 16u * tile + 4u * g4 + i, v[i], p.yfmt);
    }
    else if constexpr (EPI == opure_hip::EPI_SWIGLU)
    {
        const uint32_t F = p.out >> 1;
        const uint32_t f = 8u * tile + 2u * g4;
        store_act_rt(p.y, static_cast<uint64_t>(m) * F + f, swiglu(v[0], v[1]), p.yfmt);
        store_act_rt(p.y, static_cast<uint64_t>(m) * F + f + 1u, swiglu(v[2], v[3]), p.yfmt);
    }
    else if constexpr (EPI == opure_hip::EPI_QKV)
    {
        const opure_hip::QkvEpilogue& e = p.qkv;
        const uint32_t b = m / e.rows_per_seq, j = m - b * e.rows_per_seq;
        const uint32_t pos = static_cast<uint32_t>(e.seq_len[b]) + j;
        if (pos >= e.rope_max_pos || pos / OPURE_PAGE_SIZE >= e.max_pages) return;   // past the tables: drop
        const uint32_t o0 = 16u * tile + 4u * g4;   // even; o0..o0+3 lie in one head
        const uint32_t hd = e.head_dim, half = hd >> 1;
        if (o0 < e.qdim + e.kvdim)
        {
            // rotate the two interleaved pairs (Opure_RoPE.usf:7-10)
#pragma unroll
            for (int pr = 0; pr < 2; ++pr)
            {
                const uint32_t o = o0 + 2u * pr;
                const uint32_t d = (o < e.qdim ? o : o - e.qdim) % hd;
                const float c = e.rope_cos[static_cast<uint64_t>(pos) * half + d / 2u];
                const float s = e.rope_sin[static_cast<uint64_t>(pos) * half + d / 2u];
                const float e0 = v[2 * pr], e1 = v[2 * pr + 1];
                v[2 * pr] = __fsub_rn(__fmul_rn(e0, c), __fmul_rn(e1, s));
                v[2 * pr + 1] = __fadd_rn(__fmul_rn(e0, s), __fmul_rn(e1, c));
            }
        }
        if (o0 < e.qdim)
        {
#pragma unroll
            for (int i = 0; i < 4; ++i) store_act_rt(p.y, static_cast<uint64_t>(m) * e.qdim + o0 + i, v[i], p.yfmt);
            return;
        }
        const uint32_t kvsel = o0 < e.qdim + e.kvdim ? 0u : 1u;
        const uint32_t ok = o0 - e.qdim - kvsel * e.kvdim;
        const uint32_t kh = ok / hd, d0 = ok - kh * hd;
        const int32_t page = e.page_table[static_cast<uint64_t>(b) * e.max_pages + pos / OPURE_PAGE_SIZE];
        if (page < 0 || static_cast<uint32_t>(page) >= e.n_pages) return;
        const uint64_t base = ((((static_cast<uint64_t>(e.layer) * e.n_pages + static_cast<uint32_t>(page)) * 2u + kvsel) *
                                e.n_kv_heads + kh) * OPURE_PAGE_SIZE + pos % OPURE_PAGE_SIZE) * hd + d0;
#pragma unroll
        for (int i = 0; i < 4; ++i) store_act_rt(e.kv_pool, base + i, v[i], p.yfmt);
    }
}

template <int WF, int AF, int EPI, int NW, int T, bool NORM, bool STAGED>
int launch_k(opure_dev* dev, const KParams& kp, uint32_t lds)
{
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<WF, AF, EPI, NW, T, NORM, STAGED>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        configured = true;
    }
    const uint32_t groups = (kp.tiles + T - 1u) / T;
    hipLaunchKernelGGL((k_gemv<WF, AF, EPI, NW, T, NORM, STAGED>), dim3(groups), dim3(NW * 64), lds, dev->stream, kp);
    OPURE_LAUNCH_CHECK("k_gemv");
    return OPURE_OK;
}

template <int WF, int AF, int EPI, int NW, int T, bool NORM>
int launch_st(opure_dev* dev, const KParams& kp, bool staged, uint32_t lds)
{
    return staged ? launch_k<WF, AF, EPI, NW, T, NORM, true>(dev, kp, lds)
                  : launch_k<WF, AF, EPI, NW, T, NORM, false>(dev, kp, lds);
}

// (waves, tiles per workgroup) pairs gemv_shape can choose: T > 1 only with 4 waves
template <int WF, int AF, int EPI, bool NORM>
int launch_shape(opure_dev* dev, const KParams& kp, const opure_hip::GemvShape& s, bool staged, uint32_t lds)
{
    if (s.t == 1 && s.nw == 4) return launch_st<WF, AF, EPI, 4, 1, NORM>(dev, kp, staged, lds);
    if (s.t == 1 && s.nw == 8) return launch_st<WF, AF, EPI, 8, 1, NORM>(dev, kp, staged, lds);
    if (s.t == 1 && s.nw == 16) return launch_st<WF, AF, EPI, 16, 1, NORM>(dev, kp, staged, lds);
    if (s.t == 2 && s.nw == 4) return launch_st<WF, AF, EPI, 4, 2, NORM>(dev, kp, staged, lds);
    if (s.t == 4 && s.nw == 4) return launch_st<WF, AF, EPI, 4, 4, NORM>(dev, kp, staged, lds);
    return opure_hip::set_error(OPURE_E_INVALID, "gemv: no kernel for %u waves x %u tiles", s.nw, s.t);
}

// norm-fused variants exist for the consumers of a residual (qkv, gate/up, LM head)
template <int WF, int AF>
int launch_epi(opure_dev* dev, uint32_t epi, bool norm, const KParams& kp, const opure_hip::GemvShape& s, bool staged,
               uint32_t lds)
{
    using namespace opure_hip;
    if (!norm)
    {
        switch (epi)
        {
        case EPI_STORE: return launch_shape<WF, AF, EPI_STORE, false>(dev, kp, s, staged, lds);
        case EPI_RESIDUAL: return launch_shape<WF, AF, EPI_RESIDUAL, false>(dev, kp, s, staged, lds);
        case EPI_SWIGLU: return launch_shape<WF, AF, EPI_SWIGLU, false>(dev, kp, s, staged, lds);
        }
    }
    else
    {
        switch (epi)
        {
        case EPI_SWIGLU: return launch_shape<WF, AF, EPI_SWIGLU, true>(dev, kp, s, staged, lds);
        case EPI_QKV: return launch_shape<WF, AF, EPI_QKV, true>(dev, kp, s, staged, lds);
        case EPI_LOGITS: return launch_shape<WF, AF, EPI_LOGITS, true>(dev, kp, s, staged, lds);
        }
    }
    return set_error(OPURE_E_INVALID, "gemv: epilogue %u %s the fused norm is not built", epi, norm ? "with" : "without");
}

// blocks per wave per pass; must match U in k_gemv
uint32_t u_of(uint32_t wfmt, uint32_t t, uint32_t nw, bool norm)
{
    if (wfmt == OPURE_W_I4G128) return (t >= 4 || (norm && nw == 16)) ? 2u : 4u;
    return (t >= 4 || (norm && nw == 16)) ? 4u : 8u;
}

uint32_t kb_of(uint32_t wfmt) { return wfmt == OPURE_W_F32 ? 16u : (wfmt == OPURE_W_I8PC ? 64u : 128u); }

}  // namespace

namespace opure_hip {

// T 16-row tiles per workgroup while that still leaves >= 512 workgroups, then
// NW waves splitting K grow while the grid has fewer than 2048 waves and every
// wave keeps at least two 64-byte blocks per row.  Depends on the shape only,
// never on M, so a row's result does not depend on the rows beside it.
GemvShape gemv_shape(uint32_t wfmt, uint32_t out, uint32_t in)
{
    GemvShape s;
    s.tiles = out / 16u;
    s.blocks = in / kb_of(wfmt);
    s.t = s.tiles >= 4u * 512u ? 4u : (s.tiles >= 2u * 512u ? 2u : 1u);
    s.nw = 4u;
    const uint32_t groups = (s.tiles + s.t - 1u) / s.t;
    while (s.nw < 16u && groups * s.nw < 2048u && s.blocks >= 4u * s.nw) s.nw *= 2u;
    return s;
}

int gemv_validate(const GemvCall& c)
{
    const uint32_t wf = c.wfmt, af = c.xfmt;
    OPURE_REQUIRE(wf <= OPURE_W_I4G128 && af <= OPURE_A_BF16, OPURE_E_INVALID, "gemv: bad format (w %u, x %u)", wf, af);
    const bool ok = (wf == OPURE_W_F32 && af == OPURE_A_F32) || (wf == OPURE_W_I8PC && af == OPURE_A_F16) ||
                    (wf == OPURE_W_I4G128 && (af == OPURE_A_F16 || af == OPURE_A_BF16));
    OPURE_REQUIRE(ok, OPURE_E_UNSUPPORTED, "gemv: weights %u with %s activations are not built", wf, afmt_name(af));
    OPURE_REQUIRE(c.W.w && c.x && c.y, OPURE_E_INVALID, "gemv: null weight, input or output pointer");
    OPURE_REQUIRE(c.M >= 1 && c.M <= OPURE_MAX_ROWS, OPURE_E_CAPACITY, "gemv: M=%u outside 1..%d", c.M, OPURE_MAX_ROWS);
    OPURE_REQUIRE(c.W.out >= 16 && c.W.out % 16 == 0, OPURE_E_INVALID, "gemv: out=%u must be a positive multiple of 16",
                  c.W.out);
    const uint32_t KB = kb_of(wf);
    OPURE_REQUIRE(c.W.in >= KB && c.W.in % KB == 0, OPURE_E_INVALID, "gemv: in=%u must be a multiple of %u", c.W.in, KB);
    OPURE_REQUIRE((reinterpret_cast<uintptr_t>(c.W.w) & 15u) == 0 && (reinterpret_cast<uintptr_t>(c.x) & 15u) == 0,
                  OPURE_E_INVALID, "gemv: weight and input pointers must be 16-byte aligned");
    if (c.gain)
        OPURE_REQUIRE(c.ss_in && c.ss_tiles >= 1 && (reinterpret_cast<uintptr_t>(c.gain) & 15u) == 0 &&
                          (c.epi == EPI_SWIGLU || c.epi == EPI_QKV || c.epi == EPI_LOGITS),
                      OPURE_E_INVALID, "gemv: fused rmsnorm needs sums of squares, an aligned gain and a consumer epilogue");
    else
        OPURE_REQUIRE(c.epi != EPI_QKV && c.epi != EPI_LOGITS, OPURE_E_INVALID, "gemv: qkv/logits epilogues fuse the rmsnorm");
    if (wf == OPURE_W_I8PC) OPURE_REQUIRE(c.W.scale, OPURE_E_INVALID, "gemv: int8 weights need scales");
    if (wf == OPURE_W_I4G128) OPURE_REQUIRE(c.W.scale && c.W.zero, OPURE_E_INVALID, "gemv: int4 weights need scale and zero");
    OPURE_REQUIRE(c.yfmt <= OPURE_A_BF16, OPURE_E_INVALID, "gemv: bad output format %u", c.yfmt);
    if (c.epi == EPI_RESIDUAL || c.epi == EPI_LOGITS)
        OPURE_REQUIRE(c.yfmt == OPURE_A_F32, OPURE_E_INVALID, "gemv: residual/logits output must be f32");
    if (c.epi == EPI_SWIGLU) OPURE_REQUIRE(c.W.out % 32 == 0, OPURE_E_INVALID, "gemv: swiglu needs 2*ffn %% 32 == 0");
    if (c.epi == EPI_LOGITS) OPURE_REQUIRE(c.logits.am_val && c.logits.am_idx, OPURE_E_INVALID, "gemv: argmax partials");
    if (c.epi == EPI_QKV)
    {
        const QkvEpilogue& e = c.qkv;
        OPURE_REQUIRE(e.head_dim >= 16 && e.head_dim % 16 == 0 && e.qdim % e.head_dim == 0 && e.kvdim % e.head_dim == 0 &&
                          c.W.out == e.qdim + 2u * e.kvdim,
                      OPURE_E_INVALID, "gemv: qkv epilogue shape mismatch");
        OPURE_REQUIRE(e.rope_cos && e.rope_sin && e.seq_len && e.kv_pool && e.page_table && e.rows_per_seq >= 1 &&
                          c.M % e.rows_per_seq == 0,
                      OPURE_E_INVALID, "gemv: qkv epilogue pointers");
    }
    return OPURE_OK;
}

int gemv_launch(opure_dev* dev, const GemvCall& c)
{
    const GemvShape s = gemv_shape(c.wfmt, c.W.out, c.W.in);
    const bool norm = c.gain != nullptr;
    KParams kp;
    kp.w = static_cast<const uint8_t*>(c.W.w);
    kp.scale = c.W.scale;
    kp.zero = c.W.zero;
    kp.out = c.W.out;
    kp.in = c.W.in;
    kp.x = static_cast<const uint8_t*>(c.x);
    kp.M = c.M;
    kp.y = c.y;
    kp.yfmt = c.yfmt;
    kp.tiles = s.tiles;
    kp.gain = c.gain;
    kp.eps = c.eps;
    kp.ss_in = c.ss_in;
    kp.ss_tiles = c.ss_tiles;
    kp.ss_out = c.ss_out;
    kp.qkv = c.qkv;
    kp.lg = c.logits;

    // LDS: the X stage takes as many whole passes as fit in this workgroup's
    // share of the CU (more workgroups per CU for larger grids); if not even
    // one pass fits, fragments come straight from global memory.
    const uint32_t KB = kb_of(c.wfmt);
    const uint32_t EB = act_bytes(c.xfmt);
    const uint32_t PBK = u_of(c.wfmt, s.t, s.nw, norm) * s.nw * KB;      // k per pass
    const uint32_t npass = (c.W.in + PBK - 1u) / PBK;
    const uint32_t groups = (s.tiles + s.t - 1u) / s.t;
    const uint32_t per_cu = groups >= 1024u ? 3u : (groups >= 512u ? 2u : 1u);
    const uint32_t cap = 160u * 1024u / per_cu - 1024u;
    const uint32_t red_bytes = s.nw * s.t * 1024u;
    const uint32_t sz_bytes = c.wfmt == OPURE_W_I4G128 ? s.t * 16u * (c.W.in / 128u) * 8u : 0u;
    uint32_t lds = 0;
    bool staged = false;
    for (uint32_t P = npass; P >= 1u; --P)
    {
        const uint32_t segk = P * PBK < c.W.in ? P * PBK : c.W.in;
        const uint32_t stride = segk * EB + 16u;
        const uint32_t xsum_bytes = c.wfmt == OPURE_W_I4G128 ? c.M * (segk / 128u) * 4u : 0u;
        const uint32_t off_xsum = static_cast<uint32_t>(align_up(static_cast<uint64_t>(c.M) * stride, 16));
        const uint32_t off_sz = static_cast<uint32_t>(align_up(off_xsum + xsum_bytes, 16));
        const uint32_t total = std::max(off_sz + sz_bytes, red_bytes);
        if (total <= cap)
        {
            staged = true;
            kp.seg_passes = P;
            kp.x_stride = stride;
            kp.x_groups = segk / 128u;
            kp.off_xsum = off_xsum;
            kp.off_sz = off_sz;
            lds = total;
            break;
        }
    }
    if (!staged)
    {
        kp.seg_passes = npass;
        kp.x_stride = kp.x_groups = kp.off_xsum = 0;
        kp.off_sz = 0;
        lds = std::max(sz_bytes, red_bytes);
        OPURE_REQUIRE(lds <= 160u * 1024u, OPURE_E_UNSUPPORTED, "gemv: in=%u too long for the group-scale stage", c.W.in);
    }
    if (c.wfmt == OPURE_W_F32) return launch_epi<OPURE_W_F32, OPURE_A_F32>(dev, c.epi, norm, kp, s, staged, lds);
    if (c.wfmt == OPURE_W_I8PC) return launch_epi<OPURE_W_I8PC, OPURE_A_F16>(dev, c.epi, norm, kp, s, staged, lds);
    if (c.xfmt == OPURE_A_F16) return launch_epi<OPURE_W_I4G128, OPURE_A_F16>(dev, c.epi, norm, kp, s, staged, lds);
    return launch_epi<OPURE_W_I4G128, OPURE_A_BF16>(dev, c.epi, norm, kp, s, staged, lds);
}

}  // namespace opure_hip

using namespace opure_hip;

static int gemv_public(opure_dev* dev, const opure_gemv_args* a, uint32_t wfmt)
{
    OPURE_REQUIRE(dev && a, OPURE_E_INVALID, "gemv: null argument");
    OPURE_REQUIRE(a->epilogue <= OPURE_EPI_SWIGLU, OPURE_E_INVALID, "gemv: bad epilogue %u", a->epilogue);
    GemvCall c;
    c.W = a->W;
    c.wfmt = wfmt;
    c.x = a->x;
    c.xfmt = a->xfmt;
    c.M = a->M;
    c.y = a->y;
    c.yfmt = a->yfmt;
    c.epi = a->epilogue;
    const int rc = gemv_validate(c);
    if (rc) return rc;
    return gemv_launch(dev, c);
}

extern "C" {
int opure_gemv_batched_f32(opure_dev* dev, const opure_gemv_args* a) { return gemv_public(dev, a, OPURE_W_F32); }
int opure_gemv_batched_i8pc(opure_dev* dev, const opure_gemv_args* a) { return gemv_public(dev, a, OPURE_W_I8PC); }
int opure_gemv_batched_i4g128(opure_dev* dev, const opure_gemv_args* a) { return gemv_public(dev, a, OPURE_W_I4G128); }
}
