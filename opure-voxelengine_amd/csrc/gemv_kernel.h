// ============================================================================
//  gemv_kernel.h -- the K+1-row GEMV kernel for gfx950 matrix cores, included
//  by gemv_f32.hip / gemv_i8.hip / gemv_i4.hip (one weight format each, so the
//  instantiations compile in parallel).
//
//  Replaces GEMVMain / GEMVQuantMain (shaders/Opure_GEMV.usf:40-89,
//  shaders/Opure_GEMV_Quant.usf:39-95), which read the whole weight matrix once
//  per activation row.  Here every weight byte is read once for all M <= 16
//  rows (the K+1 draft positions of one or more sequences).
//
//  Mapping.  y^T[o][m] = sum_k W[o][k] X[m][k] is one 16 x 16 MFMA tile per 16
//  weight rows: A = 16 weight rows x 32 k, B = 32 k x 16 columns of X (columns
//  >= M compute on a copy of column M-1 and are never stored).  Weights are in
//  the tiled layout (opure_tile_linear): tile t, block b is 1 KB and lane l of
//  a wave loads bytes [16l, 16l+16) of it -- row l%16, k-slice l/16 -- so one
//  wave instruction reads 1 KB of contiguous memory.  Widening in registers:
//    f32   -> v_mfma_f32_16x16x4_f32, 4 MFMAs per block
//    int8  -> offset-binary bytes into fp16 1024+u via byte permutes, minus
//             1152 (exact), 2 x v_mfma_f32_16x16x32_f16 per block
//    uint4 -> nibbles pre-ordered so two masks and four byte permutes give
//             MAGIC|q pairs in k order, 4 MFMAs per 128-k group; the group's
//             scale and zero point are applied to the fresh group accumulator
//             through the column's group sum of X
//
//  Work split.  A workgroup of NW waves owns T tiles at a time ("a group");
//  its waves take interleaved blocks of K (U per wave per pass) and are
//  combined through LDS in wave order, then wave t runs the epilogue of tile t.
//  With STAGED, X is staged once into LDS for the whole K (rmsnorm applied
//  there for consumers of the residual) and the workgroup loops over groups
//  (persistent); otherwise X fragments are loaded from global memory with the
//  weights -- for at most 8 rows two blocks a load (XM_PAIRED: lanes of rows
//  0..7 take block u, lanes of rows 8..15 block u + 1, and a row rotation
//  brings block u + 1 under rows 0..7 when it is its turn; the rows >= M of
//  the MFMA are never read).  Weights (and X fragments) of the next pass are always in flight
//  while the current pass computes.  No workgroup talks to another, and every
//  sum has a fixed order that depends on the shape only, so results are
//  reproducible and independent of M and of the path taken.
// ============================================================================
#pragma once

#include "internal.h"
#include "rollback.h"

namespace opure_gemv {

using namespace opure_dev_math;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

struct KParams {
    const uint8_t* w;          // tiled weights
    const void* sc;            // tiled scales: int8 fp16[tiles][16]; uint4 u32[tiles][G][16]
    uint32_t out, in, tiles, nblk, groups;
    const uint8_t* x;          // X [M][in] in the activation format, or the fp32 residual with NORM
    uint32_t M;
    void* y;
    uint32_t yfmt;
    const float* gain;         // NORM: rmsnorm gain [in]
    float eps;
    const float* ss_in;        // NORM: producer's per-16-column sums of squares [ss_tiles][M]
    uint32_t ss_tiles;
    float* ss_out;             // RESIDUAL: this GEMV's per-tile sums of squares [tiles][M] (may be null)
    uint32_t x_stride;         // STAGED: LDS bytes per staged X row
    uint32_t off_xsum;         // STAGED uint4: LDS offset of the group sums [M][in/128]
    uint32_t off_red;          // LDS offset of the wave reduction [NW][T][64] f4
    uint32_t off_ring, ring;   // loader-wave kernel: LDS offset of the slot rings, slots per compute wave
    uint32_t* err;             // opure_dev::err (ERR_WAIT: a bounded wait gave up)
    uint32_t wait_limit;       // loader-wave kernel: sleeps before a wait gives up
    opure_hip::QkvEpilogue qkv;
    opure_hip::LogitsEpilogue lg;
};

template <int WF> struct Fmt;
// KB: k values per 64-byte block of a row; N: X dwords per lane per block
template <> struct Fmt<OPURE_W_F32>    { static constexpr uint32_t KB = 16, N = 4; };
template <> struct Fmt<OPURE_W_I8PC>   { static constexpr uint32_t KB = 64, N = 8; };
template <> struct Fmt<OPURE_W_I4G128> { static constexpr uint32_t KB = 128, N = 16; };

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

// 4 offset-binary bytes u = q + 128 -> fp16 pairs (q0, q1), (q2, q3), exactly:
// 0x64uu is 1024 + u, minus 1152
__device__ __forceinline__ void u8x4_to_f16(uint32_t u, uint32_t& lo, uint32_t& hi)
{
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const half2_t bias = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, a) + bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, b) + bias);
}

// A tiled uint4 word holds elements e0..e7 at nibbles 0,4,1,5,2,6,3,7 and is
// stored rotated left by 3 bits (opure_tile_linear), so the low nibble of every
// byte sits at bits 3..6 of that byte, and after a rotation right by 4 the high
// nibble does: lo bytes are (e0,e4,e1,e5) << 3, hi bytes (e2,e6,e3,e7) << 3.
// Byte permutes against MAGIC then give operand pairs in k order:
//   fp16 0x64|q<<3 = 1024 + 8q, minus 1024 exactly: 8q;
//   bf16 0x41|q<<3 = 8 + q/2 (bf16 has no packed subtract, so the 8 stays and
//        is taken out with the zero point through the group sum of X; 8 on a
//        step of 1/2 is the smallest offset a 4-bit field under the implicit
//        leading one allows -- 128 + q, with the field at the bottom of the
//        mantissa, cost about 3 more bits of every group sum).
// So operand = U4<AF>::MUL * q + U4<AF>::OFF exactly, and a group's
//   s * sum (q - z) x = (s / MUL) * (acc - (OFF + MUL z) * sum x)
// with both factors exact (MUL a power of two).
template <int AF> struct U4 {
    static constexpr uint32_t MAGIC = AF == OPURE_A_F16 ? 0x64646464u : 0x41414141u;
    static constexpr float MUL = AF == OPURE_A_F16 ? 8.0f : 0.5f;
    static constexpr float OFF = AF == OPURE_A_F16 ? 0.0f : 8.0f;
};
template <int AF>
__device__ __forceinline__ void u4x8_pairs(uint32_t d, uint32_t (&o)[4])
{
    constexpr uint32_t MAGIC = U4<AF>::MAGIC;
    const uint32_t lo = d & 0x78787878u;
    const uint32_t hi = __builtin_amdgcn_alignbit(d, d, 4) & 0x78787878u;
    o[0] = __builtin_amdgcn_perm(MAGIC, lo, 0x04020400u);   // e0 e1
    o[1] = __builtin_amdgcn_perm(MAGIC, hi, 0x04020400u);   // e2 e3
    o[2] = __builtin_amdgcn_perm(MAGIC, lo, 0x04030401u);   // e4 e5
    o[3] = __builtin_amdgcn_perm(MAGIC, hi, 0x04030401u);   // e6 e7
    if constexpr (AF == OPURE_A_F16)
    {
        const half2_t bias = {static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, o[j]) + bias);
    }
}

// a uint4 group's (scale, zero) word -> the factor and the offset the group
// accumulator is corrected with (see U4)
template <int AF>
__device__ __forceinline__ void u4_group(uint32_t sz, float& sc, float& zo)
{
    sc = __fmul_rn(__uint_as_float(sz << 16), 1.0f / U4<AF>::MUL);
    zo = __fmaf_rn(__uint_as_float(sz & 0xFFFF0000u), U4<AF>::MUL, U4<AF>::OFF);
}

// sum of 8 rounded activations (4 pairs): packed dot products with (1, 1)
template <int AF>
__device__ __forceinline__ float unit_sum(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3)
{
    const uint32_t d[4] = {d0, d1, d2, d3};
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
    {
        if constexpr (AF == OPURE_A_F16)
            s = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, d[j]), __builtin_bit_cast(half2_t, 0x3C003C00u), s,
                                       false);
        else
            s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, d[j]),
                                                __builtin_bit_cast(bf16x2_t, 0x3F803F80u), s, false);
    }
    return s;
}

// two floats rounded to nearest even into one packed pair (v_cvt_pk_f16_f32 /
// v_cvt_pk_bf16_f32)
template <int AF>
__device__ __forceinline__ uint32_t pack2(float a, float b)
{
    typedef float f2_t __attribute__((ext_vector_type(2)));
    const f2_t v = {a, b};
    if constexpr (AF == OPURE_A_F16)
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, half2_t));
    else
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// 1 / rms of column m from the producer's per-16-column sums of squares, by
// one wave in a fixed order (lane l takes tiles l, l+64, ..., then a 6-level
// butterfly) that depends on neither M nor the kernel shape
__device__ __forceinline__ float inv_rms_finish(const KParams& p, float ssum)
{
    ssum = row16_sum(ssum);
    ssum = add_xor32(add_xor16(ssum));
    return __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ssum, static_cast<float>(p.in)), p.eps)));
}

__device__ __forceinline__ float inv_rms_wave(const KParams& p, uint32_t m, uint32_t lane)
{
    float ssum = 0.0f;
    for (uint32_t t = lane; t < p.ss_tiles; t += 64u) ssum += p.ss_in[static_cast<uint64_t>(t) * p.M + m];
    return inv_rms_finish(p, ssum);
}

// 8 consecutive activations of row m at k, as 8 fp32 words (AF f32) or 4
// pairs; with NORM rmsnorm'd from the fp32 residual: round(x*inv*g)
// (Opure_RMSNorm.usf:44-78)
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
        float yv[8];
#pragma unroll
        for (int e = 0; e < 4; ++e)
        {
            yv[e] = __fmul_rn(__fmul_rn(x0[e], inv), g0[e]);
            yv[4 + e] = __fmul_rn(__fmul_rn(x1[e], inv), g1[e]);
        }
        if constexpr (AF == OPURE_A_F32)
        {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = __float_as_uint(yv[e]);
        }
        else
        {
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = pack2<AF>(yv[2 * j], yv[2 * j + 1]);
        }
    }
}

// Staging of X rows 0..M-1 (whole K) into LDS rows of x_stride bytes, natural
// k order.  A round holds KR rows in registers: stage_issue only issues the
// loads, stage_store converts and writes them, so the kernel can issue the
// first round, then its first weight loads, and wait for L2 alone (loads
// retire in issue order).  Every load instruction reads 64 consecutive 16-byte
// pieces (the memory pipeline takes 64 bytes a clock, so a strided piece costs
// as much as a whole line).
//
// 16-bit or fp32 X: thread t owns the 8-value unit column j = j0 + t % n8
// (n8 = in/8) and the rows rg, rg + RT, ... with rg = t / n8 and RT =
// max(1, NTH / n8) row groups.
// rmsnorm'd fp32 residual: thread t owns the 4-value quads q = j0 + t and
// j0 + t + NTH of every row, and the gain quads once for all rows.
template <int AF, bool NORM, int KR>
struct StageRound {
    static constexpr int XW = (NORM || AF == OPURE_A_F32) ? 2 : 1;   // 16-byte words per row
    u4_t x[KR][XW];
    u4_t g[NORM ? 2 : 1];
};

template <int NTH>
struct StageMap {
    uint32_t n8, rt, j, rg;
    bool col;                 // this thread owns a unit column
    __device__ __forceinline__ StageMap(const KParams& p, uint32_t j0)
    {
        n8 = p.in / 8u;
        rt = n8 >= NTH ? 1u : NTH / n8;
        const uint32_t t = threadIdx.x;
        rg = n8 >= NTH ? 0u : t / n8;
        j = j0 + (n8 >= NTH ? t : t - rg * n8);
        col = rg < rt && j < n8;
    }
};

// the rmsnorm'd path's rounds: quads j0 + t + h NTH (h < 2), KR rows at a time
template <int NTH>
__device__ __forceinline__ uint32_t norm_quad(uint32_t j0, int h) { return j0 + threadIdx.x + h * NTH; }

template <int AF, bool NORM, int NTH, int KR>
__device__ __forceinline__ void stage_issue(const KParams& p, StageRound<AF, NORM, KR>& r, uint32_t j0, uint32_t i0)
{
    if constexpr (NORM)
    {
        const uint32_t n4 = p.in / 4u;
        const f4_t* xf = reinterpret_cast<const f4_t*>(p.x);
#pragma unroll
        for (int h = 0; h < 2; ++h)
        {
            if (h == 1 && j0 + NTH >= n4) break;             // uniform: the round has one quad per thread
            const uint32_t q = min(norm_quad<NTH>(j0, h), n4 - 1u);   // past the end: the last quad again, never stored
            r.g[h] = __builtin_bit_cast(u4_t, reinterpret_cast<const f4_t*>(p.gain)[q]);
#pragma unroll
            for (int i = 0; i < KR; ++i)
            {
                const uint32_t m = min(i0 + i, p.M - 1u);
                r.x[i][h] = __builtin_bit_cast(u4_t, xf[static_cast<uint64_t>(m) * n4 + q]);
            }
        }
        return;
    }
    const StageMap<NTH> sm(p, j0);
    const uint32_t j = sm.col ? sm.j : 0u;           // past the end: unit 0 of row 0 again, never stored
#pragma unroll
    for (int i = 0; i < KR; ++i)
    {
        const uint32_t m = min(sm.rg + (i0 + i) * sm.rt, p.M - 1u);
        if constexpr (AF == OPURE_A_F32)
        {
            const u4_t* src = reinterpret_cast<const u4_t*>(p.x + (static_cast<uint64_t>(m) * p.in + 8u * j) * 4u);
            r.x[i][0] = src[0];
            r.x[i][1] = src[1];
        }
        else
        {
            r.x[i][0] = *reinterpret_cast<const u4_t*>(p.x + (static_cast<uint64_t>(m) * p.in + 8u * j) * 2u);
        }
    }
}

template <int WF, int AF, bool NORM, int NTH, int KR>
__device__ __forceinline__ void stage_store(const KParams& p, const StageRound<AF, NORM, KR>& r, uint32_t j0, uint32_t i0,
                                            uint8_t* lds, const float* sinv)
{
    constexpr uint32_t EB = AF == OPURE_A_F32 ? 4u : 2u;
    if constexpr (NORM)
    {
        const uint32_t n4 = p.in / 4u;
#pragma unroll
        for (int i = 0; i < KR; ++i)
        {
            const uint32_t m = i0 + i;
            if (m >= p.M) break;                         // uniform
            // round(x * inv * g) (Opure_RMSNorm.usf:44-78)
            const float inv = sinv[m];
#pragma unroll
            for (int h = 0; h < 2; ++h)
            {
                if (h == 1 && j0 + NTH >= n4) break;         // uniform
                const uint32_t q = norm_quad<NTH>(j0, h);
                const f4_t x = __builtin_bit_cast(f4_t, r.x[i][h]), g = __builtin_bit_cast(f4_t, r.g[h]);
                float yv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) yv[e] = __fmul_rn(__fmul_rn(x[e], inv), g[e]);
                uint8_t* dst = lds + static_cast<uint64_t>(m) * p.x_stride + 4u * q * EB;
                if (q >= n4) continue;
                if constexpr (AF == OPURE_A_F32)
                    *reinterpret_cast<f4_t*>(dst) = f4_t{yv[0], yv[1], yv[2], yv[3]};
                else
                {
                    typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
                    *reinterpret_cast<u2_t*>(dst) = u2_t{pack2<AF>(yv[0], yv[1]), pack2<AF>(yv[2], yv[3])};
                }
            }
        }
        return;
    }
    const StageMap<NTH> sm(p, j0);
#pragma unroll
    for (int i = 0; i < KR; ++i)
    {
        const uint32_t m = sm.rg + (i0 + i) * sm.rt;
        const bool keep = sm.col && m < p.M;
        uint8_t* dst = lds + static_cast<uint64_t>(m) * p.x_stride + 8u * sm.j * EB;
        if constexpr (AF == OPURE_A_F32)
        {
            if (keep)
            {
                reinterpret_cast<u4_t*>(dst)[0] = r.x[i][0];
                reinterpret_cast<u4_t*>(dst)[1] = r.x[i][1];
            }
        }
        else
        {
            if (keep) *reinterpret_cast<u4_t*>(dst) = r.x[i][0];
        }
    }
}

// Rows a round holds per unit column (a rmsnorm'd row costs 8 registers):
// one round for the 8 rows of a K=7 step; 16-wave workgroups have 128
// registers, 8-wave ones 256
template <int AF, bool NORM, int NTH>
constexpr int stage_rows()
{
    return NTH >= 1024 ? 4 : 8;
}

typedef float f2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

// v[0..3] into elements i .. i + 3 of an activation array (i a multiple of 4):
// one 16- or 8-byte store, the same roundings as store_act_rt
__device__ __forceinline__ void store4_act_rt(void* base, uint64_t i, const float (&v)[4], uint32_t af)
{
    if (af == OPURE_A_F32)
    {
        *reinterpret_cast<f4_t*>(static_cast<float*>(base) + i) = f4_t{v[0], v[1], v[2], v[3]};
        return;
    }
    uint32_t h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) h[k] = af == OPURE_A_F16 ? f32_to_f16(v[k]) : f32_to_bf16(v[k]);
    *reinterpret_cast<u2_t*>(static_cast<uint16_t*>(base) + i) = u2_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
}

// a, b into elements i, i + 1 (i even): one 8- or 4-byte store
__device__ __forceinline__ void store2_act_rt(void* base, uint64_t i, float a, float b, uint32_t af)
{
    if (af == OPURE_A_F32)
    {
        *reinterpret_cast<f2_t*>(static_cast<float*>(base) + i) = f2_t{a, b};
        return;
    }
    const uint32_t ha = af == OPURE_A_F16 ? f32_to_f16(a) : f32_to_bf16(a);
    const uint32_t hb = af == OPURE_A_F16 ? f32_to_f16(b) : f32_to_bf16(b);
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(base) + i) = ha | (hb << 16);
}

// EPI_LOGITS keeps the best (value, lowest index) of column m seen so far in
// (best_v, best_i); the workgroup writes one partial per column at its end.
// The thin GEMM's epilogue: lane (g4, r16) holds rows 4 g4 .. 4 g4 + 3 of the
// tile for X row m, stored with one vector store where the layout allows.
template <int WF, int EPI>
__device__ __forceinline__ void epilogue(const KParams& p, uint32_t tile, uint32_t m, uint32_t g4, f4_t tot,
                                         float& best_v, int32_t& best_i, const f4_t* scale = nullptr)
{
    const uint32_t M = p.M;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        v[i] = tot[i];
        // int8: the row scales, loaded here or passed in (the same values)
        if constexpr (WF == OPURE_W_I8PC)
            v[i] = __fmul_rn(v[i], scale ? (*scale)[i] : f16_to_f32(static_cast<const uint16_t*>(p.sc)[tile * 16u + 4u * g4 + i]));
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
        if (bv > best_v || (bv == best_v && bi < best_i)) { best_v = bv; best_i = bi; }
        return;
    }
    if constexpr (EPI == opure_hip::EPI_RESIDUAL)
    {
        // x += y, and this tile's sum of squares of the new x for the next rmsnorm
        float sq = 0.0f;
        if (m < M)
        {
            f4_t* y = reinterpret_cast<f4_t*>(static_cast<float*>(p.y) + static_cast<uint64_t>(m) * p.out + 16u * tile + 4u * g4);
            f4_t nv = *y;
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                nv[i] = __fadd_rn(nv[i], v[i]);
                sq = __fmaf_rn(nv[i], nv[i], sq);
            }
            *y = nv;
        }
        sq = add_xor32(add_xor16(sq));
        if (p.ss_out && m < M && g4 == 0) p.ss_out[static_cast<uint64_t>(tile) * M + m] = sq;
        return;
    }
    if (m >= M) return;
    if constexpr (EPI == opure_hip::EPI_STORE)
    {
        store4_act_rt(p.y, static_cast<uint64_t>(m) * p.out + 16u * tile + 4u * g4, v, p.yfmt);
    }
    else if constexpr (EPI == opure_hip::EPI_SWIGLU)
    {
        // tile rows alternate gate / up: (v0, v1) and (v2, v3) are (gate, up) pairs
        const uint32_t F = p.out >> 1;
        const uint32_t f = 8u * tile + 2u * g4;
        store2_act_rt(p.y, static_cast<uint64_t>(m) * F + f, swiglu(v[0], v[1]), swiglu(v[2], v[3]), p.yfmt);
    }
    else if constexpr (EPI == opure_hip::EPI_QKV)
    {
        const opure_hip::QkvEpilogue& e = p.qkv;
        const uint32_t b = m / e.rows_per_seq, j = m - b * e.rows_per_seq;
        const uint32_t pos = static_cast<uint32_t>(e.seq_len[b]) + j;
        if (pos >= e.rope_max_pos || pos / OPURE_PAGE_SIZE >= e.max_pages)   // past the tables: dropped, reported
        {
            if (e.err) e.err[ERR_POSITION] = 1u;
            return;
        }
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
            store4_act_rt(p.y, static_cast<uint64_t>(m) * e.qdim + o0, v, p.yfmt);
            return;
        }
        const uint32_t kvsel = o0 < e.qdim + e.kvdim ? 0u : 1u;
        const uint32_t ok = o0 - e.qdim - kvsel * e.kvdim;
        const uint32_t kh = ok / hd, d0 = ok - kh * hd;
        const int32_t page = e.page_table[static_cast<uint64_t>(b) * e.max_pages + pos / OPURE_PAGE_SIZE];
        if (page < 0 || static_cast<uint32_t>(page) >= e.n_pages)   // no page for the row: dropped, reported
        {
            if (e.err) e.err[ERR_POSITION] = 1u;
            return;
        }
        // K rows are token-major (d0 .. d0 + 3 adjacent), V channel-major
        if (kvsel == 0u)
        {
            store4_act_rt(e.kv_pool,
                          kv_elem(e.layer, e.n_pages, static_cast<uint32_t>(page), 0u, e.n_kv_heads, kh, hd,
                                  pos % OPURE_PAGE_SIZE, d0),
                          v, p.yfmt);
            return;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            store_act_rt(e.kv_pool,
                         kv_elem(e.layer, e.n_pages, static_cast<uint32_t>(page), kvsel, e.n_kv_heads, kh, hd,
                                 pos % OPURE_PAGE_SIZE, d0 + i),
                         v[i], p.yfmt);
    }
}

// Epilogue of k_gemv, one output element per thread.  The MFMAs take X as
// the A operand, so lane (g4, r16) of a wave's accumulator holds y[m][o] for
// the X rows m = 4*g4 + i and the weight row o = 16*tile + r16.  After the
// waves' partial sums meet in LDS, thread e of the workgroup takes element
// (tile t, row m, column r16) with e = 256 t + 16 m + r16 and adds the waves'
// partials in wave order; so the 16 weight rows of a tile and row m sit in
// the 16 lanes of a DPP row: a tile's sums of squares and argmax are DPP
// trees, and the (gate, up) and RoPE pairs (o even, o + 1) are lanes r16 and
// r16 ^ 1.  EPI_LOGITS keeps the best (value, lowest index) of its (t, m)
// seen so far; the workgroup writes one partial per row at its end.
__device__ __forceinline__ void best_merge(float& bv, int32_t& bi, float ov, int32_t oi)
{
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

template <int CTRL>
__device__ __forceinline__ int32_t dpp_i(int32_t v)
{
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

template <int WF, int EPI>
__device__ __forceinline__ void epilogue_elem(const KParams& p, uint32_t tile, uint32_t m, uint32_t r16, float v,
                                              float& best_v, int32_t& best_i)
{
    const uint32_t M = p.M;
    const uint32_t o = 16u * tile + r16;
    const bool live = tile < p.tiles && m < M;    // uniform over the 16 lanes of the DPP row
    if constexpr (WF == OPURE_W_I8PC) v = __fmul_rn(v, live ? f16_to_f32(static_cast<const uint16_t*>(p.sc)[o]) : 1.0f);
    if constexpr (EPI == opure_hip::EPI_LOGITS)
    {
        float bv = -__builtin_huge_valf();
        int32_t bi = 0x7FFFFFFF;
        if (live)
        {
            static_cast<float*>(p.y)[static_cast<uint64_t>(m) * p.out + o] = v;
            bv = v != v ? -__builtin_huge_valf() : v;
            bi = static_cast<int32_t>(o);
        }
        // a total order, so the tree's shape does not matter
        best_merge(bv, bi, dpp_f<0xB1>(bv), dpp_i<0xB1>(bi));
        best_merge(bv, bi, dpp_f<0x4E>(bv), dpp_i<0x4E>(bi));
        best_merge(bv, bi, dpp_f<0x141>(bv), dpp_i<0x141>(bi));
        best_merge(bv, bi, dpp_f<0x140>(bv), dpp_i<0x140>(bi));
        best_merge(best_v, best_i, bv, bi);
        return;
    }
    if constexpr (EPI == opure_hip::EPI_RESIDUAL)
    {
        // x += y, and this tile's sum of squares of the new x for the next rmsnorm
        float nv = 0.0f;
        if (live)
        {
            float* y = static_cast<float*>(p.y) + static_cast<uint64_t>(m) * p.out + o;
            nv = __fadd_rn(*y, v);
            *y = nv;
        }
        const float sq = row16_sum(__fmul_rn(nv, nv));
        if (p.ss_out && live && r16 == 0) p.ss_out[static_cast<uint64_t>(tile) * M + m] = sq;
        return;
    }
    if constexpr (EPI == opure_hip::EPI_STORE)
    {
        if (live) store_act_rt(p.y, static_cast<uint64_t>(m) * p.out + o, v, p.yfmt);
    }
    else if constexpr (EPI == opure_hip::EPI_SWIGLU)
    {
        // tile rows alternate gate / up: lane r16 even holds a gate, r16 + 1 its up
        const float up = dpp_f<0xB1>(v);
        if (live && (r16 & 1u) == 0)
            store_act_rt(p.y, static_cast<uint64_t>(m) * (p.out >> 1) + 8u * tile + (r16 >> 1), swiglu(v, up), p.yfmt);
    }
    else if constexpr (EPI == opure_hip::EPI_QKV)
    {
        const opure_hip::QkvEpilogue& e = p.qkv;
        const float other = dpp_f<0xB1>(v);
        if (!live) return;
        const uint32_t b = m / e.rows_per_seq, j = m - b * e.rows_per_seq;
        const uint32_t pos = static_cast<uint32_t>(e.seq_len[b]) + j;
        if (pos >= e.rope_max_pos || pos / OPURE_PAGE_SIZE >= e.max_pages)   // past the tables: dropped, reported
        {
            if (e.err) e.err[ERR_POSITION] = 1u;
            return;
        }
        const uint32_t hd = e.head_dim, half = hd >> 1;
        const bool rot = o < e.qdim + e.kvdim;
        if (rot)
        {
            // rotate the interleaved pair (o even, o + 1) (Opure_RoPE.usf:7-10)
            const uint32_t d = (o < e.qdim ? o : o - e.qdim) % hd;
            const float c = e.rope_cos[static_cast<uint64_t>(pos) * half + d / 2u];
            const float sn = e.rope_sin[static_cast<uint64_t>(pos) * half + d / 2u];
            const bool odd = (r16 & 1u) != 0;
            const float e0 = odd ? other : v, e1 = odd ? v : other;
            v = odd ? __fadd_rn(__fmul_rn(e0, sn), __fmul_rn(e1, c)) : __fsub_rn(__fmul_rn(e0, c), __fmul_rn(e1, sn));
        }
        if (o < e.qdim)
        {
            store_act_rt(p.y, static_cast<uint64_t>(m) * e.qdim + o, v, p.yfmt);
            return;
        }
        const uint32_t kvsel = rot ? 0u : 1u;
        const uint32_t ok = o - e.qdim - kvsel * e.kvdim;
        const uint32_t kh = ok / hd, dk = ok - kh * hd;
        const int32_t page = e.page_table[static_cast<uint64_t>(b) * e.max_pages + pos / OPURE_PAGE_SIZE];
        if (page < 0 || static_cast<uint32_t>(page) >= e.n_pages)   // no page for the row: dropped, reported
        {
            if (e.err) e.err[ERR_POSITION] = 1u;
            return;
        }
        store_act_rt(e.kv_pool,
                     kv_elem(e.layer, e.n_pages, static_cast<uint32_t>(page), kvsel, e.n_kv_heads, kh, hd,
                             pos % OPURE_PAGE_SIZE, dk),
                     v, p.yfmt);
    }
}

// A workgroup barrier for data in LDS: each wave waits for its own LDS
// accesses, not for the global loads it has in flight, which __syncthreads
// drains first (a prologue's barrier would then wait for the first weight
// blocks to land before the X staging could go on).
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The staged prologue shared by the kernels.  Issue order: the first X
// staging round, the rows' sums of squares, then `issue` (the first weight
// loads).  Loads retire in issue order, so the staging below waits for L2
// only while the weights stream from HBM.  Then the rows' 1 / rms (NORM), the
// conversion into LDS and any further rounds, `late` (weight loads that may
// use the staging registers), and a barrier.
template <int WF, int AF, bool NORM, int NW, class Issue, class Late>
__device__ __forceinline__ void staged_prologue(const KParams& p, uint8_t* lds, float* sinv, Issue issue, Late late)
{
    constexpr uint32_t NTH = NW * 64;
    constexpr int KR = stage_rows<AF, NORM, NTH>();
    constexpr int RW = (OPURE_MAX_ROWS + NW - 1) / NW;      // columns whose rms a wave computes
    constexpr int SSE = 4;                                  // sums per lane issued early: in <= 4096
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t M = p.M;
    StageRound<AF, NORM, KR> r0;
    stage_issue<AF, NORM, NTH, KR>(p, r0, 0u, 0u);
    float ssp[NORM ? RW : 1][SSE];
    if constexpr (NORM)
    {
#pragma unroll
        for (int i = 0; i < RW; ++i)
        {
            const uint32_t m = wave + i * NW;
            if (m >= M) break;                               // uniform
#pragma unroll
            for (int e = 0; e < SSE; ++e)
            {
                const uint32_t t = min(lane + 64u * e, p.ss_tiles - 1u);
                ssp[i][e] = p.ss_in[static_cast<uint64_t>(t) * M + m];
            }
        }
    }
    issue();
    if constexpr (NORM)
    {
        // one wave per column, the sums in inv_rms_wave's order (adding the
        // early sums of tiles past the end is skipped, not added as zero)
#pragma unroll
        for (int i = 0; i < RW; ++i)
        {
            const uint32_t m = wave + i * NW;
            if (m >= M) break;
            float ssum = 0.0f;
#pragma unroll
            for (int e = 0; e < SSE; ++e)
                if (lane + 64u * e < p.ss_tiles) ssum += ssp[i][e];
            for (uint32_t t = lane + 64u * SSE; t < p.ss_tiles; t += 64u) ssum += p.ss_in[static_cast<uint64_t>(t) * M + m];
            const float v = inv_rms_finish(p, ssum);
            if (lane == 0) sinv[m] = v;
        }
        lds_barrier();
    }
    stage_store<WF, AF, NORM, NTH, KR>(p, r0, 0u, 0u, lds, sinv);
    // further rounds when the rows or the columns exceed one round
    const uint32_t ncol = NORM ? p.in / 4u : p.in / 8u;             // quads or 8-value units
    const uint32_t jstep = NORM ? 2u * NTH : NTH;
    const uint32_t rt = NORM || ncol >= NTH ? 1u : NTH / ncol;
    const uint32_t rows_per = (M + rt - 1u) / rt;
    for (uint32_t j0 = 0; j0 < ncol; j0 += jstep)
        for (uint32_t i0 = 0; i0 < rows_per; i0 += KR)
        {
            if (j0 == 0 && i0 == 0) continue;
            StageRound<AF, NORM, KR> r;
            stage_issue<AF, NORM, NTH, KR>(p, r, j0, i0);
            stage_store<WF, AF, NORM, NTH, KR>(p, r, j0, i0, lds, sinv);
        }
    lds_barrier();
    late();
}

template <int WF, int AF, int T, int U, bool STAGED>
struct Payload {
    u4_t w[T][U];
    uint32_t s[T][U];                                    // uint4: scale | zero << 16 of weight row r16
    u4_t x[STAGED ? 1 : U][Fmt<WF>::N / 4u];             // direct X fragments
};

// X modes of k_gemv: fragments from global memory, staged in LDS, or from
// global memory two blocks a load (at most 8 rows)
constexpr int XM_DIRECT = 0, XM_STAGED = 1, XM_PAIRED = 2;

template <int WF, int AF, int EPI, int NW, int T, int U, bool NORM, int XM>
__global__ __launch_bounds__(NW * 64) void k_gemv(KParams p)
{
    constexpr bool STAGED = XM == XM_STAGED, PAIRED = XM == XM_PAIRED;
    static_assert(!PAIRED || U % 2 == 0, "paired X fragments come two blocks a load");
    constexpr uint32_t KB = Fmt<WF>::KB, N = Fmt<WF>::N;
    constexpr uint32_t EB = AF == OPURE_A_F32 ? 4u : 2u;
    constexpr uint32_t VALS = KB / 4u;                   // k values per lane per block
    constexpr uint32_t PB = U * NW;                      // blocks per pass
    static_assert(STAGED || !NORM, "the fused rmsnorm needs the staged X");
    __shared__ float sinv[OPURE_MAX_ROWS];
    extern __shared__ __align__(16) uint8_t lds[];
    f4_t* red = reinterpret_cast<f4_t*>(lds + p.off_red);

    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t g4 = lane >> 4, r16 = lane & 15u;
    const uint32_t M = p.M;
    const uint32_t mc = r16 < M ? r16 : M - 1u;         // columns >= M compute on a copy of column M-1
    const uint32_t nblk = p.nblk;
    const uint32_t npass = (nblk + PB - 1u) / PB;
    const uint32_t G = p.in / 128u;
    // groups of this workgroup: blockIdx.x, blockIdx.x + gridDim.x, ...  (grid <= groups)
    const uint32_t S = (p.groups - blockIdx.x + gridDim.x - 1u) / gridDim.x * npass;

    using PL = Payload<WF, AF, T, U, STAGED>;
    auto load = [&](PL& b, uint32_t s) {
        const uint32_t gi = s / npass, ps = s - gi * npass;
        const uint32_t grp = blockIdx.x + gi * gridDim.x;
#pragma unroll
        for (int t = 0; t < T; ++t)
        {
            const uint32_t tile = min(grp * T + t, p.tiles - 1u);
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                const uint32_t blk = min(ps * PB + u * NW + wave, nblk - 1u);
                b.w[t][u] = __builtin_nontemporal_load(
                    reinterpret_cast<const u4_t*>(p.w + ((static_cast<uint64_t>(tile) * nblk + blk) << 10) + (lane << 4)));
                if constexpr (WF == OPURE_W_I4G128)
                    b.s[t][u] = static_cast<const uint32_t*>(p.sc)[(static_cast<uint64_t>(tile) * G + blk) * 16u + r16];
            }
        }
        if constexpr (PAIRED)
        {
            // rows 0..7 of lanes r16 < 8 from block u, of lanes r16 >= 8 from block u + 1
            const uint32_t row = min(r16 & 7u, M - 1u), hi = r16 >> 3;
#pragma unroll
            for (int u = 0; u < U; u += 2)
            {
                const uint32_t blk = min(ps * PB + (u + hi) * NW + wave, nblk - 1u);
                const u4_t* src = reinterpret_cast<const u4_t*>(
                    p.x + (static_cast<uint64_t>(row) * p.in + blk * KB + VALS * g4) * EB);
#pragma unroll
                for (uint32_t i = 0; i < N / 4u; ++i) b.x[u][i] = src[i];
            }
        }
        else if constexpr (!STAGED)
        {
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                const uint32_t blk = min(ps * PB + u * NW + wave, nblk - 1u);
                const u4_t* src = reinterpret_cast<const u4_t*>(
                    p.x + (static_cast<uint64_t>(mc) * p.in + blk * KB + VALS * g4) * EB);
#pragma unroll
                for (uint32_t i = 0; i < N / 4u; ++i) b.x[u][i] = src[i];
            }
        }
    };

    PL A, B;
    [[maybe_unused]] PL C;
    if constexpr (STAGED)
    {
        staged_prologue<WF, AF, NORM, NW>(p, lds, sinv, [&] {
            load(A, 0);
            if (S > 1u) load(B, 1);
        }, [&] {
            if (S > 2u) load(C, 2);                         // the staging registers are free now
        });
    }
    else
    {
        load(A, 0);
        if (S > 1u) load(B, 1);
    }

    f4_t acc[T];
    float best_v = -__builtin_huge_valf();
    int32_t best_i = 0x7FFFFFFF;
    auto run = [&](const PL& b, uint32_t s) {
        const uint32_t gi = s / npass, ps = s - gi * npass;
        if (ps == 0)
        {
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            const uint32_t blk = ps * PB + u * NW + wave;
            if (blk >= nblk) continue;
            // X fragment of row mc, k-slice g4 of the block: the A operand
            uint32_t xd[N];
            if constexpr (STAGED)
            {
                const u4_t* src = reinterpret_cast<const u4_t*>(lds + mc * p.x_stride + (blk * KB + VALS * g4) * EB);
#pragma unroll
                for (uint32_t i = 0; i < N / 4u; ++i)
                {
                    const u4_t v = src[i];
                    xd[4 * i] = v[0]; xd[4 * i + 1] = v[1]; xd[4 * i + 2] = v[2]; xd[4 * i + 3] = v[3];
                }
            }
            else if constexpr (PAIRED)
            {
                // even u: the lane's own words; odd u: those of lane r16 + 8 (row rotation by 8)
#pragma unroll
                for (uint32_t i = 0; i < N / 4u; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                    {
                        const uint32_t w = b.x[u & ~1][i][j];
                        xd[4 * i + j] = (u & 1) ? static_cast<uint32_t>(dpp_i<0x128>(static_cast<int32_t>(w))) : w;
                    }
            }
            else
            {
#pragma unroll
                for (uint32_t i = 0; i < N / 4u; ++i)
                {
                    xd[4 * i] = b.x[u][i][0]; xd[4 * i + 1] = b.x[u][i][1];
                    xd[4 * i + 2] = b.x[u][i][2]; xd[4 * i + 3] = b.x[u][i][3];
                }
            }
            if constexpr (WF == OPURE_W_F32)
            {
#pragma unroll
                for (int t = 0; t < T; ++t)
                {
                    const f4_t wf = __builtin_bit_cast(f4_t, b.w[t][u]);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(xd[q]), wf[q], acc[t], 0, 0, 0);
                }
            }
            else if constexpr (WF == OPURE_W_I8PC)
            {
                const half8_t x1 = as_half8(xd[0], xd[1], xd[2], xd[3]);
                const half8_t x2 = as_half8(xd[4], xd[5], xd[6], xd[7]);
#pragma unroll
                for (int t = 0; t < T; ++t)
                {
                    uint32_t a[8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) u8x4_to_f16(b.w[t][u][j], a[2 * j], a[2 * j + 1]);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, as_half8(a[0], a[1], a[2], a[3]), acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x2, as_half8(a[4], a[5], a[6], a[7]), acc[t], 0, 0, 0);
                }
            }
            else
            {
                // one 128-k group per block.  The group sums of X rows 4*g4 + i
                // come from the matrix core too (B = ones), then per tile a
                // fresh accumulator of (MAGIC + q) * x and
                //   acc += (s / MUL) * (bacc - (OFF + MUL z) * xs)   (see U4)
                f4_t xs = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                {
                    if constexpr (AF == OPURE_A_F16)
                        xs = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]),
                                                                    as_half8(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u),
                                                                    xs, 0, 0, 0);
                    else
                        xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]),
                                                                     as_bf8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u),
                                                                     xs, 0, 0, 0);
                }
#pragma unroll
                for (int t = 0; t < T; ++t)
                {
                    f4_t bacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                    {
                        uint32_t a[4];
                        u4x8_pairs<AF>(b.w[t][u][j], a);
                        if constexpr (AF == OPURE_A_F16)
                            bacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                as_half8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]),
                                as_half8(a[0], a[1], a[2], a[3]), bacc, 0, 0, 0);
                        else
                            bacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                as_bf8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]),
                                as_bf8(a[0], a[1], a[2], a[3]), bacc, 0, 0, 0);
                    }
                    float sc, zo;
                    u4_group<AF>(b.s[t][u], sc, zo);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[t][i] = __fmaf_rn(sc, __fmaf_rn(-zo, xs[i], bacc[i]), acc[t][i]);
                }
            }
        }
        if (ps + 1u == npass)
        {
            // the waves' K slices meet in LDS (one buffer per group parity, so
            // one barrier a group: a buffer is written again only after every
            // thread has passed the next group's barrier), then every thread
            // adds its element's partials in wave order and runs its epilogue
            const uint32_t grp = blockIdx.x + gi * gridDim.x;
            f4_t* rb = red + (gi & 1u) * (NW * T * 64u);
#pragma unroll
            for (int t = 0; t < T; ++t) rb[(wave * T + t) * 64u + lane] = acc[t];
            __syncthreads();
#pragma unroll
            for (uint32_t e0 = 0; e0 < T * 256u; e0 += NW * 64u)
            {
                const uint32_t e = e0 + threadIdx.x;
                if (T * 256u % (NW * 64u) != 0 && e >= T * 256u) break;   // whole waves
                const uint32_t t = e >> 8, m = (e >> 4) & 15u, c = e & 15u;
                const uint32_t li = ((m >> 2) << 4) + c, i = m & 3u;
                const float* rf = reinterpret_cast<const float*>(rb);
                float v = rf[((0u * T + t) * 64u + li) * 4u + i];
#pragma unroll
                for (int w = 1; w < NW; ++w) v += rf[((w * T + t) * 64u + li) * 4u + i];
                epilogue_elem<WF, EPI>(p, grp * T + t, m, c, v, best_v, best_i);
            }
        }
    };

    // software pipeline over the steps (group, pass): with staged X three
    // buffers, so the two steps after the one computing are in flight; direct
    // kernels carry X fragments too and keep two.  Loads are issued only for
    // steps that exist, on straight-line paths, so each wait covers exactly
    // the buffer consumed.
    uint32_t s = 0;
    if constexpr (STAGED)
    {
        while (S - s >= 6u)
        {
            run(A, s);
            load(A, s + 3u);
            run(B, s + 1u);
            load(B, s + 4u);
            run(C, s + 2u);
            load(C, s + 5u);
            s += 3u;
        }
        switch (S - s)
        {
        case 5u:
            run(A, s); load(A, s + 3u);
            run(B, s + 1u); load(B, s + 4u);
            run(C, s + 2u); run(A, s + 3u); run(B, s + 4u);
            break;
        case 4u:
            run(A, s); load(A, s + 3u);
            run(B, s + 1u); run(C, s + 2u); run(A, s + 3u);
            break;
        case 3u: run(A, s); run(B, s + 1u); run(C, s + 2u); break;
        case 2u: run(A, s); run(B, s + 1u); break;
        case 1u: run(A, s); break;
        default: break;
        }
    }
    else
    {
        while (S - s >= 4u)
        {
            run(A, s);
            load(A, s + 2u);
            run(B, s + 1u);
            load(B, s + 3u);
            s += 2u;
        }
        switch (S - s)
        {
        case 3u: run(A, s); load(A, s + 2u); run(B, s + 1u); run(A, s + 2u); break;
        case 2u: run(A, s); run(B, s + 1u); break;
        case 1u: run(A, s); break;
        default: break;
        }
    }
    if constexpr (EPI == opure_hip::EPI_LOGITS)
    {
        // one argmax partial per row for the whole workgroup: thread (t, m, 0)
        // holds the best of column t of the tiles it finished (a total order,
        // so any merge order gives the same winner)
        __syncthreads();
        float* sv = reinterpret_cast<float*>(red);
        int32_t* si = reinterpret_cast<int32_t*>(sv + T * 16);
        if (threadIdx.x < T * 256u && (threadIdx.x & 15u) == 0)
        {
            sv[threadIdx.x >> 4] = best_v;
            si[threadIdx.x >> 4] = best_i;
        }
        __syncthreads();
        if (threadIdx.x < M)
        {
            float v = sv[threadIdx.x];
            int32_t i = si[threadIdx.x];
#pragma unroll
            for (int t = 1; t < T; ++t) best_merge(v, i, sv[t * 16 + threadIdx.x], si[t * 16 + threadIdx.x]);
            p.lg.am_val[static_cast<uint64_t>(blockIdx.x) * M + threadIdx.x] = v;
            p.lg.am_idx[static_cast<uint64_t>(blockIdx.x) * M + threadIdx.x] = i;
        }
    }
}

// Wave-per-tile GEMV for shapes with many tiles (1024 and more, so at least
// four per CU): X staged in LDS as in k_gemv, but each wave owns whole tiles --
// tile(k) = blockIdx.x + gridDim.x * (wave + NW * k) -- and runs U consecutive
// blocks per step through a ring of two buffers (one step in flight while
// the other computes), so no wave waits for another between tiles.  A tile's sum is its blocks' in block order.  The
// uint4 group sums of X are computed once per workgroup on the matrix cores
// (the same MFMAs as in k_gemv, so the same bits) into LDS xs[G][16].  At a
// tile's end the wave transposes its accumulator through its own 1 KB of LDS
// and runs the element epilogue on 4 elements a lane: lane (g4, r16) takes
// rows g4 + 4 j, so every DPP row still holds one row m.
// SPLIT = 2 (exactly four tiles a workgroup, at most one a wave): waves w and
// w + 4 take the first and the second half of tile w's blocks, and after the
// stream the second half's sum is added to the first's through LDS (lo + hi),
// so all 8 waves load.
// Greedy acceptance inside the LM head's launch, run by its last-dispatched
// workgroup (512 threads) once every workgroup has published its rows' bests
// as tagged words (acc_slots): per row the best (value, lowest index on ties)
// over the workgroups -- an order-free reduction, so the tokens are
// k_accept_greedy's -- then per sequence the accepted prefix, the emitted
// tokens and the rollback.  Workgroups are dispatched in order, so every word
// it waits for comes from a workgroup already running or finished; the wait is
// bounded (ERR_WAIT).  Every workgroup read this launch's count before
// publishing, so once all words carry it the count moves on.
__device__ inline void greedy_accept_in_launch(const KParams& p, uint32_t M, uint32_t tag, const int32_t* draft,
                                               int32_t* am, const opure_hip::RollbackPre* pre)
{
    constexpr uint32_t NW = 8;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, G = gridDim.x;
    const uint64_t* sl = p.lg.acc_slots;
    bool gave_up = false;
    for (uint32_t r = wave; r < M; r += NW)
    {
        float bv = -__builtin_huge_valf();
        int32_t bi = 0x7FFFFFFF;
        for (uint32_t n = 0;; ++n)
        {
            bv = -__builtin_huge_valf();
            bi = 0x7FFFFFFF;
            bool ok = true;
            for (uint32_t g = lane; g < G; g += 64u)
            {
                const uint64_t* w = sl + (static_cast<uint64_t>(g) * M + r) * 2u;
                const uint64_t wv = __hip_atomic_load(const_cast<uint64_t*>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint64_t wi = __hip_atomic_load(const_cast<uint64_t*>(w) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = ok && (wv >> 32) == tag && (wi >> 32) == tag;
                best_merge(bv, bi, __uint_as_float(static_cast<uint32_t>(wv)), static_cast<int32_t>(static_cast<uint32_t>(wi)));
            }
            if (__all(ok)) break;
            if (n >= p.lg.wait_limit)
            {
                gave_up = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) best_merge(bv, bi, __shfl_xor(bv, o), __shfl_xor(bi, o));
        if (lane == 0u) am[r] = bi == 0x7FFFFFFF ? 0 : bi;
    }
    if (gave_up && lane == 0u && p.err) p.err[ERR_WAIT] = 1u;
    __syncthreads();
    if (threadIdx.x == 0u)
        __hip_atomic_store(p.lg.acc_epoch, tag + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t K = p.lg.K, R = K + 1u;
    for (uint32_t b = 0; b < p.lg.batch; ++b)
    {
        uint32_t n = 0;
        while (n < K && am[b * R + n] == draft[b * K + n]) ++n;
        if (threadIdx.x < R)
            p.lg.out_tokens[b * R + threadIdx.x] =
                threadIdx.x < n ? draft[b * K + threadIdx.x] : (threadIdx.x == n ? am[b * R + n] : -1);
        if (threadIdx.x == 0u) p.lg.accepted[b] = static_cast<int32_t>(n);
        if (p.lg.rollback) opure_hip::rollback_seq(p.lg.rb, b, n, pre[b]);
    }
}

template <int WF, int AF, int EPI, int U, bool NORM, int D, int SPLIT = 1>
__global__ __launch_bounds__(512) void k_gemv_wpt(KParams p)
{
    constexpr int NW = 8;
    constexpr uint32_t TW = NW / SPLIT;                 // waves that own tiles
    constexpr uint32_t KB = Fmt<WF>::KB, N = Fmt<WF>::N;
    constexpr uint32_t EB = AF == OPURE_A_F32 ? 4u : 2u;
    constexpr uint32_t VALS = KB / 4u;
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float sinv[OPURE_MAX_ROWS];
    float* xsl = reinterpret_cast<float*>(lds + p.off_xsum);          // uint4: [G][16]
    float* slot = reinterpret_cast<float*>(lds + p.off_red);          // [NW][64 lanes][4]

    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t g4 = lane >> 4, r16 = lane & 15u;
    const uint32_t M = p.M;
    const uint32_t mc = r16 < M ? r16 : M - 1u;
    const uint32_t nblk = p.nblk;
    const uint32_t part = wave / TW, kblk = nblk / SPLIT, kb0 = part * kblk;   // this wave's blocks [kb0, kb0 + kblk)
    const uint32_t npass = (kblk + U - 1u) / U;
    const uint32_t G = p.in / 128u;
    const uint32_t first = blockIdx.x + gridDim.x * (wave % TW), stride = gridDim.x * TW;
    const uint32_t ntile = first < p.tiles ? (p.tiles - first + stride - 1u) / stride : 0u;
    const uint32_t S = ntile * npass;

    // in-launch greedy acceptance (EPI_LOGITS with acc_slots): this launch's
    // count; the last workgroup also loads the drafts and each sequence's
    // rollback reads, in flight with its weight stream
    __shared__ int32_t acc_draft[OPURE_MAX_ROWS];
    __shared__ int32_t acc_am[OPURE_MAX_ROWS];
    __shared__ opure_hip::RollbackPre acc_pre[OPURE_MAX_ROWS];
    uint32_t acc_tag = 0u;
    bool acc_last = false;
    if constexpr (EPI == opure_hip::EPI_LOGITS)
        if (p.lg.acc_slots)
        {
            acc_tag = __hip_atomic_load(p.lg.acc_epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            acc_last = blockIdx.x == gridDim.x - 1u;
            if (acc_last)
            {
                if (threadIdx.x < p.lg.batch * p.lg.K)
                {
                    const uint32_t b = threadIdx.x / p.lg.K, j = threadIdx.x - b * p.lg.K;
                    acc_draft[threadIdx.x] = p.lg.drafts[static_cast<uint64_t>(b) * p.lg.drafts_stride + j];
                }
                if (p.lg.rollback && threadIdx.x >= 64u && threadIdx.x < 64u + p.lg.batch)
                    acc_pre[threadIdx.x - 64u] = opure_hip::rollback_pre(p.lg.rb, threadIdx.x - 64u);
            }
        }

    struct PL {
        u4_t w[U];
        uint32_t s[U];
    };
    auto load = [&](PL& b, uint32_t s) {
        const uint32_t k = s / npass, ps = s - k * npass;
        const uint32_t tile = min(first + stride * k, p.tiles - 1u);   // a wave with no tile loads the last one
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            const uint32_t blk = kb0 + min(ps * U + u, kblk - 1u);
            b.w[u] = __builtin_nontemporal_load(
                reinterpret_cast<const u4_t*>(p.w + ((static_cast<uint64_t>(tile) * nblk + blk) << 10) + (lane << 4)));
            if constexpr (WF == OPURE_W_I4G128)
                b.s[u] = static_cast<const uint32_t*>(p.sc)[(static_cast<uint64_t>(tile) * G + blk) * 16u + r16];
        }
    };

    // One step's loads are in flight across the staging, the others are
    // issued after it (issuing them all first keeps the waves in the issue
    // queue until most of the stream has landed).  Every prologue load is
    // issued on every path (a wave with fewer steps loads its last again, one
    // with none the last tile): the compiler counts outstanding loads along
    // the path with the fewest, so behind a branch the waits for the staging
    // would also wait for the weights.
    PL buf[D];
    staged_prologue<WF, AF, NORM, NW>(p, lds, sinv, [&] { load(buf[0], 0); }, [&] {
#pragma unroll
        for (int d = 1; d < D; ++d) load(buf[d], min(static_cast<uint32_t>(d), S ? S - 1u : 0u));
    });
    if constexpr (WF == OPURE_W_I4G128)
    {
        // the group sums of X rows 4*g4 + i, block by block over the waves
        for (uint32_t blk = wave; blk < G; blk += NW)
        {
            const u4_t* src = reinterpret_cast<const u4_t*>(lds + mc * p.x_stride + (blk * KB + VALS * g4) * EB);
            f4_t xs = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                const u4_t v = src[j];
                if constexpr (AF == OPURE_A_F16)
                    xs = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(v[0], v[1], v[2], v[3]),
                                                                as_half8(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u),
                                                                xs, 0, 0, 0);
                else
                    xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(v[0], v[1], v[2], v[3]),
                                                                 as_bf8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u),
                                                                 xs, 0, 0, 0);
            }
            if (r16 == 0) *reinterpret_cast<f4_t*>(xsl + blk * 16u + 4u * g4) = xs;
        }
        lds_barrier();
    }

    f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float best_v[4];
    int32_t best_i[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) { best_v[j] = -__builtin_huge_valf(); best_i[j] = 0x7FFFFFFF; }
    float* my = slot + wave * 256u;
    // a tile is done: transpose its sums through this wave's LDS slot, run
    // the element epilogue, start the next tile from zero
    auto finish = [&](uint32_t tile) {
        *reinterpret_cast<f4_t*>(my + lane * 4u) = acc;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const uint32_t m = g4 + 4u * j;
            const float v = my[(((m >> 2) << 4) + r16) * 4u + (m & 3u)];
            epilogue_elem<WF, EPI>(p, tile, m, r16, v, best_v[j], best_i[j]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        acc = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    };
    auto run = [&](const PL& b, uint32_t s) {
        const uint32_t k = s / npass, ps = s - k * npass;
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            if (ps * U + u >= kblk) continue;
            const uint32_t blk = kb0 + ps * U + u;
            uint32_t xd[N];
            const u4_t* src = reinterpret_cast<const u4_t*>(lds + mc * p.x_stride + (blk * KB + VALS * g4) * EB);
#pragma unroll
            for (uint32_t i = 0; i < N / 4u; ++i)
            {
                const u4_t v = src[i];
                xd[4 * i] = v[0]; xd[4 * i + 1] = v[1]; xd[4 * i + 2] = v[2]; xd[4 * i + 3] = v[3];
            }
            if constexpr (WF == OPURE_W_F32)
            {
                const f4_t wf = __builtin_bit_cast(f4_t, b.w[u]);
#pragma unroll
                for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(xd[q]), wf[q], acc, 0, 0, 0);
            }
            else if constexpr (WF == OPURE_W_I8PC)
            {
                uint32_t a[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) u8x4_to_f16(b.w[u][j], a[2 * j], a[2 * j + 1]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(xd[0], xd[1], xd[2], xd[3]), as_half8(a[0], a[1], a[2], a[3]), acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(xd[4], xd[5], xd[6], xd[7]), as_half8(a[4], a[5], a[6], a[7]), acc, 0, 0, 0);
            }
            else
            {
                const f4_t xs = *reinterpret_cast<const f4_t*>(xsl + blk * 16u + 4u * g4);
                f4_t bacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                {
                    uint32_t a[4];
                    u4x8_pairs<AF>(b.w[u][j], a);
                    if constexpr (AF == OPURE_A_F16)
                        bacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]),
                                                                      as_half8(a[0], a[1], a[2], a[3]), bacc, 0, 0, 0);
                    else
                        bacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]),
                                                                       as_bf8(a[0], a[1], a[2], a[3]), bacc, 0, 0, 0);
                }
                float sc, zo;
                u4_group<AF>(b.s[u], sc, zo);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = __fmaf_rn(sc, __fmaf_rn(-zo, xs[i], bacc[i]), acc[i]);
            }
        }
        if (SPLIT == 1 && ps + 1u == npass) finish(first + stride * k);
    };

    // a ring of D buffers: the D - 1 steps after the one computing are in
    // flight.  The steady loop issues every load unconditionally; only the
    // last 2 D steps branch (uniformly) on whether a step exists.
    uint32_t s = 0;
    while (S - s >= 2u * D)
    {
#pragma unroll
        for (int d = 0; d < D; ++d)
        {
            run(buf[d], s + d);
            load(buf[d], s + d + D);
        }
        s += D;
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
    {
        if (s + d >= S) break;
        run(buf[d], s + d);
        if (s + d + D < S) load(buf[d], s + d + D);
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
    {
        if (s + D + d >= S) break;
        run(buf[d], s + D + d);
    }
    if constexpr (SPLIT == 2)
    {
        // the host launches this only with at most one tile a wave (S <= npass);
        // the barrier is outside every branch
        if (part == 1u && S > 0u) *reinterpret_cast<f4_t*>(my + lane * 4u) = acc;
        __syncthreads();
        if (part == 0u && S > 0u)
        {
            const f4_t hi = *reinterpret_cast<const f4_t*>(slot + (wave + TW) * 256u + lane * 4u);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], hi[i]);
            finish(first);
        }
    }

    if constexpr (EPI == opure_hip::EPI_LOGITS)
    {
        // one argmax partial per row for the workgroup: lane (g4, 0) of every
        // wave holds the best of rows g4 + 4 j over its tiles
        __syncthreads();
        float* sv = slot;
        int32_t* si = reinterpret_cast<int32_t*>(slot + NW * 16u);
        if (r16 == 0)
        {
#pragma unroll
            for (int j = 0; j < 4; ++j) { sv[wave * 16u + g4 + 4u * j] = best_v[j]; si[wave * 16u + g4 + 4u * j] = best_i[j]; }
        }
        __syncthreads();
        if (threadIdx.x < M)
        {
            float v = sv[threadIdx.x];
            int32_t i = si[threadIdx.x];
#pragma unroll
            for (int w = 1; w < NW; ++w) best_merge(v, i, sv[w * 16 + threadIdx.x], si[w * 16 + threadIdx.x]);
            if (p.lg.acc_slots)
            {
                uint64_t* w = p.lg.acc_slots + (static_cast<uint64_t>(blockIdx.x) * M + threadIdx.x) * 2u;
                __hip_atomic_store(w, (static_cast<uint64_t>(acc_tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(w + 1, (static_cast<uint64_t>(acc_tag) << 32) | static_cast<uint32_t>(i),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            else
            {
                p.lg.am_val[static_cast<uint64_t>(blockIdx.x) * M + threadIdx.x] = v;
                p.lg.am_idx[static_cast<uint64_t>(blockIdx.x) * M + threadIdx.x] = i;
            }
        }
        if (acc_last) greedy_accept_in_launch(p, M, acc_tag, acc_draft, acc_am, acc_pre);
    }
}


// Wave-per-tile GEMV with loader waves.  Waves 0..7 compute exactly as in
// k_gemv_wpt -- the same tiles, blocks and order of sums, so the same bits --
// but take their weight blocks from LDS.  Waves 8..11 only load: each fills
// a ring of `ring` slots of PC_SB blocks (and their uint4 scale words) for
// two compute waves with global_load_lds_dwordx4, so the weight stream runs
// from the first cycle, across the X staging and while the compute waves
// dequantise; no compute wave ever waits to issue a load.  Hand-off per
// compute wave: an LDS count of its steps filled (written by its loader once
// those steps' loads have landed: loads retire in issue order, s_waitcnt
// vmcnt) and of its steps consumed (written once the compute wave holds the
// slot's words in registers).  Every wait is a bounded sleep loop; a wave
// that gives up stops waiting (its results are then wrong) but still reaches
// every barrier, so the grid always drains, and reports it (ERR_WAIT), so the
// host's next sync returns an error instead of the wrong results.  The number
// of sleeps before giving up is KParams::wait_limit (opure_dev::wait_limit).
constexpr int PC_NC = 8, PC_NL = 4;                   // compute and loader waves
constexpr uint32_t PC_SB = 4;                          // blocks a slot

template <int WF>
constexpr uint32_t pc_slot_bytes() { return PC_SB * 1024u + (WF == OPURE_W_I4G128 ? 256u : 0u); }

// the hand-off counts, as LDS pointers (ds_read / ds_write: a flat access
// would count in vmcnt and make every poll wait for the loader's loads)
typedef __attribute__((address_space(3))) volatile uint32_t lds_u32;

// wait until *f >= want (a count another wave raises); false if given up
__device__ __forceinline__ bool pc_wait(const lds_u32* f, uint32_t want, uint32_t limit, bool& bail)
{
    if (bail) return false;
    // every lane reads the same count: take lane 0's, so the loop is scalar
    for (uint32_t n = 0; static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(*f))) < want; ++n)
    {
        if (n >= limit)
        {
            bail = true;
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

template <int WF, int AF, int EPI, bool NORM>
__global__ __launch_bounds__((PC_NC + PC_NL) * 64) void k_gemv_pc(KParams p)
{
    constexpr int NW = PC_NC;
    constexpr uint32_t KB = Fmt<WF>::KB, N = Fmt<WF>::N, SB = PC_SB, SLOT = pc_slot_bytes<WF>();
    constexpr uint32_t EB = AF == OPURE_A_F32 ? 4u : 2u;
    constexpr uint32_t VALS = KB / 4u;
    constexpr int NBAR = (NORM ? 1 : 0) + 1 + (WF == OPURE_W_I4G128 ? 1 : 0);   // compute waves' prologue barriers
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float sinv[OPURE_MAX_ROWS];
    float* xsl = reinterpret_cast<float*>(lds + p.off_xsum);          // uint4: [G][16]
    float* slotb = reinterpret_cast<float*>(lds + p.off_red);         // [NW][64 lanes][4]
    lds_u32* filled = (lds_u32*)(lds + p.off_ring + NW * p.ring * SLOT);
    lds_u32* consumed = filled + NW;

    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t g4 = lane >> 4, r16 = lane & 15u;
    const uint32_t M = p.M;
    const uint32_t nblk = p.nblk, npass = nblk / SB, R = p.ring;
    const uint32_t G = p.in / 128u;
    const uint32_t stride = gridDim.x * NW;
    auto first_of = [&](uint32_t c) { return blockIdx.x + gridDim.x * c; };
    auto steps_of = [&](uint32_t c) {
        const uint32_t f = first_of(c);
        return f < p.tiles ? (p.tiles - f + stride - 1u) / stride * npass : 0u;
    };
    if (threadIdx.x < 2u * NW) filled[threadIdx.x] = 0u;     // filled[0..7], consumed[0..7]
    __syncthreads();
    bool bail = false;

    if (wave >= static_cast<uint32_t>(NW))
    {
        // ---- loader wave: compute waves c0 = l, c1 = l + 4 (waves of the low
        // indices are the ones that have tiles when there are few) ---------------
        const uint32_t l = wave - NW, c0 = l, c1 = l + static_cast<uint32_t>(PC_NL);
        const uint32_t S0 = steps_of(c0), S1 = steps_of(c1), Smax = S0 > S1 ? S0 : S1;
        auto issue = [&](uint32_t c, uint32_t s) {
            const uint32_t k = s / npass, ps = s - k * npass;
            const uint32_t tile = first_of(c) + stride * k;
            uint8_t* base = lds + p.off_ring + (c * R + s % R) * SLOT;
#pragma unroll
            for (uint32_t u = 0; u < SB; ++u)
                __builtin_amdgcn_global_load_lds(
                    p.w + ((static_cast<uint64_t>(tile) * nblk + ps * SB + u) << 10) + (lane << 4),
                    (__attribute__((address_space(3))) void*)(base + u * 1024u), 16, 0, 0);
            if constexpr (WF == OPURE_W_I4G128)
                __builtin_amdgcn_global_load_lds(
                    static_cast<const uint32_t*>(p.sc) + (static_cast<uint64_t>(tile) * G + ps * SB) * 16u + lane,
                    (__attribute__((address_space(3))) void*)(base + SB * 1024u), 4, 0, 0);
        };
        // The compute waves' prologue barriers.  The first is met before any
        // weight load is issued: the compute waves' X has landed by then, and
        // weights issued earlier queue with the X loads in the CU's memory
        // pipeline and hold the prologue back.  The others are joined with
        // bare s_barrier: a loader publishes nothing through them (its
        // hand-off is the LDS counts), and __syncthreads would first wait for
        // every load it has in flight.
        __builtin_amdgcn_s_barrier();
        bool joined = false;
        auto join = [&] {
#pragma unroll
            for (int i = 1; i < NBAR; ++i) __builtin_amdgcn_s_barrier();
            joined = true;
        };
        // Steps are signalled R - 1 iterations behind the issue: after issuing
        // step s, the loads of the last R - 1 iterations may stay in flight
        // (loads retire in order), so steps <= s - R + 1 have landed.  A slot
        // is taken back for step s once step s - R is consumed, which only
        // needs steps signalled up to s - R: no wait can deadlock.
        constexpr uint32_t L = SB + (WF == OPURE_W_I4G128 ? 1u : 0u);   // loads a wave-step
        uint32_t n_prev = 0;                                             // waves issued an iteration ago
        for (uint32_t s = 0; s < Smax; ++s)
        {
            // the compute waves take slots only after their prologue: join it
            // before the first wait on a slot
            if (s == R && !joined) join();
            const bool i0 = s < S0, i1 = s < S1;
            if (i0)
            {
                if (s >= R) pc_wait(consumed + c0, s - R + 1u, p.wait_limit, bail);
                issue(c0, s);
            }
            if (i1)
            {
                if (s >= R) pc_wait(consumed + c1, s - R + 1u, p.wait_limit, bail);
                issue(c1, s);
            }
            const uint32_t n_cur = (i0 ? 1u : 0u) + (i1 ? 1u : 0u);
            const uint32_t keep = R >= 3u ? n_prev + n_cur : n_cur;      // iterations' loads left in flight
            if (keep >= 4u) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4u * L) : "memory");
            else if (keep == 3u) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3u * L) : "memory");
            else if (keep == 2u) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2u * L) : "memory");
            else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L) : "memory");
            n_prev = n_cur;
            const uint32_t lag = R >= 3u ? 2u : 1u;
            const uint32_t ready = s + 1u >= lag ? s + 1u - lag : 0u;   // steps landed
            if (lane == 0u)
            {
                filled[c0] = ready < S0 ? ready : S0;
                filled[c1] = ready < S1 ? ready : S1;
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0u)
        {
            filled[c0] = S0;
            filled[c1] = S1;
            if (bail && p.err) p.err[ERR_WAIT] = 1u;
        }
        if (!joined) join();
        if constexpr (EPI == opure_hip::EPI_LOGITS)
        {
            __syncthreads();
            __syncthreads();
        }
        return;
    }

    // ---- compute wave ------------------------------------------------------
    const uint32_t mc = r16 < M ? r16 : M - 1u;
    const uint32_t first = first_of(wave);
    const uint32_t S = steps_of(wave);
    staged_prologue<WF, AF, NORM, NW>(p, lds, sinv, [] {}, [] {});
    if constexpr (WF == OPURE_W_I4G128)
    {
        for (uint32_t blk = wave; blk < G; blk += NW)
        {
            const u4_t* src = reinterpret_cast<const u4_t*>(lds + mc * p.x_stride + (blk * KB + VALS * g4) * EB);
            f4_t xs = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                const u4_t v = src[j];
                if constexpr (AF == OPURE_A_F16)
                    xs = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(v[0], v[1], v[2], v[3]),
                                                                as_half8(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u),
                                                                xs, 0, 0, 0);
                else
                    xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(v[0], v[1], v[2], v[3]),
                                                                 as_bf8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u),
                                                                 xs, 0, 0, 0);
            }
            if (r16 == 0) *reinterpret_cast<f4_t*>(xsl + blk * 16u + 4u * g4) = xs;
        }
        lds_barrier();
    }

    f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float best_v[4];
    int32_t best_i[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) { best_v[j] = -__builtin_huge_valf(); best_i[j] = 0x7FFFFFFF; }
    float* my = slotb + wave * 256u;
    for (uint32_t s = 0; s < S; ++s)
    {
        const uint32_t k = s / npass, ps = s - k * npass;
        pc_wait(filled + wave, s + 1u, p.wait_limit, bail);
        const uint8_t* base = lds + p.off_ring + (wave * R + s % R) * SLOT;
        u4_t w[SB];
        uint32_t sz[SB];
#pragma unroll
        for (uint32_t u = 0; u < SB; ++u)
        {
            w[u] = *reinterpret_cast<const u4_t*>(base + u * 1024u + (lane << 4));
            if constexpr (WF == OPURE_W_I4G128) sz[u] = reinterpret_cast<const uint32_t*>(base + SB * 1024u)[u * 16u + r16];
        }
        // the slot's words are in registers: hand the slot back
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0u) consumed[wave] = s + 1u;
#pragma unroll
        for (uint32_t u = 0; u < SB; ++u)
        {
            const uint32_t blk = ps * SB + u;
            uint32_t xd[N];
            const u4_t* src = reinterpret_cast<const u4_t*>(lds + mc * p.x_stride + (blk * KB + VALS * g4) * EB);
#pragma unroll
            for (uint32_t i = 0; i < N / 4u; ++i)
            {
                const u4_t v = src[i];
                xd[4 * i] = v[0]; xd[4 * i + 1] = v[1]; xd[4 * i + 2] = v[2]; xd[4 * i + 3] = v[3];
            }
            if constexpr (WF == OPURE_W_I8PC)
            {
                uint32_t a[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) u8x4_to_f16(w[u][j], a[2 * j], a[2 * j + 1]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(xd[0], xd[1], xd[2], xd[3]), as_half8(a[0], a[1], a[2], a[3]), acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(xd[4], xd[5], xd[6], xd[7]), as_half8(a[4], a[5], a[6], a[7]), acc, 0, 0, 0);
            }
            else
            {
                const f4_t xs = *reinterpret_cast<const f4_t*>(xsl + blk * 16u + 4u * g4);
                f4_t bacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                {
                    uint32_t a[4];
                    u4x8_pairs<AF>(w[u][j], a);
                    if constexpr (AF == OPURE_A_F16)
                        bacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]),
                                                                      as_half8(a[0], a[1], a[2], a[3]), bacc, 0, 0, 0);
                    else
                        bacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xd[4 * j], xd[4 * j + 1], xd[4 * j + 2], xd[4 * j + 3]),
                                                                       as_bf8(a[0], a[1], a[2], a[3]), bacc, 0, 0, 0);
                }
                float sc, zo;
                u4_group<AF>(sz[u], sc, zo);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = __fmaf_rn(sc, __fmaf_rn(-zo, xs[i], bacc[i]), acc[i]);
            }
        }
        if (ps + 1u == npass)
        {
            const uint32_t tile = first + stride * k;
            *reinterpret_cast<f4_t*>(my + lane * 4u) = acc;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                const uint32_t m = g4 + 4u * j;
                const float v = my[(((m >> 2) << 4) + r16) * 4u + (m & 3u)];
                epilogue_elem<WF, EPI>(p, tile, m, r16, v, best_v[j], best_i[j]);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            acc = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    if (bail && lane == 0u && p.err) p.err[ERR_WAIT] = 1u;

    if constexpr (EPI == opure_hip::EPI_LOGITS)
    {
        __syncthreads();
        float* sv = slotb;
        int32_t* si = reinterpret_cast<int32_t*>(slotb + NW * 16u);
        if (r16 == 0)
        {
#pragma unroll
            for (int j = 0; j < 4; ++j) { sv[wave * 16u + g4 + 4u * j] = best_v[j]; si[wave * 16u + g4 + 4u * j] = best_i[j]; }
        }
        __syncthreads();
        if (threadIdx.x < M)
        {
            float v = sv[threadIdx.x];
            int32_t i = si[threadIdx.x];
#pragma unroll
            for (int w = 1; w < NW; ++w) best_merge(v, i, sv[w * 16 + threadIdx.x], si[w * 16 + threadIdx.x]);
            p.lg.am_val[static_cast<uint64_t>(blockIdx.x) * M + threadIdx.x] = v;
            p.lg.am_idx[static_cast<uint64_t>(blockIdx.x) * M + threadIdx.x] = i;
        }
    }
}

// Vector-ALU GEMV, the other side of the engine choice (opure_debug_set_gemv_engine):
// M <= 8 rows, no fused rmsnorm; fp32 weights with fp32 X (v_fma_f32), int8
// with fp16 X (v_dot2_f32_f16), uint4 g128 with fp16 or bf16 X (v_dot2_f32_f16
// / v_dot2_f32_bf16 on the same operand pairs as the matrix-core path, the
// group's scale and zero point applied to the lane's partial through the
// lane's sum of X, see U4).  One workgroup of 16 waves per tile, K split over
// the waves as in k_gemv (wave w takes blocks w, w + 16, ...).  Lane (g4, r16)
// holds its k-slice of row r16 in each block (4 fp32, 16 int8 or 32 uint4),
// widens it once and takes it against the same k values of every X row, so
// each X fragment feeds one output row per lane where the matrix core feeds
// 16.  The 4 lanes of a row add by butterfly, the waves in wave order through
// LDS; then the element epilogue.  Sums are ordered differently from the
// matrix-core path (results agree to rounding).
constexpr uint32_t VALU_NW = 16, VALU_MAXM = 8;

template <int WF, int AF, int EPI>
__global__ __launch_bounds__(VALU_NW * 64) void k_gemv_valu(KParams p)
{
    constexpr uint32_t KB = Fmt<WF>::KB;                 // k values per block
    constexpr uint32_t VALS = KB / 4u;                   // k values per lane per block
    constexpr uint32_t EB = AF == OPURE_A_F32 ? 4u : 2u;
    constexpr uint32_t XW = VALS * EB / 4u;              // X dwords per lane per block and row
    __shared__ float red[VALU_NW][VALU_MAXM][16];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t g4 = lane >> 4, r16 = lane & 15u;
    const uint32_t tile = blockIdx.x, nblk = p.nblk, M = p.M, G = p.in / 128u;
    float acc[VALU_MAXM];
#pragma unroll
    for (uint32_t m = 0; m < VALU_MAXM; ++m) acc[m] = 0.0f;
    const u4_t* wp = reinterpret_cast<const u4_t*>(p.w + (static_cast<uint64_t>(tile) * nblk << 10) + (lane << 4));
    const uint32_t* sp = static_cast<const uint32_t*>(p.sc) + static_cast<uint64_t>(tile) * G * 16u + r16;
    const uint32_t b0 = min(wave, nblk - 1u);
    u4_t wn = __builtin_nontemporal_load(wp + 64u * b0);
    uint32_t sn = WF == OPURE_W_I4G128 ? sp[16u * b0] : 0u;
    for (uint32_t blk = wave; blk < nblk; blk += VALU_NW)
    {
        const u4_t w = wn;
        const uint32_t sz = sn;
        if (blk + VALU_NW < nblk)
        {
            wn = __builtin_nontemporal_load(wp + 64u * (blk + VALU_NW));
            if constexpr (WF == OPURE_W_I4G128) sn = sp[16u * (blk + VALU_NW)];
        }
        // the widened weights of the lane's k-slice
        [[maybe_unused]] uint32_t wh[WF == OPURE_W_I4G128 ? 16 : 8];
        if constexpr (WF == OPURE_W_I8PC)
        {
#pragma unroll
            for (int j = 0; j < 4; ++j) u8x4_to_f16(w[j], wh[2 * j], wh[2 * j + 1]);
        }
        else if constexpr (WF == OPURE_W_I4G128)
        {
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                uint32_t a[4];
                u4x8_pairs<AF>(w[j], a);
#pragma unroll
                for (int t = 0; t < 4; ++t) wh[4 * j + t] = a[t];
            }
        }
        [[maybe_unused]] float sc = 0.0f, zo = 0.0f;
        if constexpr (WF == OPURE_W_I4G128) u4_group<AF>(sz, sc, zo);
#pragma unroll
        for (uint32_t m = 0; m < VALU_MAXM; ++m)
        {
            if (m >= M) break;                               // uniform
            const u4_t* xr = reinterpret_cast<const u4_t*>(p.x + (static_cast<uint64_t>(m) * p.in + KB * blk + VALS * g4) * EB);
            uint32_t xd[XW];
#pragma unroll
            for (uint32_t i = 0; i < XW / 4u; ++i)
            {
                const u4_t v = xr[i];
                xd[4 * i] = v[0]; xd[4 * i + 1] = v[1]; xd[4 * i + 2] = v[2]; xd[4 * i + 3] = v[3];
            }
            if constexpr (WF == OPURE_W_F32)
            {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[m] = __fmaf_rn(__uint_as_float(w[i]), __uint_as_float(xd[i]), acc[m]);
            }
            else if constexpr (WF == OPURE_W_I8PC)
            {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    acc[m] = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, wh[j]), __builtin_bit_cast(half2_t, xd[j]),
                                                    acc[m], false);
            }
            else
            {
                float b = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j)
                {
                    if constexpr (AF == OPURE_A_F16)
                        b = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, wh[j]), __builtin_bit_cast(half2_t, xd[j]), b,
                                                   false);
                    else
                        b = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wh[j]),
                                                            __builtin_bit_cast(bf16x2_t, xd[j]), b, false);
                }
                const float xs = __fadd_rn(__fadd_rn(unit_sum<AF>(xd[0], xd[1], xd[2], xd[3]),
                                                     unit_sum<AF>(xd[4], xd[5], xd[6], xd[7])),
                                           __fadd_rn(unit_sum<AF>(xd[8], xd[9], xd[10], xd[11]),
                                                     unit_sum<AF>(xd[12], xd[13], xd[14], xd[15])));
                acc[m] = __fmaf_rn(sc, __fmaf_rn(-zo, xs, b), acc[m]);
            }
        }
    }
#pragma unroll
    for (uint32_t m = 0; m < VALU_MAXM; ++m)
    {
        acc[m] = __fadd_rn(acc[m], __shfl_xor(acc[m], 16));
        acc[m] = __fadd_rn(acc[m], __shfl_xor(acc[m], 32));
    }
    if (g4 == 0)
    {
#pragma unroll
        for (uint32_t m = 0; m < VALU_MAXM; ++m) red[wave][m][r16] = acc[m];
    }
    __syncthreads();
    if (threadIdx.x < 16u * M)
    {
        const uint32_t m = threadIdx.x >> 4, c = threadIdx.x & 15u;
        float v = red[0][m][c];
#pragma unroll
        for (uint32_t w = 1; w < VALU_NW; ++w) v = __fadd_rn(v, red[w][m][c]);
        float bv = 0.0f;
        int32_t bi = 0;
        epilogue_elem<WF, EPI>(p, tile, m, c, v, bv, bi);
    }
}

template <int WF, int AF>
int launch_valu(opure_dev* dev, uint32_t epi, const KParams& kp)
{
    switch (epi)
    {
    case opure_hip::EPI_STORE:
        OPURE_LAUNCH(dev, (k_gemv_valu<WF, AF, opure_hip::EPI_STORE>), dim3(kp.tiles), dim3(VALU_NW * 64), 0, kp);
        break;
    case opure_hip::EPI_RESIDUAL:
        OPURE_LAUNCH(dev, (k_gemv_valu<WF, AF, opure_hip::EPI_RESIDUAL>), dim3(kp.tiles), dim3(VALU_NW * 64), 0, kp);
        break;
    case opure_hip::EPI_SWIGLU:
        OPURE_LAUNCH(dev, (k_gemv_valu<WF, AF, opure_hip::EPI_SWIGLU>), dim3(kp.tiles), dim3(VALU_NW * 64), 0, kp);
        break;
    default: return opure_hip::set_error(OPURE_E_INVALID, "gemv: the vector-ALU engine has no epilogue %u", epi);
    }
    OPURE_LAUNCH_CHECK("k_gemv_valu");
    return OPURE_OK;
}

template <int WF, int AF, int EPI, bool NORM>
int launch_pc(opure_dev* dev, const KParams& kp, uint32_t grid, uint32_t lds)
{
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_pc<WF, AF, EPI, NORM>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 159 * 1024));
        configured = true;
    }
    OPURE_LAUNCH(dev, (k_gemv_pc<WF, AF, EPI, NORM>), dim3(grid), dim3((PC_NC + PC_NL) * 64), lds, kp);
    OPURE_LAUNCH_CHECK("k_gemv_pc");
    return OPURE_OK;
}

// A ring of two steps.  Three kept one more step a wave queued behind the
// stream, and where a wave has only two steps (SPLIT 2: the 1B gate/up, 16 of
// a tile's 32 blocks, 8 a step) the prologue, which fills every slot, loaded
// the second step twice: two instead of three measured C3 0.6713 -> 0.6487 ms
// (gate/up 11.7 -> 10.2 us), then the LM heads 0.2-0.6 % faster (C3, C1).
// Whole-tile waves (the LM heads) take 4 blocks a step, 4 KB in flight a wave
// (8 blocks: C3 0.647 -> 0.646 ms, C4 2.164 -> 2.154 ms; 2 blocks or a ring
// of three slower); the split tiles keep 8 (4: C3 0.645 -> 0.650 ms).
template <int WF, int AF, int EPI, int U, bool NORM, int SPLIT = 1>
int launch_wpt(opure_dev* dev, const KParams& kp, uint32_t grid, uint32_t lds)
{
    constexpr int D = 2;
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_wpt<WF, AF, EPI, U, NORM, D, SPLIT>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 159 * 1024));
        configured = true;
    }
    OPURE_LAUNCH(dev, (k_gemv_wpt<WF, AF, EPI, U, NORM, D, SPLIT>), dim3(grid), dim3(512), lds, kp);
    OPURE_LAUNCH_CHECK("k_gemv_wpt");
    return OPURE_OK;
}

// Launch one instantiation.  grid = workgroups; lds = dynamic LDS bytes.
template <int WF, int AF, int EPI, int NW, int T, int U, bool NORM, int XM>
int launch(opure_dev* dev, const KParams& kp, uint32_t grid, uint32_t lds)
{
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<WF, AF, EPI, NW, T, U, NORM, XM>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 159 * 1024));
        configured = true;
    }
    OPURE_LAUNCH(dev, (k_gemv<WF, AF, EPI, NW, T, U, NORM, XM>), dim3(grid), dim3(NW * 64), lds, kp);
    OPURE_LAUNCH_CHECK("k_gemv");
    return OPURE_OK;
}

// The shape recipes the host chooses from (waves, tiles per workgroup, blocks
// per wave per pass of the staged kernel).  One workgroup per CU, persistent:
// each CU stages X once, and a pass of 32 blocks per tile covers a whole
// 4096-long row (int4) so a workgroup's first one or two groups are in flight
// from its start.
struct Recipe { uint32_t nw, t, u, wpt = 0; };
constexpr Recipe R_WPT{8, 1, 4, 1};   // at least four tiles per wave: waves own whole tiles (staged X)
constexpr Recipe R_WIDE{8, 2, 4};     // many tiles: 2 tiles share each X fragment
constexpr Recipe R_WIDE16{16, 2, 2};  // 320 to 1023 tiles: 2 tiles a group on 16 waves
constexpr Recipe R_MID{8, 1, 4};      // about one tile per CU, rows of 8192 or more: 8 waves (paired X)
constexpr Recipe R_NARROW{16, 1, 2};  // up to about one tile per CU: 16 waves split K (more loads
                                      // in flight per CU than 8)

// Blocks go to waves by index (wave w takes w, w+NW, ...) whatever T and U
// are, so the sums depend on NW alone.
// Direct kernels carry X fragments and keep U small (8 waves: 2, so the
// 112 blocks of a 14336-long row fill whole passes; 16 waves: 1, to stay
// within 128 VGPRs).
template <int WF, int AF, int EPI, bool NORM, bool STAGED>
int launch_recipe(opure_dev* dev, const KParams& kp, const Recipe& r, uint32_t grid, uint32_t lds)
{
    if constexpr (STAGED)
    {
        if constexpr (WF != OPURE_W_F32 && AF != OPURE_A_F32)
        {
            if (r.wpt == 2) return launch_pc<WF, AF, EPI, NORM>(dev, kp, grid, lds);
            if (r.wpt == 4) return launch_wpt<WF, AF, EPI, 8, NORM, 2>(dev, kp, grid, lds);
        }
        if (r.wpt) return launch_wpt<WF, AF, EPI, 4, NORM>(dev, kp, grid, lds);
        if (r.nw == 16 && r.t == 2) return launch<WF, AF, EPI, 16, 2, 2, NORM, XM_STAGED>(dev, kp, grid, lds);
        if (r.nw == 8 && r.t == 2) return launch<WF, AF, EPI, 8, 2, 4, NORM, XM_STAGED>(dev, kp, grid, lds);
        if (r.nw == 8) return launch<WF, AF, EPI, 8, 1, 4, NORM, XM_STAGED>(dev, kp, grid, lds);
        return launch<WF, AF, EPI, 16, 1, 2, NORM, XM_STAGED>(dev, kp, grid, lds);
    }
    else
    {
        // same blocks per wave, so the same sums, paired or not
        const bool paired = kp.M <= 8u;
        if (r.nw == 16 && r.t == 2) return launch<WF, AF, EPI, 16, 2, 1, NORM, XM_DIRECT>(dev, kp, grid, lds);
        if (r.nw == 8 && r.t == 2)
            return paired ? launch<WF, AF, EPI, 8, 2, 2, NORM, XM_PAIRED>(dev, kp, grid, lds)
                          : launch<WF, AF, EPI, 8, 2, 2, NORM, XM_DIRECT>(dev, kp, grid, lds);
        if (r.nw == 8)
            return paired ? launch<WF, AF, EPI, 8, 1, 2, NORM, XM_PAIRED>(dev, kp, grid, lds)
                          : launch<WF, AF, EPI, 8, 1, 2, NORM, XM_DIRECT>(dev, kp, grid, lds);
        return launch<WF, AF, EPI, 16, 1, 1, NORM, XM_DIRECT>(dev, kp, grid, lds);
    }
}

// every (epilogue, rmsnorm, staged) combination the host may ask for; nm 1:
// the rmsnorm is fused into the staging, 0: X is used as it is (a rmsnorm'd
// X comes from the rows pass)
template <int WF, int AF>
int launch_format(opure_dev* dev, uint32_t epi, uint32_t nm, bool staged, const KParams& kp, const Recipe& r,
                  uint32_t grid, uint32_t lds)
{
    using namespace opure_hip;
    if (nm == 1)
    {
        switch (epi)
        {
        case EPI_SWIGLU: return launch_recipe<WF, AF, EPI_SWIGLU, true, true>(dev, kp, r, grid, lds);
        case EPI_QKV: return launch_recipe<WF, AF, EPI_QKV, true, true>(dev, kp, r, grid, lds);
        case EPI_LOGITS: return launch_recipe<WF, AF, EPI_LOGITS, true, true>(dev, kp, r, grid, lds);
        }
    }
    else if (staged)
    {
        switch (epi)
        {
        case EPI_STORE: return launch_recipe<WF, AF, EPI_STORE, false, true>(dev, kp, r, grid, lds);
        case EPI_RESIDUAL: return launch_recipe<WF, AF, EPI_RESIDUAL, false, true>(dev, kp, r, grid, lds);
        case EPI_SWIGLU: return launch_recipe<WF, AF, EPI_SWIGLU, false, true>(dev, kp, r, grid, lds);
        case EPI_QKV: return launch_recipe<WF, AF, EPI_QKV, false, true>(dev, kp, r, grid, lds);
        case EPI_LOGITS: return launch_recipe<WF, AF, EPI_LOGITS, false, true>(dev, kp, r, grid, lds);
        }
    }
    else
    {
        switch (epi)
        {
        case EPI_STORE: return launch_recipe<WF, AF, EPI_STORE, false, false>(dev, kp, r, grid, lds);
        case EPI_RESIDUAL: return launch_recipe<WF, AF, EPI_RESIDUAL, false, false>(dev, kp, r, grid, lds);
        case EPI_SWIGLU: return launch_recipe<WF, AF, EPI_SWIGLU, false, false>(dev, kp, r, grid, lds);
        case EPI_QKV: return launch_recipe<WF, AF, EPI_QKV, false, false>(dev, kp, r, grid, lds);
        case EPI_LOGITS: return launch_recipe<WF, AF, EPI_LOGITS, false, false>(dev, kp, r, grid, lds);
        }
    }
    return set_error(OPURE_E_INVALID, "gemv: epilogue %u (rmsnorm %u, staged %d) is not built", epi, nm, staged);
}

}  // namespace opure_gemv
