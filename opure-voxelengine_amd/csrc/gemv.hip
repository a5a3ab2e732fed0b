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
//  (M padded to 16 with zeros).  One workgroup owns one tile; its NW waves
//  take interleaved 64-byte blocks of every row (so together they stream
//  contiguous 64*NW-byte runs) and are combined through LDS in wave order.
//  Lane l loads 16 contiguous weight bytes of row (l % 16) per block with a
//  128-bit load, and its X fragment straight from L2.  Weights are widened in
//  registers:
//    f32   -> v_mfma_f32_16x16x4_f32, 4 MFMAs per 16-byte load
//    int8  -> fp16 via the 1024+u exponent trick (exact), 2 x 16x16x32 f16
//    uint4 -> fp16/bf16 via the same trick, 4 x 16x16x32 per 128-k group,
//             the group's scale/zero applied to the fresh group accumulator
//  No workgroup talks to another (a device-scope fence on a multi-XCD part
//  writes back and invalidates L2, which cost 10-20x in a split-K version), so
//  results are bitwise reproducible and independent of M.
// ============================================================================
#include "internal.h"

using namespace opure_dev_math;

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
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

// 8 nibbles (element 2i in the high nibble of byte i) -> 4 pairs MAGIC|q.
// fp16 MAGIC 0x6400 = 1024 (subtracted exactly afterwards); bf16 0x4300 = 128
// (folded into the zero point, since bf16 cannot hold 128+q minus 128 packed).
template <int AF>
__device__ __forceinline__ void u4x8_to_pairs(uint32_t d, uint32_t (&o)[4])
{
    const uint32_t L = d & 0x0F0F0F0Fu;
    const uint32_t H = (d >> 4) & 0x0F0F0F0Fu;
    constexpr uint32_t MAGIC = AF == OPURE_A_F16 ? 0x64006400u : 0x43004300u;
    o[0] = __builtin_amdgcn_perm(H, L, 0x0C000C04u) | MAGIC;
    o[1] = __builtin_amdgcn_perm(H, L, 0x0C010C05u) | MAGIC;
    o[2] = __builtin_amdgcn_perm(H, L, 0x0C020C06u) | MAGIC;
    o[3] = __builtin_amdgcn_perm(H, L, 0x0C030C07u) | MAGIC;
    if constexpr (AF == OPURE_A_F16)
    {
        const half2_t bias = {static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, o[j]) + bias);
    }
}

template <int WF, int AF, int EPI, int NW>
__global__ __launch_bounds__(NW * 64) void k_gemv(KParams p)
{
    using T = WTraits<WF>;
    constexpr uint32_t EBX = AF == OPURE_A_F32 ? 4u : 2u;
    constexpr uint32_t U = 8;                       // blocks in flight per lane
    __shared__ f4_t red[NW][64];
    // uint4 only: this tile's 16 rows x G groups of (scale, zero + bias)
    extern __shared__ __align__(16) float sz[];

    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t g4 = lane >> 4, r16 = lane & 15u;
    const uint32_t tile = blockIdx.x;
    const uint32_t M = p.M;
    const uint32_t G = p.in / 128u;

    if constexpr (WF == OPURE_W_I4G128)
    {
        for (uint32_t e = threadIdx.x; e < 16u * G; e += NW * 64u)
        {
            const uint32_t r = e / G, g = e - r * G;
            const uint64_t gi = static_cast<uint64_t>(weight_row(EPI, tile, r, p.out)) * G + g;
            float z = bf16_to_f32(static_cast<const uint16_t*>(p.zero)[gi]);
            if constexpr (AF == OPURE_A_BF16) z += 128.0f;
            sz[(r * G + g) * 2u] = bf16_to_f32(static_cast<const uint16_t*>(p.scale)[gi]);
            sz[(r * G + g) * 2u + 1u] = z;
        }
        __syncthreads();
    }

    // ---- stream 16 weight rows; wave w takes blocks w, w+NW, ... of K -------
    constexpr uint32_t WBITS = WF == OPURE_W_F32 ? 32u : (WF == OPURE_W_I8PC ? 8u : 4u);
    const uint64_t w_row_bytes = static_cast<uint64_t>(p.in) * WBITS / 8u;
    const uint8_t* wp = p.w + weight_row(EPI, tile, r16, p.out) * w_row_bytes + 16u * g4;
    const bool xon = r16 < M;
    const uint8_t* xrow = p.x + static_cast<uint64_t>(xon ? r16 : 0u) * p.in * EBX;
    const uint32_t nblk = p.in / T::KB;
    f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t b0 = wave; b0 < nblk; b0 += U * NW)
    {
        u4_t wv[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u)
            if (b0 + u * NW < nblk) wv[u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(wp + (b0 + u * NW) * 64u));
#pragma unroll
        for (uint32_t u = 0; u < U; ++u)
        {
            const uint32_t blk = b0 + u * NW;
            if (blk >= nblk) break;
            const uint32_t kb = blk * T::KB;
            if constexpr (WF == OPURE_W_F32)
            {
                f4_t xv = {0.0f, 0.0f, 0.0f, 0.0f};
                if (xon) xv = *reinterpret_cast<const f4_t*>(xrow + (kb + 4u * g4) * 4u);
                const f4_t wf = __builtin_bit_cast(f4_t, wv[u]);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wf[t], xv[t], acc, 0, 0, 0);
            }
            else if constexpr (WF == OPURE_W_I8PC)
            {
                u4_t x0 = {0u, 0u, 0u, 0u}, x1 = {0u, 0u, 0u, 0u};
                if (xon)
                {
                    x0 = *reinterpret_cast<const u4_t*>(xrow + (kb + 16u * g4) * 2u);
                    x1 = *reinterpret_cast<const u4_t*>(xrow + (kb + 16u * g4) * 2u + 16u);
                }
                uint32_t a[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) i8x4_to_f16(wv[u][j], a[2 * j], a[2 * j + 1]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(a[0], a[1], a[2], a[3]),
                                                             as_half8(x0[0], x0[1], x0[2], x0[3]), acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(a[4], a[5], a[6], a[7]),
                                                             as_half8(x1[0], x1[1], x1[2], x1[3]), acc, 0, 0, 0);
            }
            else
            {
                // one 128-k quantisation group: fresh accumulator, then scale/zero
                f4_t blkacc = {0.0f, 0.0f, 0.0f, 0.0f};
                float xs = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                {
                    u4_t xj = {0u, 0u, 0u, 0u};
                    if (xon) xj = *reinterpret_cast<const u4_t*>(xrow + (kb + 32u * g4 + 8u * j) * 2u);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                    {
                        const uint32_t pr = xj[e];
                        if constexpr (AF == OPURE_A_F16)
                            xs += f16_to_f32(static_cast<uint16_t>(pr)) + f16_to_f32(static_cast<uint16_t>(pr >> 16));
                        else
                            xs += bf16_to_f32(static_cast<uint16_t>(pr)) + bf16_to_f32(static_cast<uint16_t>(pr >> 16));
                    }
                    uint32_t a[4];
                    u4x8_to_pairs<AF>(wv[u][j], a);
                    if constexpr (AF == OPURE_A_F16)
                        blkacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(a[0], a[1], a[2], a[3]),
                                                                        as_half8(xj[0], xj[1], xj[2], xj[3]), blkacc, 0, 0, 0);
                    else
                        blkacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(a[0], a[1], a[2], a[3]),
                                                                         as_bf8(xj[0], xj[1], xj[2], xj[3]), blkacc, 0, 0, 0);
                }
                // the group sum of column m over all 128 k: the four lane groups hold 32 each
                xs += __shfl_xor(xs, 16);
                xs += __shfl_xor(xs, 32);
                const uint32_t g = kb / 128u;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                {
                    const float s = sz[((4u * g4 + i) * G + g) * 2u], z = sz[((4u * g4 + i) * G + g) * 2u + 1u];
                    acc[i] = __fmaf_rn(s, __fsub_rn(blkacc[i], __fmul_rn(z, xs)), acc[i]);
                }
            }
        }
    }

    // ---- combine the waves' K slices in wave order -------------------------
    if constexpr (NW > 1)
    {
        red[wave][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        acc = red[0][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) acc += red[w][lane];
    }

    // ---- epilogue: lane holds D rows 4*g4 + i for column m = r16 -----------
    const uint32_t m = r16;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        v[i] = acc[i];
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
    if (m >= M) return;
    if constexpr (EPI == opure_hip::EPI_STORE)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            store_act_rt(p.y, static_cast<uint64_t>(m) * p.out + 16u * tile + 4u * g4 + i, v[i], p.yfmt);
    }
    else if constexpr (EPI == opure_hip::EPI_RESIDUAL)
    {
        float* y = static_cast<float*>(p.y) + static_cast<uint64_t>(m) * p.out + 16u * tile + 4u * g4;
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = __fadd_rn(y[i], v[i]);
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

template <int WF, int AF, int EPI, int NW>
int launch_t(opure_dev* dev, const KParams& kp, uint32_t lds)
{
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<WF, AF, EPI, NW>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024));
        configured = true;
    }
    hipLaunchKernelGGL((k_gemv<WF, AF, EPI, NW>), dim3(kp.tiles), dim3(NW * 64), lds, dev->stream, kp);
    OPURE_LAUNCH_CHECK("k_gemv");
    return OPURE_OK;
}

template <int WF, int AF, int EPI>
int launch_nw(opure_dev* dev, const KParams& kp, uint32_t nw, uint32_t lds)
{
    switch (nw)
    {
    case 4: return launch_t<WF, AF, EPI, 4>(dev, kp, lds);
    case 8: return launch_t<WF, AF, EPI, 8>(dev, kp, lds);
    case 16: return launch_t<WF, AF, EPI, 16>(dev, kp, lds);
    }
    return opure_hip::set_error(OPURE_E_INVALID, "gemv: bad wave count %u", nw);
}

template <int WF, int AF>
int launch_epi(opure_dev* dev, uint32_t epi, const KParams& kp, uint32_t nw, uint32_t lds)
{
    switch (epi)
    {
    case opure_hip::EPI_STORE: return launch_nw<WF, AF, opure_hip::EPI_STORE>(dev, kp, nw, lds);
    case opure_hip::EPI_RESIDUAL: return launch_nw<WF, AF, opure_hip::EPI_RESIDUAL>(dev, kp, nw, lds);
    case opure_hip::EPI_SWIGLU: return launch_nw<WF, AF, opure_hip::EPI_SWIGLU>(dev, kp, nw, lds);
    case opure_hip::EPI_QKV: return launch_nw<WF, AF, opure_hip::EPI_QKV>(dev, kp, nw, lds);
    case opure_hip::EPI_LOGITS: return launch_nw<WF, AF, opure_hip::EPI_LOGITS>(dev, kp, nw, lds);
    }
    return opure_hip::set_error(OPURE_E_INVALID, "gemv: unknown epilogue %u", epi);
}

uint32_t kb_of(uint32_t wfmt) { return wfmt == OPURE_W_F32 ? 16u : (wfmt == OPURE_W_I8PC ? 64u : 128u); }

}  // namespace

namespace opure_hip {

// One workgroup per 16-row tile; its NW waves split K and are combined in wave
// order.  NW grows while the grid has fewer than 2048 waves and every wave keeps
// at least two 64-byte blocks per row.  Depends on the shape only, never on M.
GemvShape gemv_shape(uint32_t wfmt, uint32_t out, uint32_t in)
{
    GemvShape s;
    s.tiles = out / 16u;
    s.blocks = in / kb_of(wfmt);
    s.nw = 4u;
    while (s.nw < 16u && s.tiles * s.nw < 2048u && s.blocks >= 4u * s.nw) s.nw *= 2u;
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
    kp.qkv = c.qkv;
    kp.lg = c.logits;
    const uint32_t lds = c.wfmt == OPURE_W_I4G128 ? 16u * (c.W.in / 128u) * 8u : 0u;
    OPURE_REQUIRE(lds <= 64u * 1024u, OPURE_E_UNSUPPORTED, "gemv: in=%u too long for the group-scale stage", c.W.in);
    if (c.wfmt == OPURE_W_F32) return launch_epi<OPURE_W_F32, OPURE_A_F32>(dev, c.epi, kp, s.nw, lds);
    if (c.wfmt == OPURE_W_I8PC) return launch_epi<OPURE_W_I8PC, OPURE_A_F16>(dev, c.epi, kp, s.nw, lds);
    if (c.xfmt == OPURE_A_F16) return launch_epi<OPURE_W_I4G128, OPURE_A_F16>(dev, c.epi, kp, s.nw, lds);
    return launch_epi<OPURE_W_I4G128, OPURE_A_BF16>(dev, c.epi, kp, s.nw, lds);
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
