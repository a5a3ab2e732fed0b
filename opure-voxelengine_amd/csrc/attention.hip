// ============================================================================
//  attention.hip -- paged decode attention for the K+1 verify rows.
//
//  Replaces AttentionMain{hd} (shaders/Opure_FlashAttention_Decode.usf:58-179),
//  which ran one workgroup per query head serially over every position, and
//  the never-dispatched SpeculativeVerifyMain{hd} (Opure_SpeculativeDecode.usf).
//
//  Split-K ("flash-decoding") over fixed 64-token chunks of the paged cache:
//  one workgroup per (KV head, chunk, sequence) scores all query rows of that
//  KV head's GQA group against the chunk (query head h reads KV head
//  h / (n_heads / n_kv_heads), Opure_FlashAttention_Decode.usf:71-72), keeps
//  a per-chunk (max, sum, unnormalised output), and a combine kernel merges
//  chunks 0..last(row) in order.  Chunk boundaries sit at fixed positions, so
//  each row's output depends only on its own position: verifying K+1 rows
//  gives bitwise the same rows as K+1 single-row decodes.  Row j of sequence b
//  is at position seq_len[b] + j and sees positions 0 .. seq_len[b] + j.
//  Scores are scaled by attn_scale (1.0 = the reference, which has no
//  1/sqrt(head_dim): Opure_FlashAttention_Decode.usf:91-104).
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
    float* part_acc;     // [B][nkv][nch][Gq][hd]
    float* part_ml;      // [B][nkv][nch][Gq][2]
    uint32_t n_heads, n_kv, hd, rows, n_pages, max_pages, layer, nch, chunk, afmt;
    float scale;
};

// wave-wide reductions with a fixed butterfly order (deterministic)
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
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
                const uint64_t idx = ((((static_cast<uint64_t>(p.layer) * p.n_pages + static_cast<uint32_t>(page)) * 2u + kvsel) *
                                       p.n_kv + kh) * OPURE_PAGE_SIZE + pos % OPURE_PAGE_SIZE) * hd + d;
                v = load_act_rt(p.pool, idx, p.afmt);
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
    const uint64_t pbase = ((static_cast<uint64_t>(b) * p.n_kv + kh) * p.nch + c) * Gq;
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
// tokens, and out[d] = sum_t p_t V[t][d] with p broadcast from LDS.
template <int HD, int AF>
__global__ __launch_bounds__(256) void k_attn_chunk(AttnParams p)
{
    constexpr uint32_t CH = 64, EB = AF == OPURE_A_F32 ? 4u : 2u;
    constexpr uint32_t ROWB = HD * EB + 16u;              // padded LDS row (bank spread)
    constexpr uint32_t DPL = (HD + 63u) / 64u;             // V channels per lane
    __shared__ __align__(16) uint8_t kt[CH * ROWB];
    __shared__ __align__(16) uint8_t vt[CH * ROWB];
    __shared__ __align__(16) float pbuf[4][CH];
    extern __shared__ __align__(16) float qs[];            // [Gq][HD]

    const uint32_t kh = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
    const uint32_t group = p.n_heads / p.n_kv, R = p.rows, Gq = group * R;
    const uint32_t ctx = static_cast<uint32_t>(p.seq_len[b]);
    const uint32_t total = ctx + R;
    const uint32_t t0 = c * CH;
    if (t0 >= total) return;
    const int32_t* pt = p.page_table + static_cast<uint64_t>(b) * p.max_pages;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;

    for (uint32_t e = threadIdx.x; e < Gq * HD; e += 256u)
    {
        const uint32_t qi = e / HD, d = e - qi * HD;
        const uint32_t j = qi / group, head = kh * group + (qi - j * group);
        qs[e] = load_act_rt(p.q, (static_cast<uint64_t>(b * R + j) * p.n_heads + head) * HD + d, AF);
    }
    // stage K and V rows: 16-byte pieces, a page's 16 tokens of this head are contiguous
    constexpr uint32_t PIECES = HD * EB / 16u;
    for (uint32_t e = threadIdx.x; e < 2u * CH * PIECES; e += 256u)
    {
        const uint32_t kvsel = e / (CH * PIECES), rem = e - kvsel * CH * PIECES;
        const uint32_t tl = rem / PIECES, pc = rem - tl * PIECES, pos = t0 + tl;
        u4v val = {0u, 0u, 0u, 0u};
        if (pos < total)
        {
            const int32_t page = pos / OPURE_PAGE_SIZE < p.max_pages ? pt[pos / OPURE_PAGE_SIZE] : -1;
            if (page >= 0 && static_cast<uint32_t>(page) < p.n_pages)
            {
                const uint64_t idx = ((((static_cast<uint64_t>(p.layer) * p.n_pages + static_cast<uint32_t>(page)) * 2u + kvsel) *
                                       p.n_kv + kh) * OPURE_PAGE_SIZE + pos % OPURE_PAGE_SIZE) * HD;
                val = *reinterpret_cast<const u4v*>(static_cast<const uint8_t*>(p.pool) + idx * EB + pc * 16u);
            }
            else
            {
                // a missing page or a length past the table reads as NaN, never out of bounds
                const uint32_t nan = AF == OPURE_A_F32 ? 0x7FC00000u : (AF == OPURE_A_F16 ? 0x7E007E00u : 0x7FC07FC0u);
                val = {nan, nan, nan, nan};
            }
        }
        *reinterpret_cast<u4v*>((kvsel ? vt : kt) + tl * ROWB + pc * 16u) = val;
    }
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
            vc[i][t] = d < HD ? load_act_rt(vt + t * ROWB, d, AF) : 0.0f;
    }
    const uint64_t pbase = ((static_cast<uint64_t>(b) * p.n_kv + kh) * p.nch + c) * Gq;
    const uint32_t pos = t0 + lane;
    for (uint32_t qi = wave; qi < Gq; qi += 4u)
    {
        const uint32_t j = qi / group;
        const float* qr = qs + qi * HD;
        float acc = 0.0f;
#pragma unroll
        for (uint32_t d = 0; d < HD; ++d) acc = __fmaf_rn(qr[d], kr[d], acc);
        const float s = pos <= ctx + j ? __fmul_rn(acc, p.scale) : -__builtin_huge_valf();
        const float mx = wave_max(s);
        const float e = s == -__builtin_huge_valf() ? 0.0f : expf_ref(__fsub_rn(s, mx));
        const float l = wave_sum(e);
        pbuf[wave][lane] = e;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
        for (uint32_t i = 0; i < DPL; ++i)
        {
            float o = 0.0f;
#pragma unroll
            for (uint32_t t = 0; t < CH; ++t) o = __fmaf_rn(pbuf[wave][t], vc[i][t], o);
            const uint32_t d = lane + 64u * i;
            if (d < HD) p.part_acc[(pbase + qi) * HD + d] = o;
        }
        if (lane == 0)
        {
            p.part_ml[(pbase + qi) * 2u] = mx;
            p.part_ml[(pbase + qi) * 2u + 1u] = l;
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// one workgroup of hd threads per (row, query head): merge chunks 0..last in
// order; the loads of each group of 16 chunks are independent and issued together
__global__ void k_attn_combine(AttnParams p)
{
    const uint32_t head = blockIdx.x, r = blockIdx.y;     // r = b * R + j
    const uint32_t R = p.rows, b = r / R, j = r - b * R;
    const uint32_t group = p.n_heads / p.n_kv, kh = head / group, qi = j * group + (head - kh * group);
    const uint32_t Gq = group * R, hd = p.hd, d = threadIdx.x;
    uint32_t last = (static_cast<uint32_t>(p.seq_len[b]) + j) / p.chunk;
    if (last >= p.nch) last = p.nch - 1u;          // length beyond the launch bound: clamp, never overrun
    const uint64_t base = (static_cast<uint64_t>(b) * p.n_kv + kh) * p.nch;
    constexpr uint32_t G = 16;
    float mx = -__builtin_huge_valf();
    for (uint32_t c0 = 0; c0 <= last; c0 += G)
    {
        float m[G];
#pragma unroll
        for (uint32_t i = 0; i < G; ++i)
            m[i] = c0 + i <= last ? p.part_ml[((base + c0 + i) * Gq + qi) * 2u] : -__builtin_huge_valf();
#pragma unroll
        for (uint32_t i = 0; i < G; ++i) mx = fmaxf(mx, m[i]);
    }
    float num = 0.0f, den = 0.0f;
    for (uint32_t c0 = 0; c0 <= last; c0 += G)
    {
        float m[G], l[G], a[G];
#pragma unroll
        for (uint32_t i = 0; i < G; ++i)
        {
            const bool on = c0 + i <= last;
            const uint64_t k = (base + c0 + i) * Gq + qi;
            m[i] = on ? p.part_ml[k * 2u] : -__builtin_huge_valf();
            l[i] = on ? p.part_ml[k * 2u + 1u] : 0.0f;
            a[i] = on ? p.part_acc[k * hd + d] : 0.0f;
        }
#pragma unroll
        for (uint32_t i = 0; i < G; ++i)
        {
            const float w = m[i] == -__builtin_huge_valf() ? 0.0f : expf_ref(__fsub_rn(m[i], mx));
            den = __fmaf_rn(w, l[i], den);
            num = __fmaf_rn(w, a[i], num);
        }
    }
    const float o = __fdiv_rn(num, den > 0.0f ? den : 1.0f);
    store_act_rt(p.out, (static_cast<uint64_t>(r) * p.n_heads + head) * hd + d, o, p.afmt);
}

template <int HD, int AF>
int launch_fast(opure_dev* dev, dim3 grid, uint32_t lds, const AttnParams& p)
{
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_chunk<HD, AF>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024));
        configured = true;
    }
    hipLaunchKernelGGL((k_attn_chunk<HD, AF>), grid, dim3(256), lds, dev->stream, p);
    OPURE_LAUNCH_CHECK("k_attn_chunk");
    return OPURE_OK;
}

}  // namespace

namespace opure_hip {

uint32_t attn_chunk(uint32_t hd) { return hd <= 128u ? 64u : 32u; }

uint64_t attn_partial_bytes(uint32_t batch, uint32_t n_kv, uint32_t group, uint32_t rows, uint32_t hd, uint32_t max_ctx)
{
    const uint32_t nch = (max_ctx + attn_chunk(hd) - 1u) / attn_chunk(hd);
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
    OPURE_REQUIRE(batch >= 1 && rows >= 1 && batch * rows <= OPURE_MAX_ROWS, OPURE_E_CAPACITY,
                  "attention: batch*rows = %u exceeds %d", batch * rows, OPURE_MAX_ROWS);
    OPURE_REQUIRE(max_ctx >= rows && max_ctx <= kv->max_pages_per_seq * OPURE_PAGE_SIZE, OPURE_E_CAPACITY,
                  "attention: max_ctx %u beyond the page-table capacity %u", max_ctx,
                  kv->max_pages_per_seq * OPURE_PAGE_SIZE);
    OPURE_REQUIRE(m->afmt <= OPURE_A_BF16, OPURE_E_INVALID, "attention: bad activation format");
    const uint32_t group = m->n_heads / m->n_kv_heads, CH = attn_chunk(m->head_dim);
    const uint64_t lds = (static_cast<uint64_t>(group) * rows * m->head_dim + static_cast<uint64_t>(group) * rows * CH +
                          static_cast<uint64_t>(CH) * (m->head_dim + 1)) * 4u;
    OPURE_REQUIRE(lds <= 160u * 1024u, OPURE_E_CAPACITY, "attention: %u query rows per KV head exceed LDS", group * rows);
    return OPURE_OK;
}

int attn_launch(opure_dev* dev, const opure_model* m, const opure_kv* kv, uint32_t layer, uint32_t batch,
                uint32_t rows, const int32_t* seq_len, uint32_t max_ctx, const void* q, void* out, float* part)
{
    AttnParams p;
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
    p.chunk = attn_chunk(m->head_dim);
    p.nch = (max_ctx + p.chunk - 1u) / p.chunk;
    p.afmt = m->afmt;
    p.scale = m->attn_scale;
    const uint32_t group = m->n_heads / m->n_kv_heads, Gq = group * rows;
    const uint64_t q_elems = static_cast<uint64_t>(batch) * p.n_kv * p.nch * Gq;
    p.part_acc = part;
    p.part_ml = part + align_up(q_elems * p.hd * 4u, 256) / 4u;
    const dim3 grid(p.n_kv, p.nch, batch);
    const uint32_t hd = p.hd;
    if (p.chunk == 64u && (hd == 64u || hd == 128u))
    {
        const uint32_t lds = Gq * hd * 4u;
        int rc;
        if (hd == 64u && p.afmt == OPURE_A_F32) rc = launch_fast<64, OPURE_A_F32>(dev, grid, lds, p);
        else if (hd == 64u && p.afmt == OPURE_A_F16) rc = launch_fast<64, OPURE_A_F16>(dev, grid, lds, p);
        else if (hd == 64u) rc = launch_fast<64, OPURE_A_BF16>(dev, grid, lds, p);
        else if (p.afmt == OPURE_A_F32) rc = launch_fast<128, OPURE_A_F32>(dev, grid, lds, p);
        else if (p.afmt == OPURE_A_F16) rc = launch_fast<128, OPURE_A_F16>(dev, grid, lds, p);
        else rc = launch_fast<128, OPURE_A_BF16>(dev, grid, lds, p);
        if (rc) return rc;
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
        hipLaunchKernelGGL(k_attn_chunk_generic, grid, dim3(256), lds, dev->stream, p);
        OPURE_LAUNCH_CHECK("k_attn_chunk_generic");
    }
    hipLaunchKernelGGL(k_attn_combine, dim3(p.n_heads, batch * rows), dim3(p.hd), 0, dev->stream, p);
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
                                                  a->max_ctx), 0);
    if (rc) return rc;
    return attn_launch(dev, a->model, a->kv, a->layer, a->batch, a->rows, a->seq_len, a->max_ctx, a->q, a->out,
                       static_cast<float*>(dev->ws));
}
