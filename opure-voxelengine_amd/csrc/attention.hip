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

__global__ __launch_bounds__(256) void k_attn_chunk(AttnParams p)
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

// one workgroup of hd threads per (row, query head): merge chunks in order
__global__ void k_attn_combine(AttnParams p)
{
    const uint32_t head = blockIdx.x, r = blockIdx.y;     // r = b * R + j
    const uint32_t R = p.rows, b = r / R, j = r - b * R;
    const uint32_t group = p.n_heads / p.n_kv, kh = head / group, qi = j * group + (head - kh * group);
    const uint32_t Gq = group * R, hd = p.hd, d = threadIdx.x;
    uint32_t last = (static_cast<uint32_t>(p.seq_len[b]) + j) / p.chunk;
    if (last >= p.nch) last = p.nch - 1u;          // length beyond the launch bound: clamp, never overrun
    const uint64_t base = (static_cast<uint64_t>(b) * p.n_kv + kh) * p.nch;
    float mx = -__builtin_huge_valf();
    for (uint32_t c = 0; c <= last; ++c) mx = fmaxf(mx, p.part_ml[((base + c) * Gq + qi) * 2u]);
    float num = 0.0f, den = 0.0f;
    for (uint32_t c = 0; c <= last; ++c)
    {
        const float m = p.part_ml[((base + c) * Gq + qi) * 2u];
        const float w = m == -__builtin_huge_valf() ? 0.0f : expf_ref(__fsub_rn(m, mx));
        den = __fmaf_rn(w, p.part_ml[((base + c) * Gq + qi) * 2u + 1u], den);
        num = __fmaf_rn(w, p.part_acc[((base + c) * Gq + qi) * hd + d], num);
    }
    const float o = __fdiv_rn(num, den > 0.0f ? den : 1.0f);
    store_act_rt(p.out, (static_cast<uint64_t>(r) * p.n_heads + head) * hd + d, o, p.afmt);
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
    const uint32_t lds = (Gq * p.hd + Gq * p.chunk + p.chunk * (p.hd + 1u)) * 4u;
    static bool configured = false;
    if (!configured)
    {
        OPURE_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_chunk),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        configured = true;
    }
    hipLaunchKernelGGL(k_attn_chunk, dim3(p.n_kv, p.nch, batch), dim3(256), lds, dev->stream, p);
    OPURE_LAUNCH_CHECK("k_attn_chunk");
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
