// ============================================================================
//  verify.hip -- one speculative-decoding verify step on the GPU.
//
//  Replaces VoxelEngine::RecordForward (src/engine/Opure_VoxelEngine.cpp:189-536),
//  which recorded 1 + 14 L + 2 barriered dispatches per token for ONE token.
//  A verify step scores K+1 rows of B sequences in one pass over the weights:
//
//    embed gather (dequantised)                        x  [MR][h]  fp32 residual
//    per layer:
//      rmsnorm(x, attn_norm) fused into the qkv load
//      gemv qkv   + RoPE, q store, paged K/V append    q  [MR][nh*hd]
//      paged attention (split-K chunks + combine)      att[MR][nh*hd]
//      gemv o     + residual add                       x += o
//      rmsnorm(x, mlp_norm) fused into the gate/up load
//      gemv gate/up + SwiGLU                           h  [MR][ffn]
//      gemv down  + residual add                       x += down
//    rmsnorm(x, final_norm) fused into the LM head; logits + per-tile argmax
//    partials
//    acceptance (greedy from the partials, or rejection sampling)
//    rollback of rejected positions
//
//  Every launch goes to the device's one stream, so a whole step can be
//  captured once into a hipGraph and replayed (opure_verify_reserve sizes the
//  workspace first, because capture cannot allocate).
// ============================================================================
#include "internal.h"

#include <algorithm>
#include <utility>

using namespace opure_dev_math;

namespace {

// Dequantised embedding rows into the fp32 residual, plus each 16-column
// tile's sum of squares for the first layer's fused RMSNorm.  One thread per
// 16-column tile: its columns are one 16-byte piece (int8), half a piece
// (uint4) or four pieces (fp32) of the tiled layout, loaded at once.
__global__ __launch_bounds__(256) void k_embed(const int32_t* tokens, opure_linear E, uint32_t wfmt, uint32_t h,
                                               uint32_t vocab, uint32_t M, uint32_t KB, float* x, float* ss,
                                               uint32_t* err)
{
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    const uint32_t r = blockIdx.x;
    const int32_t t = tokens[r];
    float* xr = x + static_cast<uint64_t>(r) * h;
    const bool bad = t < 0 || static_cast<uint32_t>(t) >= vocab;
    if (bad && threadIdx.x == 0 && err) err[ERR_TOKEN] = 1u;   // reported at the host's next sync
    const uint32_t nblk = h / KB;
    const uint32_t row = bad ? 0u : static_cast<uint32_t>(t), tile = row >> 4, rr = row & 15u;
    const uint8_t* w = static_cast<const uint8_t*>(E.w);
    for (uint32_t c16 = threadIdx.x; c16 < h / 16u; c16 += 256u)
    {
        float v[16];
        const uint32_t k0 = 16u * c16, b = k0 / KB, kk = k0 - b * KB;
        const uint64_t blk = (static_cast<uint64_t>(tile) * nblk + b) << 10;
        if (wfmt == OPURE_W_F32)
        {
#pragma unroll
            for (uint32_t gq = 0; gq < 4; ++gq)
            {
                const u4v q = *reinterpret_cast<const u4v*>(w + blk + ((16u * gq + rr) << 4));
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * gq + e] = __uint_as_float(q[e]);
            }
        }
        else if (wfmt == OPURE_W_I8PC)
        {
            const u4v q = *reinterpret_cast<const u4v*>(w + blk + ((16u * (kk / 16u) + rr) << 4));
            const float sc = f16_to_f32(static_cast<const uint16_t*>(E.scale)[tile * 16u + rr]);
#pragma unroll
            for (int e = 0; e < 16; ++e)
            {
                const int8_t qi = static_cast<int8_t>(((q[e >> 2] >> (8 * (e & 3))) & 0xFFu) ^ 0x80u);
                v[e] = __fmul_rn(static_cast<float>(qi), sc);
            }
        }
        else
        {
            // 16 columns = words 2*half, 2*half+1 of lane g's piece; element e of a
            // word sits at nibble {0,4,1,5,2,6,3,7}[e]
            const uint32_t g = kk / 32u, half = (kk % 32u) / 16u;
            const uint32_t* wd = reinterpret_cast<const uint32_t*>(w + blk + ((16u * g + rr) << 4)) + 2u * half;
            // the tiled words are stored rotated left by 3 bits: undo it
            const uint32_t w0 = __builtin_amdgcn_alignbit(wd[0], wd[0], 3), w1 = __builtin_amdgcn_alignbit(wd[1], wd[1], 3);
            const uint32_t sz = static_cast<const uint32_t*>(E.scale)[(static_cast<uint64_t>(tile) * nblk + b) * 16u + rr];
            const float s = __uint_as_float(sz << 16), z = __uint_as_float(sz & 0xFFFF0000u);
#pragma unroll
            for (int e = 0; e < 16; ++e)
            {
                const uint32_t word = e < 8 ? w0 : w1, el = e & 7;
                const uint32_t q = (word >> (4u * ((el >> 1) | ((el & 1u) << 2)))) & 0x0Fu;
                v[e] = __fmul_rn(s, __fsub_rn(static_cast<float>(q), z));
            }
        }
        float sq = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e)
        {
            // an id outside the vocabulary poisons its row instead of reading out of bounds
            const float val = bad ? __builtin_nanf("") : v[e];
            xr[k0 + e] = val;
            sq = __fmaf_rn(val, val, sq);
        }
        ss[static_cast<uint64_t>(c16) * M + r] = sq;
    }
}

// Per-16-column-tile sums of squares of a given fp32 residual [M][h] (the
// value every residual producer leaves for the next fused RMSNorm), summed in
// column order: one thread per (row, tile).
__global__ __launch_bounds__(256) void k_tile_sumsq(const float* x, uint32_t M, uint32_t h, float* ss)
{
    const uint32_t tiles = h / 16u;
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (i >= static_cast<uint64_t>(M) * tiles) return;
    const uint32_t r = static_cast<uint32_t>(i / tiles), c16 = static_cast<uint32_t>(i - static_cast<uint64_t>(r) * tiles);
    const float* xr = x + static_cast<uint64_t>(r) * h + 16u * c16;
    float sq = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) sq = __fmaf_rn(xr[e], xr[e], sq);
    ss[static_cast<uint64_t>(c16) * M + r] = sq;
}

}  // namespace

namespace opure_hip {

struct VerifyPlan {
    uint64_t x = 0, ss = 0, xn = 0, q = 0, att = 0, h = 0, am_val = 0, am_idx = 0, attn = 0, rej = 0, part = 0, total = 0;
    uint32_t lm_tiles = 0;
};

static VerifyPlan make_plan(const opure_dev* dev, const opure_model* m, uint32_t B, uint32_t R, uint32_t max_ctx)
{
    VerifyPlan p;
    const uint64_t MR = static_cast<uint64_t>(B) * R;
    const uint32_t eb = act_bytes(m->afmt);
    const uint32_t qdim = m->n_heads * m->head_dim, kvdim = m->n_kv_heads * m->head_dim;
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) { const uint64_t o = off; off += align_up(bytes ? bytes : 1, 256); return o; };
    p.x = take(MR * m->hidden * 4u);
    p.ss = take(MR * (m->hidden / 16u) * 4u);
    p.xn = take(MR * m->hidden * eb);
    p.q = take(MR * qdim * eb);
    p.att = take(MR * qdim * eb);
    p.h = take(MR * m->ffn * eb);
    // argmax partials: one per LM-head workgroup and row (at most one per tile),
    // or one per 4096 logits when more than OPURE_MAX_ROWS rows store the logits
    p.lm_tiles = m->vocab / 16u;
    const uint64_t am = std::max<uint64_t>(p.lm_tiles, argmax_parts(m->vocab)) * MR * 4u;
    p.am_val = take(am);
    p.am_idx = take(am);
    p.attn = take(attn_partial_bytes(B, m->n_kv_heads, m->n_heads / m->n_kv_heads, R, m->head_dim, m->afmt, max_ctx));
    p.rej = take(accept_ws_bytes(B, R - 1u, m->vocab, OPURE_ACCEPT_REJECTION));
    // split-K accumulators of the GEMVs over more than OPURE_MAX_ROWS rows
    uint64_t part = 0;
    for (const auto& s : {std::pair<uint32_t, uint32_t>{qdim + 2u * kvdim, m->hidden}, {m->hidden, qdim},
                          {2u * m->ffn, m->hidden}, {m->hidden, m->ffn}, {m->vocab, m->hidden}})
        part = std::max(part, gemv_scratch_bytes(dev, m->wfmt, s.first, s.second, static_cast<uint32_t>(MR)));
    p.part = take(part);
    p.total = off;
    return p;
}

static int check_linear(const opure_linear& L, uint32_t out, uint32_t in, const char* what, uint32_t wfmt,
                        uint32_t layout = OPURE_LAYOUT_TILED)
{
    OPURE_REQUIRE(L.w && L.out == out && L.in == in, OPURE_E_INVALID, "verify: %s is %ux%u (w=%p), expected %ux%u", what,
                  L.out, L.in, L.w, out, in);
    OPURE_REQUIRE(L.layout == layout, OPURE_E_INVALID, "verify: %s must be in layout %u (opure_tile_linear), got %u",
                  what, layout, L.layout);
    if (wfmt != OPURE_W_F32) OPURE_REQUIRE(L.scale, OPURE_E_INVALID, "verify: %s has no scales", what);
    return OPURE_OK;
}

static int check_model(const opure_model* m, const opure_kv* kv, uint32_t B, uint32_t R, uint32_t max_ctx)
{
    OPURE_REQUIRE(m && kv && m->layers && m->final_norm && m->rope_cos && m->rope_sin, OPURE_E_INVALID,
                  "verify: null model field");
    OPURE_REQUIRE(m->n_layers >= 1 && m->hidden >= 16 && m->hidden % 16 == 0 && m->vocab >= 16 && m->vocab % 16 == 0 &&
                      m->ffn >= 16,
                  OPURE_E_INVALID, "verify: bad model shape");
    const bool ok = (m->wfmt == OPURE_W_F32 && m->afmt == OPURE_A_F32) ||
                    (m->wfmt == OPURE_W_I8PC && m->afmt == OPURE_A_F16) ||
                    (m->wfmt == OPURE_W_I4G128 && (m->afmt == OPURE_A_F16 || m->afmt == OPURE_A_BF16));
    OPURE_REQUIRE(ok, OPURE_E_UNSUPPORTED, "verify: weights %u with %s activations are not built", m->wfmt,
                  afmt_name(m->afmt));
    int rc = attn_validate(m, kv, B, R, max_ctx);
    if (rc) return rc;
    OPURE_REQUIRE(max_ctx <= m->rope_max_pos, OPURE_E_CAPACITY, "verify: max_ctx %u beyond the RoPE table (%u)", max_ctx,
                  m->rope_max_pos);
    OPURE_REQUIRE(R >= 1 && R - 1u < 64u, OPURE_E_CAPACITY, "verify: rows %u", R);
    const uint32_t qdim = m->n_heads * m->head_dim, kvdim = m->n_kv_heads * m->head_dim;
    if ((rc = check_linear(m->embed, m->vocab, m->hidden, "embed", m->wfmt))) return rc;
    if ((rc = check_linear(m->lm_head, m->vocab, m->hidden, "lm_head", m->wfmt))) return rc;
    for (uint32_t L = 0; L < m->n_layers; ++L)
    {
        const opure_layer_weights& W = m->layers[L];
        OPURE_REQUIRE(W.attn_norm && W.mlp_norm, OPURE_E_INVALID, "verify: layer %u norm gains missing", L);
        if ((rc = check_linear(W.qkv, qdim + 2u * kvdim, m->hidden, "qkv", m->wfmt))) return rc;
        if ((rc = check_linear(W.o, m->hidden, qdim, "o_proj", m->wfmt))) return rc;
        if ((rc = check_linear(W.gate_up, 2u * m->ffn, m->hidden, "gate_up", m->wfmt, OPURE_LAYOUT_TILED_SWIGLU)))
            return rc;
        if ((rc = check_linear(W.down, m->hidden, m->ffn, "down", m->wfmt))) return rc;
    }
    return OPURE_OK;
}

// One layer of the verify step on the residual x (fp32 [B*R][hidden]) whose
// per-tile sums of squares are in ss: rmsnorm + qkv GEMV + RoPE + paged K/V
// append, attention, o_proj + residual, rmsnorm + gate/up + SwiGLU, down +
// residual.  `c` carries the step-wide GEMV fields (formats, rows, scratch).
// The body of RecordForward's layer loop (Opure_VoxelEngine.cpp:296-492).
// Above OPURE_MAX_ROWS rows a residual GEMV also writes the next rmsnorm's
// rows (GemvCall::norm_gain) into xn, so the consumer reads them instead of
// running its own normalisation pass: xn_ready says the incoming xn holds
// this layer's attention-norm rows, next_gain is the norm after the layer.
static int layer_launch(opure_dev* dev, const opure_model* m, const opure_kv* kv, uint32_t L, uint32_t B, uint32_t R,
                        const int32_t* seq_len, uint32_t max_ctx, const VerifyPlan& P, float* x, float* ss, GemvCall& c,
                        bool xn_ready = false, const float* next_gain = nullptr)
{
    const bool wide = B * R > OPURE_MAX_ROWS;
    char* ws = static_cast<char*>(dev->ws);
    void* xn = ws + P.xn;
    void* q = ws + P.q;
    void* att = ws + P.att;
    void* hbuf = ws + P.h;
    const uint32_t qdim = m->n_heads * m->head_dim, kvdim = m->n_kv_heads * m->head_dim;
    int rc;
    const opure_layer_weights& W = m->layers[L];
    c.W = W.qkv;
    c.x = xn_ready ? xn : x;
    c.gain = xn_ready ? nullptr : W.attn_norm;
    c.ss_in = ss;
    c.ss_out = nullptr;
    c.norm_gain = nullptr;
    c.y = q;
    c.yfmt = m->afmt;
    c.epi = EPI_QKV;
    c.qkv.qdim = qdim;
    c.qkv.kvdim = kvdim;
    c.qkv.head_dim = m->head_dim;
    c.qkv.n_kv_heads = m->n_kv_heads;
    c.qkv.rope_cos = m->rope_cos;
    c.qkv.rope_sin = m->rope_sin;
    c.qkv.rope_max_pos = m->rope_max_pos;
    c.qkv.seq_len = seq_len;
    c.qkv.rows_per_seq = R;
    c.qkv.kv_pool = kv->pool;
    c.qkv.page_table = kv->page_table;
    c.qkv.max_pages = kv->max_pages_per_seq;
    c.qkv.n_pages = kv->n_pages;
    c.qkv.layer = L;
    c.qkv.err = dev->err;
    if ((rc = gemv_validate(c)) || (rc = prof_begin(dev, OPURE_STAGE_QKV)) || (rc = gemv_launch(dev, c)) ||
        (rc = prof_end(dev)))
        return rc;

    if ((rc = prof_begin(dev, OPURE_STAGE_ATTN)) ||
        (rc = attn_launch(dev, m, kv, L, B, R, seq_len, max_ctx, q, att, reinterpret_cast<float*>(ws + P.attn))) ||
        (rc = prof_end(dev)))
        return rc;

    c.W = W.o;
    c.x = att;
    c.gain = nullptr;
    c.ss_out = ss;
    c.y = x;
    c.yfmt = OPURE_A_F32;
    c.epi = EPI_RESIDUAL;
    c.norm_gain = wide ? W.mlp_norm : nullptr;
    c.norm_out = xn;
    if ((rc = gemv_validate(c)) || (rc = prof_begin(dev, OPURE_STAGE_O)) || (rc = gemv_launch(dev, c)) ||
        (rc = prof_end(dev)))
        return rc;

    c.W = W.gate_up;
    c.x = wide ? xn : x;
    c.gain = wide ? nullptr : W.mlp_norm;
    c.ss_out = nullptr;
    c.norm_gain = nullptr;
    c.y = hbuf;
    c.yfmt = m->afmt;
    c.epi = EPI_SWIGLU;
    if ((rc = gemv_validate(c)) || (rc = prof_begin(dev, OPURE_STAGE_GATE_UP)) || (rc = gemv_launch(dev, c)) ||
        (rc = prof_end(dev)))
        return rc;

    c.W = W.down;
    c.x = hbuf;
    c.gain = nullptr;
    c.ss_out = ss;
    c.y = x;
    c.yfmt = OPURE_A_F32;
    c.epi = EPI_RESIDUAL;
    c.norm_gain = wide ? next_gain : nullptr;
    c.norm_out = xn;
    if ((rc = gemv_validate(c)) || (rc = prof_begin(dev, OPURE_STAGE_DOWN)) || (rc = gemv_launch(dev, c)) ||
        (rc = prof_end(dev)))
        return rc;
    return OPURE_OK;
}

// The GEMV fields shared by every launch of a step over B*R rows.
static GemvCall step_gemv(const opure_model* m, uint32_t MR, const VerifyPlan& P, char* ws, float* ss)
{
    GemvCall c;
    c.wfmt = m->wfmt;
    c.xfmt = m->afmt;
    c.M = MR;
    c.eps = m->rms_eps;
    c.ss_tiles = m->hidden / 16u;
    c.ss_in = ss;
    c.xn_scratch = ws + P.xn;
    c.part_scratch = ws + P.part;
    return c;
}

}  // namespace opure_hip

using namespace opure_hip;

extern "C" {

int opure_verify_reserve(opure_dev* dev, const opure_model* model, uint32_t batch, uint32_t rows, uint32_t max_ctx)
{
    OPURE_REQUIRE(dev && model, OPURE_E_INVALID, "opure_verify_reserve: null argument");
    OPURE_REQUIRE(batch >= 1 && rows >= 1 && rows <= OPURE_MAX_ROWS && batch * rows <= OPURE_MAX_BATCH_ROWS,
                  OPURE_E_CAPACITY, "opure_verify_reserve: %u rows x batch %u beyond %d / %d", rows, batch,
                  OPURE_MAX_ROWS, OPURE_MAX_BATCH_ROWS);
    const VerifyPlan p = make_plan(dev, model, batch, rows, max_ctx);
    return ensure_workspace(dev, p.total);
}

int opure_debug_workspace(opure_dev* dev, void** ptr, uint64_t* bytes)
{
    OPURE_REQUIRE(dev && ptr && bytes, OPURE_E_INVALID, "opure_debug_workspace: null argument");
    *ptr = dev->ws;
    *bytes = dev->ws_bytes;
    return OPURE_OK;
}

int opure_debug_verify_offsets(const opure_model* model, uint32_t batch, uint32_t rows, uint32_t max_ctx,
                               uint64_t offsets[5])
{
    OPURE_REQUIRE(model && offsets && batch && rows, OPURE_E_INVALID, "opure_debug_verify_offsets: bad argument");
    const VerifyPlan p = make_plan(nullptr, model, batch, rows, max_ctx);
    offsets[0] = p.x;
    offsets[1] = p.ss;
    offsets[2] = p.q;
    offsets[3] = p.att;
    offsets[4] = p.h;
    return OPURE_OK;
}

int opure_verify_layer(opure_dev* dev, const opure_verify_layer_args* a)
{
    OPURE_REQUIRE(dev && a && a->model && a->kv && a->seq_len && a->x, OPURE_E_INVALID,
                  "opure_verify_layer: null argument");
    const opure_model* m = a->model;
    const uint32_t B = a->batch, R = a->rows, MR = B * R;
    int rc = check_model(m, a->kv, B, R, a->max_ctx);
    if (rc) return rc;
    OPURE_REQUIRE(a->layer < m->n_layers, OPURE_E_INVALID, "opure_verify_layer: layer %u of %u", a->layer, m->n_layers);
    const VerifyPlan P = make_plan(dev, m, B, R, a->max_ctx);
    if ((rc = ensure_workspace(dev, P.total))) return rc;
    char* ws = static_cast<char*>(dev->ws);
    float* ss = reinterpret_cast<float*>(ws + P.ss);
    const uint64_t n = static_cast<uint64_t>(MR) * (m->hidden / 16u);
    OPURE_LAUNCH(dev, k_tile_sumsq, dim3(static_cast<uint32_t>((n + 255u) / 256u)), dim3(256), 0, a->x, MR,
                       m->hidden, ss);
    OPURE_LAUNCH_CHECK("k_tile_sumsq");
    GemvCall c = step_gemv(m, MR, P, ws, ss);
    return layer_launch(dev, m, a->kv, a->layer, B, R, a->seq_len, a->max_ctx, P, a->x, ss, c);
}

int opure_verify_step(opure_dev* dev, const opure_verify_args* a)
{
    OPURE_REQUIRE(dev && a && a->model && a->kv && a->tokens && a->seq_len, OPURE_E_INVALID,
                  "opure_verify_step: null argument");
    // no logits: a prefill, which stops after the last layer
    OPURE_REQUIRE(a->logits || (a->accept_mode == OPURE_ACCEPT_NONE && !a->rollback), OPURE_E_INVALID,
                  "opure_verify_step: acceptance needs logits");
    const opure_model* m = a->model;
    const opure_kv* kv = a->kv;
    const uint32_t B = a->batch, R = a->rows, MR = B * R;
    int rc = check_model(m, kv, B, R, a->max_ctx);
    if (rc) return rc;
    OPURE_REQUIRE(a->accept_mode <= OPURE_ACCEPT_REJECTION, OPURE_E_INVALID, "verify: accept_mode %u", a->accept_mode);
    if (a->accept_mode != OPURE_ACCEPT_NONE)
    {
        // one row and no drafts is a plain decode step: out_tokens[0] is the
        // argmax (greedy) or a sample at the temperature (rejection)
        OPURE_REQUIRE(a->out_tokens && a->accepted, OPURE_E_INVALID, "verify: acceptance needs out_tokens and accepted");
        if (a->accept_mode == OPURE_ACCEPT_REJECTION)
            OPURE_REQUIRE((a->draft_logits || R == 1) && a->temperature > 0.0f, OPURE_E_INVALID,
                          "verify: rejection needs draft_logits and temperature > 0");
    }
    if (a->rollback)
        OPURE_REQUIRE(a->accept_mode != OPURE_ACCEPT_NONE && a->new_seq_len, OPURE_E_INVALID,
                      "verify: rollback needs acceptance and new_seq_len");

    const VerifyPlan P = make_plan(dev, m, B, R, a->max_ctx);
    rc = ensure_workspace(dev, P.total);
    if (rc) return rc;
    char* ws = static_cast<char*>(dev->ws);
    float* x = reinterpret_cast<float*>(ws + P.x);
    float* ss = reinterpret_cast<float*>(ws + P.ss);

    if ((rc = prof_begin(dev, OPURE_STAGE_EMBED))) return rc;
    OPURE_LAUNCH(dev, k_embed, dim3(MR), dim3(256), 0, a->tokens, m->embed, m->wfmt, m->hidden, m->vocab,
                       MR, tiled_block_k(m->wfmt), x, ss, dev->err);
    OPURE_LAUNCH_CHECK("k_embed");
    if ((rc = prof_end(dev))) return rc;

    // Each residual producer (embed, o, down) leaves per-tile sums of squares in
    // `ss`; the next consumer (qkv, gate/up, LM head) applies the RMSNorm while
    // loading x.  Stream order keeps the single buffer consistent.
    GemvCall c = step_gemv(m, MR, P, ws, ss);
    const bool wide = MR > OPURE_MAX_ROWS;
    for (uint32_t L = 0; L < m->n_layers; ++L)
    {
        const float* next = L + 1u < m->n_layers ? m->layers[L + 1u].attn_norm : (a->logits ? m->final_norm : nullptr);
        if ((rc = layer_launch(dev, m, kv, L, B, R, a->seq_len, a->max_ctx, P, x, ss, c, wide && L > 0u, next)))
            return rc;
    }
    if (!a->logits) return OPURE_OK;

    c.W = m->lm_head;
    c.x = wide ? static_cast<const void*>(ws + P.xn) : x;
    c.gain = wide ? nullptr : m->final_norm;
    c.norm_gain = nullptr;
    c.ss_out = nullptr;
    c.y = a->logits;
    c.yfmt = OPURE_A_F32;
    // up to OPURE_MAX_ROWS rows the LM head also leaves per-workgroup argmax
    // partials; beyond, the logits are stored and reduced per 4096 columns
        c.epi = wide ? EPI_STORE : EPI_LOGITS;
    c.logits.am_val = reinterpret_cast<float*>(ws + P.am_val);
    c.logits.am_idx = reinterpret_cast<int32_t*>(ws + P.am_idx);
    if ((rc = gemv_validate(c))) return rc;

    opure_rollback_args rb{};
    if (a->rollback)
    {
        rb.model = m;
        rb.kv = kv;
        rb.batch = B;
        rb.k = R - 1u;
        rb.seq_len = a->seq_len;
        rb.accepted = a->accepted;
        rb.new_seq_len = a->new_seq_len;
        rb.freed = a->freed;
        rb.freed_stride = a->freed_stride;
        rb.n_freed = a->n_freed;
        rb.poison = a->poison;
        rb.poison_bits = a->poison_bits;
        if ((rc = rollback_validate(&rb))) return rc;
    }
    // greedy acceptance and the rollback inside the LM head's launch: its last
    // workgroup gathers the others' argmax words (wave-per-tile kernel only)
    const bool fused = a->accept_mode == OPURE_ACCEPT_GREEDY && !wide && dev->acc_sync &&
                       dev->greedy_mode == OPURE_GREEDY_IN_LM_HEAD && gemv_is_wave_per_tile(dev, c) &&
                       gemv_grid(dev, c) <= ACC_SYNC_WGS;
    if (fused)
    {
        c.logits.acc_slots = static_cast<uint64_t*>(dev->acc_sync);
        c.logits.acc_epoch = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(dev->acc_sync) + ACC_SYNC_SLOT_BYTES);
        c.logits.drafts = a->tokens + 1;
        c.logits.drafts_stride = R;
        c.logits.K = R - 1u;
        c.logits.batch = B;
        c.logits.wait_limit = dev->wait_limit;
        c.logits.out_tokens = a->out_tokens;
        c.logits.accepted = a->accepted;
        c.logits.rollback = a->rollback ? 1u : 0u;
        if (a->rollback) c.logits.rb = rollback_params(&rb);
    }
    if ((rc = prof_begin(dev, OPURE_STAGE_LM_HEAD)) || (rc = gemv_launch(dev, c)) || (rc = prof_end(dev))) return rc;

    if (a->accept_mode != OPURE_ACCEPT_NONE && (rc = prof_begin(dev, OPURE_STAGE_ACCEPT))) return rc;
    if (a->accept_mode == OPURE_ACCEPT_GREEDY && !fused)
    {
        // greedy acceptance and the rollback run in one kernel
        uint32_t parts = 0;
        if (wide)
        {
            parts = argmax_parts(m->vocab);
            if ((rc = argmax_partials_launch(dev, a->logits, MR, m->vocab, c.logits.am_val, c.logits.am_idx))) return rc;
        }
        else
        {
            parts = gemv_grid(dev, c);
        }
        rc = greedy_from_partials(dev, c.logits.am_val, c.logits.am_idx, parts, B, R - 1u, a->tokens + 1, R,
                                  a->out_tokens, a->accepted, a->rollback ? &rb : nullptr);
        if (rc) return rc;
    }
    else if (a->accept_mode == OPURE_ACCEPT_REJECTION)
    {
        opure_accept_args aa{};
        aa.batch = B;
        aa.k = R - 1u;
        aa.vocab = m->vocab;
        aa.target_logits = a->logits;
        aa.draft_logits = a->draft_logits;
        aa.drafts = a->tokens + 1;
        aa.drafts_stride = R;
        aa.temperature = a->temperature;
        aa.seed = a->seed;
        aa.pos_base = a->pos_base;
        aa.out_tokens = a->out_tokens;
        aa.accepted = a->accepted;
        aa.dist_out = a->dist_out;
        rc = accept_rejection_launch(dev, &aa, ws + P.rej, nullptr, nullptr);
        if (rc) return rc;
        if (a->rollback && (rc = rollback_launch(dev, &rb))) return rc;
    }
    if (a->accept_mode != OPURE_ACCEPT_NONE && (rc = prof_end(dev))) return rc;
    return OPURE_OK;
}

}  // extern "C"
