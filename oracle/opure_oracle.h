/*
 * opure_oracle.h -- CPU oracle for the Opure speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the reference restatement the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  Nothing in the product links it.
 *
 * It restates the reference's scalar CPU forward pass,
 *   src/engine/Opure_CpuReference.cpp:151-347  (Gemv, RmsNorm, RoPE, SwiGLU,
 *                                               attention, per-token order)
 * in plain scalar C++ with double accumulation, and extends it to what the
 * reference never built (it has no verify step): K+1 query rows per sequence,
 * a batch of sequences, a paged KV cache, per-channel int8 and group-128 int4
 * weights, fp16/bf16 activation storage, greedy and rejection-sampling
 * acceptance (Philox4x32-10) and KV rollback.
 *
 * Every parameterised choice (RoPE table, attention scale, activation dtype,
 * tie-break) is data, not a code fork; the defaults follow the reference.
 *
 * Pinning status of each function is listed in tests/test_oracle_*.py and in
 * the header comment of opure_oracle.cpp.
 */
#ifndef OPURE_ORACLE_H
#define OPURE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* weight formats */
enum { ORC_W_F32 = 0, ORC_W_I8PC = 1, ORC_W_I4G128 = 2 };
/* activation / KV storage formats */
enum { ORC_A_F32 = 0, ORC_A_F16 = 1, ORC_A_BF16 = 2 };
/* RoPE frequency schedules (Opure_RoPE.usf:56 vs Opure_CpuReference.cpp:179) */
enum { ORC_ROPE_GPU = 0, ORC_ROPE_CPUREF = 1 };

typedef struct orc_linear {
    const void*     w;      /* f32: float[out*in]; i8: int8[out*in];
                               i4: uint8[out*in/2], element 2i in the high nibble */
    const uint16_t* scale;  /* i8: fp16[out]; i4: bf16[out*(in/128)] */
    const uint16_t* zero;   /* i4: bf16[out*(in/128)]; unused otherwise */
    uint32_t        out, in;
} orc_linear;

typedef struct orc_layer {
    const float* attn_norm;   /* [hidden] */
    const float* mlp_norm;    /* [hidden] */
    orc_linear   qkv;         /* rows [q (nh*hd); k (nkv*hd); v (nkv*hd)] x hidden */
    orc_linear   o;           /* hidden x (nh*hd) */
    orc_linear   gate_up;     /* rows [gate (ffn); up (ffn)] x hidden */
    orc_linear   down;        /* hidden x ffn */
} orc_layer;

typedef struct orc_model {
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab;
    float    rms_eps;
    float    attn_scale;      /* 1.0 reproduces the reference (no 1/sqrt(hd)) */
    uint32_t wfmt;            /* ORC_W_* for every linear, embed and lm_head */
    uint32_t afmt;            /* ORC_A_*: activations fed to GEMVs and the KV cache */
    const float* rope_cos;    /* [rope_max_pos][head_dim/2] */
    const float* rope_sin;
    uint32_t rope_max_pos;
    orc_linear embed;         /* [vocab, hidden] */
    orc_linear lm_head;       /* [vocab, hidden]; equal to embed when tied */
    const float* final_norm;  /* [hidden] */
    const orc_layer* layers;  /* [n_layers] */
} orc_model;

typedef struct orc_kv {
    void*    pool;            /* [n_layers][n_pages][2][n_kv] planes of page_size*hd afmt elements:
                                 K plane [page_size][hd] (token-major), V plane [hd][page_size]
                                 (channel-major) */
    uint32_t n_pages;
    uint32_t page_size;
    const int32_t* page_table;/* [batch][max_pages_per_seq] */
    uint32_t max_pages_per_seq;
} orc_kv;

/* ---- scalar numerics ---------------------------------------------------- */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);          /* round to nearest even */
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);         /* round to nearest even */
float    orc_expf(float x);                /* the shared exp (see .cpp) */
void     orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
uint32_t orc_philox_u32(uint64_t seed, uint32_t pos, uint32_t seq, uint32_t stream);
/* reference harness RNG (Opure_TestHarness.cpp:36-47) */
void     orc_xorshift_fill(uint64_t seed, float* out, uint64_t n, float mul, float add);
void     orc_xorshift_u32(uint64_t seed, uint32_t* out, uint64_t n);

/* ---- building blocks (row-major, M activation rows) -------------------- */
void orc_set_threads(int n);               /* 1 = scalar reference; >1 = OpenMP over rows */
void orc_gemv(const orc_linear* L, uint32_t wfmt, const float* x, float* y, uint32_t M);
void orc_rmsnorm_rows(const float* x, const float* g, float* y, uint32_t M, uint32_t d,
                      float eps, uint32_t afmt);
void orc_round_act(float* x, uint64_t n, uint32_t afmt);
void orc_rope_table(double theta, uint32_t head_dim, uint32_t max_pos, uint32_t mode,
                    float* cos_out, float* sin_out);
void orc_rope_rows(float* vec, uint32_t n_heads, uint32_t head_dim, const float* cos_t,
                   const float* sin_t, uint32_t pos);
void orc_swiglu(const float* g, const float* u, float* h, uint64_t n);

/* attention of R query rows of one sequence over its paged cache, one layer.
 * q: [R][n_heads*hd] (already rotated, already in storage precision).
 * Row j sees positions 0 .. ctx+j.  out: [R][n_heads*hd]. */
void orc_attention_paged(const orc_model* m, const orc_kv* kv, uint32_t layer,
                         uint32_t seq, uint32_t ctx, uint32_t R, const float* q, float* out);

/* ---- the verify forward ------------------------------------------------ */
/* tokens: [B][R] input ids (row 0 = last accepted token, rows 1.. = drafts).
 * seq_len: [B] tokens already in the cache; row j is at position seq_len[b]+j.
 * Writes K/V of every row into the cache, and logits [B][R][vocab].
 * Returns 0, or a negative code on a bad argument. */
int orc_verify_forward(const orc_model* m, orc_kv* kv, uint32_t B, uint32_t R,
                       const int32_t* tokens, const int32_t* seq_len, float* logits);

/* The forward in parts: orc_verify_forward = orc_verify_embed, then
 * orc_verify_layers(0, n_layers), then orc_verify_head, bit for bit.
 * x: fp32 residual [B*R][hidden].  orc_verify_layers applies layers
 * [first, first+count) to x in place and appends the rows' K/V to the cache
 * (the checks and return codes of orc_verify_forward). */
int orc_verify_embed(const orc_model* m, uint32_t MR, const int32_t* tokens, float* x);
int orc_verify_layers(const orc_model* m, orc_kv* kv, uint32_t B, uint32_t R, const int32_t* seq_len, float* x,
                      uint32_t first, uint32_t count);
int orc_verify_head(const orc_model* m, uint32_t MR, const float* x, float* logits);

/* Test hook: after the rounding of intermediate `stage` in layer `layer`,
 * element `index` moves by one unit in the last place of the activation
 * format (layer < 0 turns it off).  It measures how far one rounding decision
 * travels through the rest of the forward. */
enum { ORC_STAGE_XN_ATTN = 0, ORC_STAGE_Q = 1, ORC_STAGE_ATT = 2, ORC_STAGE_XN_MLP = 3, ORC_STAGE_H = 4 };
void orc_set_perturbation(int32_t layer, uint32_t stage, uint64_t index);

/* As orc_verify_forward, also recording layer 0's intermediates (the
 * reference's ForwardTraced idea, Opure_CpuReference.h:48-54):
 * trace = [q (MR*nh*hd, after RoPE, rounded) | att (MR*nh*hd) | x after the
 *          attention residual (MR*h) | h (MR*ffn) | x after the layer (MR*h) |
 *          final normed x (MR*h)] */
int orc_verify_forward_traced(const orc_model* m, orc_kv* kv, uint32_t B, uint32_t R,
                              const int32_t* tokens, const int32_t* seq_len, float* logits,
                              float* trace);

/* ---- acceptance -------------------------------------------------------- */
/* greedy: target_logits [B][K+1][V]; drafts [B][K].
 * out_tokens [B][K+1] (emitted: accepted drafts then the correction/bonus,
 * rest -1); accepted [B]. Ties in argmax go to the lowest index. */
void orc_accept_greedy(const float* target_logits, const int32_t* drafts, uint32_t B,
                       uint32_t K, uint32_t V, int32_t* out_tokens, int32_t* accepted);
void orc_argmax_rows(const float* logits, uint32_t rows, uint32_t V, int32_t* idx, float* val);

/* rejection sampling (Leviathan et al. 2023; Chen et al. 2023).
 * draft_logits [B][K][V]; temperature > 0; uniforms from Philox keyed by
 * (seed, seq, pos_base[b]+j).  dist_out [B][V] receives the distribution the
 * final token was drawn from (normalised residual, or p_K after full accept). */
void orc_accept_rejection(const float* target_logits, const float* draft_logits,
                          const int32_t* drafts, uint32_t B, uint32_t K, uint32_t V,
                          float temperature, uint64_t seed, const uint32_t* pos_base,
                          int32_t* out_tokens, int32_t* accepted, float* dist_out);

/* sample one token per row from softmax(logits/temperature) on Philox stream
 * `stream`, counter (pos[r], seq[r]). */
void orc_sample_rows(const float* logits, uint32_t rows, uint32_t V, float temperature,
                     uint64_t seed, const uint32_t* pos, const uint32_t* seq,
                     uint32_t stream, int32_t* out);

/* ---- KV rollback ------------------------------------------------------- */
/* For each sequence: new length = seq_len[b] + accepted[b] + 1 (the verify
 * step wrote seq_len[b] .. seq_len[b]+K).  Slots from the new length up to
 * seq_len[b]+K+1 are overwritten with `poison` in every layer (if
 * poison_bits != 0), pages wholly past the new length are released
 * (page_table entry -> -1, id appended to freed[b][...]).  Writes new_len[b]
 * and n_freed[b]. */
void orc_kv_rollback(orc_kv* kv, const orc_model* m, uint32_t B, uint32_t K,
                     const int32_t* seq_len, const int32_t* accepted,
                     int32_t* page_table_rw, int32_t* new_len, int32_t* freed,
                     uint32_t freed_stride, int32_t* n_freed, uint32_t poison_bits);

#ifdef __cplusplus
}
#endif
#endif
