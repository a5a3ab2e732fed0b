/* ============================================================================
 *  opure_engine.h -- C-ABI of the native generation engine (libopure_engine.so)
 *
 *  The engine is the C++20 class opure::engine::VoxelEngine
 *  (opure-voxelengine_amd/engine/voxel_engine.h), which keeps the reference
 *  engine's shape -- Initialize / Prefill / DecodeStep / Generate
 *  (src/engine/Opure_VoxelEngine.h:127-200) -- and adds the speculative loop:
 *  draft K tokens with a small model, score them with one K+1-row verify step
 *  of the target (opure_verify_step), keep the accepted prefix and the
 *  correction token, roll the caches back.  These functions wrap it for
 *  callers that are not C++ (the Python tests and benchmark bind them with
 *  ctypes).  Errors: every function returns OPURE_OK or a negative
 *  OPURE_E_* code; opure_engine_last_error() holds the calling thread's
 *  message.  No exception crosses this boundary.
 *
 *  The engine borrows the device and the models (their weights and the host
 *  array of layer descriptors must outlive it) and owns its KV pools, page
 *  tables, step buffers and captured graphs.  Each model's KV pool is a set of
 *  16-token pages handed out by a free list as the sequence grows and given
 *  back by the rollback; prompts of quantised models are prefilled 256 rows a
 *  launch.
 * ========================================================================== */
#ifndef OPURE_ENGINE_H
#define OPURE_ENGINE_H

#include <stdint.h>

#include "opure_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct opure_engine opure_engine;

const char* opure_engine_last_error(void);

typedef struct opure_engine_options {
    uint32_t max_positions;   /* cache capacity per model, tokens (prompt + generated + K + 1) */
    uint32_t draft_tokens;    /* K for GenerateSpeculative (1..15) */
    uint32_t use_graphs;      /* 1: replay captured hipGraphs for the fixed-shape steps */
    int32_t  stop_token;      /* < 0: none */
} opure_engine_options;

typedef struct opure_engine_stats {
    uint32_t emitted;         /* tokens returned */
    uint32_t verify_steps;    /* target steps after the prefill */
    uint32_t draft_steps;     /* single-row draft steps */
    uint32_t accepted_total;  /* drafts accepted over all verify steps */
    double   ms_prefill;      /* prompt prefill of target (and draft) */
    double   ms_generate;     /* everything after the prefill */
} opure_engine_stats;

/* draft may be NULL (then only opure_engine_generate is available) */
int opure_engine_create(opure_dev* dev, const opure_model* target, const opure_model* draft,
                        const opure_engine_options* opts, opure_engine** out);
int opure_engine_destroy(opure_engine* e);

/* Greedy decoding of the target alone, one token per step (the reference's
 * Generate, Opure_VoxelEngine.cpp:894-958).  out[n_new]. */
int opure_engine_generate(opure_engine* e, const int32_t* prompt, uint32_t n_prompt, uint32_t n_new, int32_t* out,
                          opure_engine_stats* stats);

/* ForwardLogits of the reference (Opure_VoxelEngine.h:141-147), its parity
 * entry point: prefills tokens[0..n) into a fresh cache of the target and
 * writes the last position's logits[vocab]; *argmax (may be NULL) = their
 * argmax, ties to the lowest index. */
int opure_engine_forward_logits(opure_engine* e, const int32_t* tokens, uint32_t n, float* logits, uint32_t* argmax);

/* Greedy speculative decoding: the emitted ids equal opure_engine_generate's
 * for any draft model.  out[n_new]; accepted_hist[hist_cap] (may be NULL)
 * receives the accepted count of each verify step, in order. */
int opure_engine_generate_speculative(opure_engine* e, const int32_t* prompt, uint32_t n_prompt, uint32_t n_new,
                                      int32_t* out, uint32_t* accepted_hist, uint32_t hist_cap,
                                      opure_engine_stats* stats);

/* One verify step of the target on explicit rows: tokens[0] is the last
 * accepted token, tokens[1..n) the drafts, at positions seq_len .. seq_len +
 * n - 1 (n <= OPURE_MAX_ROWS); greedy acceptance.  *accepted = drafts kept;
 * out[0 .. *accepted] = those drafts then the target's own next token.  The
 * rows' K/V stay in the cache until opure_engine_rollback_kv.  The engine's
 * VerifyStep (the reference has none). */
int opure_engine_verify_step(opure_engine* e, const int32_t* tokens, uint32_t n, uint32_t seq_len, int32_t* out,
                             uint32_t* accepted);
/* After a verify step of k drafts at seq_len that kept `accepted`: the cache
 * keeps seq_len + accepted + 1 positions, the rest are rolled back and the
 * pages wholly past them return to the pool.  *new_len = the kept length.
 * Replaces EvictOldestKV (src/engine/Opure_VoxelEngine.cpp:721-763). */
int opure_engine_rollback_kv(opure_engine* e, uint32_t seq_len, uint32_t accepted, uint32_t k, uint32_t* new_len);
/* Page accounting of the target's (draft != 0: the draft's) KV pool: pages in
 * the pool, pages free, and the sequence's page-table row (-1 = no page) into
 * row[0 .. min(row_cap, *row_len)). */
int opure_engine_pages(const opure_engine* e, int draft, uint32_t* total, uint32_t* available, int32_t* row,
                       uint32_t row_cap, uint32_t* row_len);

/* Running totals since opure_engine_create or the last reset.  Replaces the
 * reference's speculativeAcceptance, which is declared but always -1 because
 * nothing drafts (src/engine/Opure_Metrics.cpp:65-68, set from
 * Opure_VoxelEngine.cpp:666). */
typedef struct opure_engine_metrics {
    uint64_t generate_calls;          /* generate / generate_speculative calls with n_new > 0 */
    uint64_t verify_steps;            /* speculative verify steps */
    uint64_t drafts_proposed;         /* K per speculative verify step */
    uint64_t drafts_accepted;
    uint64_t tokens_emitted;          /* ids returned by both generators */
    double   speculative_acceptance;  /* drafts_accepted / drafts_proposed; -1 before any speculative step */
} opure_engine_metrics;

int opure_engine_get_metrics(const opure_engine* e, opure_engine_metrics* out);
int opure_engine_reset_metrics(opure_engine* e);

/* ---- model directories: config.json + model.safetensors (or the shards of
 *      model.safetensors.index.json) in the Llama layout.  Replaces the
 *      reference's Graph::LoadConfigOnly / UploadWeights and
 *      ModelSpec::Resolve (src/engine/Opure_Graph.cpp:267-300, :430-530;
 *      src/engine/Opure_ModelSpec.cpp:120-320) and its safetensors reader
 *      (src/core/Opure_Streamer.h), whose packed-int4 sizes and per-tensor
 *      scale uploads are wrong (ElementBytes(I4) = 1, Opure_Streamer.cpp:
 *      104-117; every scale uploaded from one loop variable's address,
 *      Opure_Graph.cpp:521-527).
 *
 *      Stored forms (X = e.g. model.layers.0.self_attn.q_proj):
 *        float      X.weight F32 / F16 / BF16 [out][in]
 *        int8 pc    X.weight I8 [out][in], X.weight_scale F16 [out] (or [out][1])
 *        int4 g128  X.weight U8 [out][in/2] or U4 [out][in], element 2i in the
 *                   high nibble; X.weight_scale BF16 [out][in/128];
 *                   X.weight_zero BF16 [out][in/128] (absent: 0);
 *                   w = scale * (q - zero).  I4 [out][in]: signed, zero 8.
 *        the reference's form: I8 / U4 / I4 with a "scale" number in the
 *                   header entry, w = q * scale (per tensor)
 *      q/k/v and gate/up are fused on load; a float linear of a model that
 *      computes in int8 / int4 is quantised on the device at load time.
 *      config.json: vocab_size, hidden_size, intermediate_size,
 *      num_hidden_layers, num_attention_heads, num_key_value_heads, head_dim,
 *      max_position_embeddings, rms_norm_eps, rope_theta, tie_word_embeddings
 *      (default true, as the reference), quantization_config.activation_dtype
 *      ("float16" | "bfloat16" | "float32").  hidden_act other than silu,
 *      bias terms, rope_scaling and a head_dim that is not a multiple of 16 in
 *      16..256 are OPURE_E_UNSUPPORTED (the reference takes 64 and 128 only,
 *      Opure_Graph.cpp:167-174). */
enum {
    OPURE_ROLE_EMBED = 0, OPURE_ROLE_LM_HEAD = 1, OPURE_ROLE_QKV = 2, OPURE_ROLE_O = 3, OPURE_ROLE_GATE_UP = 4,
    OPURE_ROLE_DOWN = 5, OPURE_ROLE_ATTN_NORM = 6, OPURE_ROLE_MLP_NORM = 7, OPURE_ROLE_FINAL_NORM = 8
};

/* RoPE pairing the stored q_proj / k_proj rows were trained with.  The kernels
 * (and the reference: Opure_RoPE.usf:7-10, Opure_CpuReference.cpp:171-189)
 * rotate adjacent channels (2p, 2p+1) of a head.  ADJACENT uses the rows as
 * stored, which is what the reference does with every file it loads,
 * including HF checkpoints.  HALF is for checkpoints trained with
 * rotate-half pairs (p, p + head_dim/2), such as HF Llama's q_proj / k_proj:
 * each head's rows are permuted at load, new row 2p = row p and new row 2p+1
 * = row p + head_dim/2 (with their scales and zero points), so the adjacent
 * rotation computes the checkpoint's attention exactly (the same permutation
 * of q and k leaves every q.k unchanged; v and o_proj are untouched).  To
 * convert a file offline instead, apply that permutation to the rows of
 * q_proj and k_proj of every layer and load it as ADJACENT. */
enum { OPURE_ROPE_PAIRS_ADJACENT = 0, OPURE_ROPE_PAIRS_HALF = 1 };

typedef struct opure_load_options {
    uint32_t max_positions;   /* RoPE table rows; 0: config.json's max_position_embeddings */
    int32_t  wfmt;            /* OPURE_W_* to compute in; -1: as stored (the first q_proj's form) */
    int32_t  afmt;            /* OPURE_A_*; -1: quantization_config.activation_dtype, else F32 / F16 / BF16
                               * for float / int8 / int4 weights */
    float    attn_scale;      /* 0: 1/sqrt(head_dim); 1.0: the reference's unscaled scores */
    uint32_t rope_pairs;      /* OPURE_ROPE_PAIRS_*: 0 (ADJACENT, the reference) or HALF (HF rotate-half files) */
} opure_load_options;

typedef struct opure_model_info {
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_position_embeddings;
    float    rms_eps, attn_scale;
    double   rope_theta;
    uint32_t tied;
    uint32_t stored_wfmt;     /* form of the first q_proj on disk */
    uint32_t wfmt, afmt;      /* what the loaded model computes in */
    uint32_t rope_max_pos;
    uint32_t n_tensors;
    uint64_t file_bytes;
} opure_model_info;

/* Host half of loading (no device calls): config.json parsed, weights mapped,
 * every tensor found and shape-checked.  opts may be NULL (all defaults). */
typedef struct opure_model_files opure_model_files;
int opure_model_files_open(const char* model_dir, const opure_load_options* opts, opure_model_files** out);
int opure_model_files_info(const opure_model_files* f, opure_model_info* out);
/* One role (layer ignored for EMBED, LM_HEAD, FINAL_NORM) in the row-major
 * interchange form of opure_hip.h, as stored (float linears widened to fp32;
 * norms: out = hidden, in = 1, fp32).  The buffers belong to f and stay
 * valid until the next read or close. */
typedef struct opure_host_linear {
    uint32_t wfmt, out, in;
    const void* w;
    const void* scale;
    const void* zero;
    uint64_t w_bytes, scale_bytes, zero_bytes;
} opure_host_linear;
int opure_model_files_read(opure_model_files* f, uint32_t role, uint32_t layer, opure_host_linear* out);
int opure_model_files_close(opure_model_files* f);

/* A model directory on the device, tiled, with its RoPE table: *desc is
 * valid (and its weights resident) until opure_model_unload. */
typedef struct opure_loaded_model opure_loaded_model;
int opure_model_load(opure_dev* dev, const char* model_dir, const opure_load_options* opts, opure_loaded_model** out);
int opure_loaded_model_desc(const opure_loaded_model* m, const opure_model** desc, uint64_t* device_bytes);
int opure_model_unload(opure_loaded_model* m);

/* Initialize(modelDir, ...) of the reference (Opure_VoxelEngine.h:127-140):
 * loads the target (and the draft, when draft_dir is not NULL) from their
 * directories and creates an engine that owns them; opure_engine_destroy
 * frees the models too. */
int opure_engine_initialize(opure_dev* dev, const char* target_dir, const char* draft_dir,
                            const opure_load_options* load, const opure_engine_options* opts, opure_engine** out);

/* ---- safetensors files, read-only (host, no device calls) */
typedef struct opure_safetensors opure_safetensors;
enum { OPURE_DT_F32 = 0, OPURE_DT_F16 = 1, OPURE_DT_BF16 = 2, OPURE_DT_U8 = 3, OPURE_DT_I8 = 4, OPURE_DT_U4 = 5,
       OPURE_DT_I4 = 6 };
typedef struct opure_tensor_info {
    const char* name;         /* valid while the file is open */
    uint32_t dtype;           /* OPURE_DT_* */
    uint32_t ndim;            /* <= 8 */
    int64_t  shape[8];
    uint64_t offset;          /* bytes from the start of the file */
    uint64_t bytes;           /* stored bytes (packed 4-bit: two elements a byte) */
    const void* data;         /* in the read-only mapping */
    uint32_t has_scale;       /* the entry carries the reference's "scale" key */
    double   scale;
} opure_tensor_info;
/* Maps the file and checks every entry's byte span against its shape and
 * dtype; OPURE_E_INVALID names the first bad entry. */
int opure_safetensors_open(const char* path, opure_safetensors** out);
int opure_safetensors_count(const opure_safetensors* f, uint32_t* n);
int opure_safetensors_tensor(const opure_safetensors* f, uint32_t i, opure_tensor_info* out);
/* OPURE_E_INVALID when absent */
int opure_safetensors_find(const opure_safetensors* f, const char* name, opure_tensor_info* out);
int opure_safetensors_close(opure_safetensors* f);

/* ---- page pool: the free list of a paged KV pool's pages (host bookkeeping,
 *      no device calls).  Sequences own 16-token pages through their
 *      page-table rows (opure_kv.page_table); a row takes pages as the
 *      sequence grows and opure_kv_rollback's freed lists give them back.
 *      Replaces the reference's fixed contiguous cache
 *      (ModelConfig::KvCacheWords, src/engine/Opure_Graph.h:81-84) and its
 *      EvictOldestKV (src/engine/Opure_VoxelEngine.cpp:721-763).  Not
 *      thread-safe. */
typedef struct opure_page_pool opure_page_pool;

int opure_page_pool_create(uint32_t n_pages, opure_page_pool** out);
int opure_page_pool_destroy(opure_page_pool* p);
/* *out = pages free now */
int opure_page_pool_available(const opure_page_pool* p, uint32_t* out);
/* n pages into ids[n], all or none (OPURE_E_CAPACITY when fewer are free).
 * A fresh pool hands out 0, 1, 2, ...; released pages are handed out again
 * first, last released first. */
int opure_page_pool_alloc(opure_page_pool* p, uint32_t n, int32_t* ids);
/* Entries < 0 are skipped (the -1 padding of opure_kv_rollback's freed
 * lists).  An id past the pool, not handed out, or listed twice is
 * OPURE_E_INVALID and releases nothing. */
int opure_page_pool_release(opure_page_pool* p, const int32_t* ids, uint32_t n);
/* Entries [0, ceil(tokens / OPURE_PAGE_SIZE)) of one host page-table row
 * made valid, a page taken for each entry < 0; all or none (OPURE_E_CAPACITY
 * when the row or the pool is too short).  *added (may be NULL) = pages
 * taken.  The caller uploads the row before the step that writes there. */
int opure_page_pool_grow_seq(opure_page_pool* p, int32_t* row, uint32_t max_pages, uint32_t tokens,
                             uint32_t* added);

#ifdef __cplusplus
}
#endif

#endif /* OPURE_ENGINE_H */
