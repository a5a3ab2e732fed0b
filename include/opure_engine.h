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
 * VerifyStep (SURVEY's build plan; the reference has none). */
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
