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
 *  tables, step buffers and captured graphs.
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

#ifdef __cplusplus
}
#endif

#endif /* OPURE_ENGINE_H */
