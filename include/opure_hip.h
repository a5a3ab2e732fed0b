/*
 * opure_hip.h -- the C-ABI that replaces the reference's D3D12 dispatch layer
 * (src/core/Opure_Dx12.h, src/core/Opure_Shaders.h) for the speculative-
 * decoding verify path, implemented with hand-written gfx950 HIP kernels.
 *
 * Conventions
 *   - Every function returns int: OPURE_OK (0) or a negative OPURE_E_* code.
 *     opure_last_error() returns the calling thread's last message.  No C++
 *     exception crosses this boundary; the C++ engine turns codes back into
 *     opure::Error, as OPURE_CHECK / ThrowError do (Opure_Platform.h:45-85).
 *   - Device pointers are plain void* obtained from opure_buf_alloc (or any
 *     HIP allocation on the same device).  Argument structs are POD and are
 *     read during the call only.
 *   - One stream per device.  Calls on one device are not thread-safe; the
 *     caller serialises them (the reference's server does, Opure_Server.cpp:21-25).
 *   - Kernel entry points enqueue work and return; opure_stream_sync waits.
 *     Conditions only a kernel can see are reported at the next
 *     opure_stream_sync or opure_buf_download of that device, which then
 *     return a code instead of OPURE_OK (the outputs of the work before it
 *     are invalid): a token id outside the vocabulary (OPURE_E_INVALID; its
 *     row reads NaN), a row position seq_len + j at or past max_ctx or with no
 *     page in the page table (OPURE_E_CAPACITY; its K/V are not written and
 *     its attention is clamped), a bounded wait between waves that gave up
 *     (OPURE_E_DEVICE).
 *     Uploads and downloads are synchronous, like UploadToBuffer /
 *     ReadbackFromBuffer (Opure_Dx12.h:230-244).
 *
 * Data layouts (row-major interchange; the kernels read weights in the tiled
 * layout made by opure_tile_linear, see opure_linear below)
 *   linear (OPURE_W_F32)     w: float[out][in]
 *   linear (OPURE_W_I8PC)    w: int8[out][in], scale: fp16[out]; y = scale[o] * sum_i w*x
 *   linear (OPURE_W_I4G128)  w: uint8[out][in/2], element 2i in the high nibble
 *                            (Opure_Streamer.cpp:403-426 nibble order, unsigned),
 *                            scale, zero: bf16[out][in/128]; w(o,i) = s*(q - z)
 *   activations              [rows][width] in OPURE_A_F32 / F16 / BF16
 *   KV pool                  [n_layers][n_pages][2 (K,V)][n_kv_heads] planes of
 *                            page_size*head_dim elements in the model's activation
 *                            format: a K plane is token-major [page_size][head_dim],
 *                            a V plane channel-major [head_dim][page_size] (so V^T
 *                            tiles of 8 tokens are one 16-byte load); page_table
 *                            int32[batch][max_pages_per_seq] (-1 = none)
 *   rope table               float cos[max_pos][head_dim/2], sin[...] (interleaved
 *                            pairs (2p, 2p+1), Opure_RoPE.usf:7-10)
 */
#ifndef OPURE_HIP_H
#define OPURE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OPURE_OK              0
#define OPURE_E_INVALID      -1   /* null / misaligned pointer, bad shape or enum */
#define OPURE_E_NODEVICE     -2   /* no HIP device at that ordinal */
#define OPURE_E_HIP          -3   /* HIP runtime error; message has the detail */
#define OPURE_E_OOM          -4   /* device allocation failed */
#define OPURE_E_UNSUPPORTED  -5   /* weight/activation combination not built */
#define OPURE_E_CAPACITY     -6   /* rows > OPURE_MAX_ROWS, ctx past capacity, pages missing */
#define OPURE_E_DEVICE       -7   /* a kernel reported that its outputs are invalid (see below) */

#define OPURE_MAX_ROWS       16   /* rows of one sequence's verify step (K+1); GEMV rows scored by the K+1-row kernel */
#define OPURE_MAX_BATCH_ROWS 256  /* rows of one verify step or GEMV (batch * (K+1)); above OPURE_MAX_ROWS the
                                   * GEMV runs as a thin GEMM (16-bit activations, quantised weights) */
#define OPURE_PAGE_SIZE      16   /* KV tokens per page */

enum { OPURE_W_F32 = 0, OPURE_W_I8PC = 1, OPURE_W_I4G128 = 2 };
enum { OPURE_A_F32 = 0, OPURE_A_F16 = 1, OPURE_A_BF16 = 2 };
enum { OPURE_ROPE_GPU = 0, OPURE_ROPE_CPUREF = 1 };
enum { OPURE_EPI_STORE = 0, OPURE_EPI_RESIDUAL = 1, OPURE_EPI_SWIGLU = 2 };
enum { OPURE_ACCEPT_NONE = 0, OPURE_ACCEPT_GREEDY = 1, OPURE_ACCEPT_REJECTION = 2 };

typedef struct opure_dev opure_dev;
typedef struct opure_graph opure_graph;

/* ---- device: replaces dx12::Device::Initialize/Shutdown (Opure_Dx12.h:186-187) */
int         opure_dev_create(int ordinal, opure_dev** out);
int         opure_dev_destroy(opure_dev* dev);
const char* opure_dev_name(const opure_dev* dev);
uint64_t    opure_dev_hbm_bytes(const opure_dev* dev);
const char* opure_last_error(void);

/* ---- buffers: replaces GpuBuffer::Create/Destroy and the upload/readback
 *      calls (Opure_Dx12.h:155-156, :230-244) */
typedef struct opure_upload_range {
    void*       dptr;
    uint64_t    offset;
    const void* src;
    uint64_t    bytes;
} opure_upload_range;

int opure_buf_alloc(opure_dev* dev, uint64_t bytes, void** dptr);
int opure_buf_free(opure_dev* dev, void* dptr);
int opure_buf_upload(opure_dev* dev, void* dptr, uint64_t offset, const void* src, uint64_t bytes);
int opure_buf_upload_ranges(opure_dev* dev, const opure_upload_range* ranges, uint32_t n);
int opure_buf_download(opure_dev* dev, void* dst, const void* dptr, uint64_t offset, uint64_t bytes);
/* fills `count` 32-bit words with `value` using a kernel (safe inside graph capture) */
int opure_buf_fill_u32(opure_dev* dev, void* dptr, uint32_t value, uint64_t count);
int opure_buf_copy(opure_dev* dev, void* dst, const void* src, uint64_t bytes);

/* ---- stream: replaces ResetCommandList / ExecuteAndWait (Opure_Dx12.h:273-274) */
int opure_stream_begin(opure_dev* dev);
int opure_stream_sync(opure_dev* dev);

/* ---- graphs: capture a whole verify step once, replay it per step */
int opure_graph_begin(opure_dev* dev);
int opure_graph_end(opure_dev* dev, opure_graph** out);
int opure_graph_launch(opure_dev* dev, opure_graph* g);
int opure_graph_destroy(opure_graph* g);

/* ---- timing: replaces Begin/EndTimestamp + ResolveTimestampMs (Opure_Dx12.h:267-270) */
int opure_timer_begin(opure_dev* dev);
int opure_timer_end(opure_dev* dev);
int opure_timer_ms(opure_dev* dev, float* ms);

/* ---- streaming bandwidth of the device: `reps` launches that read `bytes`
 *      of src (OPURE_BW_READ) or copy them to dst (OPURE_BW_COPY), 16-byte
 *      nontemporal accesses, four 512-thread workgroups a CU, timed with the
 *      device's HIP events after one warm-up launch.  *gbs = bytes moved per
 *      second / 1e9 (a copy moves 2 * bytes).  The peak the kernels' roofline
 *      fractions are read against, beside the published 8 TB/s; the
 *      counterpart of the GEMV microbench's effective-GB/s line
 *      (Opure_TestHarness.cpp:1714-1754).  Pointers and bytes are 16-byte
 *      multiples; choose bytes well above the 256 MB last-level cache. */
enum { OPURE_BW_READ = 0, OPURE_BW_COPY = 1 };
int opure_bw_measure(opure_dev* dev, uint32_t mode, const void* src, void* dst, uint64_t bytes, uint32_t reps,
                     double* gbs);

/* ---- host helper: RoPE cos/sin table.  OPURE_ROPE_GPU uses theta^(-2p/hd)
 *      for pair p (Opure_RoPE.usf:56); OPURE_ROPE_CPUREF uses theta^(-4p/hd)
 *      (Opure_CpuReference.cpp:179).  Computed in double, stored as float. */
int opure_rope_table(double theta, uint32_t head_dim, uint32_t max_pos, uint32_t mode,
                     float* cos_out, float* sin_out);

/* ---- model description ------------------------------------------------ */
/* Weight layouts.  ROWMAJOR is the interchange format above (what loaders and
 * the quantisers produce).  Every compute entry point reads the TILED layout
 * made by opure_tile_linear:
 *   16-row tiles (out/16), each weight row cut into 64-byte blocks (16 f32,
 *   64 int8 or 128 uint4 values); tile t, block b is one 1 KB piece at
 *   (t * (in_bytes/64) + b) * 1024, and lane l = 16*g + r of a wave reads its
 *   16 bytes [16g, 16g+16) of row r's block at offset 16*l -- one contiguous
 *   1 KB load per wave, already in MFMA operand order.
 *   int8 is stored offset-binary (q ^ 0x80); uint4 elements e0..e7 of a
 *   32-bit word sit at nibbles 0,4,1,5,2,6,3,7 and the word is rotated left by
 *   3 bits, so that byte masks (one of them after a 4-bit rotation) and byte
 *   permutes yield element pairs in k order; scales follow the tiles: int8 fp16[tile][16], uint4
 *   uint32 (bf16 scale | bf16 zero << 16)[tile][in/128][16]; zero is unused.
 * TILED_SWIGLU additionally interleaves the rows of a [gate; up] linear
 * (out = 2F): tile t holds gate rows 8t..8t+7 and up rows 8t..8t+7 alternately,
 * so the SwiGLU epilogue finds each (gate, up) pair in one lane. */
#define OPURE_LAYOUT_ROWMAJOR      0u
#define OPURE_LAYOUT_TILED         1u
#define OPURE_LAYOUT_TILED_SWIGLU  2u

typedef struct opure_linear {
    const void* w;
    const void* scale;      /* ROWMAJOR I8PC: fp16[out]; I4G128: bf16[out][in/128]; TILED: see above */
    const void* zero;       /* ROWMAJOR I4G128: bf16[out][in/128]; TILED: unused */
    uint32_t    out, in;
    uint32_t    layout;     /* OPURE_LAYOUT_* */
} opure_linear;

/* Bytes of the tiled copy of an out x in linear. */
int opure_tiled_bytes(uint32_t wfmt, uint32_t out, uint32_t in, uint64_t* w_bytes, uint64_t* scale_bytes);
/* Rewrites the ROWMAJOR linear `src` into w_dst / scale_dst (device buffers of
 * opure_tiled_bytes) in layout OPURE_LAYOUT_TILED or _TILED_SWIGLU, and fills
 * *dst to describe it.  A pure permutation (plus the int8 sign flip): the
 * values the kernels compute with are exactly the row-major ones.  The
 * counterpart of the weight upload (Opure_Graph.cpp:500-528), done once at
 * load time. */
int opure_tile_linear(opure_dev* dev, uint32_t wfmt, uint32_t layout, const opure_linear* src, void* w_dst,
                      void* scale_dst, opure_linear* dst);

typedef struct opure_layer_weights {
    const float* attn_norm;   /* [hidden] fp32 */
    const float* mlp_norm;    /* [hidden] fp32 */
    opure_linear qkv;         /* rows [q; k; v] = (n_heads + 2 n_kv_heads) * head_dim, TILED */
    opure_linear o;           /* hidden x n_heads*head_dim, TILED */
    opure_linear gate_up;     /* rows [gate; up] = 2 ffn, TILED_SWIGLU */
    opure_linear down;        /* hidden x ffn, TILED */
} opure_layer_weights;

typedef struct opure_model {
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab;
    float    rms_eps;
    float    attn_scale;      /* 1.0 = the reference (no 1/sqrt(head_dim)) */
    uint32_t wfmt;            /* OPURE_W_* (all linears, embed and lm_head) */
    uint32_t afmt;            /* OPURE_A_*: activations fed to GEMVs and the KV cache */
    const float* rope_cos;    /* device [rope_max_pos][head_dim/2] */
    const float* rope_sin;
    uint32_t rope_max_pos;
    opure_linear embed;       /* [vocab][hidden], TILED (rows are gathered from the tiles) */
    opure_linear lm_head;     /* [vocab][hidden], TILED (same pointers as embed when tied) */
    const float* final_norm;  /* [hidden] */
    const opure_layer_weights* layers;   /* HOST array [n_layers] of device pointers */
} opure_model;

typedef struct opure_kv {
    void*    pool;
    uint32_t n_pages;
    uint32_t page_size;       /* must be OPURE_PAGE_SIZE */
    int32_t* page_table;      /* device [batch][max_pages_per_seq] */
    uint32_t max_pages_per_seq;
} opure_kv;

/* ---- batched GEMV: replaces GEMVMain / GEMVQuantMain (Opure_GEMV.usf:40-89,
 *      Opure_GEMV_Quant.usf:39-95).  Scores all M <= OPURE_MAX_ROWS activation
 *      rows in one pass over the weights.
 *        STORE:    y[m][o]  = sum_i W[o][i] x[m][i]            (y in yfmt)
 *        RESIDUAL: y[m][o] += sum_i W[o][i] x[m][i]            (y fp32)
 *        SWIGLU:   W rows = [gate; up] (out = 2F); y[m][f] = silu(g) * u  (y in yfmt)
 *      Weight/activation pairs built: F32/F32, I8PC/F16, I4G128/F16, I4G128/BF16. */
typedef struct opure_gemv_args {
    opure_linear W;           /* TILED (TILED_SWIGLU for the SwiGLU epilogue) */
    const void*  x;           /* [M][W.in] in xfmt */
    void*        y;
    uint32_t     M;
    uint32_t     xfmt, yfmt;
    uint32_t     epilogue;    /* OPURE_EPI_* */
} opure_gemv_args;

int opure_gemv_batched_f32(opure_dev* dev, const opure_gemv_args* a);
int opure_gemv_batched_i8pc(opure_dev* dev, const opure_gemv_args* a);
int opure_gemv_batched_i4g128(opure_dev* dev, const opure_gemv_args* a);

/* ---- paged decode attention for K+1 query rows: replaces AttentionMain{hd}
 *      and the never-dispatched SpeculativeVerifyMain{hd}
 *      (Opure_FlashAttention_Decode.usf:58-179, Opure_SpeculativeDecode.usf:60-189).
 *      q [batch*rows][n_heads*head_dim] (afmt), row j of sequence b sits at
 *      position seq_len[b]+j and sees positions 0..seq_len[b]+j; query head h
 *      reads KV head h / (n_heads/n_kv_heads).  out has q's shape and format. */
typedef struct opure_attn_args {
    const opure_model* model; /* n_heads, n_kv_heads, head_dim, attn_scale, afmt */
    const opure_kv*    kv;
    uint32_t           layer;
    uint32_t           batch, rows;
    const int32_t*     seq_len;     /* device [batch] */
    uint32_t           max_ctx;     /* host upper bound on seq_len[b] + rows */
    const void*        q;
    void*              out;
} opure_attn_args;

int opure_attn_decode_paged(opure_dev* dev, const opure_attn_args* a);

/* ---- acceptance ------------------------------------------------------- */
/* Greedy: argmax per row (ties -> lowest index; the reference's ArgMaxMain,
 * Opure_ArgMax.usf:33-86, re-specified), longest matching draft prefix, then
 * the correction (or bonus) token.  out_tokens[b][0..n] = accepted drafts then
 * the final token, -1 after.  Rejection (Leviathan et al. 2023): accept draft
 * x_j iff u_j * q_j(x_j) < p_j(x_j), u_j = Philox(seed; pos_base[b]+j, b, 1);
 * on rejection sample max(0, p - q) normalised, after K accepts sample p_K,
 * both by inverse CDF on Philox(seed; pos_base[b]+n, b, 2).  Probabilities use
 * an exact fixed-point partition sum (see accept.hip).  dist_out[b][V] (may
 * be NULL) receives the distribution the final token was drawn from. */
typedef struct opure_accept_args {
    uint32_t       batch, k, vocab;
    const float*   target_logits;   /* [batch][k+1][vocab] */
    const float*   draft_logits;    /* [batch][k][vocab] (rejection only) */
    const int32_t* drafts;          /* [batch][drafts_stride], first k used */
    uint32_t       drafts_stride;
    float          temperature;     /* rejection only, > 0 */
    uint64_t       seed;
    const uint32_t* pos_base;       /* device [batch] or NULL (all 0) */
    int32_t*       out_tokens;      /* [batch][k+1] */
    int32_t*       accepted;        /* [batch] */
    float*         dist_out;        /* [batch][vocab] or NULL */
} opure_accept_args;

int opure_accept_greedy(opure_dev* dev, const opure_accept_args* a);
int opure_accept_rejection(opure_dev* dev, const opure_accept_args* a);

/* The same rejection sampling as opure_accept_rejection, for callers that
 * cannot allocate device memory (code under hipGraph capture, serving loops,
 * harnesses that forbid hipMalloc); it has no counterpart in the reference.
 * Its scratch is a device array of OPURE_NOALLOC_SCRATCH_BYTES built into the
 * library (one per GPU, held until the process ends); the call never
 * allocates or frees.  A shape needs batch * (2k + 1) * 16, batch *
 * ceil(vocab / 4096) * 16, batch * vocab * 4 and, for the rows' slice
 * statistics, batch * (2k + 1) * (ceil(vocab / 4096) * 12 + 4) bytes of it
 * (each part rounded up to 256); one that does not fit returns
 * OPURE_E_CAPACITY (at vocab 128256, up to 65 sequences fit with one draft
 * each, 64 with 3 to 7).  Every call on one GPU shares that GPU's array, so calls
 * that overlap on one GPU (streams of two opure_dev handles) race. */
#define OPURE_NOALLOC_SCRATCH_BYTES (32ull << 20)
int opure_accept_rejection_noalloc(opure_dev* dev, const opure_accept_args* a);

/* sample one id per row from softmax(logits/temperature) (Philox stream
 * `stream`, counter (pos[r], seq[r])): drafting at temperature. */
typedef struct opure_sample_args {
    uint32_t        rows, vocab;
    const float*    logits;         /* [rows][vocab] */
    float           temperature;
    uint64_t        seed;
    const uint32_t* pos;            /* device [rows] */
    const uint32_t* seq;            /* device [rows] */
    uint32_t        stream;
    int32_t*        out;            /* device [rows] */
} opure_sample_args;

int opure_sample_rows(opure_dev* dev, const opure_sample_args* a);

/* Philox4x32-10 test hook: out[i] = word 0 of Philox(seed; pos[i], seq[i], stream, 0). */
int opure_philox_uniform(opure_dev* dev, uint64_t seed, const uint32_t* pos, const uint32_t* seq,
                         uint32_t stream, uint32_t n, uint32_t* out);

/* ---- KV rollback: after accepting accepted[b] of k drafts, the valid cache
 *      is seq_len[b] + accepted[b] + 1 tokens.  Slots past it that the verify
 *      step wrote are overwritten with poison_bits (when poison != 0), pages
 *      wholly past it are released: page_table entry -> -1 and the id appended
 *      to freed[b][...].  Replaces the broken EvictOldestKV
 *      (Opure_VoxelEngine.cpp:721-763). */
typedef struct opure_rollback_args {
    const opure_model* model;
    const opure_kv*    kv;           /* kv->page_table is updated in place */
    uint32_t           batch, k;     /* k + 1 <= OPURE_MAX_ROWS (the rows of the verify step rolled back) */
    const int32_t*     seq_len;
    const int32_t*     accepted;
    int32_t*           new_seq_len;
    int32_t*           freed;        /* [batch][freed_stride] or NULL */
    uint32_t           freed_stride; /* >= ceil(k / OPURE_PAGE_SIZE), the most pages one rollback releases */
    int32_t*           n_freed;      /* [batch] or NULL */
    uint32_t           poison;
    uint32_t           poison_bits;  /* element bits in the model's afmt */
} opure_rollback_args;

int opure_kv_rollback(opure_dev* dev, const opure_rollback_args* a);

/* ---- one verify step: embedding, every layer (RMSNorm -> fused QKV GEMV
 *      with RoPE and paged KV append -> paged attention -> o_proj + residual
 *      -> RMSNorm -> gate/up GEMV with SwiGLU -> down_proj + residual), final
 *      RMSNorm, LM head, then the acceptance stage and rollback.  Replaces
 *      VoxelEngine::RecordForward (Opure_VoxelEngine.cpp:189-536) for K+1
 *      rows and a batch of sequences. */
typedef struct opure_verify_args {
    const opure_model* model;
    const opure_kv*    kv;
    uint32_t           batch, rows;  /* rows = K + 1; batch * rows <= OPURE_MAX_ROWS */
    const int32_t*     tokens;       /* device [batch][rows]: last token, then K drafts */
    const int32_t*     seq_len;      /* device [batch] */
    uint32_t           max_ctx;      /* host upper bound on seq_len[b] + rows */
    float*             logits;       /* device [batch][rows][vocab]; NULL (with OPURE_ACCEPT_NONE): a prefill,
                                      * which writes the rows' K/V and stops before the LM head */
    uint32_t           accept_mode;  /* OPURE_ACCEPT_* */
    const float*       draft_logits; /* rejection: [batch][rows-1][vocab] */
    float              temperature;
    uint64_t           seed;
    const uint32_t*    pos_base;     /* device [batch] or NULL */
    int32_t*           out_tokens;   /* [batch][rows] */
    int32_t*           accepted;     /* [batch] */
    float*             dist_out;     /* [batch][vocab] or NULL */
    uint32_t           rollback;     /* 1: run opure_kv_rollback after acceptance */
    int32_t*           new_seq_len;  /* [batch] (required when rollback) */
    int32_t*           freed;
    uint32_t           freed_stride;
    int32_t*           n_freed;
    uint32_t           poison;
    uint32_t           poison_bits;
} opure_verify_args;

/* Sizes the device's internal workspace for this model and shape; call it
 * before capturing a verify step into a graph (capture cannot allocate). */
int opure_verify_reserve(opure_dev* dev, const opure_model* model, uint32_t batch, uint32_t rows,
                         uint32_t max_ctx);
int opure_verify_step(opure_dev* dev, const opure_verify_args* a);

/* ---- one layer of the verify step on a caller's residual: rmsnorm -> fused
 *      QKV GEMV with RoPE and paged K/V append -> paged attention -> o_proj +
 *      residual -> rmsnorm -> gate/up GEMV with SwiGLU -> down + residual, the
 *      same kernels as one iteration of opure_verify_step's layer loop.
 *      x (fp32 [batch*rows][hidden]) is updated in place; the rows' K/V are
 *      appended to layer `layer` of the cache.  The RMSNorm's sums of squares
 *      are recomputed from x (a step carries them from the previous layer), so
 *      the normalised rows can differ from a step's in the last bit.  Replaces
 *      the body of RecordForward's layer loop (Opure_VoxelEngine.cpp:296-492)
 *      and the per-layer runs of RunLayersTraced (Opure_VoxelEngine.h:226-227). */
typedef struct opure_verify_layer_args {
    const opure_model* model;
    const opure_kv*    kv;
    uint32_t           layer;
    uint32_t           batch, rows;  /* batch * rows <= OPURE_MAX_BATCH_ROWS, rows <= OPURE_MAX_ROWS */
    const int32_t*     seq_len;      /* device [batch]: row j of sequence b sits at seq_len[b] + j */
    uint32_t           max_ctx;      /* host upper bound on seq_len[b] + rows */
    float*             x;            /* device [batch*rows][hidden] fp32 residual, in and out */
} opure_verify_layer_args;

int opure_verify_layer(opure_dev* dev, const opure_verify_layer_args* a);

/* ---- stage timing of eager verify steps.  With profiling on, every stage of
 *      opure_verify_step is bracketed by HIP events on the device's stream
 *      (skipped while a graph is being captured).  opure_profile_read waits
 *      for the stream, returns per stage the number of bracketed launches and
 *      their summed milliseconds since the last read, and starts over.  The
 *      counterpart of the per-layer timings of MetricsSnapshot
 *      (src/engine/Opure_Metrics.h:42-43). */
#define OPURE_STAGE_EMBED    0u   /* embedding gather                          */
#define OPURE_STAGE_QKV      1u   /* rmsnorm + qkv GEMV + RoPE + K/V append    */
#define OPURE_STAGE_ATTN     2u   /* paged attention (chunks + combine)        */
#define OPURE_STAGE_O        3u   /* o_proj GEMV + residual                    */
#define OPURE_STAGE_GATE_UP  4u   /* rmsnorm + gate/up GEMV + SwiGLU           */
#define OPURE_STAGE_DOWN     5u   /* down GEMV + residual                      */
#define OPURE_STAGE_LM_HEAD  6u   /* final rmsnorm + LM head + argmax partials */
#define OPURE_STAGE_ACCEPT   7u   /* acceptance and KV rollback                */
#define OPURE_STAGE_COUNT    8u
int opure_profile_enable(opure_dev* dev, int on);
int opure_profile_read(opure_dev* dev, uint32_t counts[OPURE_STAGE_COUNT], double ms[OPURE_STAGE_COUNT]);

/* ---- diagnostics: the device workspace of the last verify step, so a test
 *      can read layer intermediates (run with n_layers = 1 to see layer 0).
 *      The counterpart of ReadActBank / RunLayersTraced (Opure_VoxelEngine.h:
 *      173-178, :226-227).  offsets[0..4] = byte offsets of x (fp32 residual,
 *      [rows][hidden]), ss (fp32 sums of squares of x per 16-column tile,
 *      [hidden/16][rows], feeding the fused RMSNorm), q (afmt), att (afmt),
 *      h (afmt). */
int opure_debug_workspace(opure_dev* dev, void** ptr, uint64_t* bytes);
/* Sleeps a bounded wait takes before it gives up (default 4M): between the
 * waves of a GEMV workgroup, between the slices of a sequence in the
 * one-launch rejection step, or in the LM head's greedy acceptance.  A test hook: 0 makes any wait that is not already met give
 * up at once, so the failure report can be checked while every wave still
 * runs to its end. */
int opure_debug_set_wait_limit(opure_dev* dev, uint32_t sleeps);
/* GEMV engine of opure_gemv_batched_* at M <= 8 rows with a STORE / RESIDUAL /
 * SWIGLU epilogue: the matrix-core kernels (default) or the vector-ALU kernel
 * (one output row per lane: v_fma_f32 for fp32 weights, v_dot2_f32_f16 for
 * int8 and uint4 with fp16 X, v_dot2_f32_bf16 for uint4 with bf16 X), kept for
 * the engine comparison.  The verify step always uses the matrix cores. */
enum { OPURE_GEMV_MFMA = 0, OPURE_GEMV_VALU = 1 };
int opure_debug_set_gemv_engine(opure_dev* dev, uint32_t engine);
/* Launches of opure_accept_rejection (and of the rejection step inside
 * opure_verify_step): one launch whose slices of a sequence wait for each
 * other (default), or the separate row-statistics, slice and draw launches,
 * kept for comparison.  Both give the same bits. */
enum { OPURE_REJ_ONE_LAUNCH = 0, OPURE_REJ_STAGED = 1 };
int opure_debug_set_rejection_launches(opure_dev* dev, uint32_t mode);
/* Greedy acceptance (and its rollback) inside opure_verify_step: run by the
 * LM head's own launch where its kernel allows (default: the last workgroup
 * gathers every workgroup's argmax through tagged words), or by a separate
 * launch after it, kept for comparison.  Both give the same tokens, accepted
 * lengths and rollback. */
enum { OPURE_GREEDY_IN_LM_HEAD = 0, OPURE_GREEDY_SEPARATE = 1 };
int opure_debug_set_greedy_acceptance(opure_dev* dev, uint32_t mode);
/* Evaluates the SwiGLU epilogue's branch-free exponential and the oracle-order
 * exponential the other kernels use on every one of the 2^32 fp32 bit
 * patterns and counts the results that differ (bit for bit; 0 expected). */
int opure_debug_exp_check(opure_dev* dev, uint64_t* mismatches);
int opure_debug_verify_offsets(const opure_model* model, uint32_t batch, uint32_t rows, uint32_t max_ctx,
                               uint64_t offsets[5]);

/* ---- synthetic seeded weights (N(0, std) from Philox, stream `tensor_id`)
 *      and device-side quantisers, so full-size models need no host copy. */
int opure_synth_normal_f32(opure_dev* dev, float* dst, uint64_t n, uint64_t seed, uint32_t tensor_id,
                           float std, float mean);
int opure_quantize_i8pc(opure_dev* dev, const float* w, uint32_t out, uint32_t in, int8_t* q,
                        uint16_t* scale_f16);
int opure_quantize_i4g128(opure_dev* dev, const float* w, uint32_t out, uint32_t in, uint8_t* q,
                          uint16_t* scale_bf16, uint16_t* zero_bf16);
int opure_convert_f32(opure_dev* dev, const float* src, void* dst, uint32_t afmt, uint64_t n);

#ifdef __cplusplus
}
#endif
#endif
