// ============================================================================
//  internal.h -- shared host and device internals of libopure_hip.
// ============================================================================
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/opure_hip.h"

// ---------------------------------------------------------------------------
//  Host side: device object, errors, workspace
// ---------------------------------------------------------------------------
constexpr uint32_t REJ_SYNC_SEQS = 4096;
constexpr uint64_t REJ_SYNC_BYTES = REJ_SYNC_SEQS * 4ull + REJ_SYNC_SEQS * 64ull * 6ull * 8ull;
// The LM head's in-launch greedy acceptance: tagged (value, index) words of
// up to ACC_SYNC_WGS workgroups x OPURE_MAX_ROWS rows, then the launch count
constexpr uint32_t ACC_SYNC_WGS = 4096;
constexpr uint64_t ACC_SYNC_SLOT_BYTES = uint64_t(ACC_SYNC_WGS) * 16u * 2u * 8u;
constexpr uint64_t ACC_SYNC_BYTES = ACC_SYNC_SLOT_BYTES + 256u;

struct opure_dev {
    int         ordinal = 0;
    hipStream_t stream = nullptr;
    hipEvent_t  ev_begin = nullptr, ev_end = nullptr;
    char        name[256] = {0};
    uint64_t    hbm = 0;
    int         n_cu = 0;
    bool        capturing = false;
    // Grow-only workspace used by the kernels (attention partials, acceptance
    // statistics, activations of a verify step).
    void*       ws = nullptr;
    uint64_t    ws_bytes = 0;
    // device address of opure_accept_rejection_noalloc's scratch array (looked up once)
    void*       noalloc_scratch = nullptr;
    // The one-launch rejection sampler's per-sequence state (REJ_SYNC_BYTES,
    // zeroed once at creation): a launch count a sequence [REJ_SYNC_SEQS] u32,
    // then the sequences' slots [REJ_SYNC_SEQS][64 slices][6] u64, whose tags
    // carry the launch count, so no clear is needed between launches.
    void*       rej_sync = nullptr;
    // The LM head's in-launch greedy acceptance state (ACC_SYNC_BYTES): the
    // workgroups' tagged words, zeroed, then the launch count, which starts
    // at 0x01010101 (a zero word never carries a live tag); reset after a
    // bounded wait gave up (check_device_errors)
    void*       acc_sync = nullptr;
    // greedy acceptance inside the LM head's launch where the shape allows
    // (opure_debug_set_greedy_acceptance)
    uint32_t    greedy_mode = OPURE_GREEDY_IN_LM_HEAD;
    // Conditions a kernel found that make its outputs invalid, one word each
    // (ERR_* below), in pinned host memory: a kernel sets a word with an
    // ordinary store, the host reads and clears it after the stream is idle
    // (opure_stream_sync, opure_buf_download), so nothing is added to a step
    // or a captured graph.
    uint32_t*   err = nullptr;
    // sleeps before a bounded inter-wave wait gives up (opure_debug_set_wait_limit)
    uint32_t    wait_limit = 1u << 22;
    // GEMV engine of opure_gemv_batched_i8pc for M <= 8 (opure_debug_set_gemv_engine)
    uint32_t    gemv_engine = OPURE_GEMV_MFMA;
    // launches of the rejection step (opure_debug_set_rejection_launches)
    uint32_t    rej_mode = OPURE_REJ_ONE_LAUNCH;
    // captured graphs still alive: a workspace they point into is kept, not
    // freed, when a larger call replaces it
    uint32_t    live_graphs = 0;
    std::vector<void*> retired_ws;
    // stage timing of eager verify steps: every kernel launched inside an open
    // stage gets a start/stop event pair of its own (kernel time, not launch gaps)
    bool                   prof_on = false;
    bool                   prof_open = false;       // between prof_begin and prof_end
    uint32_t               prof_cur = 0;            // the open stage
    uint32_t               prof_count[OPURE_STAGE_COUNT] = {};   // stage instances since the last read
    std::vector<hipEvent_t> prof_ev;                // pairs
    std::vector<uint32_t>  prof_stage;              // stage of each pair
    uint32_t               prof_used = 0;           // pairs recorded since the last read
};

struct opure_graph {
    hipGraph_t     graph = nullptr;
    hipGraphExec_t exec = nullptr;
    opure_dev*     dev = nullptr;
};

// words of opure_dev::err
enum : uint32_t {
    ERR_WAIT = 0,       // a bounded wait between waves gave up (loader-wave GEMV)
    ERR_TOKEN = 1,      // a token id outside the vocabulary (its embedding row is NaN)
    ERR_POSITION = 2,   // a row's position past max_ctx or the page table
    ERR_WORDS = 4
};

namespace opure_hip {

int set_error(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
const char* afmt_name(uint32_t afmt);
int  ensure_workspace(opure_dev* dev, uint64_t bytes);
// the error words a kernel reported since the last check, as an OPURE_E_* code (cleared)
int  check_device_errors(opure_dev* dev);
// zero the in-launch greedy acceptance's words and restart its launch count (async on dev->stream)
hipError_t reset_acc_sync(opure_dev* dev);
// open / close a stage of an eager verify step (no-op unless profiling, or while capturing)
int  prof_begin(opure_dev* dev, uint32_t stage);
int  prof_end(opure_dev* dev);
// a start/stop event pair for the next kernel of the open stage; false when
// nothing is being timed
bool prof_kernel_events(opure_dev* dev, hipEvent_t* start, hipEvent_t* stop);
inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }
inline uint32_t act_bytes(uint32_t afmt) { return afmt == OPURE_A_F32 ? 4u : 2u; }

#define OPURE_HIP_TRY(expr)                                                  \
    do {                                                                     \
        hipError_t _e = (expr);                                              \
        if (_e != hipSuccess) return ::opure_hip::hip_fail(_e, #expr);      \
    } while (0)

#define OPURE_REQUIRE(cond, code, ...)                                       \
    do {                                                                     \
        if (!(cond)) return ::opure_hip::set_error((code), __VA_ARGS__);     \
    } while (0)

// Every kernel launch of the library, on the device's stream.  While a stage of
// an eager verify step is profiled (opure_profile_enable), the extended launch
// stamps start/stop events from the dispatch itself: the kernel's own
// execution time, as a profiler's kernel trace reports it, without the gaps
// between launches.
#define OPURE_LAUNCH(dev, kernel, grid, block, lds, ...)                                              \
    do {                                                                                              \
        hipEvent_t _ks = nullptr, _ke = nullptr;                                                      \
        if (::opure_hip::prof_kernel_events((dev), &_ks, &_ke))                                       \
            hipExtLaunchKernelGGL(kernel, grid, block, lds, (dev)->stream, _ks, _ke, 0, __VA_ARGS__);  \
        else                                                                                          \
            hipLaunchKernelGGL(kernel, grid, block, lds, (dev)->stream, __VA_ARGS__);                 \
    } while (0)

#define OPURE_LAUNCH_CHECK(what)                                             \
    do {                                                                     \
        hipError_t _e = hipGetLastError();                                   \
        if (_e != hipSuccess) return ::opure_hip::hip_fail(_e, what);       \
    } while (0)

// ---- GEMV launcher shared by the public entry points and the verify step --
enum GemvEpi : uint32_t {
    EPI_STORE = OPURE_EPI_STORE,
    EPI_RESIDUAL = OPURE_EPI_RESIDUAL,
    EPI_SWIGLU = OPURE_EPI_SWIGLU,
    EPI_QKV = 3,       // RoPE on q/k rows, q stored, k/v appended to the paged cache
    EPI_LOGITS = 4,    // fp32 logits plus a per-tile (value, index) argmax partial
};

struct QkvEpilogue {
    uint32_t qdim = 0, kvdim = 0, head_dim = 0, n_kv_heads = 0;
    const float* rope_cos = nullptr;
    const float* rope_sin = nullptr;
    uint32_t rope_max_pos = 0;
    const int32_t* seq_len = nullptr;
    uint32_t rows_per_seq = 1;
    void* kv_pool = nullptr;
    const int32_t* page_table = nullptr;
    uint32_t max_pages = 0, n_pages = 0, layer = 0;
    uint32_t* err = nullptr;     // opure_dev::err: a row past the tables sets ERR_POSITION
};

// The KV rollback of a sequence after acceptance (rollback.h)
struct RollbackParams {
    void* pool;
    int32_t* page_table;
    uint32_t max_pages, n_pages, n_layers, n_kv, hd, afmt, K;
    const int32_t* seq_len;
    const int32_t* accepted;
    int32_t* new_len;
    int32_t* freed;
    uint32_t freed_stride;
    int32_t* n_freed;
    uint32_t poison, poison_bits;
};

struct LogitsEpilogue {
    float*   am_val = nullptr;   // [workgroups][M]: best logit of each column per workgroup
    int32_t* am_idx = nullptr;   // its vocabulary index (lowest on ties)
    // Greedy acceptance (and the rollback) inside the LM head's launch, when
    // acc_slots is set (wave-per-tile kernel): every workgroup publishes its
    // rows' bests as tagged words, the last-dispatched workgroup gathers them
    // and accepts, as k_accept_greedy does from am_val / am_idx.
    uint64_t* acc_slots = nullptr;   // [workgroups][M][2]: (tag << 32) | value bits, (tag << 32) | index
    uint32_t* acc_epoch = nullptr;   // the launch count that tags them
    const int32_t* drafts = nullptr; // [batch][drafts_stride], K of them a sequence
    uint32_t drafts_stride = 0, K = 0, batch = 0, wait_limit = 0, rollback = 0;
    int32_t* out_tokens = nullptr;   // [batch][K + 1]
    int32_t* accepted = nullptr;     // [batch]
    RollbackParams rb{};
};

struct GemvCall {
    opure_linear W{};
    uint32_t wfmt = 0;
    const void* x = nullptr;
    uint32_t xfmt = 0;
    uint32_t M = 0;
    void* y = nullptr;
    uint32_t yfmt = 0;
    uint32_t epi = EPI_STORE;
    // fused rmsnorm (Opure_RMSNorm.usf:44-78) of an fp32 residual x: gain != null
    // turns it on; ss_in holds per-16-column sums of squares [ss_tiles][M]
    const float* gain = nullptr;
    float eps = 0.0f;
    const float* ss_in = nullptr;
    uint32_t ss_tiles = 0;
    // EPI_RESIDUAL: where to write the new residual's per-tile sums of squares
    float* ss_out = nullptr;
    // fused rmsnorm whose X does not fit in LDS: [M][in] activations, written
    // by a normalisation rows pass that the GEMV then reads
    void* xn_scratch = nullptr;
    // more than OPURE_MAX_ROWS rows with K split over workgroups: the splits'
    // accumulators (gemv_scratch_bytes)
    void* part_scratch = nullptr;
    // EPI_RESIDUAL over more than OPURE_MAX_ROWS rows: also write the next
    // consumer's rmsnorm of the new residual, round(y * inv_rms * norm_gain),
    // to norm_out [M][out] in xfmt (the same bits as the consumer's own pass)
    const float* norm_gain = nullptr;
    void* norm_out = nullptr;
    QkvEpilogue qkv{};
    LogitsEpilogue logits{};
};

int gemv_validate(const GemvCall& c);
// device scratch a call needs in part_scratch (0 when it needs none)
uint64_t gemv_scratch_bytes(const opure_dev* dev, uint32_t wfmt, uint32_t out, uint32_t in, uint32_t M);
int gemv_launch(opure_dev* dev, const GemvCall& c);
// workgroups gemv_launch runs for this call (EPI_LOGITS writes one argmax
// partial per workgroup and column)
uint32_t gemv_grid(const opure_dev* dev, const GemvCall& c);
// whether gemv_launch runs this call on the wave-per-tile kernel (the one whose
// EPI_LOGITS can accept greedily in the launch)
bool gemv_is_wave_per_tile(const opure_dev* dev, const GemvCall& c);
// device-side tiled-layout helpers shared with the embedding gather
uint32_t tiled_block_k(uint32_t wfmt);      // k values per 64-byte block

// ---- attention (attention.hip) ---------------------------------------------
uint32_t attn_chunk(uint32_t head_dim, uint32_t afmt, uint32_t query_rows_per_kv_head);
uint64_t attn_partial_bytes(uint32_t batch, uint32_t n_kv, uint32_t group, uint32_t rows, uint32_t hd, uint32_t afmt,
                            uint32_t max_ctx);
int      attn_validate(const opure_model* m, const opure_kv* kv, uint32_t batch, uint32_t rows, uint32_t max_ctx);
int      attn_launch(opure_dev* dev, const opure_model* m, const opure_kv* kv, uint32_t layer, uint32_t batch,
                     uint32_t rows, const int32_t* seq_len, uint32_t max_ctx, const void* q, void* out, float* part);

// ---- acceptance and rollback (accept.hip) ----------------------------------
uint32_t argmax_parts(uint32_t vocab);
uint64_t accept_ws_bytes(uint32_t batch, uint32_t k, uint32_t vocab, uint32_t mode);
int      accept_validate(const opure_accept_args* a, bool rejection);
// `rb` (may be null): run that rollback inside the acceptance kernel
RollbackParams rollback_params(const opure_rollback_args* a);
int      greedy_from_partials(opure_dev* dev, const float* am_val, const int32_t* am_idx, uint32_t parts,
                              uint32_t batch, uint32_t K, const int32_t* drafts, uint32_t stride, int32_t* out_tokens,
                              int32_t* accepted, const opure_rollback_args* rb);
int      accept_greedy_launch(opure_dev* dev, const opure_accept_args* a, void* ws);
// per-4096-column (value, lowest index) argmax partials [parts][rows] of fp32 logits
int      argmax_partials_launch(opure_dev* dev, const float* logits, uint32_t rows, uint32_t V, float* am_val,
                                int32_t* am_idx);
int      accept_rejection_launch(opure_dev* dev, const opure_accept_args* a, void* ws, const int32_t* seq_len,
                                 int32_t* new_seq_len);
int      rollback_validate(const opure_rollback_args* a);
int      rollback_launch(opure_dev* dev, const opure_rollback_args* a);

}  // namespace opure_hip

// ---------------------------------------------------------------------------
//  Device side: numerics shared with the CPU oracle bit for bit
// ---------------------------------------------------------------------------
namespace opure_dev_math {

__device__ __forceinline__ float bits_f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f_bits(float f) { return __float_as_uint(f); }

// Sum over each row of 16 lanes with the tree of the xor butterfly 1, 2, 4, 8
// (u += lane ^ o), in DPP moves instead of LDS permutes: quad_perm [1,0,3,2]
// and [2,3,0,1] are xor 1 and 2; after them every lane of a quad holds the
// quad's sum, so the half-row mirror (lane 7 - i) and the row mirror (lane
// 15 - i) read the same values as xor 4 and xor 8.  Bit-identical to the
// butterfly, one VALU each.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Partner lanes l ^ 32 and l ^ 16 on the VALU: v_permlane32_swap and
// v_permlane16_swap with both operands = v leave every lane its own value in one
// result and its partner's in the other, so r[0] op r[1] is v op partner (op
// commutative: the bits equal those of reading the partner through LDS).
__device__ __forceinline__ float add_xor32(float v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor32(float v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor16(float v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// 64-lane butterflies in the order xor 32, 16, 8, 4, 2, 1, with no LDS
// traffic: the swaps above, then row rotations by 8 (exactly lane l ^ 8 in a
// 16-lane row) and by 4 (after the xor-8 step the values repeat every 8 lanes,
// so lane l + 4 holds lane l ^ 4's value), then the quad permutations xor 2
// and xor 1.  Same partners and order as the __shfl_xor butterfly, same bits.
__device__ __forceinline__ float wave_max64(float v)
{
    v = max_xor32(v);
    v = max_xor16(v);
    v = fmaxf(v, dpp_f<0x128>(v));   // row_ror:8
    v = fmaxf(v, dpp_f<0x124>(v));   // row_ror:4
    v = fmaxf(v, dpp_f<0x4E>(v));    // quad_perm [2,3,0,1]
    return fmaxf(v, dpp_f<0xB1>(v));  // quad_perm [1,0,3,2]
}
__device__ __forceinline__ float wave_sum64(float v)
{
    v = add_xor32(v);
    v = add_xor16(v);
    v += dpp_f<0x128>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x4E>(v);
    return v + dpp_f<0xB1>(v);
}

__device__ __forceinline__ float row16_sum(float u)
{
    u += dpp_f<0xB1>(u);    // quad_perm [1,0,3,2]
    u += dpp_f<0x4E>(u);    // quad_perm [2,3,0,1]
    u += dpp_f<0x141>(u);   // row_half_mirror
    u += dpp_f<0x140>(u);   // row_mirror
    return u;
}

// Cody-Waite reduced degree-7 Taylor exp, same operations as orc_expf.
__device__ __forceinline__ float expf_ref(float x)
{
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_huge_valf();
    if (x < -87.33654022216797f) return 0.0f;
    const float LOG2E = static_cast<float>(1.4426950408889634);
    const float LN2_HI = 0.693145751953125f;
    const float LN2_LO = static_cast<float>(0.6931471805599453 - 0.693145751953125);
    const float kf = __builtin_rintf(__fmul_rn(x, LOG2E));
    float r = __fmaf_rn(-kf, LN2_HI, x);
    r = __fmaf_rn(-kf, LN2_LO, r);
    float p = static_cast<float>(1.0 / 5040.0);
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 720.0));
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 120.0));
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 24.0));
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 6.0));
    p = __fmaf_rn(p, r, 0.5f);
    p = __fmaf_rn(p, r, 1.0f);
    p = __fmaf_rn(p, r, 1.0f);
    const int k = static_cast<int>(kf);
    if (k > 127) return __fmul_rn(__fmul_rn(p, bits_f(254u << 23)), 2.0f);
    return __fmul_rn(p, bits_f(static_cast<uint32_t>(k + 127) << 23));
}

// expf_ref restricted to x <= 0 (and NaN): the same operations in the same
// order, without the overflow paths, so the bits equal expf_ref's there
__device__ __forceinline__ float expf_ref_nonpos(float x)
{
    const float LOG2E = static_cast<float>(1.4426950408889634);
    const float LN2_HI = 0.693145751953125f;
    const float LN2_LO = static_cast<float>(0.6931471805599453 - 0.693145751953125);
    const float kf = __builtin_rintf(__fmul_rn(x, LOG2E));
    float r = __fmaf_rn(-kf, LN2_HI, x);
    r = __fmaf_rn(-kf, LN2_LO, r);
    float p = static_cast<float>(1.0 / 5040.0);
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 720.0));
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 120.0));
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 24.0));
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 6.0));
    p = __fmaf_rn(p, r, 0.5f);
    p = __fmaf_rn(p, r, 1.0f);
    p = __fmaf_rn(p, r, 1.0f);
    const int k = x < -87.33654022216797f ? 0 : static_cast<int>(kf);
    const float v = __fmul_rn(p, bits_f(static_cast<uint32_t>(k + 127) << 23));
    return x != x ? x : (x < -87.33654022216797f ? 0.0f : v);
}

__device__ __forceinline__ uint32_t philox_u32(uint64_t seed, uint32_t c0, uint32_t c1, uint32_t c2)
{
    uint32_t c3 = 0u;
    uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r)
    {
        if (r > 0) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
        const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
    }
    return c0;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return bits_f(static_cast<uint32_t>(h) << 16); }

// round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h)
{
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return static_cast<float>(v);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f)
{
    const _Float16 v = static_cast<_Float16>(f);
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

template <int AF>
__device__ __forceinline__ float load_act(const void* base, uint64_t i)
{
    if constexpr (AF == OPURE_A_F32) return static_cast<const float*>(base)[i];
    else if constexpr (AF == OPURE_A_F16) return f16_to_f32(static_cast<const uint16_t*>(base)[i]);
    else return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
}

__device__ __forceinline__ float load_act_rt(const void* base, uint64_t i, uint32_t af)
{
    if (af == OPURE_A_F32) return static_cast<const float*>(base)[i];
    const uint16_t h = static_cast<const uint16_t*>(base)[i];
    return af == OPURE_A_F16 ? f16_to_f32(h) : bf16_to_f32(h);
}

__device__ __forceinline__ void store_act_rt(void* base, uint64_t i, float v, uint32_t af)
{
    if (af == OPURE_A_F32) { static_cast<float*>(base)[i] = v; return; }
    static_cast<uint16_t*>(base)[i] = af == OPURE_A_F16 ? f32_to_f16(v) : f32_to_bf16(v);
}

__device__ __forceinline__ float round_act_rt(float v, uint32_t af)
{
    if (af == OPURE_A_F16) return f16_to_f32(f32_to_f16(v));
    if (af == OPURE_A_BF16) return bf16_to_f32(f32_to_bf16(v));
    return v;
}

// Element (slot, d) of the K (kvsel 0) or V (kvsel 1) plane of a cache page.
// K planes are token-major [16][hd]; V planes channel-major [hd][16], so a
// V^T tile of 8 consecutive tokens of one channel is 16 contiguous bytes.
__device__ __forceinline__ uint64_t kv_elem(uint32_t layer, uint32_t n_pages, uint32_t page, uint32_t kvsel,
                                            uint32_t n_kv, uint32_t head, uint32_t hd, uint32_t slot, uint32_t d)
{
    const uint64_t plane = ((((static_cast<uint64_t>(layer) * n_pages + page) * 2u + kvsel) * n_kv + head) *
                            OPURE_PAGE_SIZE) * hd;
    return kvsel == 0u ? plane + static_cast<uint64_t>(slot) * hd + d : plane + static_cast<uint64_t>(d) * OPURE_PAGE_SIZE + slot;
}

// expf_ref without branches: the same operations wherever expf_ref computes
// (x clamped into that range first, which changes nothing there), the NaN,
// overflow and underflow results chosen by selects -- so the same bits
__device__ __forceinline__ float expf_ref_sel(float x)
{
    const float LOG2E = static_cast<float>(1.4426950408889634);
    const float LN2_HI = 0.693145751953125f;
    const float LN2_LO = static_cast<float>(0.6931471805599453 - 0.693145751953125);
    const float xc = fminf(fmaxf(x, -87.33654022216797f), 88.72283935546875f);
    const float kf = __builtin_rintf(__fmul_rn(xc, LOG2E));
    float r = __fmaf_rn(-kf, LN2_HI, xc);
    r = __fmaf_rn(-kf, LN2_LO, r);
    float p = static_cast<float>(1.0 / 5040.0);
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 720.0));
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 120.0));
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 24.0));
    p = __fmaf_rn(p, r, static_cast<float>(1.0 / 6.0));
    p = __fmaf_rn(p, r, 0.5f);
    p = __fmaf_rn(p, r, 1.0f);
    p = __fmaf_rn(p, r, 1.0f);
    const int k = static_cast<int>(kf);
    // expf_ref: p * 2^k, or (p * 2^127) * 2 for k = 128 (a product by 1 is exact)
    const float v = __fmul_rn(__fmul_rn(p, bits_f(static_cast<uint32_t>(min(k, 127) + 127) << 23)), k > 127 ? 2.0f : 1.0f);
    return x != x ? x : (x > 88.72283935546875f ? __builtin_huge_valf() : (x < -87.33654022216797f ? 0.0f : v));
}

// silu(g) * u in the order of Opure_CpuReference.cpp:195-196
__device__ __forceinline__ float swiglu(float g, float u)
{
    const float s = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_ref_sel(-g)));
    return __fmul_rn(__fmul_rn(g, s), u);
}

}  // namespace opure_dev_math
