// ============================================================================
//  opure_oracle.cpp -- CPU oracle for the Opure verify path.
//
//  TEST INFRASTRUCTURE ONLY: the CPU restatement the HIP path is compared against.
//  Nothing in the product links or loads this file's library.
//
//  Restates src/engine/Opure_CpuReference.cpp (scalar C++, double
//  accumulation, float rounding at the end of each stage) and extends it to
//  the verify step.  Function-by-function provenance:
//
//    orc_gemv (f32)       Opure_CpuReference.cpp:151-161  double acc, one float
//                         round per output
//    orc_gemv (i8pc)      Opure_GEMV_Quant.usf:52-73, :93 byte order; scale applied
//                         after the dot product.  Per-channel scale replaces
//                         the per-tensor P[5].
//    orc_gemv (i4g128)    w = s_g * (q - z_g); nibble order from
//                         Opure_Streamer.cpp:403-426 (element 2i = high nibble)
//    orc_rmsnorm_rows     Opure_CpuReference.cpp:163-169
//    orc_rope_rows        Opure_CpuReference.cpp:171-189 rotation, with cos/sin
//                         taken from a table (orc_rope_table) whose schedule is
//                         Opure_RoPE.usf:56 (GPU) or Opure_CpuReference.cpp:179
//    orc_swiglu           Opure_CpuReference.cpp:191-198
//    orc_attention_paged  Opure_CpuReference.cpp:259-305 (two-pass softmax in
//                         double; V accumulated in double, see the function),
//                         GQA map Opure_FlashAttention_Decode.usf:71-72,
//                         KV append Opure_RoPE.usf:105-114 (rotated K, raw V)
//    orc_verify_forward   per-token order of Opure_CpuReference.cpp:225-345,
//                         run layer-major over R rows (equivalent: row j at
//                         layer L reads only K/V of rows <= j at layer L);
//                         composed of orc_verify_embed / _layers / _head so a
//                         test can feed any residual into any layer, as the
//                         reference harness traces layers
//                         (Opure_TestHarness.cpp:956-987)
//    orc_argmax_rows      Opure_ArgMax.usf contract, ties -> lowest index
//    orc_accept_*         absent from the reference; Leviathan et al. 2023 /
//                         Chen et al. 2023 with the fixed-point conventions
//                         documented at row_stats() below
//    orc_philox4x32_10    Salmon et al., SC'11 (Random123)
//
//  Build: oracle/Makefile (g++ -O2 -ffp-contract=off), so no expression is
//  silently fused into an fma and every float operation rounds as written.
// ============================================================================
#include "opure_oracle.h"

#include <cmath>
#include <cstring>
#include <vector>
#include <algorithm>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

int g_threads = 1;

inline float bits_f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t f_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

inline float load_act(const void* base, uint64_t idx, uint32_t afmt)
{
    if (afmt == ORC_A_F32) return static_cast<const float*>(base)[idx];
    const uint16_t h = static_cast<const uint16_t*>(base)[idx];
    return afmt == ORC_A_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
}

inline void store_act(void* base, uint64_t idx, float v, uint32_t afmt)
{
    if (afmt == ORC_A_F32) { static_cast<float*>(base)[idx] = v; return; }
    static_cast<uint16_t*>(base)[idx] = afmt == ORC_A_F16 ? orc_f32_to_f16(v) : orc_f32_to_bf16(v);
}

inline float round_act1(float v, uint32_t afmt)
{
    if (afmt == ORC_A_F16) return orc_f16_to_f32(orc_f32_to_f16(v));
    if (afmt == ORC_A_BF16) return orc_bf16_to_f32(orc_f32_to_bf16(v));
    return v;
}

// Dequantised weight (o, i) in double.  Used by the gemv and the embedding.
inline double weight_at(const orc_linear* L, uint32_t wfmt, uint32_t o, uint32_t i)
{
    const uint64_t idx = static_cast<uint64_t>(o) * L->in + i;
    switch (wfmt)
    {
    case ORC_W_F32: return static_cast<const float*>(L->w)[idx];
    case ORC_W_I8PC: return static_cast<double>(static_cast<const int8_t*>(L->w)[idx]) *
                            static_cast<double>(orc_f16_to_f32(L->scale[o]));
    default:
    {
        const uint8_t byte = static_cast<const uint8_t*>(L->w)[idx >> 1];
        const uint32_t q = (idx & 1) ? (byte & 0x0Fu) : (byte >> 4);
        const uint64_t g = static_cast<uint64_t>(o) * (L->in / 128) + i / 128;
        const double s = orc_bf16_to_f32(L->scale[g]);
        const double z = orc_bf16_to_f32(L->zero[g]);
        return s * (static_cast<double>(q) - z);
    }
    }
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
//  Conversions.  f16 -> f32 restates Opure_Streamer.cpp:49-84 (subnormals
//  renormalised); bf16 -> f32 is the shift of Opure_Streamer.h:140-146.  The
//  narrowing directions are IEEE round-to-nearest-even.
// ---------------------------------------------------------------------------
float orc_f16_to_f32(uint16_t h)
{
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (e == 0u)
    {
        if (man == 0u) bits = sign;
        else
        {
            // man * 2^-24 renormalised.  Opure_Streamer.cpp:66-69 writes the
            // exponent as 127-15-k, which halves every subnormal; IEEE needs
            // 127-15+1-k, used here.
            uint32_t k = 0u, m = man;
            while ((m & 0x400u) == 0u) { m <<= 1; ++k; }
            m &= 0x3FFu;
            bits = sign | ((127u - 15u + 1u - k) << 23) | (m << 13);
        }
    }
    else if (e == 0x1Fu) bits = sign | 0x7F800000u | (man << 13);
    else bits = sign | ((e + (127u - 15u)) << 23) | (man << 13);
    return bits_f(bits);
}

uint16_t orc_f32_to_f16(float f)
{
    const uint32_t x = f_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return static_cast<uint16_t>(sign | 0x7E00u | ((ax >> 13) & 0x1FFu));
    if (ax >= 0x47800000u) return static_cast<uint16_t>(sign | 0x7C00u);   // >= 65536 or inf
    const uint32_t e = ax >> 23;
    if (e < 113u)
    {
        // f16 subnormal (or zero): value = m24 * 2^(e-150) = m16 * 2^-24
        if (e < 102u) return static_cast<uint16_t>(sign);
        const uint32_t m24 = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;            // 14 .. 24
        uint32_t m16 = m24 >> shift;
        const uint32_t rem = m24 & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (m16 & 1u))) ++m16;
        return static_cast<uint16_t>(sign | m16);
    }
    uint32_t h = ((e - 112u) << 10) | ((ax >> 13) & 0x3FFu);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;   // carry may reach inf: correct
    return static_cast<uint16_t>(sign | h);
}

float orc_bf16_to_f32(uint16_t h) { return bits_f(static_cast<uint32_t>(h) << 16); }

uint16_t orc_f32_to_bf16(float f)
{
    const uint32_t x = f_bits(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((x >> 16) | 0x40u);
    return static_cast<uint16_t>((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

// ---------------------------------------------------------------------------
//  exp.  Cody & Waite range reduction x = k*ln2 + r, |r| <= ln2/2, followed by
//  the degree-7 Taylor polynomial of e^r (truncation error < 8e-9 relative),
//  evaluated by Horner's rule with explicit fused multiply-adds, then scaled by
//  2^k through the exponent field.  ln2 is split into LN2_HI (ln2 rounded to 16
//  significant bits, so k*LN2_HI is exact for |k| <= 256) and LN2_LO = ln2 -
//  LN2_HI.  The device kernels use the same formula with the same operations,
//  so both sides produce identical bits.  Inputs below ln(FLT_MIN) flush to 0.
// ---------------------------------------------------------------------------
float orc_expf(float x)
{
    if (x != x) return x;
    if (x > 88.72283935546875f) return HUGE_VALF;
    if (x < -87.33654022216797f) return 0.0f;
    const float LOG2E = static_cast<float>(1.4426950408889634);
    const float LN2_HI = 0.693145751953125f;
    const float LN2_LO = static_cast<float>(0.6931471805599453 - 0.693145751953125);
    const float kf = std::rint(x * LOG2E);
    float r = std::fma(-kf, LN2_HI, x);
    r = std::fma(-kf, LN2_LO, r);
    float p = static_cast<float>(1.0 / 5040.0);
    p = std::fma(p, r, static_cast<float>(1.0 / 720.0));
    p = std::fma(p, r, static_cast<float>(1.0 / 120.0));
    p = std::fma(p, r, static_cast<float>(1.0 / 24.0));
    p = std::fma(p, r, static_cast<float>(1.0 / 6.0));
    p = std::fma(p, r, 0.5f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    const int k = static_cast<int>(kf);
    if (k > 127) return (p * bits_f(static_cast<uint32_t>(254) << 23)) * 2.0f;
    return p * bits_f(static_cast<uint32_t>(k + 127) << 23);
}

// ---------------------------------------------------------------------------
//  Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11).
// ---------------------------------------------------------------------------
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r)
    {
        if (r > 0) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
        const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
        const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
        const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

uint32_t orc_philox_u32(uint64_t seed, uint32_t pos, uint32_t seq, uint32_t stream)
{
    const uint32_t ctr[4] = { pos, seq, stream, 0u };
    const uint32_t key[2] = { static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32) };
    uint32_t out[4];
    orc_philox4x32_10(ctr, key, out);
    return out[0];
}

// Opure_TestHarness.cpp:36-47
void orc_xorshift_u32(uint64_t seed, uint32_t* out, uint64_t n)
{
    uint64_t s = seed ? seed : 1;
    for (uint64_t i = 0; i < n; ++i)
    {
        s ^= s << 13; s ^= s >> 7; s ^= s << 17;
        out[i] = static_cast<uint32_t>(s >> 32);
    }
}

void orc_xorshift_fill(uint64_t seed, float* out, uint64_t n, float mul, float add)
{
    uint64_t s = seed ? seed : 1;
    for (uint64_t i = 0; i < n; ++i)
    {
        s ^= s << 13; s ^= s >> 7; s ^= s << 17;
        const float f = static_cast<float>(static_cast<uint32_t>(s >> 32)) / 2147483648.0f - 1.0f;
        out[i] = f * mul + add;
    }
}

// ---------------------------------------------------------------------------
void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

void orc_gemv(const orc_linear* L, uint32_t wfmt, const float* x, float* y, uint32_t M)
{
    const uint32_t O = L->out, K = L->in;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
#endif
    for (int64_t o = 0; o < static_cast<int64_t>(O); ++o)
    {
        for (uint32_t m = 0; m < M; ++m)
        {
            const float* xr = x + static_cast<uint64_t>(m) * K;
            double acc = 0.0;
            if (wfmt == ORC_W_F32)
            {
                const float* row = static_cast<const float*>(L->w) + static_cast<uint64_t>(o) * K;
                for (uint32_t i = 0; i < K; ++i) acc += double(row[i]) * double(xr[i]);
            }
            else if (wfmt == ORC_W_I8PC)
            {
                const int8_t* row = static_cast<const int8_t*>(L->w) + static_cast<uint64_t>(o) * K;
                for (uint32_t i = 0; i < K; ++i) acc += double(row[i]) * double(xr[i]);
                acc *= double(orc_f16_to_f32(L->scale[o]));
            }
            else
            {
                const uint8_t* row = static_cast<const uint8_t*>(L->w) + static_cast<uint64_t>(o) * (K / 2);
                const uint32_t G = K / 128;
                for (uint32_t g = 0; g < G; ++g)
                {
                    const double s = orc_bf16_to_f32(L->scale[static_cast<uint64_t>(o) * G + g]);
                    const double z = orc_bf16_to_f32(L->zero[static_cast<uint64_t>(o) * G + g]);
                    double part = 0.0;
                    for (uint32_t i = g * 128; i < g * 128 + 128; ++i)
                    {
                        const uint8_t b = row[i >> 1];
                        const uint32_t q = (i & 1) ? (b & 0x0Fu) : (b >> 4);
                        part += (double(q) - z) * double(xr[i]);
                    }
                    acc += s * part;
                }
            }
            y[static_cast<uint64_t>(m) * O + o] = static_cast<float>(acc);
        }
    }
}

void orc_round_act(float* x, uint64_t n, uint32_t afmt)
{
    if (afmt == ORC_A_F32) return;
    for (uint64_t i = 0; i < n; ++i) x[i] = round_act1(x[i], afmt);
}

void orc_rmsnorm_rows(const float* x, const float* g, float* y, uint32_t M, uint32_t d,
                      float eps, uint32_t afmt)
{
    for (uint32_t m = 0; m < M; ++m)
    {
        const float* xr = x + static_cast<uint64_t>(m) * d;
        float* yr = y + static_cast<uint64_t>(m) * d;
        double ss = 0.0;
        for (uint32_t i = 0; i < d; ++i) ss += double(xr[i]) * double(xr[i]);
        const double inv = 1.0 / std::sqrt(ss / d + eps);
        for (uint32_t i = 0; i < d; ++i)
            yr[i] = round_act1(static_cast<float>(double(xr[i]) * inv * double(g[i])), afmt);
    }
}

void orc_rope_table(double theta, uint32_t head_dim, uint32_t max_pos, uint32_t mode,
                    float* cos_out, float* sin_out)
{
    const uint32_t half = head_dim / 2;
    for (uint32_t p = 0; p < half; ++p)
    {
        const double ch = (mode == ORC_ROPE_CPUREF) ? 2.0 * p : double(p);
        const double inv_freq = std::pow(theta, -2.0 * ch / double(head_dim));
        for (uint32_t pos = 0; pos < max_pos; ++pos)
        {
            const double t = double(pos) * inv_freq;
            cos_out[static_cast<uint64_t>(pos) * half + p] = static_cast<float>(std::cos(t));
            sin_out[static_cast<uint64_t>(pos) * half + p] = static_cast<float>(std::sin(t));
        }
    }
}

void orc_rope_rows(float* vec, uint32_t n_heads, uint32_t head_dim, const float* cos_t,
                   const float* sin_t, uint32_t pos)
{
    const uint32_t half = head_dim / 2;
    for (uint32_t h = 0; h < n_heads; ++h)
    {
        float* row = vec + static_cast<uint64_t>(h) * head_dim;
        for (uint32_t p = 0; p < half; ++p)
        {
            const double ct = cos_t[static_cast<uint64_t>(pos) * half + p];
            const double st = sin_t[static_cast<uint64_t>(pos) * half + p];
            const double e0 = row[2 * p], e1 = row[2 * p + 1];
            row[2 * p]     = static_cast<float>(e0 * ct - e1 * st);
            row[2 * p + 1] = static_cast<float>(e0 * st + e1 * ct);
        }
    }
}

void orc_swiglu(const float* g, const float* u, float* h, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i)
    {
        const float s = 1.0f / (1.0f + std::exp(-g[i]));
        h[i] = (g[i] * s) * u[i];
    }
}

// Element (slot, d) of a page's K or V plane.  K planes are token-major
// [page_size][head_dim]; V planes are channel-major [head_dim][page_size], so
// the GPU reads V^T tiles of 8 tokens with one 16-byte load (see opure_hip.h).
static inline uint64_t kv_elem(const orc_model* m, const orc_kv* kv, uint32_t layer, int32_t page,
                               uint32_t kvsel, uint32_t head, uint32_t slot, uint32_t d)
{
    const uint64_t plane = (((static_cast<uint64_t>(layer) * kv->n_pages + static_cast<uint32_t>(page)) * 2 + kvsel) *
                            m->n_kv_heads + head) * kv->page_size * m->head_dim;
    return kvsel == 0 ? plane + static_cast<uint64_t>(slot) * m->head_dim + d
                      : plane + static_cast<uint64_t>(d) * kv->page_size + slot;
}

void orc_attention_paged(const orc_model* m, const orc_kv* kv, uint32_t layer,
                         uint32_t seq, uint32_t ctx, uint32_t R, const float* q, float* out)
{
    const uint32_t hd = m->head_dim, nh = m->n_heads, group = nh / m->n_kv_heads;
    const int32_t* pt = kv->page_table + static_cast<uint64_t>(seq) * kv->max_pages_per_seq;
    // (row, query head) pairs are independent: split over threads, each pair
    // computed exactly as on one thread
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(g_threads) if (g_threads > 1)
#endif
    for (uint32_t j = 0; j < R; ++j)
    {
        for (uint32_t hq = 0; hq < nh; ++hq)
        {
            const uint32_t seqLen = ctx + j + 1;
            std::vector<double> scores(seqLen, 0.0);
            std::vector<double> o(hd);
            const uint32_t kvh = hq / group;
            const float* qRow = q + (static_cast<uint64_t>(j) * nh + hq) * hd;
            double mx = -1e300;
            for (uint32_t s = 0; s < seqLen; ++s)
            {
                const int32_t pg = pt[s / kv->page_size];
                double sc = 0.0;
                for (uint32_t d = 0; d < hd; ++d)
                    sc += double(qRow[d]) *
                          double(load_act(kv->pool, kv_elem(m, kv, layer, pg, 0, kvh, s % kv->page_size, d), m->afmt));
                sc *= double(m->attn_scale);
                scores[s] = sc;
                if (sc > mx) mx = sc;
            }
            double sum = 0.0;
            for (uint32_t s = 0; s < seqLen; ++s) { const double e = std::exp(scores[s] - mx); scores[s] = e; sum += e; }
            // The reference rounds this accumulator to float after every position
            // (Opure_CpuReference.cpp:297) although its header promises double
            // throughout (Opure_CpuReference.h:19-21); the oracle keeps it in
            // double, which only removes error: an attention output over a long
            // context is a heavily cancelled sum.
            std::fill(o.begin(), o.end(), 0.0);
            for (uint32_t s = 0; s < seqLen; ++s)
            {
                const int32_t pg = pt[s / kv->page_size];
                const double w = scores[s];
                for (uint32_t d = 0; d < hd; ++d)
                    o[d] += w * double(load_act(kv->pool, kv_elem(m, kv, layer, pg, 1, kvh, s % kv->page_size, d), m->afmt));
            }
            const double invSum = 1.0 / (sum > 0.0 ? sum : 1.0);
            float* oRow = out + (static_cast<uint64_t>(j) * nh + hq) * hd;
            for (uint32_t d = 0; d < hd; ++d) oRow[d] = static_cast<float>(o[d] * invSum);
        }
    }
}

// ---------------------------------------------------------------------------
//  The verify forward, in three parts that compose to orc_verify_forward:
//  the embedding gather, layers [first, first+count) applied to a residual in
//  place, and the final RMSNorm + LM head.  A test can run the parts one at a
//  time (the reference's per-layer tracing, Opure_TestHarness.cpp:956-987) and
//  feed any residual into any layer.
// ---------------------------------------------------------------------------
namespace {

// One element of one intermediate moved by one unit in the last place of the
// activation format, after that intermediate's rounding (a test hook: it shows
// how far a single rounding decision travels through the layers).
struct Perturbation { int32_t layer = -1; uint32_t stage = 0; uint64_t index = 0; };
Perturbation g_perturb;

void perturb_at(float* a, uint64_t n, uint32_t L, uint32_t stage, uint32_t afmt)
{
    if (g_perturb.layer < 0 || static_cast<uint32_t>(g_perturb.layer) != L || g_perturb.stage != stage ||
        g_perturb.index >= n)
        return;
    float& v = a[g_perturb.index];
    if (afmt == ORC_A_F32) { v = bits_f(f_bits(v) + 1u); return; }
    if (afmt == ORC_A_F16) { v = orc_f16_to_f32(static_cast<uint16_t>(orc_f32_to_f16(v) + 1u)); return; }
    v = orc_bf16_to_f32(static_cast<uint16_t>(orc_f32_to_bf16(v) + 1u));
}

int check_step(const orc_model* m, const orc_kv* kv, uint32_t B, uint32_t R, const int32_t* seq_len)
{
    for (uint32_t b = 0; b < B; ++b)
    {
        if (seq_len[b] < 0) return -1;
        const uint32_t last = static_cast<uint32_t>(seq_len[b]) + R - 1;
        if (last >= m->rope_max_pos) return -3;
        if (last / kv->page_size >= kv->max_pages_per_seq) return -2;
        for (uint32_t p = 0; p <= last / kv->page_size; ++p)
        {
            const int32_t pg = kv->page_table[static_cast<uint64_t>(b) * kv->max_pages_per_seq + p];
            if (pg < 0 || static_cast<uint32_t>(pg) >= kv->n_pages) return -2;
        }
    }
    return 0;
}

// Layer L of Opure_CpuReference.cpp:225-345 for B*R rows: x is updated in
// place and the rows' K/V are appended to the cache.  `trace` (layer 0 only)
// receives the intermediates listed at orc_verify_forward_traced.
void run_layer(const orc_model* m, orc_kv* kv, uint32_t B, uint32_t R, const int32_t* seq_len, uint32_t L,
               float* x, float* trace)
{
    const uint32_t h = m->hidden, hd = m->head_dim, nh = m->n_heads, nkv = m->n_kv_heads;
    const uint32_t qdim = nh * hd, kvdim = nkv * hd, ff = m->ffn;
    const uint32_t MR = B * R;
    const uint64_t xs = static_cast<uint64_t>(MR) * h;
    std::vector<float> xn(xs);
    std::vector<float> qkv(static_cast<uint64_t>(MR) * (qdim + 2 * kvdim));
    std::vector<float> q(static_cast<uint64_t>(MR) * qdim), att(q.size()), proj(xs);
    std::vector<float> gu(static_cast<uint64_t>(MR) * 2 * ff), hh(static_cast<uint64_t>(MR) * ff);
    const orc_layer& P = m->layers[L];

    orc_rmsnorm_rows(x, P.attn_norm, xn.data(), MR, h, m->rms_eps, m->afmt);
    perturb_at(xn.data(), xs, L, ORC_STAGE_XN_ATTN, m->afmt);
    orc_gemv(&P.qkv, m->wfmt, xn.data(), qkv.data(), MR);
    const uint32_t qkvw = qdim + 2 * kvdim;
    for (uint32_t b = 0; b < B; ++b)
    {
        for (uint32_t j = 0; j < R; ++j)
        {
            const uint32_t r = b * R + j;
            const uint32_t pos = static_cast<uint32_t>(seq_len[b]) + j;
            float* row = qkv.data() + static_cast<uint64_t>(r) * qkvw;
            orc_rope_rows(row, nh, hd, m->rope_cos, m->rope_sin, pos);
            orc_rope_rows(row + qdim, nkv, hd, m->rope_cos, m->rope_sin, pos);
            orc_round_act(row, qkvw, m->afmt);
            std::memcpy(q.data() + static_cast<uint64_t>(r) * qdim, row, qdim * 4);
            const int32_t pg = kv->page_table[static_cast<uint64_t>(b) * kv->max_pages_per_seq + pos / kv->page_size];
            for (uint32_t kh = 0; kh < nkv; ++kh)
            {
                for (uint32_t d = 0; d < hd; ++d)
                {
                    store_act(kv->pool, kv_elem(m, kv, L, pg, 0, kh, pos % kv->page_size, d), row[qdim + kh * hd + d],
                              m->afmt);
                    store_act(kv->pool, kv_elem(m, kv, L, pg, 1, kh, pos % kv->page_size, d),
                              row[qdim + kvdim + kh * hd + d], m->afmt);
                }
            }
        }
    }
    perturb_at(q.data(), q.size(), L, ORC_STAGE_Q, m->afmt);
    for (uint32_t b = 0; b < B; ++b)
        orc_attention_paged(m, kv, L, b, static_cast<uint32_t>(seq_len[b]), R,
                            q.data() + static_cast<uint64_t>(b) * R * qdim,
                            att.data() + static_cast<uint64_t>(b) * R * qdim);
    orc_round_act(att.data(), att.size(), m->afmt);
    perturb_at(att.data(), att.size(), L, ORC_STAGE_ATT, m->afmt);
    orc_gemv(&P.o, m->wfmt, att.data(), proj.data(), MR);
    for (uint64_t i = 0; i < xs; ++i) x[i] = x[i] + proj[i];
    if (trace)
    {
        float* t = trace;
        std::memcpy(t, q.data(), q.size() * 4); t += q.size();
        std::memcpy(t, att.data(), att.size() * 4); t += att.size();
        std::memcpy(t, x, xs * 4);
    }

    orc_rmsnorm_rows(x, P.mlp_norm, xn.data(), MR, h, m->rms_eps, m->afmt);
    perturb_at(xn.data(), xs, L, ORC_STAGE_XN_MLP, m->afmt);
    orc_gemv(&P.gate_up, m->wfmt, xn.data(), gu.data(), MR);
    for (uint32_t r = 0; r < MR; ++r)
        orc_swiglu(gu.data() + static_cast<uint64_t>(r) * 2 * ff,
                   gu.data() + static_cast<uint64_t>(r) * 2 * ff + ff,
                   hh.data() + static_cast<uint64_t>(r) * ff, ff);
    orc_round_act(hh.data(), hh.size(), m->afmt);
    perturb_at(hh.data(), hh.size(), L, ORC_STAGE_H, m->afmt);
    orc_gemv(&P.down, m->wfmt, hh.data(), proj.data(), MR);
    for (uint64_t i = 0; i < xs; ++i) x[i] = x[i] + proj[i];
    if (trace)
    {
        float* t = trace + 2 * q.size() + xs;
        std::memcpy(t, hh.data(), hh.size() * 4); t += hh.size();
        std::memcpy(t, x, xs * 4);
    }
}

}  // namespace

void orc_set_perturbation(int32_t layer, uint32_t stage, uint64_t index)
{
    g_perturb.layer = layer;
    g_perturb.stage = stage;
    g_perturb.index = index;
}

// embedding (Opure_CpuReference.cpp:225; dequantised row for quantised tables)
int orc_verify_embed(const orc_model* m, uint32_t MR, const int32_t* tokens, float* x)
{
    if (!m || !tokens || !x) return -1;
    const uint32_t h = m->hidden;
    for (uint32_t r = 0; r < MR; ++r)
        if (tokens[r] < 0 || static_cast<uint32_t>(tokens[r]) >= m->vocab) return -4;
    for (uint32_t r = 0; r < MR; ++r)
    {
        const uint32_t t = static_cast<uint32_t>(tokens[r]);
        for (uint32_t i = 0; i < h; ++i)
        {
            float v;
            if (m->wfmt == ORC_W_F32) v = static_cast<const float*>(m->embed.w)[static_cast<uint64_t>(t) * h + i];
            else if (m->wfmt == ORC_W_I8PC)
                v = static_cast<float>(static_cast<const int8_t*>(m->embed.w)[static_cast<uint64_t>(t) * h + i]) *
                    orc_f16_to_f32(m->embed.scale[t]);
            else
            {
                const uint64_t idx = static_cast<uint64_t>(t) * h + i;
                const uint8_t byte = static_cast<const uint8_t*>(m->embed.w)[idx >> 1];
                const uint32_t qv = (idx & 1) ? (byte & 0x0Fu) : (byte >> 4);
                const uint64_t g = static_cast<uint64_t>(t) * (h / 128) + i / 128;
                v = orc_bf16_to_f32(m->embed.scale[g]) * (static_cast<float>(qv) - orc_bf16_to_f32(m->embed.zero[g]));
            }
            x[static_cast<uint64_t>(r) * h + i] = v;
        }
    }
    return 0;
}

int orc_verify_layers(const orc_model* m, orc_kv* kv, uint32_t B, uint32_t R, const int32_t* seq_len, float* x,
                      uint32_t first, uint32_t count)
{
    if (!m || !kv || !seq_len || !x || B == 0 || R == 0 || first + count > m->n_layers) return -1;
    const int rc = check_step(m, kv, B, R, seq_len);
    if (rc) return rc;
    for (uint32_t L = first; L < first + count; ++L) run_layer(m, kv, B, R, seq_len, L, x, nullptr);
    return 0;
}

// final RMSNorm (Opure_VoxelEngine.cpp:523-527) and the LM head (:528-532)
int orc_verify_head(const orc_model* m, uint32_t MR, const float* x, float* logits)
{
    if (!m || !x || !logits) return -1;
    std::vector<float> xn(static_cast<uint64_t>(MR) * m->hidden);
    orc_rmsnorm_rows(x, m->final_norm, xn.data(), MR, m->hidden, m->rms_eps, m->afmt);
    orc_gemv(&m->lm_head, m->wfmt, xn.data(), logits, MR);
    return 0;
}

static int verify_impl(const orc_model* m, orc_kv* kv, uint32_t B, uint32_t R,
                       const int32_t* tokens, const int32_t* seq_len, float* logits, float* trace)
{
    if (!m || !kv || !tokens || !seq_len || !logits || B == 0 || R == 0) return -1;
    int rc = check_step(m, kv, B, R, seq_len);
    if (rc) return rc;
    const uint32_t MR = B * R, h = m->hidden;
    std::vector<float> x(static_cast<uint64_t>(MR) * h);
    if ((rc = orc_verify_embed(m, MR, tokens, x.data()))) return rc;
    for (uint32_t L = 0; L < m->n_layers; ++L) run_layer(m, kv, B, R, seq_len, L, x.data(), L == 0 ? trace : nullptr);
    if (trace)
    {
        const uint64_t qs = static_cast<uint64_t>(MR) * m->n_heads * m->head_dim, xs = static_cast<uint64_t>(MR) * h;
        orc_rmsnorm_rows(x.data(), m->final_norm, trace + 2 * qs + 2 * xs + static_cast<uint64_t>(MR) * m->ffn, MR, h,
                         m->rms_eps, m->afmt);
    }
    return orc_verify_head(m, MR, x.data(), logits);
}

int orc_verify_forward(const orc_model* m, orc_kv* kv, uint32_t B, uint32_t R,
                       const int32_t* tokens, const int32_t* seq_len, float* logits)
{
    return verify_impl(m, kv, B, R, tokens, seq_len, logits, nullptr);
}

int orc_verify_forward_traced(const orc_model* m, orc_kv* kv, uint32_t B, uint32_t R,
                              const int32_t* tokens, const int32_t* seq_len, float* logits,
                              float* trace)
{
    return verify_impl(m, kv, B, R, tokens, seq_len, logits, trace);
}

// ---------------------------------------------------------------------------
//  Acceptance
// ---------------------------------------------------------------------------
void orc_argmax_rows(const float* logits, uint32_t rows, uint32_t V, int32_t* idx, float* val)
{
    for (uint32_t r = 0; r < rows; ++r)
    {
        // NaN logits count as -inf; ties and an all -inf row go to the lowest index
        const float* row = logits + static_cast<uint64_t>(r) * V;
        float best = -HUGE_VALF;
        uint32_t bi = 0;
        for (uint32_t v = 0; v < V; ++v)
        {
            const float c = row[v] != row[v] ? -HUGE_VALF : row[v];
            if (c > best) { best = c; bi = v; }
        }
        if (idx) idx[r] = static_cast<int32_t>(bi);
        if (val) val[r] = best;
    }
}

void orc_accept_greedy(const float* target_logits, const int32_t* drafts, uint32_t B,
                       uint32_t K, uint32_t V, int32_t* out_tokens, int32_t* accepted)
{
    std::vector<int32_t> am(K + 1);
    for (uint32_t b = 0; b < B; ++b)
    {
        orc_argmax_rows(target_logits + static_cast<uint64_t>(b) * (K + 1) * V, K + 1, V, am.data(), nullptr);
        uint32_t n = 0;
        while (n < K && am[n] == drafts[b * K + n]) ++n;
        for (uint32_t j = 0; j <= K; ++j)
            out_tokens[b * (K + 1) + j] = j < n ? drafts[b * K + j] : (j == n ? am[n] : -1);
        accepted[b] = static_cast<int32_t>(n);
    }
}

namespace {

// Softmax statistics of one row at temperature tau, in the fixed-point form
// shared with the device kernel:
//   l_v = logit_v / tau                      (fp32, correctly rounded)
//   e_v = orc_expf(l_v - max_v l_v)           (fp32)
//   E_v = floor(e_v * 2^32 + 0.5)             (exact in double, u64)
//   S   = sum_v E_v                           (u64: exact, order-independent)
// The probability of v is e_v / (S * 2^-32).  Because S is an exact integer
// sum, any parallel reduction order gives the same bits.
struct RowStats { std::vector<float> e; std::vector<uint64_t> E; uint64_t S = 0; };

// v in [0, 1]; NaN and non-positive values map to 0
inline uint64_t to_fixed(float v) { return v > 0.0f ? static_cast<uint64_t>(static_cast<double>(v) * 4294967296.0 + 0.5) : 0u; }

void row_stats(const float* logits, uint32_t V, float tau, RowStats& st)
{
    st.e.resize(V); st.E.resize(V);
    float mx = -HUGE_VALF;
    for (uint32_t v = 0; v < V; ++v) { const float l = logits[v] / tau; st.e[v] = l; if (l > mx) mx = l; }
    uint64_t S = 0;
    for (uint32_t v = 0; v < V; ++v)
    {
        const float e = orc_expf(st.e[v] - mx);
        st.e[v] = e;
        st.E[v] = to_fixed(e);
        S += st.E[v];
    }
    st.S = S;
}

// Inverse-CDF draw: the smallest v whose inclusive prefix of W exceeds
// floor(U * total / 2^32).  Integer-exact.
uint32_t draw_fixed(const uint64_t* W, uint32_t V, uint64_t total, uint32_t U)
{
    const unsigned __int128 prod = static_cast<unsigned __int128>(U) * total;
    const uint64_t t = static_cast<uint64_t>(prod >> 32);
    uint64_t pre = 0;
    for (uint32_t v = 0; v < V; ++v) { pre += W[v]; if (pre > t) return v; }
    return V - 1;
}

inline float uniform24(uint32_t u) { return static_cast<float>(u >> 8) * (1.0f / 16777216.0f); }

}  // namespace

void orc_accept_rejection(const float* target_logits, const float* draft_logits,
                          const int32_t* drafts, uint32_t B, uint32_t K, uint32_t V,
                          float temperature, uint64_t seed, const uint32_t* pos_base,
                          int32_t* out_tokens, int32_t* accepted, float* dist_out)
{
    RowStats P, Q;
    std::vector<uint64_t> Rw(V);
    for (uint32_t b = 0; b < B; ++b)
    {
        const uint32_t pb = pos_base ? pos_base[b] : 0u;
        uint32_t n = 0;
        for (; n < K; ++n)
        {
            row_stats(target_logits + (static_cast<uint64_t>(b) * (K + 1) + n) * V, V, temperature, P);
            row_stats(draft_logits + (static_cast<uint64_t>(b) * K + n) * V, V, temperature, Q);
            const uint32_t xv = static_cast<uint32_t>(drafts[b * K + n]);
            const float u = uniform24(orc_philox_u32(seed, pb + n, b, 1));
            // accept iff u * q(x) < p(x)  <=>  (u * e_q(x)) * S_p < e_p(x) * S_q.
            // u * e_q(x) is exact in double (24 x 24 bits); each side then
            // rounds once, identically on host and device.
            const double lhs = (static_cast<double>(u) * static_cast<double>(Q.e[xv])) * static_cast<double>(P.S);
            const double rhs = static_cast<double>(P.e[xv]) * static_cast<double>(Q.S);
            if (!(lhs < rhs)) break;
        }
        float* dist = dist_out ? dist_out + static_cast<uint64_t>(b) * V : nullptr;
        uint32_t tok;
        const uint32_t U = orc_philox_u32(seed, pb + n, b, 2);
        if (n < K)
        {
            // residual max(0, p - q) at the rejected row (P, Q hold row n)
            const double invP = 4294967296.0 / static_cast<double>(P.S);
            const double invQ = 4294967296.0 / static_cast<double>(Q.S);
            std::vector<float> r(V);
            uint64_t Rs = 0;
            for (uint32_t v = 0; v < V; ++v)
            {
                const float pf = static_cast<float>(static_cast<double>(P.e[v]) * invP);
                const float qf = static_cast<float>(static_cast<double>(Q.e[v]) * invQ);
                const float d = pf - qf;
                r[v] = d > 0.0f ? d : 0.0f;
                Rw[v] = to_fixed(r[v]);
                Rs += Rw[v];
            }
            if (Rs > 0)
            {
                tok = draw_fixed(Rw.data(), V, Rs, U);
                const double invR = 4294967296.0 / static_cast<double>(Rs);
                if (dist) for (uint32_t v = 0; v < V; ++v) dist[v] = static_cast<float>(static_cast<double>(r[v]) * invR);
            }
            else
            {
                tok = draw_fixed(P.E.data(), V, P.S, U);
                if (dist) for (uint32_t v = 0; v < V; ++v) dist[v] = static_cast<float>(static_cast<double>(P.e[v]) * invP);
            }
        }
        else
        {
            row_stats(target_logits + (static_cast<uint64_t>(b) * (K + 1) + K) * V, V, temperature, P);
            tok = draw_fixed(P.E.data(), V, P.S, U);
            const double invP = 4294967296.0 / static_cast<double>(P.S);
            if (dist) for (uint32_t v = 0; v < V; ++v) dist[v] = static_cast<float>(static_cast<double>(P.e[v]) * invP);
        }
        for (uint32_t j = 0; j <= K; ++j)
            out_tokens[b * (K + 1) + j] = j < n ? drafts[b * K + j] : (j == n ? static_cast<int32_t>(tok) : -1);
        accepted[b] = static_cast<int32_t>(n);
    }
}

void orc_sample_rows(const float* logits, uint32_t rows, uint32_t V, float temperature,
                     uint64_t seed, const uint32_t* pos, const uint32_t* seq,
                     uint32_t stream, int32_t* out)
{
    RowStats st;
    for (uint32_t r = 0; r < rows; ++r)
    {
        row_stats(logits + static_cast<uint64_t>(r) * V, V, temperature, st);
        const uint32_t U = orc_philox_u32(seed, pos[r], seq[r], stream);
        out[r] = static_cast<int32_t>(draw_fixed(st.E.data(), V, st.S, U));
    }
}

// ---------------------------------------------------------------------------
//  KV rollback.  The reference's nearest relative, EvictOldestKV
//  (Opure_VoxelEngine.cpp:721-763), is broken and not followed.
// ---------------------------------------------------------------------------
void orc_kv_rollback(orc_kv* kv, const orc_model* m, uint32_t B, uint32_t K,
                     const int32_t* seq_len, const int32_t* accepted,
                     int32_t* page_table_rw, int32_t* new_len, int32_t* freed,
                     uint32_t freed_stride, int32_t* n_freed, uint32_t poison_bits)
{
    const uint32_t ps = kv->page_size;
    for (uint32_t b = 0; b < B; ++b)
    {
        int32_t* pt = page_table_rw + static_cast<uint64_t>(b) * kv->max_pages_per_seq;
        const uint32_t old_end = static_cast<uint32_t>(seq_len[b]) + K + 1;
        const uint32_t nl = static_cast<uint32_t>(seq_len[b]) + static_cast<uint32_t>(accepted[b]) + 1;
        new_len[b] = static_cast<int32_t>(nl);
        if (poison_bits != 0)
        {
            for (uint32_t pos = nl; pos < old_end; ++pos)
            {
                const int32_t pg = pt[pos / ps];
                if (pg < 0) continue;
                for (uint32_t L = 0; L < m->n_layers; ++L)
                    for (uint32_t s = 0; s < 2; ++s)
                        for (uint32_t h = 0; h < m->n_kv_heads; ++h)
                        {
                            for (uint32_t d = 0; d < m->head_dim; ++d)
                            {
                                const uint64_t e = kv_elem(m, kv, L, pg, s, h, pos % ps, d);
                                if (m->afmt == ORC_A_F32) static_cast<uint32_t*>(kv->pool)[e] = poison_bits;
                                else static_cast<uint16_t*>(kv->pool)[e] = static_cast<uint16_t>(poison_bits);
                            }
                        }
            }
        }
        int32_t nf = 0;
        const uint32_t first_free = (nl + ps - 1) / ps;
        const uint32_t last_used = (old_end - 1) / ps;
        for (uint32_t p = first_free; p <= last_used && p < kv->max_pages_per_seq; ++p)
        {
            if (pt[p] < 0) continue;
            if (freed && static_cast<uint32_t>(nf) < freed_stride) freed[static_cast<uint64_t>(b) * freed_stride + nf] = pt[p];
            pt[p] = -1;
            ++nf;
        }
        if (n_freed) n_freed[b] = nf;
    }
}

}  // extern "C"
