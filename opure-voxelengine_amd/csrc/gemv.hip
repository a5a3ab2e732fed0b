// ============================================================================
//  gemv.hip -- host side of the K+1-row GEMV: the tiled weight layout, the
//  shape plan, validation and dispatch, and the public entry points.  The
//  kernel itself is gemv_kernel.h, instantiated per weight format in
//  gemv_f32.hip, gemv_i8.hip, gemv_i4h.hip and gemv_i4b.hip.
// ============================================================================
#include "gemm_wide.h"

#include <algorithm>

using namespace opure_dev_math;

namespace opure_gemv {

int launch_f32(opure_dev*, uint32_t, uint32_t, bool, const KParams&, const Recipe&, uint32_t, uint32_t);
int launch_i8(opure_dev*, uint32_t, uint32_t, bool, const KParams&, const Recipe&, uint32_t, uint32_t);
int launch_i4_f16(opure_dev*, uint32_t, uint32_t, bool, const KParams&, const Recipe&, uint32_t, uint32_t);
int launch_i4_bf16(opure_dev*, uint32_t, uint32_t, bool, const KParams&, const Recipe&, uint32_t, uint32_t);
int launch_wide_i8(opure_dev*, uint32_t, const WParams&, uint32_t, const float*, void*);
int launch_valu_f32(opure_dev*, uint32_t, const KParams&);
int launch_valu_i8(opure_dev*, uint32_t, const KParams&);
int launch_valu_i4_f16(opure_dev*, uint32_t, const KParams&);
int launch_valu_i4_bf16(opure_dev*, uint32_t, const KParams&);
int launch_wide_i4_f16(opure_dev*, uint32_t, const WParams&, uint32_t, const float*, void*);
int launch_wide_i4_bf16(opure_dev*, uint32_t, const WParams&, uint32_t, const float*, void*);

}  // namespace opure_gemv

namespace {

using opure_gemv::u4_t;
using opure_gemv::f4_t;

uint32_t kb_of(uint32_t wfmt) { return wfmt == OPURE_W_F32 ? 16u : (wfmt == OPURE_W_I8PC ? 64u : 128u); }
uint64_t row_bytes(uint32_t wfmt, uint32_t in)
{
    return wfmt == OPURE_W_F32 ? 4ull * in : (wfmt == OPURE_W_I8PC ? 1ull * in : in / 2ull);
}

// row of the row-major source held by row r of tile t
__device__ __forceinline__ uint32_t src_row(uint32_t layout, uint32_t t, uint32_t r, uint32_t out)
{
    if (layout == OPURE_LAYOUT_TILED_SWIGLU) return (r & 1u) ? (out >> 1) + 8u * t + (r >> 1) : 8u * t + (r >> 1);
    return 16u * t + r;
}

// one thread per 16-byte piece: tile t, block b, lane l = 16*g + r holds
// bytes [16g, 16g+16) of source row src_row(t, r), block b
__global__ __launch_bounds__(256) void k_tile_w(const uint8_t* src, uint8_t* dst, uint32_t wfmt, uint32_t layout,
                                                uint32_t out, uint32_t nblk, uint64_t rbytes, uint64_t pieces)
{
    const uint64_t id = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (id >= pieces) return;
    const uint32_t lane = static_cast<uint32_t>(id & 63u);
    const uint64_t tb = id >> 6;
    const uint32_t t = static_cast<uint32_t>(tb / nblk), b = static_cast<uint32_t>(tb % nblk);
    const uint32_t row = src_row(layout, t, lane & 15u, out);
    u4_t v = *reinterpret_cast<const u4_t*>(src + row * rbytes + 64ull * b + 16u * (lane >> 4));
    if (wfmt == OPURE_W_I8PC)
    {
        v ^= u4_t{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};   // offset binary
    }
    else if (wfmt == OPURE_W_I4G128)
    {
        // element 2i = high nibble of byte i -> element e at nibble {0,4,1,5,2,6,3,7}[e],
        // then the word rotated left by 3 bits (nibbles at bits 3..6 of a byte)
        constexpr uint32_t pos[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const uint32_t d = v[j];
            uint32_t o = 0;
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e)
            {
                const uint32_t byte = (d >> (8u * (e >> 1))) & 0xFFu;
                const uint32_t q = (e & 1u) ? (byte & 0x0Fu) : (byte >> 4);
                o |= q << (4u * pos[e]);
            }
            v[j] = (o << 3) | (o >> 29);
        }
    }
    *reinterpret_cast<u4_t*>(dst + (tb << 10) + (static_cast<uint64_t>(lane) << 4)) = v;
}

// int8: fp16[tiles][16]; uint4: (bf16 scale | bf16 zero << 16)[tiles][G][16]
__global__ __launch_bounds__(256) void k_tile_s(const uint16_t* scale, const uint16_t* zero, void* dst, uint32_t wfmt,
                                                uint32_t layout, uint32_t out, uint32_t G, uint64_t n)
{
    const uint64_t id = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (id >= n) return;
    const uint32_t r = static_cast<uint32_t>(id & 15u);
    if (wfmt == OPURE_W_I8PC)
    {
        const uint32_t t = static_cast<uint32_t>(id >> 4);
        static_cast<uint16_t*>(dst)[id] = scale[src_row(layout, t, r, out)];
        return;
    }
    const uint64_t tg = id >> 4;
    const uint32_t t = static_cast<uint32_t>(tg / G), g = static_cast<uint32_t>(tg % G);
    const uint64_t si = static_cast<uint64_t>(src_row(layout, t, r, out)) * G + g;
    static_cast<uint32_t*>(dst)[id] = static_cast<uint32_t>(scale[si]) | (static_cast<uint32_t>(zero[si]) << 16);
}

// The rmsnorm rows pass: xn[m][k] = round(x[m][k] * inv_m * g[k]), the same
// inverse rms (inv_rms_wave) and rounding as the staged fusion.  Workgroup
// (c, m) takes 2048 columns of row m, 8 per thread; every wave issues its x
// and gain loads, then computes inv_m itself, so the pass is one round trip.
template <int AF>
__global__ __launch_bounds__(256) void k_rmsnorm_rows(opure_gemv::KParams p, void* xn)
{
    constexpr uint32_t EB = AF == OPURE_A_F32 ? 4u : 2u;
    const uint32_t m = blockIdx.y, lane = threadIdx.x & 63u;
    const uint32_t j = blockIdx.x * 256u + threadIdx.x, n8 = p.in / 8u;
    const uint32_t jc = min(j, n8 - 1u);
    const f4_t* xr = reinterpret_cast<const f4_t*>(reinterpret_cast<const float*>(p.x) + static_cast<uint64_t>(m) * p.in + 8u * jc);
    const f4_t* gr = reinterpret_cast<const f4_t*>(p.gain + 8u * jc);
    const f4_t x0 = xr[0], x1 = xr[1], g0 = gr[0], g1 = gr[1];
    const float inv = opure_gemv::inv_rms_wave(p, m, lane);
    if (j >= n8) return;
    float yv[8];
#pragma unroll
    for (int e = 0; e < 4; ++e)
    {
        yv[e] = __fmul_rn(__fmul_rn(x0[e], inv), g0[e]);
        yv[4 + e] = __fmul_rn(__fmul_rn(x1[e], inv), g1[e]);
    }
    uint8_t* dst = static_cast<uint8_t*>(xn) + (static_cast<uint64_t>(m) * p.in + 8u * j) * EB;
    if constexpr (AF == OPURE_A_F32)
    {
        reinterpret_cast<u4_t*>(dst)[0] = __builtin_bit_cast(u4_t, f4_t{yv[0], yv[1], yv[2], yv[3]});
        reinterpret_cast<u4_t*>(dst)[1] = __builtin_bit_cast(u4_t, f4_t{yv[4], yv[5], yv[6], yv[7]});
    }
    else
    {
        *reinterpret_cast<u4_t*>(dst) = u4_t{opure_gemv::pack2<AF>(yv[0], yv[1]), opure_gemv::pack2<AF>(yv[2], yv[3]),
                                             opure_gemv::pack2<AF>(yv[4], yv[5]), opure_gemv::pack2<AF>(yv[6], yv[7])};
    }
}

int rmsnorm_rows_launch(opure_dev* dev, const opure_gemv::KParams& kp, uint32_t afmt, uint32_t M, void* xn)
{
    const dim3 grid((kp.in / 8u + 255u) / 256u, M);
    if (afmt == OPURE_A_F32)
        OPURE_LAUNCH(dev, k_rmsnorm_rows<OPURE_A_F32>, grid, dim3(256), 0, kp, xn);
    else if (afmt == OPURE_A_F16)
        OPURE_LAUNCH(dev, k_rmsnorm_rows<OPURE_A_F16>, grid, dim3(256), 0, kp, xn);
    else
        OPURE_LAUNCH(dev, k_rmsnorm_rows<OPURE_A_BF16>, grid, dim3(256), 0, kp, xn);
    OPURE_LAUNCH_CHECK("k_rmsnorm_rows");
    return OPURE_OK;
}

struct Plan {
    opure_gemv::Recipe r{};
    uint32_t tiles = 0, nblk = 0, groups = 0, grid = 0, lds = 0;
    bool staged = false;
    uint32_t x_stride = 0, off_xsum = 0, off_red = 0, off_ring = 0, ring = 0;
};

// The recipe depends on the shape only (so a row's result never depends on the
// rows beside it); staging, persistence and the grid only move work around.
Plan make_plan(const opure_dev* dev, uint32_t wfmt, uint32_t xfmt, uint32_t out, uint32_t in, uint32_t M)
{
    using namespace opure_gemv;
    Plan pl;
    pl.tiles = out / 16u;
    pl.nblk = in / kb_of(wfmt);
    const uint32_t EB = opure_hip::act_bytes(xfmt);
    const uint32_t stride = in * EB + 16u;
    const uint32_t xbytes = static_cast<uint32_t>(opure_hip::align_up(static_cast<uint64_t>(M) * stride, 16));
    // 1024 tiles and more: waves own whole tiles, if X, the group sums and a
    // 1 KB slot per wave fit in LDS -- judged at OPURE_MAX_ROWS rows, so that the
    // recipe (and with it every row's summation order) is the same for any M
    const uint32_t wpt_xs = wfmt == OPURE_W_I4G128 ? (in / 128u) * 64u : 0u;
    const uint32_t xbytes_max =
        static_cast<uint32_t>(opure_hip::align_up(static_cast<uint64_t>(OPURE_MAX_ROWS) * stride, 16));
    const bool wpt = pl.tiles >= 1024u && xbytes_max + wpt_xs + R_WPT.nw * 1024u <= 159u * 1024u;
    pl.r = wpt ? R_WPT
               : (pl.tiles >= 1024u ? R_WIDE
                                    : (pl.tiles >= 320u ? R_WIDE16 : (pl.tiles > 192u && in >= 8192u ? R_MID : R_NARROW)));
    pl.groups = (pl.tiles + pl.r.t - 1u) / pl.r.t;
    // the K-split kernels: one reduction buffer per group parity; the
    // wave-per-tile kernel: a 1 KB transposition slot per wave
    const uint32_t red = wpt ? pl.r.nw * 1024u : 2u * pl.r.nw * pl.r.t * 1024u;
    const uint32_t xsum = wpt ? wpt_xs : 0u;
    const uint32_t off_xsum = xbytes;
    const uint32_t off_red = static_cast<uint32_t>(opure_hip::align_up(off_xsum + xsum, 16));
    const uint32_t total = off_red + red;
    pl.staged = total <= 159u * 1024u;
    if (pl.staged)
    {
        pl.x_stride = stride;
        pl.off_xsum = off_xsum;
        pl.off_red = off_red;
        pl.lds = total;
    }
    else
    {
        pl.off_red = 0;
        pl.lds = red;
    }
    // wave-per-tile shapes of quantised weights and 16-bit X where most of the
    // 8 compute waves of a CU own one tile (6 to 8 tiles a CU: the 8B gate/up):
    // loader waves feed them through LDS rings, 3 slots each if they fit, else
    // 2.  Longer streams (the LM head) keep the wave-per-tile kernel, whose
    // waves keep more loads in flight, and so do fewer tiles (the 1B gate/up,
    // 4 a CU, measured slower in graph replay with loader waves).
    const uint32_t n_cu_pc = dev->n_cu > 0 ? static_cast<uint32_t>(dev->n_cu) : 256u;
    if (wpt && pl.staged && wfmt != OPURE_W_F32 && xfmt != OPURE_A_F32 && pl.nblk % PC_SB == 0 &&
        pl.tiles >= static_cast<uint32_t>(PC_NC - 2) * n_cu_pc && pl.tiles <= static_cast<uint32_t>(PC_NC) * n_cu_pc)
    {
        const uint32_t slot = wfmt == OPURE_W_I4G128 ? pc_slot_bytes<OPURE_W_I4G128>() : pc_slot_bytes<OPURE_W_I8PC>();
        const uint32_t off_ring = static_cast<uint32_t>(opure_hip::align_up(total, 16));
        for (uint32_t ring : {3u, 2u})
        {
            const uint32_t pc_total = off_ring + static_cast<uint32_t>(PC_NC) * ring * slot + 2u * PC_NC * 4u;
            if (pc_total <= 159u * 1024u)
            {
                pl.r.wpt = 2;
                pl.ring = ring;
                pl.off_ring = off_ring;
                pl.lds = pc_total;
                break;
            }
        }
    }
    // at most four tiles a workgroup (the 1B gate/up: 1024 tiles on 256 CUs,
    // so 4 of the 8 waves would own a tile): two waves a tile, each streaming
    // half of its blocks, so every wave loads
    if (wpt && pl.r.wpt == 1u && wfmt != OPURE_W_F32 && xfmt != OPURE_A_F32 && pl.nblk % 2u == 0 &&
        pl.tiles <= 4u * n_cu_pc)
        pl.r.wpt = 4;
    // persistent workgroups, one per CU
    const uint32_t n_cu = dev->n_cu > 0 ? static_cast<uint32_t>(dev->n_cu) : 256u;
    pl.grid = std::min(pl.groups, n_cu);
    return pl;
}

// Shape plan of the GEMV over more than OPURE_MAX_ROWS rows: row groups of 8
// tiles, column groups of at most 8 column tiles, and K splits for shapes
// with few row groups.  The splits depend on the weight shape only (not on
// the row count), so a row's sums do not depend on the batch around it.
struct WidePlan {
    uint32_t tiles = 0, nblk = 0, mt = 0, nrg = 0, ncg = 0, cgs = 0, splits = 1, bps = 0;
    uint64_t part_bytes = 0;
};

WidePlan wide_plan(const opure_dev* dev, uint32_t wfmt, uint32_t out, uint32_t in, uint32_t M)
{
    using namespace opure_gemv;
    WidePlan w;
    const uint32_t KB = kb_of(wfmt);
    const uint32_t U = wfmt == OPURE_W_I8PC ? WideDepth<OPURE_W_I8PC>::U : WideDepth<OPURE_W_I4G128>::U;
    w.tiles = out / 16u;
    w.nblk = in / KB;
    w.mt = (M + 15u) / 16u;
    w.nrg = (w.tiles + WIDE_RT - 1u) / WIDE_RT;
    w.ncg = (w.mt + WIDE_CG - 1u) / WIDE_CG;
    w.cgs = (w.mt + w.ncg - 1u) / w.ncg;
    // split K while there are fewer row groups than half the CUs (a batch
    // over 128 rows has two column groups), at most 8 ways and U blocks a split
    const uint32_t n_cu = dev && dev->n_cu > 0 ? static_cast<uint32_t>(dev->n_cu) : 256u;
    const uint32_t want = std::max(1u, n_cu / 2u);
    if (w.nrg < want) w.splits = std::min({(want + w.nrg - 1u) / w.nrg, std::max(1u, w.nblk / U), 8u});
    w.bps = (w.nblk + w.splits - 1u) / w.splits;
    w.bps = (w.bps + U - 1u) / U * U;
    w.splits = (w.nblk + w.bps - 1u) / w.bps;
    w.part_bytes = w.splits > 1u ? static_cast<uint64_t>(w.splits) * w.tiles * w.mt * 64u * 16u : 0u;
    return w;
}

}  // namespace

namespace opure_hip {

uint32_t tiled_block_k(uint32_t wfmt) { return kb_of(wfmt); }

uint64_t gemv_scratch_bytes(const opure_dev* dev, uint32_t wfmt, uint32_t out, uint32_t in, uint32_t M)
{
    if (M <= OPURE_MAX_ROWS || wfmt == OPURE_W_F32 || out % 16u || in % kb_of(wfmt)) return 0;
    return wide_plan(dev, wfmt, out, in, M).part_bytes;
}

uint32_t gemv_grid(const opure_dev* dev, const GemvCall& c)
{
    return make_plan(dev, c.wfmt, c.xfmt, c.W.out, c.W.in, c.M).grid;
}

bool gemv_is_wave_per_tile(const opure_dev* dev, const GemvCall& c)
{
    const Plan pl = make_plan(dev, c.wfmt, c.xfmt, c.W.out, c.W.in, c.M);
    // wpt 2 is the loader-wave kernel (k_gemv_pc)
    return pl.staged && (pl.r.wpt == 1u || pl.r.wpt == 4u);
}

int gemv_validate(const GemvCall& c)
{
    const uint32_t wf = c.wfmt, af = c.xfmt;
    OPURE_REQUIRE(wf <= OPURE_W_I4G128 && af <= OPURE_A_BF16, OPURE_E_INVALID, "gemv: bad format (w %u, x %u)", wf, af);
    const bool ok = (wf == OPURE_W_F32 && af == OPURE_A_F32) || (wf == OPURE_W_I8PC && af == OPURE_A_F16) ||
                    (wf == OPURE_W_I4G128 && (af == OPURE_A_F16 || af == OPURE_A_BF16));
    OPURE_REQUIRE(ok, OPURE_E_UNSUPPORTED, "gemv: weights %u with %s activations are not built", wf, afmt_name(af));
    OPURE_REQUIRE(c.W.w && c.x && c.y, OPURE_E_INVALID, "gemv: null weight, input or output pointer");
    const uint32_t want = c.epi == EPI_SWIGLU ? OPURE_LAYOUT_TILED_SWIGLU : OPURE_LAYOUT_TILED;
    OPURE_REQUIRE(c.W.layout == want, OPURE_E_INVALID,
                  "gemv: weights must be in layout %u (opure_tile_linear), got %u", want, c.W.layout);
    OPURE_REQUIRE(c.M >= 1 && c.M <= OPURE_MAX_BATCH_ROWS, OPURE_E_CAPACITY, "gemv: M=%u outside 1..%d", c.M,
                  OPURE_MAX_BATCH_ROWS);
    if (c.M > OPURE_MAX_ROWS)
    {
        OPURE_REQUIRE(wf != OPURE_W_F32 && af != OPURE_A_F32, OPURE_E_UNSUPPORTED,
                      "gemv: more than %d rows needs quantised weights and 16-bit activations", OPURE_MAX_ROWS);
        OPURE_REQUIRE(c.epi != EPI_LOGITS, OPURE_E_UNSUPPORTED,
                      "gemv: argmax partials are built for at most %d rows (store the logits instead)", OPURE_MAX_ROWS);
        OPURE_REQUIRE(!c.gain || c.xn_scratch, OPURE_E_INVALID, "gemv: rmsnorm over %u rows needs xn_scratch", c.M);
        OPURE_REQUIRE(!c.norm_gain || (c.epi == EPI_RESIDUAL && c.norm_out && c.ss_out &&
                                       (reinterpret_cast<uintptr_t>(c.norm_gain) & 15u) == 0),
                      OPURE_E_INVALID, "gemv: a fused next rmsnorm needs the residual epilogue, norm_out, ss_out and "
                      "a 16-byte aligned gain");
    }
    else
    {
        OPURE_REQUIRE(!c.norm_gain, OPURE_E_INVALID, "gemv: a fused next rmsnorm is built for more than %d rows",
                      OPURE_MAX_ROWS);
    }
    OPURE_REQUIRE(c.W.out >= 16 && c.W.out % 16 == 0, OPURE_E_INVALID, "gemv: out=%u must be a positive multiple of 16",
                  c.W.out);
    const uint32_t KB = kb_of(wf);
    OPURE_REQUIRE(c.W.in >= KB && c.W.in % KB == 0, OPURE_E_INVALID, "gemv: in=%u must be a multiple of %u", c.W.in, KB);
    OPURE_REQUIRE((reinterpret_cast<uintptr_t>(c.W.w) & 15u) == 0 && (reinterpret_cast<uintptr_t>(c.x) & 15u) == 0,
                  OPURE_E_INVALID, "gemv: weight and input pointers must be 16-byte aligned");
    if (wf != OPURE_W_F32)
        OPURE_REQUIRE(c.W.scale && (reinterpret_cast<uintptr_t>(c.W.scale) & 15u) == 0, OPURE_E_INVALID,
                      "gemv: quantised weights need 16-byte aligned tiled scales");
    OPURE_REQUIRE(c.yfmt <= OPURE_A_BF16, OPURE_E_INVALID, "gemv: bad output format %u", c.yfmt);
    if (c.epi == EPI_RESIDUAL || c.epi == EPI_LOGITS)
        OPURE_REQUIRE(c.yfmt == OPURE_A_F32, OPURE_E_INVALID, "gemv: residual/logits output must be f32");
    if (c.epi == EPI_SWIGLU) OPURE_REQUIRE(c.W.out % 32 == 0, OPURE_E_INVALID, "gemv: swiglu needs 2*ffn %% 32 == 0");
    if (c.epi == EPI_LOGITS) OPURE_REQUIRE(c.logits.am_val && c.logits.am_idx, OPURE_E_INVALID, "gemv: argmax partials");
    if (c.gain)
        OPURE_REQUIRE(c.ss_in && c.ss_tiles >= 1 && (reinterpret_cast<uintptr_t>(c.gain) & 15u) == 0 &&
                          (c.epi == EPI_SWIGLU || c.epi == EPI_QKV || c.epi == EPI_LOGITS || c.M > OPURE_MAX_ROWS),
                      OPURE_E_INVALID, "gemv: fused rmsnorm needs sums of squares, an aligned gain and a consumer epilogue");

    if (c.epi == EPI_QKV)
    {
        const QkvEpilogue& e = c.qkv;
        OPURE_REQUIRE(e.head_dim >= 16 && e.head_dim % 16 == 0 && e.qdim % e.head_dim == 0 && e.kvdim % e.head_dim == 0 &&
                          c.W.out == e.qdim + 2u * e.kvdim,
                      OPURE_E_INVALID, "gemv: qkv epilogue shape mismatch");
        OPURE_REQUIRE(e.rope_cos && e.rope_sin && e.seq_len && e.kv_pool && e.page_table && e.rows_per_seq >= 1 &&
                          c.M % e.rows_per_seq == 0,
                      OPURE_E_INVALID, "gemv: qkv epilogue pointers");
    }
    return OPURE_OK;
}

static int gemv_launch_wide(opure_dev* dev, const GemvCall& c)
{
    using namespace opure_gemv;
    const WidePlan w = wide_plan(dev, c.wfmt, c.W.out, c.W.in, c.M);
    OPURE_REQUIRE(w.splits == 1u || c.part_scratch, OPURE_E_INVALID, "gemv: %u x %u over %u rows needs part_scratch",
                  c.W.out, c.W.in, c.M);
    WParams wp{};
    KParams& kp = wp.p;
    kp.w = static_cast<const uint8_t*>(c.W.w);
    kp.sc = c.W.scale;
    kp.out = c.W.out;
    kp.in = c.W.in;
    kp.tiles = w.tiles;
    kp.nblk = w.nblk;
    kp.x = static_cast<const uint8_t*>(c.x);
    kp.M = c.M;
    kp.y = c.y;
    kp.yfmt = c.yfmt;
    kp.ss_out = c.ss_out;
    kp.err = dev->err;
    kp.wait_limit = dev->wait_limit;
    kp.qkv = c.qkv;
    wp.mt = w.mt;
    wp.nrg = w.nrg;
    wp.ncg = w.ncg;
    wp.cgs = w.cgs;
    wp.splits = w.splits;
    wp.bps = w.bps;
    wp.part = static_cast<f4_t*>(c.part_scratch);
    kp.eps = c.eps;
    // a residual with K splits and the next rmsnorm: row-major partials, added
    // and normalised per row by k_wide_reduce_norm (outputs up to 4096)
    const bool fused_norm = c.norm_gain && c.epi == EPI_RESIDUAL && w.splits > 1u && w.splits <= 8u && c.W.out <= 4096u;
    wp.part_rows = fused_norm ? 1u : 0u;
    if (c.gain)
    {
        // rmsnorm into the scratch rows first, then the GEMV reads them
        kp.gain = c.gain;
        kp.eps = c.eps;
        kp.ss_in = c.ss_in;
        kp.ss_tiles = c.ss_tiles;
        const int rc = rmsnorm_rows_launch(dev, kp, c.xfmt, c.M, c.xn_scratch);
        if (rc) return rc;
        kp.x = static_cast<const uint8_t*>(c.xn_scratch);
        kp.gain = nullptr;
    }
    const float* ng = fused_norm ? c.norm_gain : nullptr;
    int rc;
    if (c.wfmt == OPURE_W_I8PC) rc = launch_wide_i8(dev, c.epi, wp, 0, ng, c.norm_out);
    else if (c.xfmt == OPURE_A_F16) rc = launch_wide_i4_f16(dev, c.epi, wp, 0, ng, c.norm_out);
    else rc = launch_wide_i4_bf16(dev, c.epi, wp, 0, ng, c.norm_out);
    if (rc || !c.norm_gain || fused_norm) return rc;
    // the same normalised rows from the residual just written (no splits to fuse into)
    KParams np = kp;
    np.x = static_cast<const uint8_t*>(c.y);
    np.in = c.W.out;
    np.gain = c.norm_gain;
    np.ss_in = c.ss_out;
    np.ss_tiles = c.W.out / 16u;
    return rmsnorm_rows_launch(dev, np, c.xfmt, c.M, c.norm_out);
}

int gemv_launch(opure_dev* dev, const GemvCall& c)
{
    using namespace opure_gemv;
    if (c.M > OPURE_MAX_ROWS) return gemv_launch_wide(dev, c);
    const bool norm = c.gain != nullptr;
    Plan pl = make_plan(dev, c.wfmt, c.xfmt, c.W.out, c.W.in, c.M);
    KParams kp{};
    kp.w = static_cast<const uint8_t*>(c.W.w);
    kp.sc = c.W.scale;
    kp.out = c.W.out;
    kp.in = c.W.in;
    kp.tiles = pl.tiles;
    kp.nblk = pl.nblk;
    kp.groups = pl.groups;
    kp.x = static_cast<const uint8_t*>(c.x);
    kp.M = c.M;
    kp.y = c.y;
    kp.yfmt = c.yfmt;
    kp.gain = c.gain;
    kp.eps = c.eps;
    kp.ss_in = c.ss_in;
    kp.ss_tiles = c.ss_tiles;
    kp.ss_out = c.ss_out;
    kp.err = dev->err;
    kp.wait_limit = dev->wait_limit;
    kp.x_stride = pl.x_stride;
    kp.off_xsum = pl.off_xsum;
    kp.off_red = pl.off_red;
    kp.off_ring = pl.off_ring;
    kp.ring = pl.ring;
    kp.qkv = c.qkv;
    kp.lg = c.logits;
    // the vector-ALU engine, where it is chosen (at most 8 rows, a plain epilogue)
    if (dev->gemv_engine == OPURE_GEMV_VALU && c.M <= VALU_MAXM && !norm &&
        (c.epi == EPI_STORE || c.epi == EPI_RESIDUAL || c.epi == EPI_SWIGLU))
    {
        if (c.wfmt == OPURE_W_F32) return launch_valu_f32(dev, c.epi, kp);
        if (c.wfmt == OPURE_W_I8PC) return launch_valu_i8(dev, c.epi, kp);
        return c.xfmt == OPURE_A_F16 ? launch_valu_i4_f16(dev, c.epi, kp) : launch_valu_i4_bf16(dev, c.epi, kp);
    }
    // Without the fused rmsnorm, shapes under 320 tiles (at most one group a
    // CU) take their X fragments from memory with the weights instead of
    // staging X in LDS: the first blocks then wait for no barrier and no
    // staging round trip (the 1B o_proj and down run 0.4-0.7 us faster).  The
    // waves take the same blocks either way, so the sums are the same.
    if (!norm && pl.staged && pl.r.wpt == 0u && pl.tiles < 320u)
    {
        pl.staged = false;
        pl.off_red = 0;
        pl.lds = 2u * pl.r.nw * pl.r.t * 1024u;
        kp.off_red = 0;
        kp.x_stride = 0;
    }
    uint32_t nm = norm ? 1u : 0u;
    if (norm && !pl.staged)
    {
        // the rows pass into the scratch rows, then a plain GEMV
        OPURE_REQUIRE(c.xn_scratch, OPURE_E_UNSUPPORTED, "gemv: rmsnorm over %u x %u needs a scratch buffer", c.M,
                      c.W.in);
        const int rc = rmsnorm_rows_launch(dev, kp, c.xfmt, c.M, c.xn_scratch);
        if (rc) return rc;
        kp.x = static_cast<const uint8_t*>(c.xn_scratch);
        kp.gain = nullptr;
        nm = 0u;
    }
    if (c.wfmt == OPURE_W_F32) return launch_f32(dev, c.epi, nm, pl.staged, kp, pl.r, pl.grid, pl.lds);
    if (c.wfmt == OPURE_W_I8PC) return launch_i8(dev, c.epi, nm, pl.staged, kp, pl.r, pl.grid, pl.lds);
    if (c.xfmt == OPURE_A_F16) return launch_i4_f16(dev, c.epi, nm, pl.staged, kp, pl.r, pl.grid, pl.lds);
    return launch_i4_bf16(dev, c.epi, nm, pl.staged, kp, pl.r, pl.grid, pl.lds);
}

}  // namespace opure_hip

using namespace opure_hip;

static int gemv_public(opure_dev* dev, const opure_gemv_args* a, uint32_t wfmt)
{
    OPURE_REQUIRE(dev && a, OPURE_E_INVALID, "gemv: null argument");
    OPURE_REQUIRE(a->epilogue <= OPURE_EPI_SWIGLU, OPURE_E_INVALID, "gemv: bad epilogue %u", a->epilogue);
    GemvCall c;
    c.W = a->W;
    c.wfmt = wfmt;
    c.x = a->x;
    c.xfmt = a->xfmt;
    c.M = a->M;
    c.y = a->y;
    c.yfmt = a->yfmt;
    c.epi = a->epilogue;
    int rc = gemv_validate(c);
    if (rc) return rc;
    const uint64_t scratch = gemv_scratch_bytes(dev, wfmt, c.W.out, c.W.in, c.M);
    if (scratch)
    {
        if ((rc = ensure_workspace(dev, scratch))) return rc;
        c.part_scratch = dev->ws;
    }
    return gemv_launch(dev, c);
}

extern "C" {

int opure_gemv_batched_f32(opure_dev* dev, const opure_gemv_args* a) { return gemv_public(dev, a, OPURE_W_F32); }
int opure_gemv_batched_i8pc(opure_dev* dev, const opure_gemv_args* a) { return gemv_public(dev, a, OPURE_W_I8PC); }
int opure_gemv_batched_i4g128(opure_dev* dev, const opure_gemv_args* a) { return gemv_public(dev, a, OPURE_W_I4G128); }

int opure_tiled_bytes(uint32_t wfmt, uint32_t out, uint32_t in, uint64_t* w_bytes, uint64_t* scale_bytes)
{
    OPURE_REQUIRE(w_bytes && scale_bytes && wfmt <= OPURE_W_I4G128, OPURE_E_INVALID, "opure_tiled_bytes: bad argument");
    OPURE_REQUIRE(out % 16 == 0 && out > 0 && in % kb_of(wfmt) == 0 && in > 0, OPURE_E_INVALID,
                  "opure_tiled_bytes: %u x %u is not a whole number of 16-row tiles and 64-byte blocks", out, in);
    *w_bytes = static_cast<uint64_t>(out) * row_bytes(wfmt, in);
    *scale_bytes = wfmt == OPURE_W_F32 ? 0 : (wfmt == OPURE_W_I8PC ? 2ull * out : 4ull * out * (in / 128u));
    return OPURE_OK;
}

int opure_tile_linear(opure_dev* dev, uint32_t wfmt, uint32_t layout, const opure_linear* src, void* w_dst,
                      void* scale_dst, opure_linear* dst)
{
    OPURE_REQUIRE(dev && src && dst && w_dst, OPURE_E_INVALID, "opure_tile_linear: null argument");
    OPURE_REQUIRE(layout == OPURE_LAYOUT_TILED || layout == OPURE_LAYOUT_TILED_SWIGLU, OPURE_E_INVALID,
                  "opure_tile_linear: layout %u", layout);
    OPURE_REQUIRE(src->layout == OPURE_LAYOUT_ROWMAJOR && src->w, OPURE_E_INVALID,
                  "opure_tile_linear: the source must be a row-major linear");
    uint64_t wb = 0, sb = 0;
    int rc = opure_tiled_bytes(wfmt, src->out, src->in, &wb, &sb);
    if (rc) return rc;
    if (layout == OPURE_LAYOUT_TILED_SWIGLU)
        OPURE_REQUIRE(src->out % 32 == 0, OPURE_E_INVALID, "opure_tile_linear: [gate; up] needs out %% 32 == 0");
    if (wfmt != OPURE_W_F32) OPURE_REQUIRE(src->scale && scale_dst, OPURE_E_INVALID, "opure_tile_linear: scales");
    if (wfmt == OPURE_W_I4G128) OPURE_REQUIRE(src->zero, OPURE_E_INVALID, "opure_tile_linear: zero points");
    OPURE_REQUIRE((reinterpret_cast<uintptr_t>(src->w) & 15u) == 0 && (reinterpret_cast<uintptr_t>(w_dst) & 15u) == 0,
                  OPURE_E_INVALID, "opure_tile_linear: 16-byte aligned weights");
    const uint32_t nblk = src->in / kb_of(wfmt);
    const uint64_t pieces = static_cast<uint64_t>(src->out / 16u) * nblk * 64u;
    OPURE_LAUNCH(dev, k_tile_w, dim3(static_cast<uint32_t>((pieces + 255u) / 256u)), dim3(256), 0,
                       static_cast<const uint8_t*>(src->w), static_cast<uint8_t*>(w_dst), wfmt, layout, src->out, nblk,
                       row_bytes(wfmt, src->in), pieces);
    OPURE_LAUNCH_CHECK("k_tile_w");
    if (wfmt != OPURE_W_F32)
    {
        const uint64_t n = wfmt == OPURE_W_I8PC ? src->out : static_cast<uint64_t>(src->out) * (src->in / 128u);
        OPURE_LAUNCH(dev, k_tile_s, dim3(static_cast<uint32_t>((n + 255u) / 256u)), dim3(256), 0,
                           static_cast<const uint16_t*>(src->scale), static_cast<const uint16_t*>(src->zero), scale_dst,
                           wfmt, layout, src->out, src->in / 128u, n);
        OPURE_LAUNCH_CHECK("k_tile_s");
    }
    dst->w = w_dst;
    dst->scale = wfmt == OPURE_W_F32 ? nullptr : scale_dst;
    dst->zero = nullptr;
    dst->out = src->out;
    dst->in = src->in;
    dst->layout = layout;
    return OPURE_OK;
}

}  // extern "C"
