// ============================================================================
//  model_loader.cpp -- ModelConfig, ModelFiles (host) and LoadedModel (device).
// ============================================================================
#include "model_loader.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <set>

#include "voxel_engine.h"

namespace opure::engine {

namespace {

[[noreturn]] void fail(int code, const std::string& what) { throw Error(code, "model loader: " + what); }

// ---- number formats --------------------------------------------------------
float f16_to_f32(uint16_t h)
{
    const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1Fu) bits = s | 0x7F800000u | (m << 13);
    else if (e != 0) bits = s | ((e + 112u) << 23) | (m << 13);
    else if (m == 0) bits = s;
    else
    {
        // subnormal: m * 2^-24, exact in fp32
        float v = static_cast<float>(m) * 5.9604644775390625e-8f;
        std::memcpy(&bits, &v, 4);
        bits |= s;
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

float bf16_to_f32(uint16_t h)
{
    const uint32_t bits = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// round to nearest even; NaN stays NaN
uint16_t f32_to_bf16(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// round to nearest even, with fp16 subnormals and overflow to infinity
uint16_t f32_to_f16(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint16_t s = static_cast<uint16_t>((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return static_cast<uint16_t>(s | 0x7E00u);
    if (a >= 0x477FF000u) return static_cast<uint16_t>(s | 0x7C00u);   // rounds past 65504
    if (a < 0x38800000u)                                               // below 2^-14: subnormal
    {
        float x;
        std::memcpy(&x, &a, 4);
        const float q = std::nearbyint(x * 16777216.0f);                // units of 2^-24, ties to even
        return static_cast<uint16_t>(s | static_cast<uint16_t>(q));
    }
    const uint32_t r = a + 0xFFFu + ((a >> 13) & 1u);
    return static_cast<uint16_t>(s | ((r - 0x38000000u) >> 13));
}

// a 16-bit float tensor's value at element i, as fp32
float load_float(Dtype d, const uint8_t* p, uint64_t i)
{
    uint16_t h;
    switch (d)
    {
    case Dtype::F32:
    {
        float f;
        std::memcpy(&f, p + 4 * i, 4);
        return f;
    }
    case Dtype::F16: std::memcpy(&h, p + 2 * i, 2); return f16_to_f32(h);
    case Dtype::BF16: std::memcpy(&h, p + 2 * i, 2); return bf16_to_f32(h);
    default: break;
    }
    fail(OPURE_E_INVALID, "not a float tensor");
}

bool is_float(Dtype d) { return d == Dtype::F32 || d == Dtype::F16 || d == Dtype::BF16; }

// A stored scale narrowed to the fp16 (int8) or bf16 (int4) the kernels read:
// a finite nonzero scale that would round to zero or overflow to infinity
// (and silently zero or blow up its whole linear) is refused.
uint16_t narrow_scale(double v, bool to_bf16, const std::string& tensor)
{
    const float f = static_cast<float>(v);
    const uint16_t h = to_bf16 ? f32_to_bf16(f) : f32_to_f16(f);
    const uint16_t mag = h & 0x7FFFu, inf = to_bf16 ? 0x7F80u : 0x7C00u;
    if (std::isfinite(v) && v != 0.0 && (mag == 0 || mag == inf))
        fail(OPURE_E_UNSUPPORTED, tensor + ": scale " + std::to_string(v) + " is outside the " +
                                      (to_bf16 ? "bf16" : "fp16") + " range the kernels read");
    return h;
}

std::string shape_str(const std::vector<int64_t>& s)
{
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

bool shape_is(const Tensor& t, std::initializer_list<int64_t> want)
{
    return t.shape.size() == want.size() && std::equal(want.begin(), want.end(), t.shape.begin());
}

uint32_t get_u32(const Json& root, const char* key, bool required, uint32_t dflt = 0)
{
    const Json* v = root.Find(key);
    if (!v || v->kind == Json::Null)
    {
        if (required) fail(OPURE_E_INVALID, std::string("config.json: '") + key + "' is missing");
        return dflt;
    }
    if (v->kind != Json::Number || v->num < 0 || v->num > 4294967295.0 || v->num != std::floor(v->num))
        fail(OPURE_E_INVALID, std::string("config.json: '") + key + "' is not a non-negative integer");
    return static_cast<uint32_t>(v->num);
}

bool get_bool(const Json& root, const char* key, bool dflt)
{
    const Json* v = root.Find(key);
    if (!v || v->kind == Json::Null) return dflt;
    if (v->kind != Json::Bool) fail(OPURE_E_INVALID, std::string("config.json: '") + key + "' is not a boolean");
    return v->b;
}

uint32_t default_afmt(uint32_t wfmt)
{
    return wfmt == OPURE_W_F32 ? OPURE_A_F32 : wfmt == OPURE_W_I8PC ? OPURE_A_F16 : OPURE_A_BF16;
}

const char* role_name(Role r)
{
    switch (r)
    {
    case Role::Embed: return "embed";
    case Role::LmHead: return "lm_head";
    case Role::Qkv: return "qkv";
    case Role::O: return "o_proj";
    case Role::GateUp: return "gate_up";
    case Role::Down: return "down_proj";
    case Role::AttnNorm: return "input_layernorm";
    case Role::MlpNorm: return "post_attention_layernorm";
    case Role::FinalNorm: return "final norm";
    }
    return "?";
}

std::string layer_prefix(uint32_t i) { return "model.layers." + std::to_string(i) + "."; }

// Rows [row0, row0 + heads * hd) of h, head by head: new row 2p = row p, new
// row 2p + 1 = row p + hd/2, with the rows' scales and zero points (a
// rotate-half checkpoint's q / k rows in the adjacent-pair order the kernels
// rotate).
void permute_half_to_adjacent(HostLinear& h, uint32_t row0, uint32_t heads, uint32_t hd)
{
    for (std::vector<uint8_t>* v : {&h.w, &h.scale, &h.zero})
    {
        if (v->empty()) continue;
        const uint64_t rb = v->size() / h.out;                   // bytes per row of this array
        std::vector<uint8_t> head(rb * hd);
        for (uint32_t i = 0; i < heads; ++i)
        {
            uint8_t* base = v->data() + (static_cast<uint64_t>(row0) + static_cast<uint64_t>(i) * hd) * rb;
            std::memcpy(head.data(), base, head.size());
            for (uint32_t p = 0; p < hd / 2; ++p)
            {
                std::memcpy(base + (2ull * p) * rb, head.data() + static_cast<uint64_t>(p) * rb, rb);
                std::memcpy(base + (2ull * p + 1) * rb, head.data() + (static_cast<uint64_t>(p) + hd / 2) * rb, rb);
            }
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
//  config.json
// ---------------------------------------------------------------------------
ModelConfig ModelConfig::Parse(const std::string& text)
{
    const Json root = Json::Parse(text);
    if (root.kind != Json::Object) fail(OPURE_E_INVALID, "config.json is not a JSON object");
    ModelConfig c;
    c.vocab = get_u32(root, "vocab_size", true);
    c.hidden = get_u32(root, "hidden_size", true);
    c.ffn = get_u32(root, "intermediate_size", true);
    c.nLayers = get_u32(root, "num_hidden_layers", true);
    c.nHeads = get_u32(root, "num_attention_heads", true);
    // MHA checkpoints omit num_key_value_heads; HF then uses num_attention_heads
    c.nKvHeads = get_u32(root, "num_key_value_heads", false, c.nHeads);
    c.headDim = get_u32(root, "head_dim", false, c.nHeads ? c.hidden / c.nHeads : 0);
    c.maxPositionEmbeddings = get_u32(root, "max_position_embeddings", false, 0);
    const Json* eps = root.Find("rms_norm_eps");
    if (!eps || eps->kind != Json::Number) fail(OPURE_E_INVALID, "config.json: 'rms_norm_eps' is missing");
    c.rmsEps = static_cast<float>(eps->num);
    if (const Json* t = root.Find("rope_theta"); t && t->kind == Json::Number) c.ropeTheta = t->num;
    c.tied = get_bool(root, "tie_word_embeddings", true);

    if (const Json* act = root.Find("hidden_act"); act && act->kind == Json::String && act->str != "silu")
        fail(OPURE_E_UNSUPPORTED, "hidden_act '" + act->str + "' is not implemented (only silu / SwiGLU is)");
    if (get_bool(root, "attention_bias", false) || get_bool(root, "mlp_bias", false))
        fail(OPURE_E_UNSUPPORTED, "bias terms are not implemented");
    // any RoPE scaling changes the frequency schedule, not just theta: refused, as the reference does
    if (const Json* rs = root.Find("rope_scaling"); rs && rs->kind == Json::Object)
    {
        const Json* ty = rs->Find("rope_type");
        if (!ty) ty = rs->Find("type");
        const std::string t = ty && ty->kind == Json::String ? ty->str : "unknown";
        if (t != "default" && t != "none") fail(OPURE_E_UNSUPPORTED, "rope_scaling '" + t + "' is not implemented");
    }
    if (const Json* q = root.Find("quantization_config"); q && q->kind == Json::Object)
    {
        if (const Json* a = q->Find("activation_dtype"); a && a->kind == Json::String)
        {
            if (a->str == "float16") c.activationAfmt = OPURE_A_F16;
            else if (a->str == "bfloat16") c.activationAfmt = OPURE_A_BF16;
            else if (a->str == "float32") c.activationAfmt = OPURE_A_F32;
            else fail(OPURE_E_UNSUPPORTED, "quantization_config.activation_dtype '" + a->str + "'");
        }
    }

    if (!c.vocab || !c.hidden || !c.ffn || !c.nLayers || !c.nHeads || !c.nKvHeads)
        fail(OPURE_E_INVALID, "config.json is missing a required dimension");
    if (c.nHeads % c.nKvHeads)
        fail(OPURE_E_INVALID, "num_attention_heads " + std::to_string(c.nHeads) + " is not a multiple of num_key_value_heads " +
                                  std::to_string(c.nKvHeads));
    // the reference accepts 64 and 128 only (Opure_Graph.cpp:167-174); the
    // attention here takes any multiple of 16 up to 256 (64 and 128 on the
    // matrix cores, the others on the vector path)
    if (c.headDim < 16 || c.headDim > 256 || c.headDim % 16)
        fail(OPURE_E_UNSUPPORTED, "head_dim " + std::to_string(c.headDim) + " (attention takes multiples of 16 up to 256)");
    return c;
}

// ---------------------------------------------------------------------------
//  ModelFiles
// ---------------------------------------------------------------------------
ModelFiles::ModelFiles(const std::string& dir, const LoadOptions& opts) : dir_(dir)
{
    namespace fs = std::filesystem;
    cfg_ = ModelConfig::Parse(ReadTextFile((fs::path(dir) / "config.json").string()));

    std::vector<std::string> shards;
    const fs::path index = fs::path(dir) / "model.safetensors.index.json";
    if (fs::exists(index))
    {
        const Json j = Json::Parse(ReadTextFile(index.string()));
        const Json* map = j.Find("weight_map");
        if (!map || map->kind != Json::Object) fail(OPURE_E_INVALID, "model.safetensors.index.json has no weight_map");
        std::set<std::string> seen;
        for (const auto& [name, file] : map->obj)
        {
            if (file.kind != Json::String) fail(OPURE_E_INVALID, "weight_map entry of '" + name + "' is not a file name");
            // a shard is a file inside the model directory: no absolute path, no '..'
            const fs::path sp(file.str);
            bool up = false;
            for (const fs::path& c : sp) up = up || c == "..";
            if (file.str.empty() || sp.is_absolute() || up)
                fail(OPURE_E_INVALID, "weight_map names shard '" + file.str + "' outside the model directory");
            if (seen.insert(file.str).second) shards.push_back(file.str);
        }
    }
    else
    {
        shards.push_back("model.safetensors");
    }
    const fs::path root = fs::weakly_canonical(fs::path(dir));
    for (const std::string& s : shards)
    {
        // ... and it does not leave the directory through a link either
        const fs::path full = fs::weakly_canonical(fs::path(dir) / s);
        const auto [r_end, f_it] = std::mismatch(root.begin(), root.end(), full.begin(), full.end());
        if (r_end != root.end()) fail(OPURE_E_INVALID, "shard '" + s + "' resolves outside the model directory");
        (void)f_it;
        auto f = std::make_unique<WeightStreamer>();
        f->Open((fs::path(dir) / s).string());
        fileBytes_ += fs::file_size(fs::path(dir) / s);
        files_.push_back(std::move(f));
    }

    // the stored format is the first layer's q_proj's; every quantised linear must share it
    storedWfmt_ = Resolve(layer_prefix(0) + "self_attn.q_proj", cfg_.nHeads * cfg_.headDim, cfg_.hidden).wfmt;
    wfmt_ = opts.wfmt < 0 ? storedWfmt_ : static_cast<uint32_t>(opts.wfmt);
    if (wfmt_ > OPURE_W_I4G128) fail(OPURE_E_INVALID, "wfmt " + std::to_string(wfmt_));
    afmt_ = opts.afmt >= 0 ? static_cast<uint32_t>(opts.afmt)
                           : cfg_.activationAfmt >= 0 ? static_cast<uint32_t>(cfg_.activationAfmt) : default_afmt(wfmt_);
    if (afmt_ > OPURE_A_BF16) fail(OPURE_E_INVALID, "afmt " + std::to_string(afmt_));
    attnScale_ = opts.attnScale > 0.0f ? opts.attnScale : static_cast<float>(1.0 / std::sqrt(static_cast<double>(cfg_.headDim)));
    if (opts.ropePairs > OPURE_ROPE_PAIRS_HALF) fail(OPURE_E_INVALID, "rope_pairs " + std::to_string(opts.ropePairs));
    ropePairs_ = opts.ropePairs;
    maxPos_ = opts.maxPositions ? opts.maxPositions : cfg_.maxPositionEmbeddings;
    if (!maxPos_) fail(OPURE_E_INVALID, "no RoPE length: config.json has no max_position_embeddings and none was given");

    // every tensor found and shape-checked now, so a bad file fails before any upload
    auto check = [&](Role r, uint32_t layer) {
        uint32_t out = 0, in = 0;
        for (const Part& p : Parts(r, layer, &out, &in))
            if (p.wfmt != OPURE_W_F32 && p.wfmt != wfmt_)
                fail(OPURE_E_UNSUPPORTED, p.w->name + " is stored quantised in another format than the model computes in");
    };
    check(Role::Embed, 0);
    if (!cfg_.tied) check(Role::LmHead, 0);
    for (uint32_t i = 0; i < cfg_.nLayers; ++i)
        for (Role r : {Role::Qkv, Role::O, Role::GateUp, Role::Down}) check(r, i);
    for (uint32_t i = 0; i < cfg_.nLayers; ++i)
    {
        for (const char* n : {"input_layernorm.weight", "post_attention_layernorm.weight"})
        {
            const Tensor* t = Lookup(layer_prefix(i) + n, nullptr);
            if (!t || !is_float(t->dtype) || !shape_is(*t, {cfg_.hidden}))
                fail(OPURE_E_INVALID, layer_prefix(i) + n + " missing or not a float [" + std::to_string(cfg_.hidden) + "]");
        }
    }
    const Tensor* fn = Lookup("model.norm.weight", nullptr);
    if (!fn || !is_float(fn->dtype) || !shape_is(*fn, {cfg_.hidden}))
        fail(OPURE_E_INVALID, "model.norm.weight missing or not a float [" + std::to_string(cfg_.hidden) + "]");
}

uint32_t ModelFiles::TensorCount() const
{
    uint32_t n = 0;
    for (const auto& f : files_) n += static_cast<uint32_t>(f->Tensors().size());
    return n;
}

const Tensor* ModelFiles::Lookup(const std::string& name, const WeightStreamer** file) const
{
    for (const auto& f : files_)
        if (const Tensor* t = f->TryFind(name))
        {
            if (file) *file = f.get();
            return t;
        }
    return nullptr;
}

ModelFiles::Part ModelFiles::Resolve(const std::string& base, uint32_t out, uint32_t in) const
{
    Part p;
    p.out = out;
    p.w = Lookup(base + ".weight", &p.file);
    if (!p.w) fail(OPURE_E_INVALID, "tensor '" + base + ".weight' not found");
    const Tensor& w = *p.w;
    const std::string want = "[" + std::to_string(out) + ", " + std::to_string(in) + "]";
    auto bad_shape = [&](const std::string& expect) {
        fail(OPURE_E_INVALID, w.name + " is " + DtypeName(w.dtype) + " " + shape_str(w.shape) + ", expected " + expect);
    };
    p.scale = Lookup(base + ".weight_scale", nullptr);
    p.zero = Lookup(base + ".weight_zero", nullptr);
    if (is_float(w.dtype))
    {
        if (!shape_is(w, {out, in})) bad_shape(want);
        p.wfmt = OPURE_W_F32;
        return p;
    }
    if (!p.scale && !w.hasHeaderScale) fail(OPURE_E_INVALID, w.name + " is quantised but has no weight_scale tensor or scale key");
    if (p.scale && !is_float(p.scale->dtype)) fail(OPURE_E_INVALID, p.scale->name + " is not a float tensor");
    if (w.dtype == Dtype::I8)
    {
        if (!shape_is(w, {out, in})) bad_shape(want);
        if (p.scale && !shape_is(*p.scale, {out}) && !shape_is(*p.scale, {out, 1}))
            fail(OPURE_E_INVALID, p.scale->name + " is " + shape_str(p.scale->shape) + ", expected [" + std::to_string(out) + "]");
        if (p.zero) fail(OPURE_E_UNSUPPORTED, p.zero->name + ": int8 per-channel weights are symmetric");
        p.wfmt = OPURE_W_I8PC;
        return p;
    }
    if (w.dtype == Dtype::U8 || w.dtype == Dtype::U4 || w.dtype == Dtype::I4)
    {
        if (w.dtype == Dtype::U8 ? !shape_is(w, {out, in / 2}) || in % 2 : !shape_is(w, {out, in}))
            bad_shape(w.dtype == Dtype::U8 ? "[" + std::to_string(out) + ", " + std::to_string(in / 2) + "] packed" : want);
        if (in % 128) fail(OPURE_E_UNSUPPORTED, w.name + ": int4 groups of 128 need in % 128 == 0");
        const uint32_t groups = in / 128;
        if (p.scale && !shape_is(*p.scale, {out, groups}))
            fail(OPURE_E_INVALID, p.scale->name + " is " + shape_str(p.scale->shape) + ", expected [" + std::to_string(out) + ", " +
                                      std::to_string(groups) + "]");
        if (p.zero)
        {
            if (w.dtype == Dtype::I4) fail(OPURE_E_UNSUPPORTED, p.zero->name + ": signed int4 takes no zero points");
            if (!is_float(p.zero->dtype) || !shape_is(*p.zero, {out, groups}))
                fail(OPURE_E_INVALID, p.zero->name + " is not a float [" + std::to_string(out) + ", " + std::to_string(groups) + "]");
        }
        p.wfmt = OPURE_W_I4G128;
        return p;
    }
    fail(OPURE_E_UNSUPPORTED, w.name + " has dtype " + DtypeName(w.dtype) + ", which no weight format takes");
}

std::vector<ModelFiles::Part> ModelFiles::Parts(Role role, uint32_t layer, uint32_t* out, uint32_t* in) const
{
    const ModelConfig& c = cfg_;
    if (layer >= c.nLayers && (role == Role::Qkv || role == Role::O || role == Role::GateUp || role == Role::Down))
        fail(OPURE_E_INVALID, "layer " + std::to_string(layer) + " past num_hidden_layers");
    const std::string pre = layer_prefix(layer);
    std::vector<std::pair<std::string, uint32_t>> names;
    switch (role)
    {
    case Role::Embed: *in = c.hidden; names = {{"model.embed_tokens", c.vocab}}; break;
    case Role::LmHead:
        *in = c.hidden;
        names = {{c.tied ? "model.embed_tokens" : "lm_head", c.vocab}};
        break;
    case Role::Qkv:
        *in = c.hidden;
        names = {{pre + "self_attn.q_proj", c.nHeads * c.headDim},
                 {pre + "self_attn.k_proj", c.nKvHeads * c.headDim},
                 {pre + "self_attn.v_proj", c.nKvHeads * c.headDim}};
        break;
    case Role::O: *in = c.nHeads * c.headDim; names = {{pre + "self_attn.o_proj", c.hidden}}; break;
    case Role::GateUp: *in = c.hidden; names = {{pre + "mlp.gate_proj", c.ffn}, {pre + "mlp.up_proj", c.ffn}}; break;
    case Role::Down: *in = c.ffn; names = {{pre + "mlp.down_proj", c.hidden}}; break;
    default: fail(OPURE_E_INVALID, std::string("role ") + role_name(role) + " is not a linear");
    }
    std::vector<Part> parts;
    *out = 0;
    for (const auto& [name, rows] : names)
    {
        parts.push_back(Resolve(name, rows, *in));
        if (parts.back().wfmt != parts[0].wfmt) fail(OPURE_E_UNSUPPORTED, name + ".weight is stored in another format than the first part of its fused linear");
        *out += rows;
    }
    return parts;
}

void ModelFiles::ReadPart(const Part& p, uint32_t in, HostLinear& h, uint32_t row0) const
{
    const Tensor& w = *p.w;
    const auto* src = static_cast<const uint8_t*>(p.file->Data(w));
    const uint64_t n = static_cast<uint64_t>(p.out) * in;
    const uint32_t wfmt = p.wfmt;
    if (wfmt == OPURE_W_F32)
    {
        float* dst = reinterpret_cast<float*>(h.w.data()) + static_cast<uint64_t>(row0) * in;
        if (w.dtype == Dtype::F32) std::memcpy(dst, src, n * 4);
        else
            for (uint64_t i = 0; i < n; ++i) dst[i] = load_float(w.dtype, src, i);
        return;
    }
    const WeightStreamer* sf = nullptr;
    const uint8_t* sc = nullptr;
    if (p.scale)
    {
        (void)Lookup(p.scale->name, &sf);
        sc = static_cast<const uint8_t*>(sf->Data(*p.scale));
    }
    if (wfmt == OPURE_W_I8PC)
    {
        std::memcpy(h.w.data() + static_cast<uint64_t>(row0) * in, src, n);
        auto* s = reinterpret_cast<uint16_t*>(h.scale.data()) + row0;
        for (uint32_t o = 0; o < p.out; ++o)
        {
            if (!p.scale) s[o] = narrow_scale(w.headerScale, false, w.name);
            else if (p.scale->dtype == Dtype::F16) std::memcpy(&s[o], sc + 2 * o, 2);
            else s[o] = narrow_scale(load_float(p.scale->dtype, sc, o), false, p.scale->name);
        }
        return;
    }
    // int4 g128: packed bytes, element 2i in the high nibble
    uint8_t* dst = h.w.data() + static_cast<uint64_t>(row0) * (in / 2);
    std::memcpy(dst, src, n / 2);
    if (w.dtype == Dtype::I4)
        for (uint64_t i = 0; i < n / 2; ++i) dst[i] ^= 0x88u;   // signed nibble v -> v + 8
    const uint32_t groups = in / 128;
    auto* s = reinterpret_cast<uint16_t*>(h.scale.data()) + static_cast<uint64_t>(row0) * groups;
    auto* z = reinterpret_cast<uint16_t*>(h.zero.data()) + static_cast<uint64_t>(row0) * groups;
    const uint8_t* zs = nullptr;
    if (p.zero)
    {
        const WeightStreamer* zf = nullptr;
        (void)Lookup(p.zero->name, &zf);
        zs = static_cast<const uint8_t*>(zf->Data(*p.zero));
    }
    const uint16_t zero_const = w.dtype == Dtype::I4 ? f32_to_bf16(8.0f) : 0u;
    for (uint64_t i = 0; i < static_cast<uint64_t>(p.out) * groups; ++i)
    {
        if (!p.scale) s[i] = narrow_scale(w.headerScale, true, w.name);
        else if (p.scale->dtype == Dtype::BF16) std::memcpy(&s[i], sc + 2 * i, 2);
        else s[i] = narrow_scale(load_float(p.scale->dtype, sc, i), true, p.scale->name);
        if (!zs) z[i] = zero_const;
        else if (p.zero->dtype == Dtype::BF16) std::memcpy(&z[i], zs + 2 * i, 2);
        else z[i] = f32_to_bf16(load_float(p.zero->dtype, zs, i));
    }
}

void ModelFiles::ReadNorm(const std::string& name, HostLinear& h) const
{
    const WeightStreamer* f = nullptr;
    const Tensor* t = Lookup(name, &f);
    if (!t) fail(OPURE_E_INVALID, "tensor '" + name + "' not found");
    h.wfmt = OPURE_W_F32;
    h.out = cfg_.hidden;
    h.in = 1;
    h.w.resize(4ull * cfg_.hidden);
    const auto* src = static_cast<const uint8_t*>(f->Data(*t));
    auto* dst = reinterpret_cast<float*>(h.w.data());
    for (uint32_t i = 0; i < cfg_.hidden; ++i) dst[i] = load_float(t->dtype, src, i);
}

HostLinear ModelFiles::Read(Role role, uint32_t layer) const
{
    HostLinear h;
    if (role == Role::AttnNorm || role == Role::MlpNorm)
    {
        if (layer >= cfg_.nLayers) fail(OPURE_E_INVALID, "layer " + std::to_string(layer) + " past num_hidden_layers");
        ReadNorm(layer_prefix(layer) + (role == Role::AttnNorm ? "input_layernorm.weight" : "post_attention_layernorm.weight"), h);
        return h;
    }
    if (role == Role::FinalNorm)
    {
        ReadNorm("model.norm.weight", h);
        return h;
    }
    const std::vector<Part> parts = Parts(role, layer, &h.out, &h.in);
    const uint32_t wfmt = parts[0].wfmt;
    h.wfmt = wfmt;
    const uint64_t n = static_cast<uint64_t>(h.out) * h.in;
    if (wfmt == OPURE_W_F32) h.w.resize(4 * n);
    else if (wfmt == OPURE_W_I8PC)
    {
        h.w.resize(n);
        h.scale.resize(2ull * h.out);
    }
    else
    {
        h.w.resize(n / 2);
        h.scale.resize(2ull * h.out * (h.in / 128));
        h.zero.resize(h.scale.size());
    }
    uint32_t row = 0;
    for (const Part& p : parts)
    {
        ReadPart(p, h.in, h, row);
        row += p.out;
    }
    if (role == Role::Qkv && ropePairs_ == OPURE_ROPE_PAIRS_HALF)
    {
        permute_half_to_adjacent(h, 0, cfg_.nHeads, cfg_.headDim);                          // q
        permute_half_to_adjacent(h, cfg_.nHeads * cfg_.headDim, cfg_.nKvHeads, cfg_.headDim);  // k
    }
    return h;
}

// ---------------------------------------------------------------------------
//  LoadedModel
// ---------------------------------------------------------------------------
void* LoadedModel::Alloc(uint64_t bytes)
{
    void* p = nullptr;
    Check(opure_buf_alloc(dev_, bytes, &p), "model loader: weight buffer");
    bufs_.push_back(p);
    deviceBytes_ += bytes;
    return p;
}

namespace {

// device buffers freed when the scope ends (upload staging)
struct Staging {
    opure_dev* dev;
    std::vector<void*> bufs;
    void* alloc(uint64_t bytes)
    {
        void* p = nullptr;
        Check(opure_buf_alloc(dev, bytes, &p), "model loader: staging buffer");
        bufs.push_back(p);
        return p;
    }
    void* upload(const std::vector<uint8_t>& v)
    {
        void* p = alloc(v.size());
        Check(opure_buf_upload(dev, p, 0, v.data(), v.size()), "model loader: upload");
        return p;
    }
    ~Staging()
    {
        for (void* p : bufs) (void)opure_buf_free(dev, p);
    }
};

}  // namespace

opure_linear LoadedModel::Linear(const ModelFiles& files, Role role, uint32_t layer, uint32_t layout)
{
    const HostLinear h = files.Read(role, layer);
    const uint32_t wfmt = files.Wfmt();
    Staging st{dev_, {}};
    opure_linear src{};
    src.out = h.out;
    src.in = h.in;
    src.layout = OPURE_LAYOUT_ROWMAJOR;
    if (h.wfmt == wfmt)
    {
        src.w = st.upload(h.w);
        if (!h.scale.empty()) src.scale = st.upload(h.scale);
        if (!h.zero.empty()) src.zero = st.upload(h.zero);
    }
    else
    {
        // a float tensor of a quantised model: quantised on the device
        if (h.wfmt != OPURE_W_F32) fail(OPURE_E_UNSUPPORTED, std::string(role_name(role)) + " is stored in another quantised format");
        const float* f = static_cast<const float*>(st.upload(h.w));
        const uint64_t n = static_cast<uint64_t>(h.out) * h.in;
        if (wfmt == OPURE_W_I8PC)
        {
            auto* q = static_cast<int8_t*>(st.alloc(n));
            auto* s = static_cast<uint16_t*>(st.alloc(2ull * h.out));
            Check(opure_quantize_i8pc(dev_, f, h.out, h.in, q, s), "model loader: int8 quantiser");
            src.w = q;
            src.scale = s;
        }
        else
        {
            if (h.in % 128) fail(OPURE_E_UNSUPPORTED, std::string(role_name(role)) + ": int4 groups of 128 need in % 128 == 0");
            auto* q = static_cast<uint8_t*>(st.alloc(n / 2));
            auto* s = static_cast<uint16_t*>(st.alloc(2ull * h.out * (h.in / 128)));
            auto* z = static_cast<uint16_t*>(st.alloc(2ull * h.out * (h.in / 128)));
            Check(opure_quantize_i4g128(dev_, f, h.out, h.in, q, s, z), "model loader: int4 quantiser");
            src.w = q;
            src.scale = s;
            src.zero = z;
        }
    }
    uint64_t wb = 0, sb = 0;
    Check(opure_tiled_bytes(wfmt, h.out, h.in, &wb, &sb), role_name(role));
    void* tw = Alloc(wb);
    void* ts = sb ? Alloc(sb) : nullptr;
    opure_linear dst{};
    Check(opure_tile_linear(dev_, wfmt, layout, &src, tw, ts, &dst), role_name(role));
    Check(opure_stream_sync(dev_), "model loader: tiling");
    return dst;   // staging freed here, after the sync
}

const float* LoadedModel::Norm(const ModelFiles& files, Role role, uint32_t layer)
{
    const HostLinear h = files.Read(role, layer);
    void* p = Alloc(h.w.size());
    Check(opure_buf_upload(dev_, p, 0, h.w.data(), h.w.size()), "model loader: norm upload");
    return static_cast<const float*>(p);
}

LoadedModel::LoadedModel(opure_dev* dev, const ModelFiles& files) : dev_(dev)
{
    if (!dev) fail(OPURE_E_INVALID, "null device");
    const ModelConfig& c = files.Config();
    try
    {
        desc_.n_layers = c.nLayers;
        desc_.hidden = c.hidden;
        desc_.n_heads = c.nHeads;
        desc_.n_kv_heads = c.nKvHeads;
        desc_.head_dim = c.headDim;
        desc_.ffn = c.ffn;
        desc_.vocab = c.vocab;
        desc_.rms_eps = c.rmsEps;
        desc_.attn_scale = files.AttnScale();
        desc_.wfmt = files.Wfmt();
        desc_.afmt = files.Afmt();
        desc_.embed = Linear(files, Role::Embed, 0, OPURE_LAYOUT_TILED);
        desc_.lm_head = c.tied ? desc_.embed : Linear(files, Role::LmHead, 0, OPURE_LAYOUT_TILED);
        desc_.final_norm = Norm(files, Role::FinalNorm, 0);
        layers_.resize(c.nLayers);
        for (uint32_t i = 0; i < c.nLayers; ++i)
        {
            opure_layer_weights& L = layers_[i];
            L.attn_norm = Norm(files, Role::AttnNorm, i);
            L.mlp_norm = Norm(files, Role::MlpNorm, i);
            L.qkv = Linear(files, Role::Qkv, i, OPURE_LAYOUT_TILED);
            L.o = Linear(files, Role::O, i, OPURE_LAYOUT_TILED);
            L.gate_up = Linear(files, Role::GateUp, i, OPURE_LAYOUT_TILED_SWIGLU);
            L.down = Linear(files, Role::Down, i, OPURE_LAYOUT_TILED);
        }
        desc_.layers = layers_.data();
        // RoPE pairs (2p, 2p+1) at theta^(-2p/head_dim), the GPU reference's schedule
        const uint32_t mp = files.MaxPositions(), half = c.headDim / 2;
        std::vector<float> cs(static_cast<size_t>(mp) * half), sn(cs.size());
        Check(opure_rope_table(c.ropeTheta, c.headDim, mp, OPURE_ROPE_GPU, cs.data(), sn.data()), "model loader: RoPE table");
        void* pc = Alloc(cs.size() * 4);
        void* ps = Alloc(sn.size() * 4);
        Check(opure_buf_upload(dev_, pc, 0, cs.data(), cs.size() * 4), "model loader: RoPE upload");
        Check(opure_buf_upload(dev_, ps, 0, sn.data(), sn.size() * 4), "model loader: RoPE upload");
        desc_.rope_cos = static_cast<const float*>(pc);
        desc_.rope_sin = static_cast<const float*>(ps);
        desc_.rope_max_pos = mp;
    }
    catch (...)
    {
        for (void* p : bufs_) (void)opure_buf_free(dev_, p);
        bufs_.clear();
        throw;
    }
}

LoadedModel::~LoadedModel()
{
    for (void* p : bufs_) (void)opure_buf_free(dev_, p);
}

}  // namespace opure::engine
