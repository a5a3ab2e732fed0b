// ============================================================================
//  model_loader.h -- a model directory (config.json + safetensors) onto the
//  device in the tiled layout the verify step reads.
//
//  Counterpart of the reference's Graph::LoadConfigOnly / UploadWeights and
//  ModelSpec::Resolve (src/engine/Opure_Graph.cpp:267-300, :430-530,
//  src/engine/Opure_ModelSpec.cpp:120-320): parse config.json, map the
//  weights, find every tensor of the Llama layout, check its shape, upload.
//  Here the upload is per linear: q/k/v and gate/up are fused into one
//  row-major interchange linear on the host, copied to the device and
//  rewritten into the tiled layout by opure_tile_linear; a float tensor in a
//  model loaded as int8 / int4 is quantised on the device first, by the
//  same quantisers as the synthetic models.
//
//  Stored forms read (tensor X = e.g. model.layers.0.self_attn.q_proj):
//    float     X.weight F32 / F16 / BF16 [out][in]
//    int8 pc   X.weight I8 [out][in] + X.weight_scale F16 (F32, BF16) [out] or [out][1]
//    int4 g128 X.weight U8 [out][in/2] or U4 [out][in] (element 2i in the high
//              nibble) + X.weight_scale BF16 [out][in/128] + X.weight_zero
//              BF16 [out][in/128] (absent: 0); w = scale * (q - zero);
//              I4 [out][in] (signed nibbles) is read as U4 with zero 8
//    the reference's files: I8 / U4 / I4 with a per-tensor "scale" key in the
//              header entry, w = q * scale (Opure_Streamer.cpp:403-426), read
//              as the per-channel / per-group forms with that scale everywhere
//              (rounded to the fp16 / bf16 the kernels read)
//  Norm gains are F32 / F16 / BF16 [hidden], widened to fp32.
// ============================================================================
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "opure_engine.h"
#include "opure_hip.h"
#include "weight_streamer.h"

namespace opure::engine {

struct LoadOptions {
    uint32_t maxPositions = 0;   // RoPE table rows; 0: config.json's max_position_embeddings
    int32_t  wfmt = -1;          // OPURE_W_* to compute in; -1: the format the linears are stored in
    int32_t  afmt = -1;          // OPURE_A_*; -1: quantization_config.activation_dtype, else the format's default
    float    attnScale = 0.0f;   // 0: 1/sqrt(head_dim) (HF Llama); 1: the reference's unscaled scores
    uint32_t ropePairs = OPURE_ROPE_PAIRS_ADJACENT;   // HALF: q/k rows of each head permuted at load
};

// config.json (the fields the reference's ModelConfig::Parse reads,
// Opure_Graph.cpp:73-138, plus head_dim and quantization_config)
struct ModelConfig {
    uint32_t nLayers = 0, hidden = 0, nHeads = 0, nKvHeads = 0, headDim = 0, ffn = 0, vocab = 0;
    uint32_t maxPositionEmbeddings = 0;
    float    rmsEps = 1e-5f;
    double   ropeTheta = 10000.0;
    bool     tied = true;
    int32_t  activationAfmt = -1;   // quantization_config.activation_dtype, -1 when absent

    static ModelConfig Parse(const std::string& text);
};

// Roles of the tensors the loader reads (the C-ABI's OPURE_ROLE_*)
enum class Role : uint32_t { Embed = 0, LmHead, Qkv, O, GateUp, Down, AttnNorm, MlpNorm, FinalNorm };

// One linear (or norm: out = hidden, in = 1, fp32) in the row-major
// interchange form of opure_hip.h, on the host.
struct HostLinear {
    uint32_t wfmt = OPURE_W_F32;    // as stored; float tensors are fp32 here
    uint32_t out = 0, in = 0;
    std::vector<uint8_t> w, scale, zero;
};

// config.json and the mapped weights of one model directory: the host half
// of loading, no device calls.
class ModelFiles {
public:
    // Reads config.json, maps model.safetensors (or every shard named by
    // model.safetensors.index.json), finds every tensor and checks its shape
    // and dtype; throws Error naming the first problem.
    ModelFiles(const std::string& dir, const LoadOptions& opts);

    [[nodiscard]] const ModelConfig& Config() const { return cfg_; }
    [[nodiscard]] uint32_t StoredWfmt() const { return storedWfmt_; }
    [[nodiscard]] uint32_t Wfmt() const { return wfmt_; }
    [[nodiscard]] uint32_t Afmt() const { return afmt_; }
    [[nodiscard]] float AttnScale() const { return attnScale_; }
    [[nodiscard]] uint32_t MaxPositions() const { return maxPos_; }
    [[nodiscard]] uint32_t RopePairs() const { return ropePairs_; }
    [[nodiscard]] uint32_t TensorCount() const;
    [[nodiscard]] uint64_t FileBytes() const { return fileBytes_; }

    // The interchange form of one role (layer ignored for Embed, LmHead and
    // FinalNorm; LmHead of a tied model is the embedding).
    [[nodiscard]] HostLinear Read(Role role, uint32_t layer) const;

private:
    struct Part {                   // one stored tensor of a (fused) linear
        const WeightStreamer* file = nullptr;
        const Tensor* w = nullptr;
        const Tensor* scale = nullptr;
        const Tensor* zero = nullptr;
        uint32_t out = 0;
        uint32_t wfmt = OPURE_W_F32;   // the form it is stored in
    };
    [[nodiscard]] const Tensor* Lookup(const std::string& name, const WeightStreamer** file) const;
    [[nodiscard]] Part Resolve(const std::string& base, uint32_t out, uint32_t in) const;
    [[nodiscard]] std::vector<Part> Parts(Role role, uint32_t layer, uint32_t* out, uint32_t* in) const;
    void ReadPart(const Part& p, uint32_t in, HostLinear& dst, uint32_t row0) const;
    void ReadNorm(const std::string& name, HostLinear& dst) const;

    std::string dir_;
    ModelConfig cfg_;
    std::vector<std::unique_ptr<WeightStreamer>> files_;
    uint64_t fileBytes_ = 0;
    uint32_t storedWfmt_ = OPURE_W_F32, wfmt_ = OPURE_W_F32, afmt_ = OPURE_A_F32;
    float attnScale_ = 1.0f;
    uint32_t maxPos_ = 0;
    uint32_t ropePairs_ = OPURE_ROPE_PAIRS_ADJACENT;
};

// A model on the device: tiled linears, fp32 norms, the RoPE table and the
// opure_model that describes them.  Owns every buffer.
class LoadedModel {
public:
    LoadedModel(opure_dev* dev, const ModelFiles& files);
    ~LoadedModel();
    LoadedModel(const LoadedModel&) = delete;
    LoadedModel& operator=(const LoadedModel&) = delete;

    [[nodiscard]] const opure_model& Desc() const { return desc_; }
    [[nodiscard]] uint64_t DeviceBytes() const { return deviceBytes_; }

private:
    void* Alloc(uint64_t bytes);
    opure_linear Linear(const ModelFiles& files, Role role, uint32_t layer, uint32_t layout);
    const float* Norm(const ModelFiles& files, Role role, uint32_t layer);

    opure_dev* dev_ = nullptr;
    std::vector<void*> bufs_;
    std::vector<opure_layer_weights> layers_;
    opure_model desc_{};
    uint64_t deviceBytes_ = 0;
};

}  // namespace opure::engine
