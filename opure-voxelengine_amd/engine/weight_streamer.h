// ============================================================================
//  weight_streamer.h -- a zero-copy .safetensors reader and the config.json
//  reader the model loader needs.
//
//  Counterpart of the reference's WeightStreamer (src/core/Opure_Streamer.h),
//  on POSIX mmap instead of CreateFileMappingW / MapViewOfFile.  The file is
//
//      u64  header_len (little endian)
//      u8[header_len]  JSON {"__metadata__": {...}, name: {"dtype", "shape", "data_offsets": [a, b]}}
//      payload; data_offsets are relative to its first byte
//
//  and every tensor's declared byte span is checked against its shape and
//  dtype.  Differences from the reference, each a fix:
//    - packed 4-bit dtypes (U4 / I4) take half a byte per element (the
//      reference's ElementBytes(I4) = 1, Opure_Streamer.cpp:104-117, made every
//      int4 tensor fail its size check or be read at the wrong offsets);
//    - a quantised tensor's scales are tensors of their own (standard
//      safetensors); the reference's non-standard per-tensor "scale" key
//      (Opure_Streamer.cpp:275-282) is still read, into the Tensor itself,
//      so nothing points at a temporary (the reference uploads every scale
//      from the address of one loop variable, Opure_Graph.cpp:521-527).
// ============================================================================
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

namespace opure::engine {

// ---- a small JSON value: enough for safetensors headers and config.json ----
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;   // in file order

    [[nodiscard]] const Json* Find(std::string_view key) const;
    // parses a whole document; throws Error(OPURE_E_INVALID) with the offset on a syntax error
    static Json Parse(std::string_view text);
};

enum class Dtype : uint8_t { F32, F16, BF16, U8, I8, U4, I4 };

[[nodiscard]] const char* DtypeName(Dtype d);
// stored bytes of n elements (packed 4-bit: two a byte)
[[nodiscard]] uint64_t StoredBytes(Dtype d, uint64_t n);

struct Tensor {
    std::string name;
    Dtype dtype = Dtype::F32;
    std::vector<int64_t> shape;     // row-major, as stored
    uint64_t byteBegin = 0;         // absolute offsets into the mapping
    uint64_t byteEnd = 0;
    // the reference's per-tensor "scale" key (w = q * scale), when the entry
    // has one; files in the standard form carry scales as tensors instead
    bool hasHeaderScale = false;
    double headerScale = 1.0;

    [[nodiscard]] uint64_t ElementCount() const;
    [[nodiscard]] uint64_t ByteCount() const { return byteEnd - byteBegin; }
};

class WeightStreamer {
public:
    WeightStreamer() = default;
    ~WeightStreamer() { Close(); }
    WeightStreamer(const WeightStreamer&) = delete;
    WeightStreamer& operator=(const WeightStreamer&) = delete;

    // Maps the file read-only and parses its header; throws Error on any problem.
    void Open(const std::string& path);
    void Close();

    [[nodiscard]] bool IsOpen() const { return base_ != nullptr; }
    [[nodiscard]] const std::vector<Tensor>& Tensors() const { return tensors_; }
    // exact-name lookup: Find throws when absent, TryFind returns null
    [[nodiscard]] const Tensor& Find(std::string_view name) const;
    [[nodiscard]] const Tensor* TryFind(std::string_view name) const;
    // the tensor's bytes, straight out of the mapping
    [[nodiscard]] const void* Data(const Tensor& t) const { return base_ + t.byteBegin; }

private:
    void ParseHeader(const uint8_t* header, uint64_t len);

    uint8_t* base_ = nullptr;
    uint64_t size_ = 0;
    std::vector<Tensor> tensors_;
    std::map<std::string, size_t, std::less<>> index_;
};

// The file's contents as a string (config.json); throws Error when unreadable.
std::string ReadTextFile(const std::string& path);

}  // namespace opure::engine
