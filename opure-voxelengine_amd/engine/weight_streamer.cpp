// ============================================================================
//  weight_streamer.cpp -- WeightStreamer (mmap + header parse) and Json.
// ============================================================================
#include "weight_streamer.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>
#include <fstream>
#include <sstream>

#include "opure_hip.h"
#include "voxel_engine.h"

namespace opure::engine {

// ---------------------------------------------------------------------------
//  Json: a recursive-descent reader (objects, arrays, strings with the common
//  escapes, numbers, true / false / null)
// ---------------------------------------------------------------------------
namespace {

struct Reader {
    std::string_view s;
    size_t i = 0;
    int depth = 0;                       // open objects and arrays
    static constexpr int kMaxDepth = 64;  // deeper headers are refused, not recursed into

    [[noreturn]] void fail(const char* what) const
    {
        throw Error(OPURE_E_INVALID, std::string("json: ") + what + " at offset " + std::to_string(i));
    }
    void ws()
    {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
    }
    bool eat(char c)
    {
        ws();
        if (i < s.size() && s[i] == c)
        {
            ++i;
            return true;
        }
        return false;
    }
    std::string string()
    {
        if (!eat('"')) fail("expected a string");
        std::string out;
        while (i < s.size() && s[i] != '"')
        {
            char c = s[i++];
            if (c == '\\')
            {
                if (i >= s.size()) fail("truncated escape");
                const char e = s[i++];
                switch (e)
                {
                case '"': case '\\': case '/': out.push_back(e); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u':
                {
                    if (i + 4 > s.size()) fail("truncated \\u escape");
                    const unsigned cp = static_cast<unsigned>(std::stoul(std::string(s.substr(i, 4)), nullptr, 16));
                    i += 4;
                    // UTF-8 of a basic-plane code point (surrogate pairs are not used in these files)
                    if (cp < 0x80) out.push_back(static_cast<char>(cp));
                    else if (cp < 0x800)
                    {
                        out.push_back(static_cast<char>(0xC0 | (cp >> 6)));
                        out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
                    }
                    else
                    {
                        out.push_back(static_cast<char>(0xE0 | (cp >> 12)));
                        out.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
                        out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
                    }
                    break;
                }
                default: fail("bad escape");
                }
            }
            else
            {
                out.push_back(c);
            }
        }
        if (i >= s.size()) fail("unterminated string");
        ++i;
        return out;
    }
    Json value()
    {
        ws();
        if (i >= s.size()) fail("unexpected end");
        Json v;
        const char c = s[i];
        if ((c == '{' || c == '[') && ++depth > kMaxDepth) fail("nesting deeper than 64 levels");
        if (c == '{')
        {
            ++i;
            v.kind = Json::Object;
            if (eat('}'))
            {
                --depth;
                return v;
            }
            do
            {
                std::string k = string();
                if (!eat(':')) fail("expected ':'");
                v.obj.emplace_back(std::move(k), value());
            } while (eat(','));
            if (!eat('}')) fail("expected '}'");
            --depth;
        }
        else if (c == '[')
        {
            ++i;
            v.kind = Json::Array;
            if (eat(']'))
            {
                --depth;
                return v;
            }
            do
            {
                v.arr.push_back(value());
            } while (eat(','));
            if (!eat(']')) fail("expected ']'");
            --depth;
        }
        else if (c == '"')
        {
            v.kind = Json::String;
            v.str = string();
        }
        else if (s.compare(i, 4, "true") == 0)
        {
            v.kind = Json::Bool;
            v.b = true;
            i += 4;
        }
        else if (s.compare(i, 5, "false") == 0)
        {
            v.kind = Json::Bool;
            i += 5;
        }
        else if (s.compare(i, 4, "null") == 0)
        {
            i += 4;
        }
        else
        {
            const size_t b = i;
            while (i < s.size() && (std::strchr("+-0123456789.eE", s[i]) != nullptr)) ++i;
            if (b == i) fail("unexpected character");
            v.kind = Json::Number;
            const std::string t(s.substr(b, i - b));
            char* end = nullptr;
            v.num = std::strtod(t.c_str(), &end);
            if (!end || *end) fail("bad number");
        }
        return v;
    }
};

}  // namespace

const Json* Json::Find(std::string_view key) const
{
    if (kind != Object) return nullptr;
    for (const auto& [k, v] : obj)
        if (k == key) return &v;
    return nullptr;
}

Json Json::Parse(std::string_view text)
{
    Reader r{text, 0};
    Json v = r.value();
    r.ws();
    if (r.i != text.size()) r.fail("trailing characters");
    return v;
}

// ---------------------------------------------------------------------------
//  dtypes
// ---------------------------------------------------------------------------
const char* DtypeName(Dtype d)
{
    switch (d)
    {
    case Dtype::F32: return "F32";
    case Dtype::F16: return "F16";
    case Dtype::BF16: return "BF16";
    case Dtype::U8: return "U8";
    case Dtype::I8: return "I8";
    case Dtype::U4: return "U4";
    case Dtype::I4: return "I4";
    }
    return "?";
}

uint64_t StoredBytes(Dtype d, uint64_t n)
{
    uint64_t per = 1;
    switch (d)
    {
    case Dtype::F32: per = 4; break;
    case Dtype::F16:
    case Dtype::BF16: per = 2; break;
    case Dtype::U8:
    case Dtype::I8: return n;
    case Dtype::U4:
    case Dtype::I4: return n / 2u + (n & 1u);
    }
    uint64_t b = 0;
    if (__builtin_mul_overflow(n, per, &b)) throw Error(OPURE_E_INVALID, "safetensors: tensor size overflows 64 bits");
    return b;
}

namespace {

Dtype parse_dtype(const std::string& s, const std::string& tensor)
{
    if (s == "F32") return Dtype::F32;
    if (s == "F16") return Dtype::F16;
    if (s == "BF16") return Dtype::BF16;
    if (s == "U8") return Dtype::U8;
    if (s == "I8") return Dtype::I8;
    if (s == "U4") return Dtype::U4;
    if (s == "I4") return Dtype::I4;
    throw Error(OPURE_E_UNSUPPORTED, "safetensors: tensor '" + tensor + "' has dtype " + s + ", not read here");
}

}  // namespace

uint64_t Tensor::ElementCount() const
{
    uint64_t n = 1;
    for (int64_t d : shape)
        if (__builtin_mul_overflow(n, static_cast<uint64_t>(d), &n))
            throw Error(OPURE_E_INVALID, "safetensors: element count of '" + name + "' overflows 64 bits");
    return n;
}

// ---------------------------------------------------------------------------
//  WeightStreamer
// ---------------------------------------------------------------------------
void WeightStreamer::Open(const std::string& path)
{
    Close();
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw Error(OPURE_E_INVALID, "safetensors: cannot open " + path + ": " + std::strerror(errno));
    struct stat st {};
    if (::fstat(fd, &st) != 0 || st.st_size < 8)
    {
        ::close(fd);
        throw Error(OPURE_E_INVALID, "safetensors: " + path + " is shorter than its 8-byte header length");
    }
    void* p = ::mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) throw Error(OPURE_E_INVALID, "safetensors: cannot map " + path + ": " + std::strerror(errno));
    base_ = static_cast<uint8_t*>(p);
    size_ = static_cast<uint64_t>(st.st_size);
    try
    {
        uint64_t len = 0;
        std::memcpy(&len, base_, 8);    // little endian, as the format states (and this host is)
        if (len > size_ - 8) throw Error(OPURE_E_INVALID, "safetensors: header length runs past the end of " + path);
        ParseHeader(base_ + 8, len);
    }
    catch (...)
    {
        Close();
        throw;
    }
}

void WeightStreamer::Close()
{
    if (base_) ::munmap(base_, static_cast<size_t>(size_));
    base_ = nullptr;
    size_ = 0;
    tensors_.clear();
    index_.clear();
}

void WeightStreamer::ParseHeader(const uint8_t* header, uint64_t len)
{
    const Json root = Json::Parse(std::string_view(reinterpret_cast<const char*>(header), len));
    if (root.kind != Json::Object) throw Error(OPURE_E_INVALID, "safetensors: the header is not a JSON object");
    const uint64_t payload = 8u + len, payloadBytes = size_ - payload;
    for (const auto& [name, v] : root.obj)
    {
        if (name == "__metadata__") continue;
        const Json* dt = v.Find("dtype");
        const Json* sh = v.Find("shape");
        const Json* off = v.Find("data_offsets");
        if (!dt || dt->kind != Json::String || !sh || sh->kind != Json::Array || !off || off->kind != Json::Array ||
            off->arr.size() != 2)
            throw Error(OPURE_E_INVALID, "safetensors: tensor '" + name + "' lacks dtype, shape or two data_offsets");
        Tensor t;
        t.name = name;
        t.dtype = parse_dtype(dt->str, name);
        // dimensions and offsets are integers below 2^53 (exact in the double a JSON number is read into)
        constexpr double kMaxInt = 9007199254740992.0;
        auto integral = [&](const Json& d) { return d.kind == Json::Number && d.num >= 0 && d.num < kMaxInt && d.num == std::floor(d.num); };
        for (const Json& d : sh->arr)
        {
            if (!integral(d)) throw Error(OPURE_E_INVALID, "safetensors: bad shape of '" + name + "'");
            t.shape.push_back(static_cast<int64_t>(d.num));
        }
        const double b = off->arr[0].num, e = off->arr[1].num;
        if (!integral(off->arr[0]) || !integral(off->arr[1]) || e < b || e > static_cast<double>(payloadBytes))
            throw Error(OPURE_E_INVALID, "safetensors: data_offsets of '" + name + "' out of order or past the payload");
        const uint64_t expect = StoredBytes(t.dtype, t.ElementCount());
        if (static_cast<uint64_t>(e - b) != expect)
            throw Error(OPURE_E_INVALID, "safetensors: '" + name + "' declares " + std::to_string(static_cast<uint64_t>(e - b)) +
                                             " bytes, its shape and " + DtypeName(t.dtype) + " imply " +
                                             std::to_string(expect));
        if (const Json* sc = v.Find("scale"))
        {
            if (sc->kind != Json::Number) throw Error(OPURE_E_INVALID, "safetensors: 'scale' of '" + name + "' is not a number");
            t.hasHeaderScale = true;
            t.headerScale = sc->num;
        }
        t.byteBegin = payload + static_cast<uint64_t>(b);
        t.byteEnd = payload + static_cast<uint64_t>(e);
        index_.emplace(t.name, tensors_.size());
        tensors_.push_back(std::move(t));
    }
    if (tensors_.empty()) throw Error(OPURE_E_INVALID, "safetensors: the header declares no tensors");
}

const Tensor* WeightStreamer::TryFind(std::string_view name) const
{
    const auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

const Tensor& WeightStreamer::Find(std::string_view name) const
{
    const Tensor* t = TryFind(name);
    if (!t) throw Error(OPURE_E_INVALID, "safetensors: tensor '" + std::string(name) + "' not found");
    return *t;
}

std::string ReadTextFile(const std::string& path)
{
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error(OPURE_E_INVALID, "cannot read " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

}  // namespace opure::engine
