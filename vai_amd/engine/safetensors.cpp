// safetensors.cpp -- memory-mapped .safetensors reader and checkpoint folder.
#include "safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <filesystem>
#include <stdexcept>

namespace vai {

namespace {

struct Meta {
    std::string dtype;
    std::vector<uint32_t> shape;
    size_t begin = 0, end = 0;   // byte offsets into the data section
};

// The JSON subset a safetensors header uses: objects, arrays, strings,
// integers, and (inside __metadata__ only) anything else, which is skipped.
class HeaderReader
{
    const char* p_;
    const char* end_;

    [[noreturn]] void fail(const std::string& what) const
    {
        throw std::runtime_error("Invalid Safetensors header: " + what);
    }
    void ws()
    {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool peek(char c)
    {
        ws();
        return p_ < end_ && *p_ == c;
    }
    void expect(char c)
    {
        if (!peek(c)) fail(std::string("expected '") + c + "'");
        ++p_;
    }

public:
    HeaderReader(const char* p, size_t n) : p_(p), end_(p + n) {}

    std::string string()
    {
        expect('"');
        std::string s;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c == '\\') {
                if (p_ >= end_) fail("unterminated escape");
                const char e = *p_++;
                switch (e) {
                case '"': case '\\': case '/': s += e; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    if (end_ - p_ < 4) fail("short \\u escape");
                    const unsigned cp = std::stoul(std::string(p_, p_ + 4), nullptr, 16);
                    p_ += 4;
                    // names are ASCII in practice; encode the BMP code point as UTF-8
                    if (cp < 0x80) s += char(cp);
                    else if (cp < 0x800) { s += char(0xC0 | (cp >> 6)); s += char(0x80 | (cp & 0x3F)); }
                    else { s += char(0xE0 | (cp >> 12)); s += char(0x80 | ((cp >> 6) & 0x3F)); s += char(0x80 | (cp & 0x3F)); }
                    break;
                }
                default: fail("bad escape");
                }
            } else {
                s += c;
            }
        }
        if (p_ >= end_) fail("unterminated string");
        ++p_;
        return s;
    }

    uint64_t integer()
    {
        ws();
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') fail("expected a non-negative integer");
        uint64_t v = 0;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = uint64_t(*p_++ - '0');
            if (v > (UINT64_MAX - d) / 10) fail("integer overflow");
            v = v * 10 + d;
        }
        return v;
    }

    std::vector<uint64_t> intArray()
    {
        std::vector<uint64_t> v;
        expect('[');
        if (peek(']')) { ++p_; return v; }
        for (;;) {
            v.push_back(integer());
            if (peek(',')) { ++p_; continue; }
            expect(']');
            return v;
        }
    }

    void skipValue()
    {
        ws();
        if (p_ >= end_) fail("unexpected end");
        if (*p_ == '"') { string(); return; }
        if (*p_ == '{' || *p_ == '[') {
            const char close = *p_ == '{' ? '}' : ']';
            ++p_;
            if (peek(close)) { ++p_; return; }
            for (;;) {
                if (close == '}') { string(); expect(':'); }
                skipValue();
                if (peek(',')) { ++p_; continue; }
                expect(close);
                return;
            }
        }
        while (p_ < end_ && *p_ != ',' && *p_ != '}' && *p_ != ']') ++p_;   // number, true, false, null
    }

    // {"name": {"dtype": ..., "shape": [...], "data_offsets": [b, e]}, ...}
    void tensors(std::vector<std::pair<std::string, Meta>>& out)
    {
        expect('{');
        if (peek('}')) { ++p_; return; }
        for (;;) {
            std::string name = string();
            expect(':');
            if (name == "__metadata__") {
                skipValue();
            } else {
                Meta m;
                bool dt = false, sh = false, off = false;
                expect('{');
                for (;;) {
                    const std::string field = string();
                    expect(':');
                    if (field == "dtype") { m.dtype = string(); dt = true; }
                    else if (field == "shape") {
                        for (uint64_t d : intArray()) {
                            if (d > UINT32_MAX) fail(name + ": dimension too large");
                            m.shape.push_back(uint32_t(d));
                        }
                        sh = true;
                    } else if (field == "data_offsets") {
                        const auto o = intArray();
                        if (o.size() != 2 || o[1] < o[0]) fail(name + ": bad data_offsets");
                        m.begin = o[0];
                        m.end = o[1];
                        off = true;
                    } else {
                        skipValue();
                    }
                    if (peek(',')) { ++p_; continue; }
                    expect('}');
                    break;
                }
                if (!dt || !sh || !off) fail("incomplete entry " + name);
                out.emplace_back(std::move(name), std::move(m));
            }
            if (peek(',')) { ++p_; continue; }
            expect('}');
            return;
        }
    }
};

size_t dtypeBytes(const std::string& dt)
{
    if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
    if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
    if (dt == "F16" || dt == "BF16" || dt == "I16" || dt == "U16") return 2;
    if (dt == "I8" || dt == "U8" || dt == "BOOL" || dt == "F8_E4M3" || dt == "F8_E5M2") return 1;
    return 0;   // unknown: sized by its offsets alone
}

float halfToFloat(uint16_t h)
{
    const uint32_t s = uint32_t(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = s;
        else {   // subnormal: normalise
            int sh = 0;
            uint32_t mm = m;
            while (!(mm & 0x400)) { mm <<= 1; ++sh; }
            bits = s | uint32_t(127 - 15 - sh + 1) << 23 | (mm & 0x3FF) << 13;
        }
    } else if (e == 31) {
        bits = s | 0x7F800000u | m << 13;
    } else {
        bits = s | (e + 127 - 15) << 23 | m << 13;
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}   // namespace

struct SafetensorsParser::Impl
{
    std::string path;
    const unsigned char* map = nullptr;
    size_t mapBytes = 0;
    size_t dataStart = 0;
    std::vector<std::string> order;
    std::unordered_map<std::string, Meta> tensors;

    explicit Impl(const char* file) : path(file)
    {
        const int fd = ::open(file, O_RDONLY);
        if (fd < 0) throw std::runtime_error("Could not open Safetensors file: " + path);
        struct stat st{};
        if (::fstat(fd, &st) != 0) { ::close(fd); throw std::runtime_error("Could not stat " + path); }
        mapBytes = size_t(st.st_size);
        if (mapBytes < 8) { ::close(fd); throw std::runtime_error("Failed to read header length: " + path); }
        void* m = ::mmap(nullptr, mapBytes, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (m == MAP_FAILED) throw std::runtime_error("Could not map " + path);
        map = static_cast<const unsigned char*>(m);
        uint64_t headerLen = 0;
        std::memcpy(&headerLen, map, 8);   // little-endian host
        if (headerLen > mapBytes - 8) { release(); throw std::runtime_error("Failed to read header string: " + path); }
        dataStart = 8 + headerLen;
        std::vector<std::pair<std::string, Meta>> entries;
        try {
            HeaderReader(reinterpret_cast<const char*>(map + 8), headerLen).tensors(entries);
        } catch (...) {
            release();
            throw;
        }
        for (auto& [name, meta] : entries) {
            size_t n = 1;
            for (uint32_t d : meta.shape) n *= d;
            const size_t eb = dtypeBytes(meta.dtype);
            if (meta.end > mapBytes - dataStart || (eb && n * eb != meta.end - meta.begin)) {
                release();
                throw std::runtime_error("Data size mismatch for tensor " + name + " in " + path);
            }
            order.push_back(name);
            tensors.emplace(name, std::move(meta));
        }
    }
    ~Impl() { release(); }
    void release()
    {
        if (map) ::munmap(const_cast<unsigned char*>(map), mapBytes);
        map = nullptr;
    }
    const Meta& meta(std::string_view key) const
    {
        auto it = tensors.find(std::string(key));
        if (it == tensors.end()) throw std::out_of_range("Tensor key not found: " + std::string(key));
        return it->second;
    }
};

SafetensorsParser::SafetensorsParser(const char* safetensorsFilePath)
: impl_(std::make_unique<Impl>(safetensorsFilePath)) {}
SafetensorsParser::~SafetensorsParser() = default;

std::vector<std::string> SafetensorsParser::getTensorNames() const { return impl_->order; }
std::vector<uint32_t> SafetensorsParser::getShape(std::string_view key) const { return impl_->meta(key).shape; }
std::string SafetensorsParser::getDataType(std::string_view key) const { return impl_->meta(key).dtype; }
size_t SafetensorsParser::byteSize(std::string_view key) const
{
    const Meta& m = impl_->meta(key);
    return m.end - m.begin;
}
const void* SafetensorsParser::data(std::string_view key) const
{
    return impl_->map + impl_->dataStart + impl_->meta(key).begin;
}
void SafetensorsParser::readInto(std::string_view key, void* dst) const
{
    readInto(key, dst, 0, byteSize(key));
}
void SafetensorsParser::readInto(std::string_view key, void* dst, size_t byteOffset, size_t byteCount) const
{
    const Meta& m = impl_->meta(key);
    if (byteOffset > m.end - m.begin || byteCount > m.end - m.begin - byteOffset)
        throw std::runtime_error("Tensor read runs past the end of the tensor.");
    std::memcpy(dst, impl_->map + impl_->dataStart + m.begin + byteOffset, byteCount);
}

Checkpoint::Checkpoint(const std::string& dir)
{
    std::vector<std::filesystem::path> files;
    for (const auto& e : std::filesystem::directory_iterator(dir))
        if (e.path().extension() == ".safetensors") files.push_back(e.path());
    std::sort(files.begin(), files.end());   // a fixed owner for keys present twice
    for (const auto& f : files) {
        auto& shard = shards_.emplace_back(std::make_unique<SafetensorsParser>(f.string().c_str()));
        for (const std::string& key : shard->getTensorNames()) owner_.emplace(key, shard.get());
    }
    if (owner_.empty()) throw std::runtime_error("no *.safetensors under " + dir);
}

SafetensorRef Checkpoint::operator[](std::string_view key) const
{
    auto it = owner_.find(std::string(key));
    if (it == owner_.end()) throw std::runtime_error("checkpoint has no tensor " + std::string(key));
    return (*it->second)[key];
}

std::vector<std::string> Checkpoint::getTensorNames() const
{
    std::vector<std::string> v;
    for (const auto& [k, _] : owner_) v.push_back(k);
    std::sort(v.begin(), v.end());
    return v;
}

Tensor loadTensor(const SafetensorRef& ref, Dtype dtype)
{
    const std::string dt = ref.getDataType();
    std::vector<uint32_t> shape = ref.getShape();
    if (shape.empty()) shape = {1};   // a scalar
    Tensor t(shape, dtype);
    const void* src = ref.parser->data(ref.key);
    const size_t n = t.numElements();
    if ((dt == "F32" && dtype == Dtype::Fp32) || (dt == "F16" && dtype == Dtype::Fp16)) {
        if (dtype == Dtype::Fp32) t.setData(static_cast<const float*>(src));
        else t.setData(static_cast<const uint16_t*>(src));
        return t;
    }
    std::vector<float> f(n);
    if (dt == "F32") {
        std::memcpy(f.data(), src, n * 4);
    } else if (dt == "F16") {
        const uint16_t* h = static_cast<const uint16_t*>(src);
        for (size_t i = 0; i < n; ++i) f[i] = halfToFloat(h[i]);
    } else if (dt == "BF16") {
        const uint16_t* h = static_cast<const uint16_t*>(src);
        for (size_t i = 0; i < n; ++i) {
            const uint32_t bits = uint32_t(h[i]) << 16;
            std::memcpy(&f[i], &bits, 4);
        }
    } else {
        throw std::runtime_error("Unsupported dtype: " + dt + " (tensor " + ref.key + ")");
    }
    t.setFloats(f);
    return t;
}

}   // namespace vai
