// weights_hip.cpp - see weights_hip.h.
#include "weights_hip.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <utility>
#include <vector>

#include "sd_hip.hpp"

namespace sdh {
namespace {

// ---- a small JSON reader for the safetensors header ----------------------
struct JValue {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    double num = 0;
    std::string str;
    std::vector<JValue> arr;
    std::vector<std::pair<std::string, JValue>> obj;
    const JValue* find(const std::string& key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonReader {
public:
    JsonReader(const char* p, const char* end) : p_(p), end_(end) {}
    JValue document() {
        JValue v = value();
        ws();
        if (p_ != end_) fail("trailing characters");
        return v;
    }

private:
    const char* p_;
    const char* end_;
    int depth_ = 0;  // open objects and arrays; a header nests two or three deep
    static constexpr int kMaxDepth = 64;
    [[noreturn]] void fail(const char* what) { throw std::runtime_error(std::string("safetensors header: ") + what); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool take(char c) {
        ws();
        if (p_ < end_ && *p_ == c) {
            ++p_;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!take(c)) fail("unexpected character");
    }
    static void put_utf8(std::string& s, unsigned cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    unsigned hex4() {
        if (end_ - p_ < 4) fail("short \\u escape");
        unsigned v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else fail("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string s;
        while (true) {
            if (p_ >= end_) fail("unterminated string");
            const char c = *p_++;
            if (c == '"') break;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) fail("unterminated escape");
            const char e = *p_++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    unsigned cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                        p_ += 2;
                        const unsigned lo = hex4();
                        if (lo < 0xDC00 || lo > 0xDFFF) fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(s, cp);
                    break;
                }
                default: fail("bad escape");
            }
        }
        return s;
    }
    JValue value() {
        ws();
        if (p_ >= end_) fail("unexpected end");
        JValue v;
        const char c = *p_;
        if ((c == '{' || c == '[') && ++depth_ > kMaxDepth) fail("nesting too deep");
        if (c == '{') {
            ++p_;
            v.kind = JValue::Object;
            if (take('}')) {
                --depth_;
                return v;
            }
            do {
                ws();
                std::string k = string();
                expect(':');
                v.obj.emplace_back(std::move(k), value());
            } while (take(','));
            expect('}');
            --depth_;
        } else if (c == '[') {
            ++p_;
            v.kind = JValue::Array;
            if (take(']')) {
                --depth_;
                return v;
            }
            do v.arr.push_back(value());
            while (take(','));
            expect(']');
            --depth_;
        } else if (c == '"') {
            v.kind = JValue::String;
            v.str = string();
        } else if (end_ - p_ >= 4 && std::strncmp(p_, "true", 4) == 0) {
            p_ += 4;
            v.kind = JValue::Bool;
            v.num = 1;
        } else if (end_ - p_ >= 5 && std::strncmp(p_, "false", 5) == 0) {
            p_ += 5;
            v.kind = JValue::Bool;
        } else if (end_ - p_ >= 4 && std::strncmp(p_, "null", 4) == 0) {
            p_ += 4;
        } else {
            const char* s = p_;
            while (p_ < end_ && *p_ != '\0' && std::strchr("+-0123456789.eE", *p_) != nullptr) ++p_;
            if (s == p_) fail("unexpected character");
            v.kind = JValue::Number;
            const std::string t(s, p_);
            char* stop = nullptr;
            v.num = std::strtod(t.c_str(), &stop);
            if (stop != t.c_str() + t.size()) fail("bad number");
        }
        return v;
    }
};

// IEEE half -> float (subnormals, inf and NaN included).
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {  // subnormal: normalise
        int e = -1;
        do {
            man <<= 1;
            ++e;
        } while (!(man & 0x400u));
        bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}
float bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}
// tensor.cpp:114-121 rounding
uint16_t f32_to_bf16(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    if ((b & 0x7F800000u) == 0x7F800000u) return (uint16_t)(b >> 16);
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

struct Mapped {
    void* base = nullptr;
    size_t size = 0;
    explicit Mapped(const std::string& path) {
        const int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) throw std::runtime_error("cannot open " + path);
        struct stat st;
        if (fstat(fd, &st) != 0) {
            ::close(fd);
            throw std::runtime_error("cannot stat " + path);
        }
        size = (size_t)st.st_size;
        base = size ? mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
        ::close(fd);
        if (base == MAP_FAILED) {
            base = nullptr;
            throw std::runtime_error("mmap failed for " + path);
        }
    }
    ~Mapped() {
        if (base) munmap(base, size);
    }
};

}  // namespace

void Weights::load_safetensors(const std::string& path, bool keep_bf16, int64_t bf16_min_numel) {
    Mapped f(path);
    if (f.size < 8) throw std::runtime_error("safetensors: file too small: " + path);
    uint64_t hlen = 0;
    std::memcpy(&hlen, f.base, 8);
    if (hlen > f.size - 8) throw std::runtime_error("safetensors: bad header length in " + path);
    const char* hdr = (const char*)f.base + 8;
    const JValue meta = JsonReader(hdr, hdr + hlen).document();
    if (meta.kind != JValue::Object) throw std::runtime_error("safetensors: header is not an object in " + path);
    const uint8_t* data = (const uint8_t*)f.base + 8 + hlen;
    const size_t data_size = f.size - 8 - (size_t)hlen;
    for (const auto& kv : meta.obj) {
        const std::string& name = kv.first;
        if (name == "__metadata__") continue;
        const JValue* dt = kv.second.find("dtype");
        const JValue* sh = kv.second.find("shape");
        const JValue* off = kv.second.find("data_offsets");
        if (!dt || !sh || !off || off->arr.size() != 2) throw std::runtime_error("safetensors: bad entry for " + name);
        const std::string& dtype = dt->str;
        // Dimensions and offsets must be non-negative integers that fit the
        // file; the element count is formed with overflow checks, so a shape
        // can never disagree with the bytes it describes.
        auto whole = [&](const JValue& v, double hi, const char* what) {
            if (v.kind != JValue::Number || !(v.num >= 0.0) || v.num > hi || v.num != (double)(int64_t)v.num)
                throw std::runtime_error(std::string("safetensors: bad ") + what + " for " + name);
            return (int64_t)v.num;
        };
        std::vector<int64_t> shape;
        int64_t n = 1;
        for (const JValue& d : sh->arr) {
            shape.push_back(whole(d, 9.0e15, "dimension"));
            if (__builtin_mul_overflow(n, shape.back(), &n))
                throw std::runtime_error("safetensors: element count overflows for " + name);
        }
        const size_t b = (size_t)whole(off->arr[0], 9.0e15, "offset"), e = (size_t)whole(off->arr[1], 9.0e15, "offset");
        if (e > data_size || b > e) throw std::runtime_error("safetensors: bad offsets for " + name);
        if (dtype != "F32" && dtype != "F16" && dtype != "BF16") {
            std::fprintf(stderr, "  skipping %s (dtype %s)\n", name.c_str(), dtype.c_str());
            continue;
        }
        const size_t elem = dtype == "F32" ? 4 : 2;
        int64_t nbytes = 0;
        if (__builtin_mul_overflow(n, (int64_t)elem, &nbytes) || (size_t)nbytes != e - b)
            throw std::runtime_error("safetensors: size mismatch for " + name);
        const uint8_t* src = data + b;
        Tensor t(shape);  // host staging
        if (keep_bf16 && n >= bf16_min_numel) {
            t.data.clear();
            t.dtype = DType::BF16;
            t.data16.resize((size_t)n);
            if (dtype == "BF16") {
                std::memcpy(t.data16.data(), src, (size_t)n * 2);
            } else {
                for (int64_t j = 0; j < n; ++j) {
                    float v;
                    if (dtype == "F32") {
                        std::memcpy(&v, src + 4 * j, 4);
                    } else {
                        uint16_t h;
                        std::memcpy(&h, src + 2 * j, 2);
                        v = f16_to_f32(h);
                    }
                    t.data16[(size_t)j] = f32_to_bf16(v);
                }
            }
        } else if (dtype == "F32") {
            std::memcpy(t.data.data(), src, (size_t)n * 4);
        } else {
            const bool bf = dtype == "BF16";
            for (int64_t j = 0; j < n; ++j) {
                uint16_t h;
                std::memcpy(&h, src + 2 * j, 2);
                t.data[(size_t)j] = bf ? bf16_to_f32(h) : f16_to_f32(h);
            }
        }
        tensors[name] = t.to(Device::HIP);
    }
}

void Weights::add_random(const std::string& name, std::vector<int64_t> shape, uint64_t seed, float mean, float std,
                         bool keep_bf16, int64_t bf16_min_numel) {
    Tensor f = Tensor::empty(shape, Device::HIP);
    const int64_t n = f.numel();
    if (n) sd::hip::fill_normal(f.dptr(), n, seed, mean, std);
    if (keep_bf16 && n >= bf16_min_numel) {
        Tensor h;
        h.shape = shape;
        h.device = Device::HIP;
        h.dtype = DType::BF16;
        // a BF16 device tensor holds n uint16 values in a float-sized block of ceil(n / 2) floats
        Tensor store = Tensor::empty({(n + 1) / 2}, Device::HIP);
        h.dev = store.dev;
        if (n) sd::hip::to_bf16(f.dptr(), (uint16_t*)store.dptr(), n);
        tensors[name] = h;
    } else {
        tensors[name] = f;
    }
}

const Tensor& Weights::get(const std::string& name) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) throw std::runtime_error("missing weight: " + name);
    return it->second;
}

const Tensor* Weights::try_get(const std::string& name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : &it->second;
}

size_t Weights::total_params() const {
    size_t n = 0;
    for (const auto& kv : tensors) n += (size_t)kv.second.numel();
    return n;
}

}  // namespace sdh
