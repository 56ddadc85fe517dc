// theano_serialize.cpp -- safetensors container (see theano_serialize.hpp).
#include "theano_serialize.hpp"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <limits>
#include <sstream>

namespace theano {
namespace serialize {
namespace {

// ------------------------------------------------------------- minimal JSON
// Objects (key order kept), arrays, strings with escapes, integers (exact in
// 64 bits), other numbers, true/false/null -- what a safetensors header holds.
struct Json {
    enum class Kind { Null, Bool, Int, Num, Str, Arr, Obj } kind = Kind::Null;
    bool b = false;
    int64_t i = 0;
    double d = 0.0;
    std::string s;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const std::string& key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class Parser {
   public:
    Parser(const char* p, const char* e) : p_(p), e_(e) {}
    bool parse(Json& out) {
        if (!value(out, 0)) return false;
        ws();
        return p_ == e_;
    }
    std::string error() const { return err_; }

   private:
    const char* p_;
    const char* e_;
    std::string err_;

    bool fail(const char* m) {
        if (err_.empty()) err_ = m;
        return false;
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = std::strlen(w);
        if (static_cast<size_t>(e_ - p_) < n || std::memcmp(p_, w, n) != 0) return fail("bad literal");
        p_ += n;
        return true;
    }
    static void put_utf8(std::string& s, uint32_t c) {
        if (c < 0x80) {
            s += static_cast<char>(c);
        } else if (c < 0x800) {
            s += static_cast<char>(0xC0 | (c >> 6));
            s += static_cast<char>(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += static_cast<char>(0xE0 | (c >> 12));
            s += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (c & 0x3F));
        } else {
            s += static_cast<char>(0xF0 | (c >> 18));
            s += static_cast<char>(0x80 | ((c >> 12) & 0x3F));
            s += static_cast<char>(0x80 | ((c >> 6) & 0x3F));
            s += static_cast<char>(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t& v) {
        if (e_ - p_ < 4) return fail("short \\u escape");
        v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool str(std::string& out) {
        if (p_ >= e_ || *p_ != '"') return fail("expected a string");
        ++p_;
        while (p_ < e_ && *p_ != '"') {
            const unsigned char c = static_cast<unsigned char>(*p_++);
            if (c < 0x20) return fail("control character in a string");
            if (c != '\\') {
                out += static_cast<char>(c);
                continue;
            }
            if (p_ >= e_) return fail("unterminated escape");
            const char x = *p_++;
            switch (x) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t v;
                    if (!hex4(v)) return false;
                    if (v >= 0xD800 && v < 0xDC00) {  // surrogate pair
                        uint32_t lo;
                        if (e_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
                        p_ += 2;
                        if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate");
                        v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(out, v);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p_ >= e_) return fail("unterminated string");
        ++p_;
        return true;
    }
    bool num(Json& out) {
        const char* b = p_;
        if (p_ < e_ && *p_ == '-') ++p_;
        bool integral = true;
        while (p_ < e_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                           *p_ == '-')) {
            if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') integral = false;
            ++p_;
        }
        const std::string t(b, p_);
        if (t.empty() || t == "-") return fail("bad number");
        try {
            if (integral) {
                out.kind = Json::Kind::Int;
                out.i = std::stoll(t);
            } else {
                out.kind = Json::Kind::Num;
                out.d = std::stod(t);
            }
        } catch (...) {
            return fail("number out of range");
        }
        return true;
    }
    bool value(Json& out, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p_ >= e_) return fail("unexpected end");
        const char c = *p_;
        if (c == '{') {
            ++p_;
            out.kind = Json::Kind::Obj;
            ws();
            if (p_ < e_ && *p_ == '}') {
                ++p_;
                return true;
            }
            while (true) {
                ws();
                std::string key;
                if (!str(key)) return false;
                ws();
                if (p_ >= e_ || *p_ != ':') return fail("expected ':'");
                ++p_;
                Json v;
                if (!value(v, depth + 1)) return false;
                out.obj.emplace_back(std::move(key), std::move(v));
                ws();
                if (p_ < e_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < e_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p_;
            out.kind = Json::Kind::Arr;
            ws();
            if (p_ < e_ && *p_ == ']') {
                ++p_;
                return true;
            }
            while (true) {
                Json v;
                if (!value(v, depth + 1)) return false;
                out.arr.push_back(std::move(v));
                ws();
                if (p_ < e_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < e_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            out.kind = Json::Kind::Str;
            return str(out.s);
        }
        if (c == 't') {
            out.kind = Json::Kind::Bool;
            out.b = true;
            return lit("true");
        }
        if (c == 'f') {
            out.kind = Json::Kind::Bool;
            return lit("false");
        }
        if (c == 'n') return lit("null");
        return num(out);
    }
};

void put_json_string(std::string& o, const std::string& s) {
    o += '"';
    for (const char ch : s) {
        const unsigned char c = static_cast<unsigned char>(ch);
        if (c == '"') o += "\\\"";
        else if (c == '\\') o += "\\\\";
        else if (c < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", c);
            o += buf;
        } else {
            o += ch;
        }
    }
    o += '"';
}

// the reference's DType names (dtype.rs:79-100) -> standard code of the same element type
std::string standard_code(const std::string& d) {
    static const std::map<std::string, std::string> ref = {
        {"float64", "F64"}, {"float32", "F32"}, {"float16", "F16"}, {"bfloat16", "BF16"}, {"int64", "I64"},
        {"int32", "I32"},   {"int16", "I16"},   {"int8", "I8"},     {"uint8", "U8"},      {"bool", "BOOL"},
        {"qint8", "I8"},    {"quint8", "U8"},   {"qint32", "I32"}};
    const auto it = ref.find(d);
    return it == ref.end() ? d : it->second;
}

bool is_reference_name(const std::string& d) { return standard_code(d) != d; }

size_t numel_of(const std::vector<size_t>& shape) {
    size_t n = 1;
    for (const size_t s : shape) n *= s;
    return n;
}

std::string shape_text(const std::vector<size_t>& shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

// element `i` of a raw payload of standard code `code` as f64
double decode(const std::string& code, const uint8_t* p, size_t i) {
    if (code == "F64") { double v; std::memcpy(&v, p + 8 * i, 8); return v; }
    if (code == "F32") { float v; std::memcpy(&v, p + 4 * i, 4); return v; }
    if (code == "F16") { _Float16 v; std::memcpy(&v, p + 2 * i, 2); return static_cast<double>(v); }
    if (code == "BF16") { uint16_t v; std::memcpy(&v, p + 2 * i, 2); return nn::bf16_to_f32(v); }
    if (code == "I64") { int64_t v; std::memcpy(&v, p + 8 * i, 8); return static_cast<double>(v); }
    if (code == "I32") { int32_t v; std::memcpy(&v, p + 4 * i, 4); return v; }
    if (code == "I16") { int16_t v; std::memcpy(&v, p + 2 * i, 2); return v; }
    if (code == "I8") return static_cast<int8_t>(p[i]);
    if (code == "U8") return p[i];
    if (code == "F8_E4M3") return quantize::e4m3_value(p[i]);
    return p[i] != 0 ? 1.0 : 0.0;  // BOOL
}

}  // namespace

size_t element_size(const std::string& dtype) {
    static const std::map<std::string, size_t> sz = {{"F64", 8}, {"F32", 4}, {"F16", 2}, {"BF16", 2}, {"I64", 8},
                                                     {"I32", 4}, {"I16", 2}, {"I8", 1},  {"U8", 1},   {"BOOL", 1},
                                                     {"F8_E4M3", 1}};
    const auto it = sz.find(standard_code(dtype));
    return it == sz.end() ? 0 : it->second;
}

void SafeTensorsFile::add_tensor(const std::string& name, const Tensor& tensor) {
    const size_t start = data.size();
    for (size_t i = 0; i < tensor.numel(); ++i) {
        const double v = tensor.data()[i];
        uint8_t b[8];
        std::memcpy(b, &v, 8);  // little-endian host
        data.insert(data.end(), b, b + 8);
    }
    tensors[name] = TensorInfo{name, "F64", tensor.shape(), {start, data.size()}};
}

Result<void> SafeTensorsFile::add_raw(const std::string& name, const std::string& dtype, std::vector<size_t> shape,
                                      const void* bytes, size_t nbytes) {
    const size_t es = element_size(dtype);
    if (es == 0 || is_reference_name(dtype))
        return TheanoError::invalid_argument("add_raw: '" + dtype + "' is not a standard dtype code");
    if (numel_of(shape) * es != nbytes)
        return TheanoError::shape_mismatch("add_raw: " + std::to_string(nbytes) + " bytes for " + shape_text(shape) +
                                           " of " + dtype);
    const size_t start = data.size();
    const auto* p = static_cast<const uint8_t*>(bytes);
    data.insert(data.end(), p, p + nbytes);
    tensors[name] = TensorInfo{name, dtype, std::move(shape), {start, data.size()}};
    return {};
}

Result<Tensor> SafeTensorsFile::get_tensor(const std::string& name) const {
    const auto it = tensors.find(name);
    if (it == tensors.end()) return TheanoError::runtime("tensor '" + name + "' not found");
    const TensorInfo& t = it->second;
    const size_t n = numel_of(t.shape), nbytes = t.data_offsets.second - t.data_offsets.first;
    std::string code = standard_code(t.dtype);
    if (is_reference_name(t.dtype) && nbytes == 8 * n) code = "F64";  // the reference's f64 payload
    const size_t es = element_size(code);
    if (es == 0 || nbytes != n * es)
        return TheanoError::runtime("tensor '" + name + "': " + std::to_string(nbytes) + " bytes for " +
                                    shape_text(t.shape) + " of " + t.dtype);
    std::vector<double> v(n);
    const uint8_t* p = data.data() + t.data_offsets.first;
    for (size_t i = 0; i < n; ++i) v[i] = decode(code, p, i);
    return Tensor::from_slice(std::move(v), t.shape);
}

Result<std::vector<uint8_t>> SafeTensorsFile::get_raw(const std::string& name, const std::string& dtype,
                                                      const std::vector<size_t>& shape) const {
    const auto it = tensors.find(name);
    if (it == tensors.end()) return TheanoError::runtime("tensor '" + name + "' not found");
    const TensorInfo& t = it->second;
    if (standard_code(t.dtype) != standard_code(dtype) || t.shape != shape)
        return TheanoError::shape_mismatch("tensor '" + name + "' is " + t.dtype + " " + shape_text(t.shape) +
                                           ", expected " + dtype + " " + shape_text(shape));
    const size_t nbytes = t.data_offsets.second - t.data_offsets.first;
    if (nbytes != numel_of(shape) * element_size(dtype))
        return TheanoError::runtime("tensor '" + name + "' does not hold a raw " + dtype + " payload");
    return std::vector<uint8_t>(data.begin() + static_cast<std::ptrdiff_t>(t.data_offsets.first),
                                data.begin() + static_cast<std::ptrdiff_t>(t.data_offsets.second));
}

std::vector<std::string> SafeTensorsFile::tensor_names() const {
    std::vector<std::string> out;
    for (const auto& kv : tensors) out.push_back(kv.first);
    return out;
}

std::vector<uint8_t> SafeTensorsFile::to_bytes() const {
    std::string h = "{";
    bool first = true;
    for (const auto& kv : tensors) {  // name order
        const TensorInfo& t = kv.second;
        if (!first) h += ',';
        first = false;
        put_json_string(h, kv.first);
        h += ":{\"dtype\":";
        put_json_string(h, t.dtype);
        h += ",\"shape\":[";
        for (size_t i = 0; i < t.shape.size(); ++i) h += (i ? "," : "") + std::to_string(t.shape[i]);
        h += "],\"data_offsets\":[" + std::to_string(t.data_offsets.first) + "," +
             std::to_string(t.data_offsets.second) + "]}";
    }
    if (!metadata.empty()) {
        if (!first) h += ',';
        h += "\"__metadata__\":{";
        bool f2 = true;
        for (const auto& kv : metadata) {
            if (!f2) h += ',';
            f2 = false;
            put_json_string(h, kv.first);
            h += ':';
            put_json_string(h, kv.second);
        }
        h += '}';
    }
    h += '}';
    h.append((8 - h.size() % 8) % 8, ' ');
    std::vector<uint8_t> out(8);
    const uint64_t len = h.size();
    std::memcpy(out.data(), &len, 8);
    out.insert(out.end(), h.begin(), h.end());
    out.insert(out.end(), data.begin(), data.end());
    return out;
}

Result<SafeTensorsFile> SafeTensorsFile::from_bytes(const std::vector<uint8_t>& bytes) {
    if (bytes.size() < 8) return TheanoError::runtime("invalid safetensors: too short");
    uint64_t len;
    std::memcpy(&len, bytes.data(), 8);
    if (len > bytes.size() - 8) return TheanoError::runtime("invalid safetensors: truncated header");
    const char* h = reinterpret_cast<const char*>(bytes.data() + 8);
    Json root;
    Parser parser(h, h + len);
    if (!parser.parse(root) || root.kind != Json::Kind::Obj)
        return TheanoError::runtime("invalid safetensors header: " +
                                    (parser.error().empty() ? std::string("not an object") : parser.error()));
    SafeTensorsFile f;
    f.data.assign(bytes.begin() + 8 + static_cast<std::ptrdiff_t>(len), bytes.end());
    for (const auto& kv : root.obj) {
        const Json& v = kv.second;
        if (kv.first == "__metadata__") {
            if (v.kind != Json::Kind::Obj) return TheanoError::runtime("invalid safetensors: __metadata__");
            for (const auto& m : v.obj) {
                if (m.second.kind != Json::Kind::Str)
                    return TheanoError::runtime("invalid safetensors: metadata value of '" + m.first + "'");
                f.metadata[m.first] = m.second.s;
            }
            continue;
        }
        const Json* dt = v.get("dtype");
        const Json* sh = v.get("shape");
        const Json* of = v.get("data_offsets");
        if (v.kind != Json::Kind::Obj || !dt || dt->kind != Json::Kind::Str || !sh || sh->kind != Json::Kind::Arr ||
            !of || of->kind != Json::Kind::Arr || of->arr.size() != 2)
            return TheanoError::runtime("invalid safetensors entry '" + kv.first + "'");
        TensorInfo t;
        t.name = kv.first;
        t.dtype = dt->s;
        for (const Json& d : sh->arr) {
            if (d.kind != Json::Kind::Int || d.i < 0)
                return TheanoError::runtime("invalid safetensors shape of '" + kv.first + "'");
            t.shape.push_back(static_cast<size_t>(d.i));
        }
        if (of->arr[0].kind != Json::Kind::Int || of->arr[1].kind != Json::Kind::Int || of->arr[0].i < 0 ||
            of->arr[1].i < of->arr[0].i || static_cast<uint64_t>(of->arr[1].i) > f.data.size())
            return TheanoError::runtime("invalid safetensors data_offsets of '" + kv.first + "'");
        t.data_offsets = {static_cast<size_t>(of->arr[0].i), static_cast<size_t>(of->arr[1].i)};
        const size_t es = element_size(t.dtype);
        const size_t nbytes = t.data_offsets.second - t.data_offsets.first, n = numel_of(t.shape);
        if (es == 0) return TheanoError::runtime("safetensors '" + kv.first + "': unknown dtype " + t.dtype);
        if (nbytes != n * es && !(is_reference_name(t.dtype) && nbytes == 8 * n))
            return TheanoError::runtime("safetensors '" + kv.first + "' holds " + std::to_string(nbytes) +
                                        " bytes for " + shape_text(t.shape) + " of " + t.dtype);
        f.tensors[t.name] = std::move(t);
    }
    return std::move(f);
}

std::vector<uint8_t> save_safetensors(const std::map<std::string, Tensor>& tensors) {
    SafeTensorsFile f;
    for (const auto& kv : tensors) f.add_tensor(kv.first, kv.second);
    return f.to_bytes();
}

Result<std::map<std::string, Tensor>> load_safetensors(const std::vector<uint8_t>& bytes) {
    auto r = SafeTensorsFile::from_bytes(bytes);
    if (r.is_err()) return r.unwrap_err();
    const SafeTensorsFile& f = r.unwrap();
    std::map<std::string, Tensor> out;
    for (const auto& name : f.tensor_names()) {
        auto t = f.get_tensor(name);
        if (t.is_err()) return t.unwrap_err();
        out.emplace(name, std::move(t).unwrap());
    }
    return std::move(out);
}

}  // namespace serialize
}  // namespace theano
