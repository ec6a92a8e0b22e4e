// safetensors header parsing and layer plans (see fw_safetensors.h).
//
// Follows the format rules the reference's readers enforce:
// src/checkpoint_catalog.rs:146-245 (MappedShard::open: header length,
// dtype sizes, exact payload sizes, no overlaps), src/expert.rs:362-442
// (read_expert_slice: BF16 [E, rows, columns]) and src/expert.rs:444-512
// (read_tensor_2d), src/checkpoint_catalog.rs:124-127 (shard names are plain
// file names) and src/checkpoint_catalog.rs:405-443 (tensor -> shard through
// the index's weight_map).
#include "fw_safetensors.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <utility>

namespace fw::st {
namespace {

[[noreturn]] void fault(const std::string& what) { throw std::runtime_error(what); }

// ---- a small JSON reader: what safetensors headers and index files hold ----

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool boolean = false;
    bool integer = false;  // a non-negative integer that fits in 64 bits
    uint64_t u = 0;
    std::string str;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;  // in file order; duplicates rejected

    const Json* get(const std::string& key) const {
        for (const auto& m : members)
            if (m.first == key) return &m.second;
        return nullptr;
    }
};

class Parser {
   public:
    Parser(const char* p, size_t n, std::string where) : p_(p), end_(p + n), where_(std::move(where)) {}

    Json document() {
        Json v = value(0);
        skip_ws();
        if (p_ != end_) error("trailing characters after the JSON value");
        return v;
    }

   private:
    [[noreturn]] void error(const std::string& what) { fault(where_ + ": " + what); }

    void skip_ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }

    bool take(char c) {
        skip_ws();
        if (p_ < end_ && *p_ == c) {
            ++p_;
            return true;
        }
        return false;
    }

    void expect(char c) {
        if (!take(c)) error(std::string("expected '") + c + "'");
    }

    void literal(const char* word) {
        size_t n = std::strlen(word);
        if ((size_t)(end_ - p_) < n || std::memcmp(p_, word, n) != 0) error("invalid literal");
        p_ += n;
    }

    static void put_utf8(std::string& s, uint32_t cp) {
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

    uint32_t hex4() {
        if (end_ - p_ < 4) error("truncated \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) {
            char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else error("invalid \\u escape");
        }
        return v;
    }

    std::string string_body() {
        std::string s;
        while (true) {
            if (p_ >= end_) error("unterminated string");
            char c = *p_++;
            if (c == '"') return s;
            if ((unsigned char)c < 0x20) error("control character in string");
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) error("unterminated escape");
            char e = *p_++;
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
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') error("unpaired surrogate");
                        p_ += 2;
                        uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo >= 0xE000) error("unpaired surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        error("unpaired surrogate");
                    }
                    put_utf8(s, cp);
                    break;
                }
                default: error("invalid escape");
            }
        }
    }

    Json number() {
        Json v;
        v.kind = Json::Number;
        const char* start = p_;
        bool negative = false;
        if (p_ < end_ && *p_ == '-') {
            negative = true;
            ++p_;
        }
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') error("invalid number");
        if (*p_ == '0' && p_ + 1 < end_ && p_[1] >= '0' && p_[1] <= '9') error("leading zero in number");
        bool overflow = false;
        uint64_t u = 0;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            uint64_t d = (uint64_t)(*p_ - '0');
            if (u > (UINT64_MAX - d) / 10) overflow = true;
            u = u * 10 + d;
            ++p_;
        }
        bool fraction = false;
        if (p_ < end_ && *p_ == '.') {
            fraction = true;
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') error("invalid number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            fraction = true;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') error("invalid number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        (void)start;
        v.integer = !negative && !fraction && !overflow;
        v.u = v.integer ? u : 0;
        return v;
    }

    Json value(int depth) {
        if (depth > 64) error("nesting too deep");
        skip_ws();
        if (p_ >= end_) error("unexpected end of JSON");
        Json v;
        char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Json::Object;
            if (take('}')) return v;
            do {
                skip_ws();
                if (p_ >= end_ || *p_ != '"') error("expected a member name");
                ++p_;
                std::string key = string_body();
                if (v.get(key)) error("duplicate member " + key);
                expect(':');
                v.members.emplace_back(std::move(key), value(depth + 1));
            } while (take(','));
            expect('}');
        } else if (c == '[') {
            ++p_;
            v.kind = Json::Array;
            if (take(']')) return v;
            do {
                v.items.push_back(value(depth + 1));
            } while (take(','));
            expect(']');
        } else if (c == '"') {
            ++p_;
            v.kind = Json::String;
            v.str = string_body();
        } else if (c == 't') {
            literal("true");
            v.kind = Json::Bool;
            v.boolean = true;
        } else if (c == 'f') {
            literal("false");
            v.kind = Json::Bool;
        } else if (c == 'n') {
            literal("null");
        } else {
            v = number();
        }
        return v;
    }

    const char* p_;
    const char* end_;
    std::string where_;
};

// element sizes of the safetensors dtypes
int dtype_bytes(const std::string& d) {
    if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E4M3" || d == "F8_E4M3FN" || d == "F8_E5M2") return 1;
    if (d == "U16" || d == "I16" || d == "F16" || d == "BF16") return 2;
    if (d == "U32" || d == "I32" || d == "F32") return 4;
    if (d == "U64" || d == "I64" || d == "F64") return 8;
    return 0;
}

struct Fd {
    int fd = -1;
    explicit Fd(const std::string& path) : fd(::open(path.c_str(), O_RDONLY | O_CLOEXEC)) {}
    ~Fd() {
        if (fd >= 0) ::close(fd);
    }
};

void read_exact(int fd, void* dst, size_t n, uint64_t offset, const std::string& path) {
    auto* p = static_cast<char*>(dst);
    while (n) {
        ssize_t got = ::pread(fd, p, n, (off_t)offset);
        if (got <= 0) fault(path + ": short read");
        p += got;
        n -= (size_t)got;
        offset += (uint64_t)got;
    }
}

std::string read_text(const std::string& path) {
    Fd f(path);
    if (f.fd < 0) fault(path + ": cannot open");
    struct stat st {};
    if (::fstat(f.fd, &st) != 0) fault(path + ": cannot stat");
    if (st.st_size > (off_t)(64u << 20)) fault(path + ": index file too large");
    std::string s((size_t)st.st_size, '\0');
    read_exact(f.fd, s.data(), s.size(), 0, path);
    return s;
}

bool plain_file_name(const std::string& name) {
    return !name.empty() && name != "." && name != ".." && name.find('/') == std::string::npos &&
           name.find('\0') == std::string::npos;
}

std::string shape_text(const std::vector<uint64_t>& shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

}  // namespace

Shard read_shard(const std::string& path) {
    Fd f(path);
    if (f.fd < 0) fault(path + ": cannot open");
    struct stat st {};
    if (::fstat(f.fd, &st) != 0 || !S_ISREG(st.st_mode)) fault(path + ": not a regular file");
    Shard shard;
    shard.path = path;
    shard.file_bytes = (uint64_t)st.st_size;
    if (shard.file_bytes < 16) fault(path + " is too short");
    uint8_t raw[8];
    read_exact(f.fd, raw, 8, 0, path);
    uint64_t header_len = 0;
    for (int i = 7; i >= 0; --i) header_len = (header_len << 8) | raw[i];
    if (header_len == 0 || header_len > (16u << 20) || 8 + header_len > shard.file_bytes)
        fault("invalid safetensors header in " + path);
    std::string text((size_t)header_len, '\0');
    read_exact(f.fd, text.data(), text.size(), 8, path);
    Json header = Parser(text.data(), text.size(), path + " header").document();
    if (header.kind != Json::Object) fault(path + ": safetensors header is not an object");
    const uint64_t payload_start = 8 + header_len;
    const uint64_t payload_bytes = shard.file_bytes - payload_start;
    std::vector<std::pair<std::pair<uint64_t, uint64_t>, std::string>> ranges;
    for (const auto& [name, item] : header.members) {
        if (name == "__metadata__") {
            if (item.kind != Json::Object) fault(path + ": safetensors __metadata__ is not an object");
            continue;
        }
        if (item.kind != Json::Object) fault(name + ": tensor entry is not an object");
        const Json* dtype = item.get("dtype");
        if (!dtype || dtype->kind != Json::String) fault(name + ": missing dtype");
        const int esize = dtype_bytes(dtype->str);
        if (!esize) fault(name + ": unknown dtype " + dtype->str);
        const Json* shape = item.get("shape");
        if (!shape || shape->kind != Json::Array) fault(name + ": missing shape");
        TensorInfo t;
        t.dtype = dtype->str;
        unsigned __int128 bytes = (unsigned)esize;
        for (const Json& d : shape->items) {
            if (d.kind != Json::Number || !d.integer) fault(name + ": invalid shape");
            if (d.u == 0) fault(name + ": empty shape");
            t.shape.push_back(d.u);
            bytes *= d.u;
            if (bytes > ((unsigned __int128)1 << 62)) fault(name + ": tensor size overflow");
        }
        if (t.shape.empty()) fault(name + ": empty shape");
        const Json* off = item.get("data_offsets");
        if (!off || off->kind != Json::Array) fault(name + ": missing offsets");
        if (off->items.size() != 2) fault(name + ": invalid offsets");
        const Json& a = off->items[0];
        const Json& b = off->items[1];
        if (a.kind != Json::Number || !a.integer) fault(name + ": invalid start");
        if (b.kind != Json::Number || !b.integer) fault(name + ": invalid end");
        if (b.u < a.u || b.u - a.u != (uint64_t)bytes || b.u > payload_bytes)
            fault(name + ": payload layout mismatch");
        t.offset = payload_start + a.u;
        t.bytes = (uint64_t)bytes;
        ranges.push_back({{a.u, b.u}, name});
        shard.tensors.emplace(name, std::move(t));
    }
    std::sort(ranges.begin(), ranges.end());
    uint64_t previous_end = 0;
    for (const auto& r : ranges) {
        if (r.first.first < previous_end) fault("overlapping tensor " + r.second + " in " + path);
        previous_end = r.first.second;
    }
    return shard;
}

Checkpoint::Checkpoint(const std::string& path) {
    const size_t slash = path.find_last_of('/');
    dir_ = slash == std::string::npos ? std::string(".") : path.substr(0, slash == 0 ? 1 : slash);
    const std::string suffix = ".json";
    if (path.size() >= suffix.size() && path.compare(path.size() - suffix.size(), suffix.size(), suffix) == 0) {
        std::string text = read_text(path);
        Json index = Parser(text.data(), text.size(), path).document();
        const Json* map = index.kind == Json::Object ? index.get("weight_map") : nullptr;
        if (!map || map->kind != Json::Object) fault(path + ": checkpoint index has no weight_map object");
        for (const auto& [tensor, file] : map->members) {
            if (file.kind != Json::String) fault(path + ": weight_map entry " + tensor + " is not a file name");
            if (!plain_file_name(file.str)) fault("unbound checkpoint shard: " + file.str);
            weight_map_.emplace(tensor, file.str);
        }
    } else {
        single_ = path;
    }
}

const Shard& Checkpoint::shard(const std::string& file) {
    auto it = shards_.find(file);
    if (it != shards_.end()) return *it->second;
    auto s = std::make_unique<Shard>(read_shard(file));
    const Shard& ref = *s;
    shards_.emplace(file, std::move(s));
    return ref;
}

const TensorInfo& Checkpoint::bf16(const std::string& name, const std::vector<uint64_t>& shape, std::string* file) {
    std::string path;
    if (!single_.empty()) {
        path = single_;
    } else {
        auto it = weight_map_.find(name);
        if (it == weight_map_.end()) fault("tensor absent from index: " + name);
        path = dir_ + "/" + it->second;
    }
    const Shard& s = shard(path);
    auto t = s.tensors.find(name);
    if (t == s.tensors.end()) fault("tensor absent from shard: " + name);
    if (t->second.dtype != "BF16") fault(name + ": expected BF16, got " + t->second.dtype);
    if (t->second.shape != shape)
        fault(name + ": shape " + shape_text(t->second.shape) + ", expected " + shape_text(shape));
    if (file) *file = path;
    return t->second;
}

std::vector<Span> layer_plan(Checkpoint& ckpt, const std::string& prefix, uint64_t H, uint64_t I, uint64_t E,
                             uint64_t Is) {
    const std::pair<const char*, std::vector<uint64_t>> wanted[7] = {
        {".mlp.gate.weight", {E, H}},
        {".mlp.experts.gate_up_proj", {E, 2 * I, H}},
        {".mlp.experts.down_proj", {E, H, I}},
        {".mlp.shared_expert.gate_proj.weight", {Is, H}},
        {".mlp.shared_expert.up_proj.weight", {Is, H}},
        {".mlp.shared_expert.down_proj.weight", {H, Is}},
        {".mlp.shared_expert_gate.weight", {1, H}},
    };
    std::vector<Span> plan;
    for (const auto& [suffix, shape] : wanted) {
        Span sp;
        const TensorInfo& t = ckpt.bf16(prefix + suffix, shape, &sp.file);
        sp.offset = t.offset;
        sp.bytes = t.bytes;
        plan.push_back(std::move(sp));
    }
    return plan;
}

}  // namespace fw::st
