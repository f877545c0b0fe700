// Checkpoint ingest: the safetensors format as SafetensorsReader / SafetensorsCheckpoint read it
// (SafetensorsReader.cs:110-160, :188-235, :300-430; SafetensorsCheckpoint.cs:41-150).
//
// A file is an 8-byte little-endian header length, a JSON header mapping tensor names to
// {dtype, shape, data_offsets} (plus an optional "__metadata__" object), then the data section.
// Opening validates the header against the format: the announced length fits the file and
// 100 MB, every entry has a known dtype, a non-negative shape whose byte size matches its
// data_offsets, offsets inside the data section, no name twice and no two tensors sharing bytes
// (the checks SafetensorsReader.Open makes; the validator here is organised its own way).
// Tensors are read with pread in 1 MiB chunks and converted to fp32 (F32, F16, BF16, F64 sources).
// A directory opens model.safetensors.index.json (its weight_map names the shard of every
// tensor; shards and index must agree) or else model.safetensors.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/l0hip.h"
#include "host.h"

namespace l0h {
void clear_error();
int fail(int code, const std::string& msg);

#define L0H_CHECK_ARG(cond, msg)                                  \
    do {                                                          \
        if (!(cond)) return ::l0h::fail(L0H_ERR_INVALID_ARG, msg); \
    } while (0)

namespace {

// ---- a small JSON reader (objects keep their order) -------------------------------------------

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0;
    bool integral = false;
    long long ival = 0;
    std::string str;
    std::vector<Json> items;                            // Array
    std::vector<std::pair<std::string, Json>> members;  // Object
};

class JsonParser {
public:
    JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}

    bool parse(Json& out, std::string& err) {
        if (!value(out, 0)) {
            err = err_.empty() ? "malformed JSON" : err_;
            return false;
        }
        ws();
        // The safetensors header may be padded with spaces after the object.
        if (p_ != end_) {
            err = "trailing characters after the JSON value";
            return false;
        }
        return true;
    }

private:
    const char* p_;
    const char* end_;
    std::string err_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool lit(const char* s) {
        const size_t n = std::strlen(s);
        if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(std::string& s, unsigned cp) {
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
    bool hex4(unsigned& v) {
        if (end_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& s) {
        if (p_ >= end_ || *p_ != '"') return false;
        p_++;
        while (p_ < end_) {
            const char c = *p_++;
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return false;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) return false;
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
                unsigned cp;
                if (!hex4(cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                    unsigned lo;
                    if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(s, cp);
                break;
            }
            default: return false;
            }
        }
        return false;
    }
    bool number(Json& v) {
        const char* s = p_;
        if (p_ < end_ && *p_ == '-') p_++;
        bool any = false, frac = false;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                             *p_ == '-')) {
            frac |= *p_ == '.' || *p_ == 'e' || *p_ == 'E';
            any = true;
            p_++;
        }
        if (!any) return false;
        const std::string t(s, p_);
        char* e = nullptr;
        v.kind = Json::Number;
        v.num = std::strtod(t.c_str(), &e);
        if (e != t.c_str() + t.size()) return false;
        if (!frac) {
            errno = 0;
            const long long iv = std::strtoll(t.c_str(), &e, 10);
            v.integral = errno == 0 && e == t.c_str() + t.size();
            v.ival = iv;
        }
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) {
            err_ = "JSON nested too deeply";
            return false;
        }
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            p_++;
            v.kind = Json::Object;
            ws();
            if (p_ < end_ && *p_ == '}') {
                p_++;
                return true;
            }
            for (;;) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                p_++;
                Json child;
                if (!value(child, depth + 1)) return false;
                v.members.emplace_back(std::move(key), std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    p_++;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            p_++;
            v.kind = Json::Array;
            ws();
            if (p_ < end_ && *p_ == ']') {
                p_++;
                return true;
            }
            for (;;) {
                Json child;
                if (!value(child, depth + 1)) return false;
                v.items.push_back(std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    p_++;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            v.kind = Json::String;
            return string(v.str);
        }
        if (lit("true")) {
            v.kind = Json::Bool;
            v.b = true;
            return true;
        }
        if (lit("false")) {
            v.kind = Json::Bool;
            return true;
        }
        if (lit("null")) return true;
        return number(v);
    }
};

const Json* member(const Json& obj, const char* key) {
    for (const auto& kv : obj.members)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

// ---- one file -------------------------------------------------------------------------------------

constexpr long long kMaxHeaderBytes = 100000000;
constexpr size_t kChunkBytes = 1 << 20;

// Codes follow the reference's SafetensorsDType order (SafetensorsReader.cs:10-25).
const char* const kDtypeNames[] = {"BOOL", "U8", "I8", "I16", "U16", "F16", "BF16", "I32", "U32", "F32", "F64", "I64", "U64"};
const int kDtypeSizes[] = {1, 1, 1, 2, 2, 2, 2, 4, 4, 4, 8, 8, 8};
constexpr int kDtypeF16 = 5, kDtypeBF16 = 6, kDtypeF32 = 9, kDtypeF64 = 10;

struct TensorInfo {
    std::string name;
    int dtype = 0;
    std::vector<long long> shape;
    long long offset = 0, bytes = 0, count = 1;
};

struct File {
    std::string path;
    int fd = -1;
    long long data_start = 0;
    std::map<std::string, TensorInfo> tensors;
    ~File() {
        if (fd >= 0) ::close(fd);
    }
};

int bad(const std::string& path, const std::string& what) { return fail(L0H_ERR_INVALID_DATA, "'" + path + "': " + what); }

const char* kind_name(Json::Kind k) {
    static const char* const names[] = {"null", "boolean", "number", "string", "array", "object"};
    return names[k];
}

bool is_count(const Json& j) { return j.kind == Json::Number && j.integral && j.ival >= 0; }

// Checks one header entry against the format: {"dtype": one of the 13 type names, "shape": a list
// of non-negative integers, "data_offsets": [begin, end] inside the data section with end - begin
// equal to the element count times the element size}. Returns "" and fills t, or what is wrong.
// A dtype the format does not define sets *unknown_dtype instead.
std::string check_entry(const std::string& name, const Json& e, long long data_len, TensorInfo& t,
                        std::string* unknown_dtype) {
    if (e.kind != Json::Object) return std::string("entry is a ") + kind_name(e.kind) + ", not an object";
    const Json* dt = member(e, "dtype");
    const Json* sh = member(e, "shape");
    const Json* off = member(e, "data_offsets");
    if (!dt || dt->kind != Json::String) return "\"dtype\" is missing or not a string";
    if (!sh || sh->kind != Json::Array) return "\"shape\" is missing or not a list";
    if (!off || off->kind != Json::Array || off->items.size() != 2 || !is_count(off->items[0]) ||
        !is_count(off->items[1]))
        return "\"data_offsets\" is not a pair of non-negative integers";
    t.name = name;
    t.dtype = -1;
    for (int i = 0; i < (int)(sizeof kDtypeSizes / sizeof kDtypeSizes[0]); i++)
        if (dt->str == kDtypeNames[i]) t.dtype = i;
    if (t.dtype < 0) {
        *unknown_dtype = dt->str;
        return "";
    }
    t.count = 1;
    for (const Json& d : sh->items) {
        if (!is_count(d)) return "a dimension of \"shape\" is not a non-negative integer";
        if (d.ival != 0 && t.count > INT64_MAX / d.ival) return "the element count does not fit 64 bits";
        t.count *= d.ival;
        t.shape.push_back(d.ival);
    }
    const long long begin = off->items[0].ival, end = off->items[1].ival;
    if (end < begin || end > data_len)
        return "bytes " + std::to_string(begin) + ".." + std::to_string(end) + " are not within the " +
               std::to_string(data_len) + "-byte data section";
    const int es = kDtypeSizes[t.dtype];
    if (t.count > INT64_MAX / es) return "the byte size does not fit 64 bits";
    if (end - begin != t.count * es)
        return std::to_string(t.count) + " x " + kDtypeNames[t.dtype] + " needs " + std::to_string(t.count * es) +
               " bytes; data_offsets give " + std::to_string(end - begin);
    t.offset = begin;
    t.bytes = end - begin;
    return "";
}

// Reads the 8-byte length prefix and the JSON header, then every entry; the data extents of the
// tensors must be pairwise disjoint (checked by one sweep in offset order).
int open_file(const std::string& path, std::unique_ptr<File>& out) {
    auto f = std::make_unique<File>();
    f->path = path;
    f->fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) return fail(L0H_ERR_INVALID_ARG, "cannot open '" + path + "': " + std::strerror(errno));
    struct stat sb;
    if (::fstat(f->fd, &sb) != 0) return fail(L0H_ERR_INVALID_ARG, "cannot stat '" + path + "'");
    const long long size = (long long)sb.st_size;
    if (size < 8) return bad(path, std::to_string(size) + " bytes is shorter than the 8-byte length prefix");
    unsigned char prefix[8];
    if (::pread(f->fd, prefix, 8, 0) != 8) return bad(path, "read error in the length prefix");
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | prefix[i];  // little-endian u64
    if (hlen > (uint64_t)kMaxHeaderBytes)
        return bad(path, "the length prefix announces " + std::to_string(hlen) + " header bytes (limit " +
                             std::to_string(kMaxHeaderBytes) + ")");
    if ((long long)hlen > size - 8)
        return bad(path, "the length prefix announces " + std::to_string(hlen) + " header bytes; only " +
                             std::to_string(size - 8) + " follow it");
    std::string header((size_t)hlen, '\0');
    if (hlen && ::pread(f->fd, &header[0], (size_t)hlen, 8) != (ssize_t)hlen) return bad(path, "read error in the header");
    f->data_start = 8 + (long long)hlen;
    const long long data_len = size - f->data_start;

    Json root;
    std::string jerr;
    if (!JsonParser(header.data(), header.size()).parse(root, jerr)) return bad(path, "header JSON: " + jerr);
    if (root.kind != Json::Object) return bad(path, std::string("the header is a JSON ") + kind_name(root.kind) + ", not an object");
    for (const auto& kv : root.members) {
        if (kv.first == "__metadata__") continue;
        TensorInfo t;
        std::string unknown;
        const std::string problem = check_entry(kv.first, kv.second, data_len, t, &unknown);
        if (!problem.empty()) return bad(path, "tensor '" + kv.first + "': " + problem);
        if (!unknown.empty())
            return fail(L0H_ERR_UNSUPPORTED, "'" + path + "': tensor '" + kv.first + "' has element type '" + unknown +
                                                 "', which safetensors does not define");
        if (!f->tensors.emplace(kv.first, std::move(t)).second)
            return bad(path, "the header declares '" + kv.first + "' twice");
    }
    std::vector<const TensorInfo*> by_offset;
    for (const auto& kv : f->tensors)
        if (kv.second.bytes > 0) by_offset.push_back(&kv.second);
    std::sort(by_offset.begin(), by_offset.end(), [](const TensorInfo* x, const TensorInfo* y) { return x->offset < y->offset; });
    long long covered = 0;  // end of the extents seen so far
    const TensorInfo* last = nullptr;
    for (const TensorInfo* t : by_offset) {
        if (last && t->offset < covered)
            return bad(path, "the data of '" + last->name + "' and '" + t->name + "' share bytes");
        covered = t->offset + t->bytes;
        last = t;
    }
    out = std::move(f);
    return L0H_OK;
}

}  // namespace
}  // namespace l0h

using namespace l0h;

struct l0h_safetensors {
    std::vector<std::unique_ptr<File>> files;
    std::vector<std::pair<std::string, const File*>> names;  // sorted by name
    const TensorInfo* find(const char* name, const File** owner) const {
        auto it = std::lower_bound(names.begin(), names.end(), std::string(name),
                                   [](const std::pair<std::string, const File*>& a, const std::string& b) { return a.first < b; });
        if (it == names.end() || it->first != name) return nullptr;
        if (owner) *owner = it->second;
        return &it->second->tensors.at(it->first);
    }
};

namespace {

bool is_dir(const std::string& p) {
    struct stat sb;
    return ::stat(p.c_str(), &sb) == 0 && S_ISDIR(sb.st_mode);
}
bool is_file(const std::string& p) {
    struct stat sb;
    return ::stat(p.c_str(), &sb) == 0 && S_ISREG(sb.st_mode);
}

int read_text(const std::string& path, std::string& out) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(L0H_ERR_INVALID_ARG, "cannot open '" + path + "'");
    char buf[65536];
    ssize_t n;
    while ((n = ::read(fd, buf, sizeof buf)) > 0) out.append(buf, (size_t)n);
    ::close(fd);
    return n < 0 ? fail(L0H_ERR_INVALID_DATA, "cannot read '" + path + "'") : L0H_OK;
}

}  // namespace

extern "C" {

int l0h_safetensors_open(const char* path, l0h_safetensors** out) {
    clear_error();
    L0H_CHECK_ARG(out, "out is null");
    *out = nullptr;
    L0H_CHECK_ARG(path && *path, "path is empty");
    auto ck = std::make_unique<l0h_safetensors>();
    std::string p = path;
    std::map<std::string, std::string> weight_map;  // name -> shard file (index only)
    std::vector<std::string> files;
    if (is_dir(p)) {
        const std::string index = p + "/model.safetensors.index.json";
        if (is_file(index)) {
            std::string text;
            int st = read_text(index, text);
            if (st) return st;
            Json root;
            std::string jerr;
            if (!JsonParser(text.data(), text.size()).parse(root, jerr) || root.kind != Json::Object)
                return fail(L0H_ERR_INVALID_DATA, "'" + index + "': not a JSON object");
            const Json* wm = member(root, "weight_map");
            if (!wm || wm->kind != Json::Object) return fail(L0H_ERR_INVALID_DATA, "'" + index + "': \"weight_map\" is missing or not an object");
            for (const auto& kv : wm->members) {
                const std::string& f = kv.second.str;
                if (kv.second.kind != Json::String || f.empty() || f.find('/') != std::string::npos || f == "." || f == "..")
                    return fail(L0H_ERR_INVALID_DATA, "'" + index + "': the shard of '" + kv.first + "' must be a file name in the same directory");
                weight_map[kv.first] = f;
                if (std::find(files.begin(), files.end(), f) == files.end()) files.push_back(f);
            }
            for (auto& f : files) f = p + "/" + f;
        } else if (is_file(p + "/model.safetensors")) {
            files.push_back(p + "/model.safetensors");
        } else {
            return fail(L0H_ERR_INVALID_ARG, "'" + p + "': no model.safetensors.index.json and no model.safetensors inside");
        }
    } else {
        files.push_back(p);
    }
    std::map<std::string, const File*> owner;
    for (const auto& fp : files) {
        std::unique_ptr<File> f;
        int st = open_file(fp, f);
        if (st) return st;
        for (const auto& kv : f->tensors)
            if (!owner.emplace(kv.first, f.get()).second)
                return fail(L0H_ERR_INVALID_DATA, "'" + kv.first + "' is stored in more than one shard");
        ck->files.push_back(std::move(f));
    }
    // The index and the shards must agree: every mapped tensor is in the shard it names.
    for (const auto& kv : weight_map) {
        auto it = owner.find(kv.first);
        if (it == owner.end() || it->second->path != p + "/" + kv.second)
            return fail(L0H_ERR_INVALID_DATA, "the index places '" + kv.first + "' in '" + kv.second + "', but that shard does not contain it");
    }
    for (const auto& kv : owner) ck->names.emplace_back(kv.first, kv.second);  // std::map: sorted
    *out = ck.release();
    return L0H_OK;
}

int l0h_safetensors_close(l0h_safetensors* st) {
    delete st;
    return L0H_OK;
}

int l0h_safetensors_count(const l0h_safetensors* st, int* count) {
    clear_error();
    L0H_CHECK_ARG(st && count, "null argument");
    *count = (int)st->names.size();
    return L0H_OK;
}

int l0h_safetensors_info(const l0h_safetensors* st, int index, char* name, size_t name_bytes, int* dtype, int* rank,
                         long long* shape, int max_rank) {
    clear_error();
    L0H_CHECK_ARG(st, "null argument");
    L0H_CHECK_ARG(index >= 0 && index < (int)st->names.size(), "tensor index out of range");
    const auto& e = st->names[(size_t)index];
    const TensorInfo& t = e.second->tensors.at(e.first);
    if (name) {
        L0H_CHECK_ARG(name_bytes > t.name.size(), "name buffer too small");
        std::memcpy(name, t.name.c_str(), t.name.size() + 1);
    }
    if (dtype) *dtype = t.dtype;
    if (rank) *rank = (int)t.shape.size();
    if (shape) {
        L0H_CHECK_ARG(max_rank >= (int)t.shape.size(), "shape buffer too small");
        for (size_t i = 0; i < t.shape.size(); i++) shape[i] = t.shape[i];
    }
    return L0H_OK;
}

int l0h_safetensors_find(const l0h_safetensors* st, const char* name, int* index) {
    clear_error();
    L0H_CHECK_ARG(st && name && index, "null argument");
    auto it = std::lower_bound(st->names.begin(), st->names.end(), std::string(name),
                               [](const std::pair<std::string, const File*>& a, const std::string& b) { return a.first < b; });
    *index = (it != st->names.end() && it->first == name) ? (int)(it - st->names.begin()) : -1;
    return L0H_OK;
}

int l0h_safetensors_read_f32(const l0h_safetensors* st, const char* name, float* dst, size_t count) {
    clear_error();
    L0H_CHECK_ARG(st && name && dst, "null argument");
    const File* f = nullptr;
    const TensorInfo* t = st->find(name, &f);
    if (!t) return fail(L0H_ERR_INVALID_ARG, std::string("no tensor named '") + name + "'");
    if ((long long)count != t->count)
        return fail(L0H_ERR_INVALID_ARG, "'" + t->name + "' holds " + std::to_string(t->count) +
                                             " values; the destination was sized for " + std::to_string(count));
    if (t->dtype != kDtypeF32 && t->dtype != kDtypeF16 && t->dtype != kDtypeBF16 && t->dtype != kDtypeF64)
        return fail(L0H_ERR_UNSUPPORTED, "'" + t->name + "' is stored as " + kDtypeNames[t->dtype] +
                                             ": only F32, F16, BF16 and F64 convert to fp32");
    const int es = kDtypeSizes[t->dtype];
    const size_t per = kChunkBytes / es;
    std::vector<unsigned char> buf(kChunkBytes);
    for (size_t done = 0; done < count;) {
        const size_t n = std::min(count - done, per), bytes = n * es;
        const off_t at = (off_t)(f->data_start + t->offset + (long long)(done * es));
        size_t got = 0;
        while (got < bytes) {
            const ssize_t r = ::pread(f->fd, buf.data() + got, bytes - got, at + (off_t)got);
            if (r <= 0) return fail(L0H_ERR_INVALID_DATA, "'" + f->path + "': read error in the data of '" + t->name + "'");
            got += (size_t)r;
        }
        float* d = dst + done;
        switch (t->dtype) {
        case kDtypeF32: std::memcpy(d, buf.data(), bytes); break;
        case kDtypeF16:
            for (size_t i = 0; i < n; i++) {
                uint16_t h;
                std::memcpy(&h, buf.data() + 2 * i, 2);
                d[i] = host_f16_to_f32(h);
            }
            break;
        case kDtypeBF16:
            for (size_t i = 0; i < n; i++) {
                uint16_t h;
                std::memcpy(&h, buf.data() + 2 * i, 2);
                const uint32_t bits = (uint32_t)h << 16;
                std::memcpy(&d[i], &bits, 4);
            }
            break;
        default:
            for (size_t i = 0; i < n; i++) {
                double v;
                std::memcpy(&v, buf.data() + 8 * i, 8);
                d[i] = (float)v;
            }
        }
        done += n;
    }
    return L0H_OK;
}

}  // extern "C"
