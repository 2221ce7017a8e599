// .pkl4 artifact reader and load-time layout derivation (host code).
//
// The artifact (artifact.rs:11-16, :98-157): a 24-byte prefix ("PKL4AOT\0",
// u32 schema version 2, u32 flags 0, u64 header length, little-endian), a JSON
// header, then the payload from the first 4096-byte boundary after the header;
// every tensor sits at a 256-byte aligned payload offset.  Linear weights are
// stored as fp16 [ceil128(N) x ceil128(K)] zero padded ("sm89_fp16_linear"),
// their biases as fp32 [ceil128(N)] ("sm89_fp32_bias"), everything else as
// plain fp16 / fp32.  open() applies the reference's header and layout checks
// (artifact.rs:514-650); derive() reads one linear, uploads it and packs it on
// the GPU into the FP8 / INT8 / INT4 layouts the GEMMs consume.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <cstdint>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "../../include/pk_linear.h"
#include "pk_kernels.hpp"

namespace pk {
namespace {

// ---- a strict JSON reader (RFC 8259 subset serde_json writes) ---------------------

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    std::string num;  // the number's text, kept exact
    std::string s;
    std::vector<Json> a;
    std::vector<std::pair<std::string, Json>> o;

    const Json* get(const char* key) const {
        for (const auto& kv : o)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class Parser {
  public:
    Parser(const char* p, size_t n) : p_(p), end_(p + n) {}
    bool parse(Json& out, std::string& err) {
        if (!value(out, 0)) {
            err = err_;
            return false;
        }
        ws();
        if (p_ != end_) {
            err = "trailing bytes after the JSON header";
            return false;
        }
        return true;
    }

  private:
    const char* p_;
    const char* end_;
    std::string err_;

    bool fail(const char* m) {
        if (err_.empty()) err_ = m;
        return false;
    }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if ((size_t)(end_ - p_) < n || memcmp(p_, w, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(uint32_t c, std::string& s) {
        if (c < 0x80) {
            s += (char)c;
        } else if (c < 0x800) {
            s += (char)(0xc0 | (c >> 6));
            s += (char)(0x80 | (c & 0x3f));
        } else if (c < 0x10000) {
            s += (char)(0xe0 | (c >> 12));
            s += (char)(0x80 | ((c >> 6) & 0x3f));
            s += (char)(0x80 | (c & 0x3f));
        } else {
            s += (char)(0xf0 | (c >> 18));
            s += (char)(0x80 | ((c >> 12) & 0x3f));
            s += (char)(0x80 | ((c >> 6) & 0x3f));
            s += (char)(0x80 | (c & 0x3f));
        }
    }
    bool hex4(uint32_t& v) {
        if (end_ - p_ < 4) return fail("truncated \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string& s) {
        if (p_ >= end_ || *p_ != '"') return fail("expected a string");
        ++p_;
        while (true) {
            if (p_ >= end_) return fail("unterminated string");
            const unsigned char c = (unsigned char)*p_++;
            if (c == '"') return true;
            if (c < 0x20) return fail("control character in string");
            if (c != '\\') {
                s += (char)c;
                continue;
            }
            if (p_ >= end_) return fail("unterminated escape");
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
                uint32_t c1;
                if (!hex4(c1)) return false;
                if (c1 >= 0xd800 && c1 < 0xdc00) {
                    uint32_t c2;
                    if (!lit("\\u") || !hex4(c2) || c2 < 0xdc00 || c2 >= 0xe000) return fail("bad surrogate pair");
                    c1 = 0x10000 + ((c1 - 0xd800) << 10) + (c2 - 0xdc00);
                } else if (c1 >= 0xdc00 && c1 < 0xe000) {
                    return fail("lone low surrogate");
                }
                utf8(c1, s);
                break;
            }
            default: return fail("bad escape");
            }
        }
    }
    bool number(std::string& t) {
        const char* b = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad number");
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' || *p_ == '-')) ++p_;
        t.assign(b, p_);
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) return fail("JSON nested too deeply");
        ws();
        if (p_ >= end_) return fail("unexpected end of JSON");
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Json::Object;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            while (true) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
                ++p_;
                Json item;
                if (!value(item, depth + 1)) return false;
                v.o.emplace_back(std::move(key), std::move(item));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = Json::Array;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            while (true) {
                Json item;
                if (!value(item, depth + 1)) return false;
                v.a.push_back(std::move(item));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Json::String;
            return string(v.s);
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
        v.kind = Json::Number;
        return number(v.num);
    }
};

// ---- the artifact -------------------------------------------------------------------

constexpr char kMagic[8] = {'P', 'K', 'L', '4', 'A', 'O', 'T', '\0'};
constexpr uint32_t kSchemaVersion = 2;
constexpr uint64_t kPrefixBytes = 24;
constexpr uint64_t kHeaderAlignment = 4096;
constexpr uint64_t kTensorAlignment = 256;
constexpr uint64_t kMaxHeaderBytes = 128ull * 1024 * 1024;

struct Profile {
    const char* json;
    const char* repository;
    const char* revision;
    size_t blank;
};
// config.rs:7-10, :41-46
const Profile kProfiles[2] = {
    {"v2_english", "nvidia/parakeet-tdt-0.6b-v2", "ae9ad07059c7c739ffaf932226a8fe64ae2620b0", 1024},
    {"v3_multilingual", "nvidia/parakeet-tdt-0.6b-v3", "541d1f99c6b0c3cd0b11a95167540bb8edefd82b", 8192},
};

struct Tensor {
    std::string name;
    int storage = 0;
    std::vector<uint64_t> logical, physical;
    uint64_t offset = 0, bytes = 0;
};

bool align_up(uint64_t v, uint64_t a, uint64_t& out) {
    if (v > UINT64_MAX - (a - 1)) return false;
    out = (v + a - 1) / a * a;
    return true;
}

bool as_u64(const Json* j, uint64_t& out) {
    if (!j || j->kind != Json::Number || j->num.empty()) return false;
    uint64_t v = 0;
    for (char c : j->num) {
        if (c < '0' || c > '9') return false;  // non-negative integers only
        if (v > (UINT64_MAX - (uint64_t)(c - '0')) / 10) return false;
        v = v * 10 + (uint64_t)(c - '0');
    }
    out = v;
    return true;
}

bool as_str(const Json* j, std::string& out) {
    if (!j || j->kind != Json::String) return false;
    out = j->s;
    return true;
}

bool as_shape(const Json* j, std::vector<uint64_t>& out) {
    if (!j || j->kind != Json::Array) return false;
    out.clear();
    for (const auto& d : j->a) {
        uint64_t v;
        if (!as_u64(&d, v)) return false;
        out.push_back(v);
    }
    return true;
}

}  // namespace

struct Artifact {
    std::string path;
    uint64_t file_bytes = 0, data_start = 0, payload_bytes = 0, source_payload_bytes = 0;
    int profile = -1;
    std::string target, precision_plan;
    std::vector<std::string> vocabulary;
    std::vector<Tensor> tensors;
};

namespace {

// artifact.rs:20-33 storage names (serde snake_case) and element sizes.
int storage_code(const std::string& s) {
    if (s == "fp16") return PK_STORAGE_FP16;
    if (s == "fp32") return PK_STORAGE_FP32;
    if (s == "sm89_fp16_linear") return PK_STORAGE_FP16_LINEAR;
    if (s == "sm89_fp32_bias") return PK_STORAGE_FP32_BIAS;
    return -1;
}
uint64_t element_bytes(int storage) { return (storage == PK_STORAGE_FP16 || storage == PK_STORAGE_FP16_LINEAR) ? 2 : 4; }

int invalid(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    set_error("invalid L4 artifact: %s", buf);
    return PK_E_FORMAT;
}

// artifact.rs:614-650
int validate_layout(const Tensor& t) {
    auto a128 = [](uint64_t d, uint64_t& out) { return align_up(d, 128, out); };
    switch (t.storage) {
    case PK_STORAGE_FP16:
    case PK_STORAGE_FP32:
        if (t.physical != t.logical) return invalid("%s: plain storage cannot change its logical shape", t.name.c_str());
        return PK_OK;
    case PK_STORAGE_FP16_LINEAR: {
        uint64_t o, i;
        if (t.logical.size() != 2 || t.logical[0] == 0 || t.logical[1] == 0 || !a128(t.logical[0], o) || !a128(t.logical[1], i) ||
            t.physical.size() != 2 || t.physical[0] != o || t.physical[1] != i)
            return invalid("%s: invalid sm_89 FP16 linear shapes", t.name.c_str());
        return PK_OK;
    }
    default: {
        uint64_t o;
        if (t.logical.size() != 1 || t.logical[0] == 0 || !a128(t.logical[0], o) || t.physical.size() != 1 || t.physical[0] != o)
            return invalid("%s: invalid sm_89 FP32 bias shapes", t.name.c_str());
        return PK_OK;
    }
    }
}

// artifact.rs:514-592 (header), :594-612 (vocabulary)
int validate_header(const Json& h, Artifact& a, uint64_t payload_bytes) {
    uint64_t schema, alignment;
    std::string profile, repository, revision;
    if (!as_u64(h.get("schema_version"), schema)) return invalid("header has no schema_version");
    if (schema != kSchemaVersion) return invalid("header schema is %llu, expected %u", (unsigned long long)schema, kSchemaVersion);
    if (!as_str(h.get("target"), a.target)) return invalid("header has no target");
    if (a.target != "sm_89") return invalid("target is \"%s\", expected sm_89", a.target.c_str());
    if (!as_str(h.get("profile"), profile) || !as_str(h.get("source_repository"), repository) ||
        !as_str(h.get("source_revision"), revision))
        return invalid("header has no profile / source repository / revision");
    a.profile = -1;
    for (int i = 0; i < 2; ++i)
        if (profile == kProfiles[i].json) a.profile = i;
    if (a.profile < 0) return invalid("unknown profile \"%s\"", profile.c_str());
    if (repository != kProfiles[a.profile].repository || revision != kProfiles[a.profile].revision)
        return invalid("profile does not match source repository and revision");
    if (!as_u64(h.get("source_payload_bytes"), a.source_payload_bytes)) return invalid("header has no source_payload_bytes");
    if (!as_str(h.get("precision_plan"), a.precision_plan)) return invalid("header has no precision_plan");
    if (!as_u64(h.get("tensor_alignment"), alignment)) return invalid("header has no tensor_alignment");
    if (alignment != kTensorAlignment) return invalid("tensor alignment is %llu, expected 256", (unsigned long long)alignment);
    if (!as_u64(h.get("payload_bytes"), a.payload_bytes)) return invalid("header has no payload_bytes");
    if (a.payload_bytes != payload_bytes)
        return invalid("header declares %llu payload bytes, file contains %llu", (unsigned long long)a.payload_bytes,
                       (unsigned long long)payload_bytes);
    const Json* vocab = h.get("vocabulary");
    if (!vocab || vocab->kind != Json::Array) return invalid("header has no vocabulary");
    if (vocab->a.size() != kProfiles[a.profile].blank)
        return invalid("%s requires %zu vocabulary entries before the blank token, got %zu", profile.c_str(),
                       kProfiles[a.profile].blank, vocab->a.size());
    a.vocabulary.clear();
    for (size_t i = 0; i < vocab->a.size(); ++i) {
        std::string piece;
        if (!as_str(&vocab->a[i], piece)) return invalid("vocabulary entry %zu is not a string", i);
        if (piece.empty() || piece.find_first_of("\n\r\t") != std::string::npos)
            return invalid("vocabulary entry %zu is empty or contains control separators", i);
        a.vocabulary.push_back(std::move(piece));
    }
    const Json* tensors = h.get("tensors");
    if (!tensors || tensors->kind != Json::Array) return invalid("header has no tensors");
    std::set<std::string> names;
    uint64_t cursor = 0;
    a.tensors.clear();
    for (const auto& tj : tensors->a) {
        Tensor t;
        std::string storage;
        if (tj.kind != Json::Object || !as_str(tj.get("name"), t.name) || !as_str(tj.get("storage"), storage) ||
            !as_shape(tj.get("logical_shape"), t.logical) || !as_shape(tj.get("physical_shape"), t.physical) ||
            !as_u64(tj.get("offset"), t.offset) || !as_u64(tj.get("bytes"), t.bytes))
            return invalid("malformed tensor entry %zu", a.tensors.size());
        t.storage = storage_code(storage);
        if (t.storage < 0) return invalid("%s: unknown storage \"%s\"", t.name.c_str(), storage.c_str());
        if (t.name.empty() || !names.insert(t.name).second) return invalid("empty or duplicate tensor name \"%s\"", t.name.c_str());
        if (t.offset % kTensorAlignment != 0 || t.offset < cursor)
            return invalid("%s: invalid aligned offset %llu after %llu", t.name.c_str(), (unsigned long long)t.offset,
                           (unsigned long long)cursor);
        const int st = validate_layout(t);
        if (st != PK_OK) return st;
        uint64_t elements = 1;
        for (uint64_t d : t.physical) {
            if (d != 0 && elements > UINT64_MAX / d) return invalid("%s: element count overflow", t.name.c_str());
            elements *= d;
        }
        const uint64_t eb = element_bytes(t.storage);
        if (elements > UINT64_MAX / eb) return invalid("%s: byte count overflow", t.name.c_str());
        if (t.bytes != elements * eb)
            return invalid("%s: physical shape and storage require %llu bytes, header declares %llu", t.name.c_str(),
                           (unsigned long long)(elements * eb), (unsigned long long)t.bytes);
        if (t.offset > UINT64_MAX - t.bytes) return invalid("%s: range overflow", t.name.c_str());
        cursor = t.offset + t.bytes;
        if (cursor > payload_bytes)
            return invalid("%s: range ends at %llu, beyond %llu-byte payload", t.name.c_str(), (unsigned long long)cursor,
                           (unsigned long long)payload_bytes);
        a.tensors.push_back(std::move(t));
    }
    if (cursor != payload_bytes)
        return invalid("last tensor ends at %llu, payload ends at %llu", (unsigned long long)cursor, (unsigned long long)payload_bytes);
    return PK_OK;
}

uint32_t le32(const unsigned char* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
uint64_t le64(const unsigned char* p) { return (uint64_t)le32(p) | ((uint64_t)le32(p + 4) << 32); }

struct FileCloser {
    void operator()(FILE* f) const {
        if (f) fclose(f);
    }
};

}  // namespace

// artifact.rs:98-157 AotArtifactIndex::open
int artifact_open(const char* path, Artifact** out) {
    *out = nullptr;
    std::unique_ptr<FILE, FileCloser> f(fopen(path, "rb"));
    if (!f) {
        set_error("failed to open %s", path);
        return PK_E_IO;
    }
    if (fseeko(f.get(), 0, SEEK_END) != 0) {
        set_error("failed to seek %s", path);
        return PK_E_IO;
    }
    const uint64_t file_bytes = (uint64_t)ftello(f.get());
    rewind(f.get());
    if (file_bytes < kPrefixBytes) return invalid("file has %llu bytes; prefix requires 24", (unsigned long long)file_bytes);
    unsigned char prefix[kPrefixBytes];
    if (fread(prefix, 1, kPrefixBytes, f.get()) != kPrefixBytes) {
        set_error("failed to read the prefix of %s", path);
        return PK_E_IO;
    }
    if (memcmp(prefix, kMagic, 8) != 0) return invalid("bad magic");
    const uint32_t version = le32(prefix + 8), flags = le32(prefix + 12);
    const uint64_t header_bytes = le64(prefix + 16);
    if (version != kSchemaVersion) return invalid("expected schema version 2, got %u", version);
    if (flags != 0) return invalid("unsupported prefix flags %#x", flags);
    if (header_bytes == 0 || header_bytes > kMaxHeaderBytes)
        return invalid("header length %llu is outside 1..=%llu", (unsigned long long)header_bytes, (unsigned long long)kMaxHeaderBytes);
    uint64_t data_start;
    if (!align_up(kPrefixBytes + header_bytes, kHeaderAlignment, data_start)) return invalid("header offset overflow");
    if (data_start > file_bytes)
        return invalid("aligned header ends at %llu, beyond file length %llu", (unsigned long long)data_start,
                       (unsigned long long)file_bytes);
    std::vector<char> text(header_bytes);
    if (fread(text.data(), 1, header_bytes, f.get()) != header_bytes) {
        set_error("failed to read the header of %s", path);
        return PK_E_IO;
    }
    Json h;
    std::string err;
    Parser parser(text.data(), text.size());
    if (!parser.parse(h, err)) return invalid("header JSON: %s", err.c_str());
    if (h.kind != Json::Object) return invalid("header is not a JSON object");
    std::unique_ptr<Artifact> a(new Artifact);
    a->path = path;
    a->file_bytes = file_bytes;
    a->data_start = data_start;
    const int st = validate_header(h, *a, file_bytes - data_start);
    if (st != PK_OK) return st;
    *out = a.release();
    return PK_OK;
}

int artifact_read(const Artifact& a, const Tensor& t, void* dst, uint64_t capacity) {
    if (capacity < t.bytes) {
        set_error("%s needs %llu bytes, the buffer holds %llu", t.name.c_str(), (unsigned long long)t.bytes,
                  (unsigned long long)capacity);
        return PK_E_SHAPE;
    }
    std::unique_ptr<FILE, FileCloser> f(fopen(a.path.c_str(), "rb"));
    if (!f || fseeko(f.get(), (off_t)(a.data_start + t.offset), SEEK_SET) != 0 || fread(dst, 1, t.bytes, f.get()) != t.bytes) {
        set_error("failed to read %s from %s", t.name.c_str(), a.path.c_str());
        return PK_E_IO;
    }
    return PK_OK;
}

}  // namespace pk

using pk::Artifact;

extern "C" {

int32_t pk_artifact_open(const char* path, pk_artifact** out) {
    if (!path || !out) {
        pk::set_error("path and out are required");
        return PK_E_ARG;
    }
    Artifact* a = nullptr;
    const int st = pk::artifact_open(path, &a);
    *out = reinterpret_cast<pk_artifact*>(a);
    return st;
}

void pk_artifact_close(pk_artifact* artifact) { delete reinterpret_cast<Artifact*>(artifact); }

int32_t pk_artifact_info(const pk_artifact* artifact, pk_artifact_summary* out) {
    const Artifact* a = reinterpret_cast<const Artifact*>(artifact);
    if (!a || !out) {
        pk::set_error("artifact and out are required");
        return PK_E_ARG;
    }
    out->profile = a->profile;
    out->blank_token_id = (int32_t)pk::kProfiles[a->profile].blank;
    out->tensor_count = (int32_t)a->tensors.size();
    out->vocabulary_size = (int32_t)a->vocabulary.size();
    out->data_start = a->data_start;
    out->payload_bytes = a->payload_bytes;
    out->file_bytes = a->file_bytes;
    return PK_OK;
}

int32_t pk_artifact_tensor(const pk_artifact* artifact, int32_t index, pk_tensor_info* out) {
    const Artifact* a = reinterpret_cast<const Artifact*>(artifact);
    if (!a || !out) {
        pk::set_error("artifact and out are required");
        return PK_E_ARG;
    }
    if (index < 0 || (size_t)index >= a->tensors.size()) {
        pk::set_error("tensor index %d outside 0..%zu", index, a->tensors.size());
        return PK_E_ARG;
    }
    const pk::Tensor& t = a->tensors[index];
    memset(out, 0, sizeof *out);
    out->name = t.name.c_str();
    out->storage = t.storage;
    out->rank = (int32_t)t.logical.size();
    for (size_t i = 0; i < t.logical.size() && i < 4; ++i) out->logical_shape[i] = t.logical[i];
    for (size_t i = 0; i < t.physical.size() && i < 4; ++i) out->physical_shape[i] = t.physical[i];
    out->offset = t.offset;
    out->bytes = t.bytes;
    return PK_OK;
}

int32_t pk_artifact_find(const pk_artifact* artifact, const char* name) {
    const Artifact* a = reinterpret_cast<const Artifact*>(artifact);
    if (!a || !name) {
        pk::set_error("artifact and name are required");
        return PK_E_ARG;
    }
    for (size_t i = 0; i < a->tensors.size(); ++i)
        if (a->tensors[i].name == name) return (int32_t)i;
    pk::set_error("missing tensor %s", name);
    return PK_E_ARG;
}

const char* pk_artifact_vocabulary(const pk_artifact* artifact, int32_t index) {
    const Artifact* a = reinterpret_cast<const Artifact*>(artifact);
    if (!a || index < 0 || (size_t)index >= a->vocabulary.size()) return nullptr;
    return a->vocabulary[index].c_str();
}

int32_t pk_artifact_read(const pk_artifact* artifact, int32_t index, void* host_dst, uint64_t capacity) {
    const Artifact* a = reinterpret_cast<const Artifact*>(artifact);
    if (!a || !host_dst || index < 0 || (size_t)index >= a->tensors.size()) {
        pk::set_error("artifact, a tensor index and a destination are required");
        return PK_E_ARG;
    }
    return pk::artifact_read(*a, a->tensors[index], host_dst, capacity);
}

int32_t pk_artifact_derive_linear(const pk_artifact* artifact, int32_t index, int32_t format, void* host_staging,
                                  uint64_t staging_bytes, uint16_t* device_fp16, void* packed, void* scales, uint16_t* zeros,
                                  void* stream) {
    const Artifact* a = reinterpret_cast<const Artifact*>(artifact);
    if (!a || index < 0 || (size_t)index >= a->tensors.size() || !host_staging || !device_fp16) {
        pk::set_error("artifact, a tensor index, host staging and a device fp16 buffer are required");
        return PK_E_ARG;
    }
    const pk::Tensor& t = a->tensors[index];
    if (t.storage != PK_STORAGE_FP16_LINEAR) {
        pk::set_error("%s is not an sm89_fp16_linear tensor", t.name.c_str());
        return PK_E_ARG;
    }
    if (t.physical[0] > INT32_MAX || t.physical[1] > INT32_MAX) {
        pk::set_error("%s: shape exceeds the packers' int32 sizes", t.name.c_str());
        return PK_E_SHAPE;
    }
    const int32_t n = (int32_t)t.physical[0], k = (int32_t)t.physical[1];
    if (format != PK_DERIVE_FP16 && !packed) {
        pk::set_error("packed output required");
        return PK_E_ARG;
    }
    int st = pk::artifact_read(*a, t, host_staging, staging_bytes);
    if (st != PK_OK) return st;
    const hipError_t e = hipMemcpyAsync(device_fp16, host_staging, t.bytes, hipMemcpyHostToDevice, (hipStream_t)stream);
    if (e != hipSuccess) {
        pk::set_error("upload of %s failed: %s", t.name.c_str(), hipGetErrorString(e));
        return PK_E_LAUNCH;
    }
    switch (format) {
    case PK_DERIVE_FP16: return PK_OK;
    case PK_DERIVE_FP8_ROWS: return pk_pack_fp8_rows(device_fp16, n, k, (uint8_t*)packed, (float*)scales, stream);
    case PK_DERIVE_INT8_ROWS: return pk_pack_int8_rows(device_fp16, n, k, (int8_t*)packed, (float*)scales, stream);
    case PK_DERIVE_INT4_ROWS: return pk_pack_int4_rows(device_fp16, n, k, (uint8_t*)packed, (float*)scales, stream);
    case PK_DERIVE_INT4_G128: return pk_pack_int4_g128(device_fp16, n, k, (uint32_t*)packed, (uint16_t*)scales, zeros, stream);
    default:
        pk::set_error("unknown derived format %d", format);
        return PK_E_ARG;
    }
}

}  // extern "C"
