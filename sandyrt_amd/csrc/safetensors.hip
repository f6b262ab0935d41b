// safetensors.hip -- safetensors weight files: header parsing and the upload
// of every tensor to device memory (host code only).
//
// Format and semantics follow the reference loader (src/weight/
// SafeTensorWeights.cpp:44-117): an 8-byte little-endian header length, a
// JSON object mapping tensor names to {dtype, shape, data_offsets} (plus an
// optional "__metadata__" entry, skipped), then the raw data section;
// dtypes F32, F16, BF16, I32, I64, U8/BOOL.  Tensors are listed in name
// order, the iteration order of the reference's parsed JSON object.
//
// The reference reads the whole file into a host vector and uploads tensor
// by tensor from pageable memory.  Here the file is never held whole: the
// upload streams it through two pinned staging buffers (hipHostMalloc), so
// the read of chunk n + 1 overlaps the DMA of chunk n, and every tensor lands
// at a 256-byte-aligned offset of one device arena (the kernels' 128-bit
// paths need 16-byte alignment; safetensors offsets guarantee none).
#include "common.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace sandy_hip {
namespace {

// ---------------------------------------------------------------- JSON subset
// Values of a safetensors header: objects, arrays, strings, numbers, true /
// false / null.  Numbers are kept as text; only non-negative integers are
// interpreted (shapes and offsets).
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    std::string text;                                  // string value or number text
    std::vector<Json> items;                           // array elements
    std::vector<std::pair<std::string, Json>> fields;  // object members in file order
};

struct Parser {
    const char* p;
    const char* end;
    std::string error;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool fail(const char* msg) {
        if (error.empty()) error = msg;
        return false;
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
        if (end - p < 4) return fail("truncated \\u escape");
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string& out) {
        if (p >= end || *p != '"') return fail("expected a string");
        p++;
        while (p < end && *p != '"') {
            const char c = *p++;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p >= end) return fail("truncated escape");
            const char e = *p++;
            switch (e) {
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
                    if (v >= 0xD800 && v < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        uint32_t lo;
                        if (!hex4(lo)) return false;
                        v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(out, v);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool literal(const char* word, Json::Kind kind, Json& v) {
        const size_t n = std::strlen(word);
        if (static_cast<size_t>(end - p) < n || std::strncmp(p, word, n) != 0) return fail("bad literal");
        p += n;
        v.kind = kind;
        v.text = word;
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end of header");
        const char c = *p;
        if (c == '{') {
            v.kind = Json::Object;
            p++;
            ws();
            if (p < end && *p == '}') {
                p++;
                return true;
            }
            while (true) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p >= end || *p != ':') return fail("expected ':'");
                p++;
                Json item;
                if (!value(item, depth + 1)) return false;
                v.fields.emplace_back(std::move(key), std::move(item));
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == '}') {
                    p++;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = Json::Array;
            p++;
            ws();
            if (p < end && *p == ']') {
                p++;
                return true;
            }
            while (true) {
                Json item;
                if (!value(item, depth + 1)) return false;
                v.items.push_back(std::move(item));
                ws();
                if (p < end && *p == ',') {
                    p++;
                    continue;
                }
                if (p < end && *p == ']') {
                    p++;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Json::String;
            return string(v.text);
        }
        if (c == 't') return literal("true", Json::Bool, v);
        if (c == 'f') return literal("false", Json::Bool, v);
        if (c == 'n') return literal("null", Json::Null, v);
        if (c == '-' || (c >= '0' && c <= '9')) {
            v.kind = Json::Number;
            const char* s = p;
            while (p < end && (std::strchr("+-.eE", *p) || (*p >= '0' && *p <= '9'))) p++;
            v.text.assign(s, p);
            return true;
        }
        return fail("unexpected character in header");
    }
};

bool to_u64(const Json& v, uint64_t& out) {
    if (v.kind != Json::Number || v.text.empty()) return false;
    uint64_t r = 0;
    for (char c : v.text) {
        if (c < '0' || c > '9') return false;
        const uint64_t d = static_cast<uint64_t>(c - '0');
        if (r > (UINT64_MAX - d) / 10) return false;
        r = r * 10 + d;
    }
    out = r;
    return true;
}

// SafeTensorWeights.cpp:14-23 parse_dtype
bool parse_dtype(const std::string& s, int32_t& dt) {
    if (s == "F32") dt = SANDY_F32;
    else if (s == "F16") dt = SANDY_F16;
    else if (s == "BF16") dt = SANDY_BF16;
    else if (s == "I32") dt = SANDY_I32;
    else if (s == "I64") dt = SANDY_I64;
    else if (s == "U8" || s == "BOOL") dt = SANDY_U8;
    else return false;
    return true;
}

constexpr uint64_t kArenaAlign = 256;
constexpr size_t kStageBytes = 32u << 20;  // per pinned staging buffer

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

struct SandySafetensors {
    std::string path;
    int fd = -1;
    uint64_t file_size = 0;
    uint64_t data_offset = 0;  // 8 + header length
    std::vector<SandySafetensorInfo> tensors;  // name order
    std::map<std::string, size_t> index;
    uint64_t arena_bytes = 0;
};

extern "C" {

int sandy_hip_safetensors_open(const char* path, SandySafetensors** out, char* err, size_t err_cap) {
    Err e{err, err_cap};
    if (!path || !out) return fail(e, SANDY_ERR_INVALID, "safetensors open needs a path and an output handle");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(e, SANDY_ERR_INVALID, "cannot open %s", path);
    std::unique_ptr<SandySafetensors> h(new SandySafetensors());
    h->path = path;
    h->fd = fd;
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        return fail(e, SANDY_ERR_INVALID, "cannot open %s", path);
    }
    h->file_size = static_cast<uint64_t>(st.st_size);
    auto close_fail = [&](const char* fmt, const char* arg) {
        ::close(h->fd);
        h->fd = -1;
        return fail(e, SANDY_ERR_INVALID, fmt, arg);
    };
    if (h->file_size < 8) return close_fail("%s", "safetensors file too small");
    uint64_t header_len = 0;
    if (pread(fd, &header_len, 8, 0) != 8) return close_fail("%s", "safetensors file too small");
    if (header_len > h->file_size - 8) return close_fail("%s", "safetensors header size exceeds file");
    h->data_offset = 8 + header_len;
    std::string header(header_len, '\0');
    uint64_t got = 0;
    while (got < header_len) {
        const ssize_t n = pread(fd, &header[got], header_len - got, static_cast<off_t>(8 + got));
        if (n <= 0) return close_fail("%s", "safetensors header read failed");
        got += static_cast<uint64_t>(n);
    }
    Parser ps{header.data(), header.data() + header.size(), {}};
    Json root;
    if (!ps.value(root, 0)) return close_fail("safetensors header is not valid JSON: %s", ps.error.c_str());
    ps.ws();
    if (root.kind != Json::Object) return close_fail("%s", "safetensors header must be a JSON object");
    const uint64_t data_bytes = h->file_size - h->data_offset;
    for (auto& kv : root.fields) {
        if (kv.first == "__metadata__") continue;
        const Json& v = kv.second;
        const Json *dt = nullptr, *shape = nullptr, *offs = nullptr;
        if (v.kind == Json::Object)
            for (auto& f : v.fields) {
                if (f.first == "dtype") dt = &f.second;
                else if (f.first == "shape") shape = &f.second;
                else if (f.first == "data_offsets") offs = &f.second;
            }
        if (!dt || dt->kind != Json::String || !shape || shape->kind != Json::Array || !offs ||
            offs->kind != Json::Array || offs->items.size() != 2)
            return close_fail("safetensors entry %s lacks dtype, shape or data_offsets", kv.first.c_str());
        SandySafetensorInfo info{};
        if (kv.first.size() >= sizeof(info.name))
            return close_fail("safetensors tensor name too long: %s", kv.first.c_str());
        std::memcpy(info.name, kv.first.c_str(), kv.first.size() + 1);
        if (!parse_dtype(dt->text, info.dtype))
            return close_fail("unsupported safetensors dtype: %s", dt->text.c_str());
        if (shape->items.size() > SANDY_HIP_MAX_RANK)
            return close_fail("safetensors tensor %s rank too large", kv.first.c_str());
        info.rank = static_cast<int32_t>(shape->items.size());
        uint64_t elems = 1;
        for (size_t i = 0; i < shape->items.size(); i++) {
            uint64_t d;
            if (!to_u64(shape->items[i], d)) return close_fail("safetensors tensor %s has a bad shape", kv.first.c_str());
            info.dims[i] = static_cast<int64_t>(d);
            elems *= d;
        }
        uint64_t b, en;
        if (!to_u64(offs->items[0], b) || !to_u64(offs->items[1], en) || en < b || en > data_bytes)
            return close_fail("safetensors tensor %s data_offsets outside the data section", kv.first.c_str());
        info.file_offset = b;
        info.nbytes = en - b;
        if (info.nbytes != elems * dtype_size(info.dtype))
            return close_fail("safetensors tensor %s size does not match its shape", kv.first.c_str());
        h->tensors.push_back(info);
    }
    std::sort(h->tensors.begin(), h->tensors.end(),
              [](const SandySafetensorInfo& a, const SandySafetensorInfo& b) { return std::strcmp(a.name, b.name) < 0; });
    uint64_t at = 0;
    for (size_t i = 0; i < h->tensors.size(); i++) {
        if (!h->index.emplace(h->tensors[i].name, i).second)
            return close_fail("safetensors tensor %s appears twice", h->tensors[i].name);
        h->tensors[i].arena_offset = at;
        at += (h->tensors[i].nbytes + kArenaAlign - 1) / kArenaAlign * kArenaAlign;
    }
    h->arena_bytes = at;
    *out = h.release();
    return ok(e);
}

void sandy_hip_safetensors_close(SandySafetensors* h) {
    if (!h) return;
    if (h->fd >= 0) ::close(h->fd);
    delete h;
}

int64_t sandy_hip_safetensors_count(const SandySafetensors* h) {
    return h ? static_cast<int64_t>(h->tensors.size()) : -1;
}

uint64_t sandy_hip_safetensors_arena_bytes(const SandySafetensors* h) { return h ? h->arena_bytes : 0; }

int sandy_hip_safetensors_info(const SandySafetensors* h, int64_t i, SandySafetensorInfo* info, char* err,
                               size_t err_cap) {
    Err e{err, err_cap};
    if (!h || !info || i < 0 || i >= static_cast<int64_t>(h->tensors.size()))
        return fail(e, SANDY_ERR_INVALID, "safetensors tensor index out of range");
    *info = h->tensors[static_cast<size_t>(i)];
    return ok(e);
}

int64_t sandy_hip_safetensors_find(const SandySafetensors* h, const char* name) {
    if (!h || !name) return -1;
    auto it = h->index.find(name);
    return it == h->index.end() ? -1 : static_cast<int64_t>(it->second);
}

// Streams the data section through two pinned buffers into the arena: chunk
// c is read from the file while chunk c - 1's copies run; a staging buffer is
// refilled only after the event recorded behind its copies has completed.
int sandy_hip_safetensors_upload(SandySafetensors* h, void* arena, uint64_t arena_bytes, void* stream_, char* err,
                                 size_t err_cap) {
    Err e{err, err_cap};
    if (!h || !arena) return fail(e, SANDY_ERR_INVALID, "safetensors upload needs a handle and a device arena");
    if (arena_bytes < h->arena_bytes)
        return fail(e, SANDY_ERR_INVALID, "safetensors arena too small: %llu < %llu bytes",
                    static_cast<unsigned long long>(arena_bytes), static_cast<unsigned long long>(h->arena_bytes));
    if (reinterpret_cast<uintptr_t>(arena) % kArenaAlign)
        return fail(e, SANDY_ERR_INVALID, "safetensors arena must be %llu-byte aligned",
                    static_cast<unsigned long long>(kArenaAlign));
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    // tensors in file order: one pass over the data section
    std::vector<const SandySafetensorInfo*> order;
    for (auto& t : h->tensors) order.push_back(&t);
    std::sort(order.begin(), order.end(),
              [](const SandySafetensorInfo* a, const SandySafetensorInfo* b) { return a->file_offset < b->file_offset; });
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    auto cleanup = [&]() {
        for (int i = 0; i < 2; i++) {
            if (done[i]) {
                hipEventSynchronize(done[i]);
                hipEventDestroy(done[i]);
            }
            if (stage[i]) hipHostFree(stage[i]);
        }
    };
    for (int i = 0; i < 2; i++) {
        hipError_t st = hipHostMalloc(&stage[i], kStageBytes, hipHostMallocDefault);
        if (st == hipSuccess) st = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
        if (st != hipSuccess) {
            cleanup();
            return fail(e, SANDY_ERR_HIP, "safetensors staging: %s", hipGetErrorString(st));
        }
    }
    bool used[2] = {false, false};
    size_t ti = 0;
    uint64_t t_done = 0;  // bytes of order[ti] already copied
    int buf = 0;
    while (ti < order.size()) {
        if (used[buf]) {
            hipError_t st = hipEventSynchronize(done[buf]);
            if (st != hipSuccess) {
                cleanup();
                return fail(e, SANDY_ERR_HIP, "safetensors upload: %s", hipGetErrorString(st));
            }
        }
        // fill the staging buffer with the next run of tensor bytes (file order,
        // contiguous in the file up to gaps between tensors)
        char* s = static_cast<char*>(stage[buf]);
        size_t fill = 0;
        struct Piece { uint64_t dev; size_t at; size_t n; };
        std::vector<Piece> pieces;
        while (ti < order.size() && fill < kStageBytes) {
            const SandySafetensorInfo* t = order[ti];
            const size_t n = static_cast<size_t>(std::min<uint64_t>(t->nbytes - t_done, kStageBytes - fill));
            size_t got = 0;
            while (got < n) {
                const ssize_t r = pread(h->fd, s + fill + got, n - got,
                                        static_cast<off_t>(h->data_offset + t->file_offset + t_done + got));
                if (r <= 0) {
                    cleanup();
                    return fail(e, SANDY_ERR_INVALID, "safetensors read failed for %s", t->name);
                }
                got += static_cast<size_t>(r);
            }
            pieces.push_back({t->arena_offset + t_done, fill, n});
            fill += n;
            t_done += n;
            if (t_done == t->nbytes) {
                ti++;
                t_done = 0;
            }
        }
        for (auto& pc : pieces) {
            hipError_t st = hipMemcpyAsync(static_cast<char*>(arena) + pc.dev, s + pc.at, pc.n, hipMemcpyHostToDevice,
                                           stream);
            if (st != hipSuccess) {
                cleanup();
                return fail(e, SANDY_ERR_HIP, "safetensors upload: %s", hipGetErrorString(st));
            }
        }
        hipError_t st = hipEventRecord(done[buf], stream);
        if (st != hipSuccess) {
            cleanup();
            return fail(e, SANDY_ERR_HIP, "safetensors upload: %s", hipGetErrorString(st));
        }
        used[buf] = true;
        buf ^= 1;
    }
    cleanup();  // waits for the last copies: the staging buffers are freed here
    return ok(e);
}

} // extern "C"
