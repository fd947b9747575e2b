// GGUF v3 directory parser and Qwen2 model loader (host code).
//
// The directory rules follow Shard::parse (driver/src/frontier_gguf.rs:145-200):
// a bounded prefix (16 MiB) holds magic, version 3, counts, metadata and tensor
// infos; limits of 4096 tensors, 1024 keys, 256-byte keys and names, 16 MiB
// strings, 1,000,000-element (non-nested) arrays; duplicate keys and names are
// rejected; split.no / split.count / split.tensors.count are validated;
// general.alignment (default 32) must be a power of two <= 4096 and every
// tensor offset a multiple of it; rank 1..4 with non-zero dims; a tensor's
// bytes are row_bytes(kind, dims[0]) times the other dims with overflow checks;
// the data section starts at the aligned end of the directory; every tensor
// lies inside the file and no two overlap. Error categories are the
// reference's Error enum (frontier_gguf.rs:7-8).
//
// The loader reads a Qwen2 model's tensors by GGUF name (the names the
// reference's llm.rs:52-100 reader looks up) and hands them to the model
// (uq_model_set_tensor): Q8_0 matrices and F32 vectors.
#include "../../include/uq.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <set>
#include <string>
#include <vector>

namespace uq {
int set_error(int status, const std::string& msg);  // uq_runtime.hip
}

namespace {

enum GgufErr {
    G_OK = 0, G_TRUNCATED = UQ_GGUF_TRUNCATED, G_MAGIC = UQ_GGUF_MAGIC, G_VERSION = UQ_GGUF_VERSION,
    G_LIMIT = UQ_GGUF_LIMIT, G_TYPE = UQ_GGUF_TYPE, G_UTF8 = UQ_GGUF_UTF8, G_ALIGNMENT = UQ_GGUF_ALIGNMENT,
    G_SHAPE = UQ_GGUF_SHAPE, G_OVERFLOW = UQ_GGUF_OVERFLOW, G_TENSOR_BOUNDS = UQ_GGUF_TENSOR_BOUNDS,
    G_OVERLAP = UQ_GGUF_OVERLAP, G_DUPLICATE = UQ_GGUF_DUPLICATE, G_MISSING = UQ_GGUF_MISSING, G_SPLIT = UQ_GGUF_SPLIT
};

constexpr uint64_t PREFIX_MAX = 16ull << 20;

const char* gguf_err_name(int e) {
    static const char* n[] = {"ok", "truncated", "bad magic", "unsupported version", "limit exceeded", "bad type",
                              "invalid UTF-8", "bad alignment", "bad shape", "overflow", "tensor out of bounds",
                              "overlapping tensors", "duplicate", "missing", "bad split"};
    return e >= 0 && e <= 14 ? n[e] : "?";
}

// Block size and bytes per block of a ggml type: the reference's row_bytes
// (frontier_core.rs:53-58: F32, Q8_0, Q6_K, IQ3_XXS, IQ4_NL, IQ4_XS, BF16)
// plus F16, Q3_K and Q4_K.
bool type_block(uint32_t kind, uint64_t* block, uint64_t* bytes) {
    switch (kind) {
    case 0: *block = 1; *bytes = 4; return true;
    case 1: *block = 1; *bytes = 2; return true;
    case 8: *block = 32; *bytes = 34; return true;
    case 11: *block = 256; *bytes = 110; return true;
    case 12: *block = 256; *bytes = 144; return true;
    case 14: *block = 256; *bytes = 210; return true;
    case 18: *block = 256; *bytes = 98; return true;
    case 20: *block = 32; *bytes = 18; return true;
    case 23: *block = 256; *bytes = 136; return true;
    case 30: *block = 1; *bytes = 2; return true;
    default: return false;
    }
}

bool mul_ovf(uint64_t a, uint64_t b, uint64_t* out) { return __builtin_mul_overflow(a, b, out); }
bool add_ovf(uint64_t a, uint64_t b, uint64_t* out) { return __builtin_add_overflow(a, b, out); }

bool valid_utf8(const uint8_t* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        int len = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
        if (!len || i + len > n) return false;
        uint32_t cp = len == 1 ? c : c & (0x7f >> len);
        for (int k = 1; k < len; k++) {
            if ((s[i + k] & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3f);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && (cp < 0x10000 || cp > 0x10ffff)) ||
            (cp >= 0xd800 && cp <= 0xdfff))
            return false;
        i += len;
    }
    return true;
}

struct Reader {
    const uint8_t* d;
    uint64_t n, pos = 0;
    int take(uint64_t k, const uint8_t** p) {
        uint64_t end;
        if (add_ovf(pos, k, &end)) return G_OVERFLOW;
        if (end > n) return G_TRUNCATED;
        *p = d + pos;
        pos = end;
        return G_OK;
    }
    int u32(uint32_t* v) {
        const uint8_t* p;
        if (int e = take(4, &p)) return e;
        memcpy(v, p, 4);
        return G_OK;
    }
    int u64(uint64_t* v) {
        const uint8_t* p;
        if (int e = take(8, &p)) return e;
        memcpy(v, p, 8);
        return G_OK;
    }
    int string(std::string* s) {
        uint64_t len;
        if (int e = u64(&len)) return e;
        if (len > PREFIX_MAX) return G_LIMIT;
        const uint8_t* p;
        if (int e = take(len, &p)) return e;
        if (!valid_utf8(p, len)) return G_UTF8;
        if (s) s->assign((const char*)p, len);
        return G_OK;
    }
    int skip(uint32_t kind, bool nested) {
        const uint8_t* p;
        switch (kind) {
        case 0: case 1: case 7: return take(1, &p);
        case 2: case 3: return take(2, &p);
        case 4: case 5: case 6: return take(4, &p);
        case 10: case 11: case 12: return take(8, &p);
        case 8: return string(nullptr);
        case 9: {
            if (nested) return G_TYPE;
            uint32_t elem;
            uint64_t count;
            if (int e = u32(&elem)) return e;
            if (int e = u64(&count)) return e;
            if (count > 1000000) return G_LIMIT;
            for (uint64_t i = 0; i < count; i++)
                if (int e = skip(elem, true)) return e;
            return G_OK;
        }
        default: return G_TYPE;
        }
    }
};

struct Meta {
    std::string key;
    uint32_t kind;
    std::vector<uint8_t> data;  // the raw value bytes
};

struct TensorInfo {
    std::string name;
    uint64_t dims[4];
    int32_t rank;
    uint32_t kind;
    uint64_t offset, bytes, row_bytes;  // offset: absolute file offset
};

int meta_unsigned(const Meta& m, uint64_t* v) {
    const uint8_t* p = m.data.data();
    switch (m.kind) {
    case 0: if (m.data.size() < 1) return G_TRUNCATED; *v = p[0]; return G_OK;
    case 2: { uint16_t x; if (m.data.size() < 2) return G_TRUNCATED; memcpy(&x, p, 2); *v = x; return G_OK; }
    case 4: { uint32_t x; if (m.data.size() < 4) return G_TRUNCATED; memcpy(&x, p, 4); *v = x; return G_OK; }
    case 10: { if (m.data.size() < 8) return G_TRUNCATED; memcpy(v, p, 8); return G_OK; }
    default: return G_TYPE;
    }
}

}  // namespace

struct uq_gguf {
    std::vector<Meta> meta;
    std::vector<TensorInfo> tensors;
    uint64_t data_offset = 0, logical_bytes = 0, split_no = 0, split_count = 1, total_tensors = 0;
    std::string path;  // set when opened from a file
    // byte offsets of the elements of one string array, built on first use
    std::string str_index_key;
    std::vector<uint64_t> str_index;
};

namespace {

const Meta* find_meta(const uq_gguf* g, const char* key) {
    for (const auto& m : g->meta)
        if (m.key == key) return &m;
    return nullptr;
}

int parse_dir(const uint8_t* d, uint64_t len, uint64_t logical, uq_gguf* g) {
    if (len > PREFIX_MAX) return G_LIMIT;
    Reader r{d, len};
    const uint8_t* p;
    if (int e = r.take(4, &p)) return e;
    if (memcmp(p, "GGUF", 4) != 0) return G_MAGIC;
    uint32_t version;
    if (int e = r.u32(&version)) return e;
    if (version != 3) return G_VERSION;
    uint64_t nt, nk;
    if (int e = r.u64(&nt)) return e;
    if (int e = r.u64(&nk)) return e;
    if (nt > 4096 || nk > 1024) return G_LIMIT;
    for (uint64_t i = 0; i < nk; i++) {
        Meta m;
        if (int e = r.string(&m.key)) return e;
        if (m.key.size() > 256) return G_LIMIT;
        if (find_meta(g, m.key.c_str())) return G_DUPLICATE;
        if (int e = r.u32(&m.kind)) return e;
        const uint64_t start = r.pos;
        if (int e = r.skip(m.kind, false)) return e;
        m.data.assign(d + start, d + r.pos);
        g->meta.push_back(std::move(m));
    }
    g->logical_bytes = logical;
    g->total_tensors = nt;
    if (const Meta* m = find_meta(g, "split.no"))
        if (int e = meta_unsigned(*m, &g->split_no)) return e;
    if (const Meta* m = find_meta(g, "split.count"))
        if (int e = meta_unsigned(*m, &g->split_count)) return e;
    if (const Meta* m = find_meta(g, "split.tensors.count")) {
        if (m->kind == 5) {  // int32 in standard split files
            int32_t v;
            if (m->data.size() < 4) return G_TYPE;
            memcpy(&v, m->data.data(), 4);
            if (v < 0) return G_SPLIT;
            g->total_tensors = (uint64_t)v;
        } else if (int e = meta_unsigned(*m, &g->total_tensors)) {
            return e;
        }
    }
    if (g->split_count == 0 || g->split_count > 64 || g->split_no >= g->split_count || g->total_tensors < nt ||
        g->total_tensors > 65536)
        return G_SPLIT;
    uint64_t alignment = 32;
    if (const Meta* m = find_meta(g, "general.alignment"))
        if (int e = meta_unsigned(*m, &alignment)) return e;
    if (alignment == 0 || (alignment & (alignment - 1)) || alignment > 4096) return G_ALIGNMENT;
    for (uint64_t i = 0; i < nt; i++) {
        TensorInfo t;
        if (int e = r.string(&t.name)) return e;
        if (t.name.size() > 256) return G_LIMIT;
        for (const auto& o : g->tensors)
            if (o.name == t.name) return G_DUPLICATE;
        uint32_t rank;
        if (int e = r.u32(&rank)) return e;
        if (rank < 1 || rank > 4) return G_SHAPE;
        t.rank = (int32_t)rank;
        for (int k = 0; k < 4; k++) t.dims[k] = 1;
        for (uint32_t k = 0; k < rank; k++) {
            if (int e = r.u64(&t.dims[k])) return e;
            if (t.dims[k] == 0) return G_SHAPE;
        }
        if (int e = r.u32(&t.kind)) return e;
        if (int e = r.u64(&t.offset)) return e;
        if (t.offset % alignment) return G_ALIGNMENT;
        uint64_t block, bb;
        if (!type_block(t.kind, &block, &bb)) return G_TYPE;
        if (t.dims[0] % block) return G_SHAPE;
        if (mul_ovf(t.dims[0] / block, bb, &t.row_bytes)) return G_OVERFLOW;
        t.bytes = t.row_bytes;
        for (uint32_t k = 1; k < rank; k++)
            if (mul_ovf(t.bytes, t.dims[k], &t.bytes)) return G_OVERFLOW;
        g->tensors.push_back(std::move(t));
    }
    uint64_t end;
    if (add_ovf(r.pos, alignment - 1, &end)) return G_OVERFLOW;
    g->data_offset = end & ~(alignment - 1);
    if (g->data_offset > logical) return G_TENSOR_BOUNDS;
    std::vector<std::pair<uint64_t, uint64_t>> ranges;
    for (auto& t : g->tensors) {
        if (add_ovf(t.offset, g->data_offset, &t.offset)) return G_OVERFLOW;
        uint64_t e;
        if (add_ovf(t.offset, t.bytes, &e)) return G_OVERFLOW;
        if (e > logical) return G_TENSOR_BOUNDS;
        ranges.emplace_back(t.offset, e);
    }
    std::sort(ranges.begin(), ranges.end());
    for (size_t i = 1; i < ranges.size(); i++)
        if (ranges[i - 1].second > ranges[i].first) return G_OVERLAP;
    return G_OK;
}

int fail_gguf(int e, int* gguf_error, const char* what) {
    if (gguf_error) *gguf_error = e;
    return uq::set_error(UQ_ERR_FORMAT, std::string(what) + ": " + gguf_err_name(e));
}

int read_at(const std::string& path, uint64_t off, uint64_t n, void* dst) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return uq::set_error(UQ_ERR_ARG, "gguf: cannot open " + path);
    int rc = UQ_OK;
    if (fseeko(f, (off_t)off, SEEK_SET) != 0 || std::fread(dst, 1, n, f) != n)
        rc = uq::set_error(UQ_ERR_FORMAT, "gguf: short read of " + path);
    std::fclose(f);
    return rc;
}

}  // namespace

extern "C" {

int uq_gguf_parse(const void* prefix, size_t len, uint64_t logical_bytes, uq_gguf_t* out, int* gguf_error) {
    if (gguf_error) *gguf_error = 0;
    if (!out || (!prefix && len)) return uq::set_error(UQ_ERR_ARG, "gguf_parse: null pointer");
    *out = nullptr;
    uq_gguf* g = new uq_gguf();
    const int e = parse_dir((const uint8_t*)prefix, len, logical_bytes, g);
    if (e) {
        delete g;
        return fail_gguf(e, gguf_error, "gguf_parse");
    }
    *out = g;
    return UQ_OK;
}

int uq_gguf_open(const char* path, uq_gguf_t* out, int* gguf_error) {
    if (gguf_error) *gguf_error = 0;
    if (!path || !out) return uq::set_error(UQ_ERR_ARG, "gguf_open: null pointer");
    *out = nullptr;
    FILE* f = std::fopen(path, "rb");
    if (!f) return uq::set_error(UQ_ERR_ARG, std::string("gguf_open: cannot open ") + path);
    fseeko(f, 0, SEEK_END);
    const uint64_t size = (uint64_t)ftello(f);
    fseeko(f, 0, SEEK_SET);
    std::vector<uint8_t> head((size_t)std::min<uint64_t>(size, PREFIX_MAX));
    const size_t got = std::fread(head.data(), 1, head.size(), f);
    std::fclose(f);
    if (got != head.size()) return uq::set_error(UQ_ERR_FORMAT, std::string("gguf_open: short read of ") + path);
    uq_gguf* g = new uq_gguf();
    const int e = parse_dir(head.data(), head.size(), size, g);
    if (e) {
        delete g;
        return fail_gguf(e, gguf_error, "gguf_open");
    }
    g->path = path;
    *out = g;
    return UQ_OK;
}

int uq_gguf_free(uq_gguf_t g) {
    delete g;
    return UQ_OK;
}

int64_t uq_gguf_tensor_count(uq_gguf_t g) { return g ? (int64_t)g->tensors.size() : -1; }

uint64_t uq_gguf_data_offset(uq_gguf_t g) { return g ? g->data_offset : 0; }

int uq_gguf_split_info(uq_gguf_t g, uint64_t* split_no, uint64_t* split_count, uint64_t* total_tensors) {
    if (!g) return uq::set_error(UQ_ERR_ARG, "gguf_split_info: null handle");
    if (split_no) *split_no = g->split_no;
    if (split_count) *split_count = g->split_count;
    if (total_tensors) *total_tensors = g->total_tensors;
    return UQ_OK;
}

int uq_gguf_tensor_info(uq_gguf_t g, int64_t index, const char** name, uint32_t* kind, int32_t* rank, uint64_t* dims,
                        uint64_t* offset, uint64_t* bytes) {
    if (!g || index < 0 || index >= (int64_t)g->tensors.size())
        return uq::set_error(UQ_ERR_ARG, "gguf_tensor_info: bad handle or index");
    const TensorInfo& t = g->tensors[(size_t)index];
    if (name) *name = t.name.c_str();
    if (kind) *kind = t.kind;
    if (rank) *rank = t.rank;
    if (dims)
        for (int k = 0; k < 4; k++) dims[k] = t.dims[k];
    if (offset) *offset = t.offset;
    if (bytes) *bytes = t.bytes;
    return UQ_OK;
}

int64_t uq_gguf_find_tensor(uq_gguf_t g, const char* name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (g->tensors[i].name == name) return (int64_t)i;
    return -1;
}

int uq_gguf_meta_u64(uq_gguf_t g, const char* key, uint64_t* out) {
    if (!g || !key || !out) return uq::set_error(UQ_ERR_ARG, "gguf_meta_u64: null pointer");
    const Meta* m = find_meta(g, key);
    if (!m) return uq::set_error(UQ_ERR_FORMAT, std::string("gguf: missing key ") + key);
    if (int e = meta_unsigned(*m, out)) return fail_gguf(e, nullptr, key);
    return UQ_OK;
}

int uq_gguf_meta_f32(uq_gguf_t g, const char* key, float* out) {
    if (!g || !key || !out) return uq::set_error(UQ_ERR_ARG, "gguf_meta_f32: null pointer");
    const Meta* m = find_meta(g, key);
    if (!m) return uq::set_error(UQ_ERR_FORMAT, std::string("gguf: missing key ") + key);
    if (m->kind != 6 || m->data.size() < 4) return fail_gguf(G_TYPE, nullptr, key);
    memcpy(out, m->data.data(), 4);
    return UQ_OK;
}

int uq_gguf_meta_str(uq_gguf_t g, const char* key, const char** out, uint64_t* len) {
    if (!g || !key || !out || !len) return uq::set_error(UQ_ERR_ARG, "gguf_meta_str: null pointer");
    const Meta* m = find_meta(g, key);
    if (!m) return uq::set_error(UQ_ERR_FORMAT, std::string("gguf: missing key ") + key);
    if (m->kind != 8 || m->data.size() < 8) return fail_gguf(G_TYPE, nullptr, key);
    memcpy(len, m->data.data(), 8);
    *out = (const char*)m->data.data() + 8;
    return UQ_OK;
}

int uq_gguf_meta_array(uq_gguf_t g, const char* key, uint32_t* elem_kind, uint64_t* count) {
    if (!g || !key || !elem_kind || !count) return uq::set_error(UQ_ERR_ARG, "gguf_meta_array: null pointer");
    const Meta* m = find_meta(g, key);
    if (!m) return uq::set_error(UQ_ERR_FORMAT, std::string("gguf: missing key ") + key);
    if (m->kind != 9 || m->data.size() < 12) return fail_gguf(G_TYPE, nullptr, key);
    memcpy(elem_kind, m->data.data(), 4);
    memcpy(count, m->data.data() + 4, 8);
    return UQ_OK;
}

int uq_gguf_meta_array_str(uq_gguf_t g, const char* key, uint64_t index, const char** out, uint64_t* len) {
    if (!g || !key || !out || !len) return uq::set_error(UQ_ERR_ARG, "gguf_meta_array_str: null pointer");
    const Meta* m = find_meta(g, key);
    if (!m) return uq::set_error(UQ_ERR_FORMAT, std::string("gguf: missing key ") + key);
    uint32_t elem = 0;
    uint64_t count = 0;
    if (m->kind != 9 || m->data.size() < 12) return fail_gguf(G_TYPE, nullptr, key);
    memcpy(&elem, m->data.data(), 4);
    memcpy(&count, m->data.data() + 4, 8);
    if (elem != 8) return fail_gguf(G_TYPE, nullptr, key);
    if (index >= count) return uq::set_error(UQ_ERR_ARG, "gguf_meta_array_str: index out of range");
    if (g->str_index_key != key) {
        // the parser checked every length against the value's bytes
        g->str_index.clear();
        g->str_index.reserve((size_t)count);
        uint64_t pos = 12;
        for (uint64_t i = 0; i < count; i++) {
            uint64_t l;
            memcpy(&l, m->data.data() + pos, 8);
            g->str_index.push_back(pos);
            pos += 8 + l;
        }
        g->str_index_key = key;
    }
    const uint64_t pos = g->str_index[(size_t)index];
    memcpy(len, m->data.data() + pos, 8);
    *out = (const char*)m->data.data() + pos + 8;
    return UQ_OK;
}

// Model::text (driver/src/llm.rs:87-99): the GPT-2 byte-level string of token
// `id` back to bytes. A character below 256 is that byte; character 256 + i
// is the i-th byte (ascending) outside the printable ranges 33-126, 161-172
// and 174-255; any other character is its own UTF-8 encoding.
int uq_gguf_token_text(uq_gguf_t g, uint32_t id, uint8_t* out, uint64_t cap, uint64_t* len) {
    if (!g || !len || (cap && !out)) return uq::set_error(UQ_ERR_ARG, "gguf_token_text: null pointer");
    const char* s = nullptr;
    uint64_t n = 0;
    if (int rc = uq_gguf_meta_array_str(g, "tokenizer.ggml.tokens", id, &s, &n)) return rc;
    uint8_t unprintable[68];
    int nun = 0;
    for (int b = 0; b < 256; b++)
        if (!((b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255))) unprintable[nun++] = (uint8_t)b;
    uint64_t w = 0;
    auto put = [&](uint8_t b) {
        if (w < cap) out[w] = b;
        w++;
    };
    const uint8_t* p = (const uint8_t*)s;
    uint64_t i = 0;
    while (i < n) {
        // the parser checked the string is valid UTF-8
        uint32_t c = p[i], extra = 0;
        if (c >= 0xF0) { c &= 0x07; extra = 3; }
        else if (c >= 0xE0) { c &= 0x0F; extra = 2; }
        else if (c >= 0xC0) { c &= 0x1F; extra = 1; }
        const uint64_t start = i;
        i++;
        for (uint32_t k = 0; k < extra; k++, i++) c = (c << 6) | (p[i] & 0x3F);
        if (c < 256) put((uint8_t)c);
        else if (c - 256 < (uint32_t)nun) put(unprintable[c - 256]);
        else
            for (uint64_t k = start; k < i; k++) put(p[k]);
    }
    *len = w;
    if (w > cap) return uq::set_error(UQ_ERR_ARG, "gguf_token_text: buffer too small");
    return UQ_OK;
}

int uq_gguf_qwen2_config(uq_gguf_t g, int32_t max_seq, uq_qwen2_config* cfg) {
    if (!g || !cfg) return uq::set_error(UQ_ERR_ARG, "gguf_qwen2_config: null pointer");
    const char* arch = nullptr;
    uint64_t alen = 0;
    if (int rc = uq_gguf_meta_str(g, "general.architecture", &arch, &alen)) return rc;
    if (std::string(arch, alen) != "qwen2") return uq::set_error(UQ_ERR_FORMAT, "gguf: architecture is not qwen2");
    uint64_t layers, dim, hidden, heads, kv, ctx;
    float theta, eps;
    if (int rc = uq_gguf_meta_u64(g, "qwen2.block_count", &layers)) return rc;
    if (int rc = uq_gguf_meta_u64(g, "qwen2.embedding_length", &dim)) return rc;
    if (int rc = uq_gguf_meta_u64(g, "qwen2.feed_forward_length", &hidden)) return rc;
    if (int rc = uq_gguf_meta_u64(g, "qwen2.attention.head_count", &heads)) return rc;
    if (int rc = uq_gguf_meta_u64(g, "qwen2.attention.head_count_kv", &kv)) return rc;
    if (int rc = uq_gguf_meta_u64(g, "qwen2.context_length", &ctx)) return rc;
    if (int rc = uq_gguf_meta_f32(g, "qwen2.rope.freq_base", &theta)) return rc;
    if (int rc = uq_gguf_meta_f32(g, "qwen2.attention.layer_norm_rms_epsilon", &eps)) return rc;
    const int64_t te = uq_gguf_find_tensor(g, "token_embd.weight");
    if (te < 0) return uq::set_error(UQ_ERR_FORMAT, "gguf: token_embd.weight missing");
    const TensorInfo& t = g->tensors[(size_t)te];
    if (t.rank != 2 || t.dims[0] != dim || !heads || dim % heads)
        return uq::set_error(UQ_ERR_SHAPE, "gguf: inconsistent qwen2 shapes");
    if (layers > 4096 || dim > (1u << 20) || hidden > (1u << 20) || heads > 4096 || kv > 4096 || t.dims[1] > (1u << 30))
        return uq::set_error(UQ_ERR_SHAPE, "gguf: qwen2 shapes out of range");
    cfg->layers = (int32_t)layers;
    cfg->dim = (int32_t)dim;
    cfg->hidden = (int32_t)hidden;
    cfg->heads = (int32_t)heads;
    cfg->kv_heads = (int32_t)kv;
    cfg->head_dim = (int32_t)(dim / heads);
    cfg->vocab = (int32_t)t.dims[1];
    cfg->max_seq = max_seq > 0 ? max_seq : (int32_t)std::min<uint64_t>(ctx, 1u << 30);
    cfg->eps = eps;
    cfg->theta = theta;
    return UQ_OK;
}

// Tensor::rows (frontier_gguf.rs:86-94): the absolute file range of `count`
// contiguous rows from `start`.
static int tensor_rows(const TensorInfo& t, uint64_t start, uint64_t count, uint64_t* off, uint64_t* n) {
    const uint64_t total = t.bytes / t.row_bytes;
    uint64_t end;
    if (add_ovf(start, count, &end)) return G_OVERFLOW;
    if (count == 0 || end > total) return G_TENSOR_BOUNDS;
    uint64_t skip, o, len;
    if (mul_ovf(start, t.row_bytes, &skip) || add_ovf(t.offset, skip, &o) || mul_ovf(count, t.row_bytes, &len))
        return G_OVERFLOW;
    *off = o;
    *n = len;
    return G_OK;
}

// Tensor::expert (frontier_gguf.rs:95-98): the rows of expert `id` of a
// rank-3 [n, rows, experts] tensor.
static int tensor_expert(const TensorInfo& t, uint64_t id, uint64_t* off, uint64_t* n) {
    if (t.rank != 3 || id >= t.dims[2]) return G_SHAPE;
    uint64_t start;
    if (mul_ovf(id, t.dims[1], &start)) return G_OVERFLOW;
    return tensor_rows(t, start, t.dims[1], off, n);
}

int uq_gguf_tensor_rows(uq_gguf_t g, int64_t index, uint64_t start, uint64_t count, uint64_t* offset, uint64_t* bytes,
                        int* gguf_error) {
    if (gguf_error) *gguf_error = 0;
    if (!g || index < 0 || index >= (int64_t)g->tensors.size() || !offset || !bytes)
        return uq::set_error(UQ_ERR_ARG, "gguf_tensor_rows: bad handle, index or pointer");
    if (int e = tensor_rows(g->tensors[(size_t)index], start, count, offset, bytes))
        return fail_gguf(e, gguf_error, "gguf_tensor_rows");
    return UQ_OK;
}

int uq_gguf_tensor_expert(uq_gguf_t g, int64_t index, uint32_t expert, uint64_t* offset, uint64_t* bytes,
                          int* gguf_error) {
    if (gguf_error) *gguf_error = 0;
    if (!g || index < 0 || index >= (int64_t)g->tensors.size() || !offset || !bytes)
        return uq::set_error(UQ_ERR_ARG, "gguf_tensor_expert: bad handle, index or pointer");
    if (int e = tensor_expert(g->tensors[(size_t)index], expert, offset, bytes))
        return fail_gguf(e, gguf_error, "gguf_tensor_expert");
    return UQ_OK;
}

}  // extern "C"

// ModelIndex (frontier_gguf.rs:101-137): the directories of every split file
// of one model, ordered by split.no. The shard handles stay the caller's.
struct uq_gguf_index {
    std::vector<uq_gguf_t> shards;
};

extern "C" {

int uq_gguf_index_create(const uq_gguf_t* shards, int count, uq_gguf_index_t* out, int* gguf_error) {
    if (gguf_error) *gguf_error = 0;
    if (!out || (count > 0 && !shards)) return uq::set_error(UQ_ERR_ARG, "gguf_index_create: null pointer");
    *out = nullptr;
    if (count <= 0) return fail_gguf(G_SPLIT, gguf_error, "gguf_index_create");
    std::vector<uq_gguf_t> v(shards, shards + count);
    for (uq_gguf_t g : v)
        if (!g) return uq::set_error(UQ_ERR_ARG, "gguf_index_create: null shard");
    std::sort(v.begin(), v.end(), [](uq_gguf_t a, uq_gguf_t b) { return a->split_no < b->split_no; });
    const uint64_t total = v[0]->total_tensors, n = (uint64_t)count;
    std::set<std::string> names;
    for (size_t i = 0; i < v.size(); i++) {
        if (v[i]->split_no != i || v[i]->split_count != n || v[i]->total_tensors != total)
            return fail_gguf(G_SPLIT, gguf_error, "gguf_index_create");
        for (const auto& t : v[i]->tensors)
            if (!names.insert(t.name).second) return fail_gguf(G_DUPLICATE, gguf_error, "gguf_index_create");
    }
    if ((uint64_t)names.size() != total) return fail_gguf(G_SPLIT, gguf_error, "gguf_index_create");
    *out = new uq_gguf_index{std::move(v)};
    return UQ_OK;
}

int uq_gguf_index_free(uq_gguf_index_t ix) {
    delete ix;
    return UQ_OK;
}

int uq_gguf_index_shard_count(uq_gguf_index_t ix) { return ix ? (int)ix->shards.size() : UQ_ERR_ARG; }

uq_gguf_t uq_gguf_index_shard(uq_gguf_index_t ix, int i) {
    return ix && i >= 0 && i < (int)ix->shards.size() ? ix->shards[(size_t)i] : nullptr;
}

int uq_gguf_index_find(uq_gguf_index_t ix, const char* name, int* shard, int64_t* index, int* gguf_error) {
    if (gguf_error) *gguf_error = 0;
    if (!ix || !name || !shard || !index) return uq::set_error(UQ_ERR_ARG, "gguf_index_find: null pointer");
    for (size_t i = 0; i < ix->shards.size(); i++) {
        const int64_t t = uq_gguf_find_tensor(ix->shards[i], name);
        if (t >= 0) {
            *shard = (int)i;
            *index = t;
            return UQ_OK;
        }
    }
    return fail_gguf(G_MISSING, gguf_error, (std::string("gguf_index_find ") + name).c_str());
}

int uq_gguf_index_inventory(uq_gguf_index_t ix, uint64_t* bytes3, int* gguf_error) {
    if (gguf_error) *gguf_error = 0;
    if (!ix || !bytes3) return uq::set_error(UQ_ERR_ARG, "gguf_index_inventory: null pointer");
    uint64_t c[3] = {0, 0, 0};
    for (uq_gguf_t g : ix->shards)
        for (const auto& t : g->tensors) {
            const size_t L = t.name.size();
            const int k = t.name == "per_layer_token_embd.weight"
                              ? 1
                              : (L >= 12 && t.name.compare(L - 12, 12, "_exps.weight") == 0 ? 2 : 0);
            if (add_ovf(c[k], t.bytes, &c[k])) return fail_gguf(G_OVERFLOW, gguf_error, "gguf_index_inventory");
        }
    for (int k = 0; k < 3; k++) bytes3[k] = c[k];
    return UQ_OK;
}

int uq_gguf_load_weight(uq_gguf_t g, int64_t index, int32_t expert, uq_weight_t* out) {
    if (!g || !out || index < 0 || index >= (int64_t)g->tensors.size())
        return uq::set_error(UQ_ERR_ARG, "gguf_load_weight: bad handle or index");
    if (g->path.empty()) return uq::set_error(UQ_ERR_ARG, "gguf_load_weight: the GGUF handle was not opened from a file");
    const TensorInfo& t = g->tensors[(size_t)index];
    uint64_t off, n;
    int e = expert < 0 ? tensor_rows(t, 0, t.bytes / t.row_bytes, &off, &n) : tensor_expert(t, (uint64_t)expert, &off, &n);
    if (e) return fail_gguf(e, nullptr, "gguf_load_weight");
    if (expert < 0 && t.rank > 2) return uq::set_error(UQ_ERR_SHAPE, "gguf_load_weight: rank-3 tensor needs an expert id");
    std::vector<uint8_t> buf((size_t)n);
    if (int rc = read_at(g->path, off, n, buf.data())) return rc;
    return uq_weight_upload(t.kind, (int64_t)t.dims[0], (int64_t)(n / t.row_bytes), buf.data(), buf.size(), out);
}

// The expert bank of one MoE layer from a split model: the rank-3
// blk.L.ffn_{gate,up,down}_exps.weight tensors ([dim, ff, experts] and
// [ff, dim, experts]) expert by expert (Tensor::expert), then the shared
// expert blk.L.ffn_{gate,up,down}_shexp.weight and its optional f32 gate
// blk.L.ffn_gate_inp_shexp.weight -- the tensors Backend::expert streams
// (frontier_backend.rs:98-128), here made resident once. Before reading,
// the bank's bytes are checked against the free HBM of the device (twice,
// for the verified upload's staging).
int uq_moe_load_gguf(uq_moe_t m, uq_gguf_index_t ix, int32_t layer) {
    if (!m || !ix || layer < 0) return uq::set_error(UQ_ERR_ARG, "moe_load_gguf: bad arguments");
    int32_t D, Fd, E, K;
    uint32_t kind;
    if (int rc = uq_moe_info(m, &D, &Fd, &E, &K, &kind)) return rc;
    struct Found { uq_gguf_t g = nullptr; const TensorInfo* t = nullptr; };
    auto find = [&](const std::string& name, bool required, Found* f) -> int {
        int sh = 0;
        int64_t ti = 0;
        if (uq_gguf_index_find(ix, name.c_str(), &sh, &ti, nullptr) != UQ_OK) {
            if (!required) return UQ_OK;
            return uq::set_error(UQ_ERR_FORMAT, "moe_load_gguf: " + name + " missing");
        }
        f->g = ix->shards[(size_t)sh];
        f->t = &f->g->tensors[(size_t)ti];
        if (f->g->path.empty()) return uq::set_error(UQ_ERR_ARG, "moe_load_gguf: shard not opened from a file");
        return UQ_OK;
    };
    const std::string b = "blk." + std::to_string(layer) + ".ffn_";
    Found eg, eu, ed, sg, su, sd, gi;
    if (int rc = find(b + "gate_exps.weight", true, &eg)) return rc;
    if (int rc = find(b + "up_exps.weight", true, &eu)) return rc;
    if (int rc = find(b + "down_exps.weight", true, &ed)) return rc;
    if (int rc = find(b + "gate_shexp.weight", true, &sg)) return rc;
    if (int rc = find(b + "up_shexp.weight", true, &su)) return rc;
    if (int rc = find(b + "down_shexp.weight", true, &sd)) return rc;
    if (int rc = find(b + "gate_inp_shexp.weight", false, &gi)) return rc;
    auto dims_are = [](const TensorInfo* t, int rank, uint64_t a, uint64_t b2, uint64_t c) {
        return t->rank == rank && t->dims[0] == a && t->dims[1] == b2 && (rank < 3 || t->dims[2] == c);
    };
    for (const Found* f : {&eg, &eu, &ed})
        if (f->t->kind != kind) return uq::set_error(UQ_ERR_QUANT_TYPE, "moe_load_gguf: " + f->t->name + " kind != bank kind");
    if (!dims_are(eg.t, 3, D, Fd, E) || !dims_are(eu.t, 3, D, Fd, E) || !dims_are(ed.t, 3, Fd, D, E))
        return uq::set_error(UQ_ERR_SHAPE, "moe_load_gguf: expert tensor shapes != the layer's dim/ff/experts");
    const uint32_t skind = sg.t->kind;
    if (su.t->kind != skind || sd.t->kind != skind) return uq::set_error(UQ_ERR_QUANT_TYPE, "moe_load_gguf: shared expert kinds differ");
    if (!dims_are(sg.t, 2, D, Fd, 0) || !dims_are(su.t, 2, D, Fd, 0) || !dims_are(sd.t, 2, Fd, D, 0))
        return uq::set_error(UQ_ERR_SHAPE, "moe_load_gguf: shared expert shapes != the layer's dim/ff");
    if (gi.t && (gi.t->kind != 0 || gi.t->rank != 1 || gi.t->dims[0] != (uint64_t)D))
        return uq::set_error(UQ_ERR_SHAPE, "moe_load_gguf: ffn_gate_inp_shexp must be f32 [dim]");
    uint64_t need = 0;
    for (const Found* f : {&eg, &eu, &ed, &sg, &su, &sd}) need += f->t->bytes;
    size_t free_b = 0, total_b = 0;
    if (int rc = uq_device_memory(&free_b, &total_b)) return rc;
    if (2 * need > (uint64_t)free_b)
        return uq::set_error(UQ_ERR_DEVICE, "moe_load_gguf: the layer's " + std::to_string(need) +
                                                " expert bytes do not fit the free HBM (" + std::to_string(free_b) + ")");
    auto read_all = [&](const Found& f, std::vector<uint8_t>* buf) -> int {
        buf->resize((size_t)f.t->bytes);
        return read_at(f.g->path, f.t->offset, f.t->bytes, buf->data());
    };
    std::vector<uint8_t> bg, bu, bd;
    if (int rc = read_all(eg, &bg)) return rc;
    if (int rc = read_all(eu, &bu)) return rc;
    if (int rc = read_all(ed, &bd)) return rc;
    for (int32_t e = 0; e < E; e++) {
        uint64_t og, ng, ou, nu, od, nd;
        if (tensor_expert(*eg.t, (uint64_t)e, &og, &ng) || tensor_expert(*eu.t, (uint64_t)e, &ou, &nu) ||
            tensor_expert(*ed.t, (uint64_t)e, &od, &nd))
            return uq::set_error(UQ_ERR_FORMAT, "moe_load_gguf: expert range");
        if (int rc = uq_moe_set_expert(m, e, bg.data() + (og - eg.t->offset), bu.data() + (ou - eu.t->offset),
                                       bd.data() + (od - ed.t->offset)))
            return rc;
    }
    std::vector<uint8_t> sbg, sbu, sbd, sgi;
    if (int rc = read_all(sg, &sbg)) return rc;
    if (int rc = read_all(su, &sbu)) return rc;
    if (int rc = read_all(sd, &sbd)) return rc;
    if (gi.t)
        if (int rc = read_all(gi, &sgi)) return rc;
    return uq_moe_set_shared(m, skind, sbg.data(), sbu.data(), sbd.data(), gi.t ? (const float*)sgi.data() : nullptr);
}

// Tensors of a Qwen2 decoder by GGUF name. output.weight falls back to
// token_embd.weight when the file ties them (no output.weight tensor).
int uq_model_load_gguf(uq_model_t m, uq_gguf_t g) {
    if (!m || !g) return uq::set_error(UQ_ERR_ARG, "model_load_gguf: null pointer");
    if (g->path.empty()) return uq::set_error(UQ_ERR_ARG, "model_load_gguf: the GGUF handle was not opened from a file");
    std::vector<uint8_t> buf;
    auto load = [&](const TensorInfo& t, const char* as) -> int {
        const uint64_t rows = t.bytes / t.row_bytes;
        buf.resize((size_t)t.bytes);
        if (int rc = read_at(g->path, t.offset, t.bytes, buf.data())) return rc;
        return uq_model_set_tensor(m, as, t.kind, (int64_t)t.dims[0], (int64_t)rows, buf.data(), buf.size());
    };
    bool have_output = false;
    for (const auto& t : g->tensors) {
        const bool wanted = t.name.rfind("blk.", 0) == 0 || t.name == "token_embd.weight" ||
                            t.name == "output_norm.weight" || t.name == "output.weight";
        if (!wanted) continue;
        if (int rc = load(t, t.name.c_str())) return rc;
        have_output |= t.name == "output.weight";
    }
    if (!have_output) {
        const int64_t te = uq_gguf_find_tensor(g, "token_embd.weight");
        if (te < 0) return uq::set_error(UQ_ERR_FORMAT, "model_load_gguf: token_embd.weight missing");
        if (int rc = load(g->tensors[(size_t)te], "output.weight")) return rc;
    }
    return UQ_OK;
}

}  // extern "C"
