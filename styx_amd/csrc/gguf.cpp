// gguf.cpp -- GGUF reader (see gguf.h).
#include "gguf.h"

#include <cstdio>
#include <cstring>

namespace styx {

namespace {

struct Reader {
    FILE *f = nullptr;
    bool ok = true;
    uint64_t pos = 0;
    bool read(void *dst, size_t n)
    {
        if (!ok) return false;
        if (n && fread(dst, 1, n, f) != n) {
            ok = false;
            return false;
        }
        pos += n;
        return true;
    }
    template <typename T> bool rd(T &v) { return read(&v, sizeof(T)); }
};

bool valid_utf8(const std::string &s)
{
    // Strict UTF-8 (no overlong forms, surrogates or code points > U+10FFFF),
    // as Rust's String::from_utf8 enforces.
    const unsigned char *p = (const unsigned char *)s.data();
    const size_t n = s.size();
    size_t i = 0;
    while (i < n) {
        const unsigned c = p[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int extra;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) { extra = 1; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { extra = 2; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { extra = 3; cp = c & 0x07; }
        else return false;
        if (i + extra >= n) return false;
        for (int k = 1; k <= extra; k++) {
            if ((p[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (p[i + k] & 0x3F);
        }
        if ((extra == 1 && cp < 0x80) || (extra == 2 && cp < 0x800) ||
            (extra == 3 && cp < 0x10000) || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        i += extra + 1;
    }
    return true;
}

bool read_string(Reader &r, std::string &s, std::string &err)
{
    uint64_t len;
    if (!r.rd(len)) { err = "failed to fill whole buffer"; return false; }
    if (len > (1ull << 24)) { err = "String too long"; return false; }
    s.resize(len);
    if (!r.read(&s[0], len)) { err = "failed to fill whole buffer"; return false; }
    if (!valid_utf8(s)) { err = "Invalid UTF-8"; return false; }
    return true;
}

bool read_value(Reader &r, uint32_t type, GgufValue &v, std::string &err, int depth = 0)
{
    auto fail_io = [&]() { err = "failed to fill whole buffer"; return false; };
    switch (type) {
    case 0: { uint8_t x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::U8; v.u = x; return true; }
    case 1: { int8_t x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::I8; v.i = x; return true; }
    case 2: { uint16_t x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::U16; v.u = x; return true; }
    case 3: { int16_t x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::I16; v.i = x; return true; }
    case 4: { uint32_t x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::U32; v.u = x; return true; }
    case 5: { int32_t x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::I32; v.i = x; return true; }
    case 6: { float x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::F32; v.f = x; return true; }
    case 7: { uint8_t x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::BOOL; v.u = x != 0; return true; }
    case 8: v.kind = GgufValue::STR; return read_string(r, v.s, err);
    case 9: {
        uint32_t et;
        uint64_t n;
        if (!r.rd(et) || !r.rd(n)) return fail_io();
        if (n > (1ull << 28)) { err = "Array too long"; return false; }
        v.kind = GgufValue::ARR;
        v.arr.clear();
        for (uint64_t k = 0; k < n; k++) {
            GgufValue e;
            if (!read_value(r, et, e, err, depth + 1)) return false;
            v.arr.push_back(std::move(e));
        }
        return true;
    }
    case 10: { uint64_t x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::U64; v.u = x; return true; }
    case 11: { int64_t x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::I64; v.i = x; return true; }
    case 12: { double x; if (!r.rd(x)) return fail_io(); v.kind = GgufValue::F64; v.f = x; return true; }
    default:
        err = "Unknown value type: " + std::to_string(type);
        return false;
    }
}

}  // namespace

bool ggml_block(uint32_t t, uint64_t &el, uint64_t &by)
{
    // crates/gguf-rs/src/lib.rs:242-332
    static const struct { uint32_t t, el, by; } tab[] = {
        {0, 1, 4},     {1, 1, 2},     {2, 32, 18},   {3, 32, 20},   {6, 32, 22},
        {7, 32, 24},   {8, 32, 34},   {9, 32, 36},   {10, 256, 84}, {11, 256, 110},
        {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {16, 256, 66},
        {17, 256, 74}, {18, 256, 98},  {19, 256, 50},  {20, 32, 18},  {21, 256, 110},
        {22, 256, 82}, {23, 256, 136}, {24, 1, 1},     {25, 1, 2},    {26, 1, 4},
        {27, 1, 8},    {28, 1, 8},    {29, 256, 56},  {30, 1, 2},
    };
    for (const auto &e : tab)
        if (e.t == t) {
            el = e.el;
            by = e.by;
            return true;
        }
    return false;
}

const GgufTensor *Gguf::find(const std::string &name) const
{
    for (const auto &t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

bool Gguf::get_u32(const std::string &key, uint32_t &out) const
{
    auto it = metadata.find(key);
    if (it == metadata.end() || it->second.kind != GgufValue::U32) return false;
    out = (uint32_t)it->second.u;
    return true;
}

bool Gguf::get_f32(const std::string &key, float &out) const
{
    auto it = metadata.find(key);
    if (it == metadata.end() || it->second.kind != GgufValue::F32) return false;
    out = (float)it->second.f;
    return true;
}

bool Gguf::get_str(const std::string &key, std::string &out) const
{
    auto it = metadata.find(key);
    if (it == metadata.end() || it->second.kind != GgufValue::STR) return false;
    out = it->second.s;
    return true;
}

bool gguf_open(const std::string &path, Gguf &g, std::string &err)
{
    Reader r;
    r.f = fopen(path.c_str(), "rb");
    if (!r.f) {
        err = "open " + path + ": " + strerror(errno);
        return false;
    }
    struct Closer { FILE *f; ~Closer() { fclose(f); } } closer{r.f};
    uint32_t magic, version;
    uint64_t ntens, nkv;
    if (!r.rd(magic)) { err = "failed to fill whole buffer"; return false; }
    if (magic != 0x46554747u) { err = "Invalid GGUF magic"; return false; }
    if (!r.rd(version)) { err = "failed to fill whole buffer"; return false; }
    if (version != 2 && version != 3) { err = "Unsupported GGUF version"; return false; }
    if (!r.rd(ntens) || !r.rd(nkv)) { err = "failed to fill whole buffer"; return false; }
    g.version = version;
    g.metadata.clear();
    g.tensors.clear();
    for (uint64_t i = 0; i < nkv; i++) {
        std::string key;
        if (!read_string(r, key, err)) return false;
        uint32_t vt;
        if (!r.rd(vt)) { err = "failed to fill whole buffer"; return false; }
        GgufValue v;
        if (!read_value(r, vt, v, err)) return false;
        g.metadata[key] = std::move(v);
    }
    for (uint64_t i = 0; i < ntens; i++) {
        GgufTensor t;
        if (!read_string(r, t.name, err)) return false;
        uint32_t nd;
        if (!r.rd(nd)) { err = "failed to fill whole buffer"; return false; }
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t dim;
            if (!r.rd(dim)) { err = "failed to fill whole buffer"; return false; }
            t.dims.push_back(dim);
        }
        if (!r.rd(t.ggml_type) || !r.rd(t.offset)) { err = "failed to fill whole buffer"; return false; }
        uint64_t el, by;
        if (!ggml_block(t.ggml_type, el, by)) {
            err = "Unknown ggml_type: " + std::to_string(t.ggml_type);
            return false;
        }
        // the reference multiplies unchecked (lib.rs:319-331); a product or
        // byte size past 2^64 is rejected here instead of wrapping
        uint64_t prod = 1;
        for (uint64_t d : t.dims)
            if (__builtin_mul_overflow(prod, d, &prod)) {
                err = "Tensor dimensions overflow: " + t.name;
                return false;
            }
        if (prod % el) { err = "First dimension not multiple of block size"; return false; }
        if (__builtin_mul_overflow(prod / el, by, &t.size_bytes)) {
            err = "Tensor size overflows: " + t.name;
            return false;
        }
        g.tensors.push_back(std::move(t));
    }
    uint64_t align = 32;
    uint32_t a32;
    if (g.get_u32("general.alignment", a32)) align = a32;
    if (align == 0) align = 32;
    g.data_start = (r.pos + align - 1) / align * align;
    return true;
}

}  // namespace styx

// --------------------------------------------------------------- C ABI ----
#include "runtime.h"

namespace {

void json_str(std::string &o, const std::string &s)
{
    o += '"';
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') {
            o += '\\';
            o += (char)c;
        } else if (c < 0x20) {
            char b[8];
            snprintf(b, sizeof b, "\\u%04x", c);
            o += b;
        } else {
            o += (char)c;
        }
    }
    o += '"';
}

}  // namespace

extern "C" int styx_gguf_inspect(const char *path, char *out, uint64_t cap)
{
    using namespace styx;
    if (!path || !out) return fail(STYX_E_INVALID, "styx_gguf_inspect: NULL argument");
    Gguf g;
    std::string err;
    if (!gguf_open(path, g, err)) return fail(STYX_E_FORMAT, err);
    std::string o = "{\"version\":" + std::to_string(g.version) +
                    ",\"data_start\":" + std::to_string(g.data_start) + ",\"metadata\":[";
    bool first = true;
    for (auto &kv : g.metadata) {
        if (!first) o += ',';
        first = false;
        json_str(o, kv.first);
    }
    o += "],\"tensors\":[";
    first = true;
    for (auto &t : g.tensors) {
        if (!first) o += ',';
        first = false;
        o += "{\"name\":";
        json_str(o, t.name);
        o += ",\"dims\":[";
        for (size_t i = 0; i < t.dims.size(); i++) o += (i ? "," : "") + std::to_string(t.dims[i]);
        o += "],\"type\":" + std::to_string(t.ggml_type) + ",\"offset\":" +
             std::to_string(t.offset) + ",\"size_bytes\":" + std::to_string(t.size_bytes) + "}";
    }
    o += "]}";
    if (o.size() + 1 > cap) return fail(STYX_E_INVALID, "styx_gguf_inspect: buffer too small");
    memcpy(out, o.c_str(), o.size() + 1);
    return STYX_OK;
}
