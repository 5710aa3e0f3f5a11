// ref_gguf_shim.cpp -- extern "C" view of the reference's own GGUF reader,
// compiled from /root/reference sources in place (oracle/Makefile, target
// `ref`) into oracle/_ref/libflref_gguf.so.  TEST INFRASTRUCTURE ONLY: used by
// tests/golden/make_gguf_golden.py (in this container) to record what
// fastllm::Gguf (src/model/gguf.cpp) reads from each fixture file.  No
// reference source is copied: its headers are included from the tree by -I.
#include "model/gguf.h"
#include <cstdio>
#include <cstring>
#include <string>

using namespace fastllm;

namespace {
void put_str(std::string & o, const std::string & s) {
    o += '"';
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') { o += '\\'; o += (char)c; }
        else if (c < 0x20 || c >= 0x7f) { char b[8]; snprintf(b, sizeof b, "\\u%04x", c); o += b; }
        else o += (char)c;
    }
    o += '"';
}
uint64_t fnv1a(const uint8_t * p, uint64_t n) {
    uint64_t h = 1469598103934665603ull;
    for (uint64_t i = 0; i < n; ++i) { h ^= p[i]; h *= 1099511628211ull; }
    return h;
}
}  // namespace

extern "C" {

// Opens `path` with Gguf::open and writes a JSON record of everything the
// reader exposes: alignment, shard count, every tensor info with an FNV-1a
// hash of its payload bytes, and for each key of `keys` (newline-separated)
// has / kv_i / kv_f / kv_s / kv_sarr.  Returns the JSON length (truncated to
// cap-1), or -1 when open() returns false.
long ref_gguf_dump(const char * path, const char * keys, char * out, size_t cap) {
    Gguf g;
    if (!g.open(path)) return -1;
    std::string o = "{\"alignment\":" + std::to_string(g.alignment()) +
                    ",\"n_shards\":" + std::to_string(g.n_shards()) + ",\"tensors\":[";
    bool first = true;
    for (const GgufTensor & t : g.tensors()) {
        if (!first) o += ',';
        first = false;
        Fmt f;
        const bool known = Gguf::fmt_of(t.type, &f);
        o += "{\"name\":";
        put_str(o, t.name);
        o += ",\"type\":" + std::to_string(t.type) + ",\"type_name\":";
        put_str(o, Gguf::type_name(t.type));
        o += ",\"fmt\":" + std::to_string(known ? (int)f : -1);
        o += ",\"n_dims\":" + std::to_string(t.n_dims) + ",\"ne\":[";
        for (int d = 0; d < 4; ++d) o += std::to_string(t.ne[d]) + (d < 3 ? "," : "]");
        o += ",\"offset\":" + std::to_string(t.offset) + ",\"nbytes\":" + std::to_string(t.nbytes) +
             ",\"shard\":" + std::to_string(t.shard) + ",\"fnv\":\"" +
             std::to_string(fnv1a(g.data(t), t.nbytes)) + "\"";
        const GgufTensor * ft = g.find(t.name);
        o += ",\"find_is_self\":" + std::string(ft == &t ? "true" : "false") + "}";
    }
    o += "],\"kv\":{";
    first = true;
    std::string ks = keys ? keys : "";
    size_t pos = 0;
    while (pos < ks.size()) {
        size_t nl = ks.find('\n', pos);
        if (nl == std::string::npos) nl = ks.size();
        const std::string k = ks.substr(pos, nl - pos);
        pos = nl + 1;
        if (k.empty()) continue;
        if (!first) o += ',';
        first = false;
        put_str(o, k);
        char fb[64];
        snprintf(fb, sizeof fb, "%.17g", g.kv_f(k, -777.5));
        o += ":{\"has\":" + std::string(g.has(k) ? "true" : "false") +
             ",\"i\":" + std::to_string(g.kv_i(k, -777)) + ",\"f\":" + fb + ",\"s\":";
        put_str(o, g.kv_s(k, "<none>"));
        o += ",\"sarr\":";
        if (const auto * v = g.kv_sarr(k)) {
            o += '[';
            for (size_t i = 0; i < v->size(); ++i) { if (i) o += ','; put_str(o, (*v)[i]); }
            o += ']';
        } else {
            o += "null";
        }
        o += '}';
    }
    o += "}}";
    const size_t n = o.size() < cap ? o.size() : cap - 1;
    memcpy(out, o.data(), n);
    out[n] = 0;
    return (long)n;
}

}  // extern "C"
