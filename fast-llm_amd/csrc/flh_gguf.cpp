// flh_gguf.cpp -- GGUF v2/v3 reader and the host->HBM weight upload.
//
// Behaviour follows the reference's Gguf (src/model/gguf.h:28-79,
// src/model/gguf.cpp:133-303): the file is mmapped read-only, KV metadata is
// captured as int64 / double / string / string-array maps, tensor infos keep
// (type, dims, offset relative to their shard's data section, payload bytes),
// and split models "<stem>-NNNNN-of-MMMMM.gguf" are mapped shard by shard with
// the named shard's metadata kept.  Where the reference aborts on a malformed
// file this returns FLH_ERR_FORMAT; a missing file or shard is FLH_ERR_IO (the
// reference returns false).
//
// The reference then uses the weights in place (unified memory,
// src/model/decoder.cpp:203).  On MI355X the weights are streamed at HBM rate
// only from device memory, so flh_gguf_upload_all copies each shard's whole
// tensor payload span to the device in one pass: the file bytes go through a
// ring of pinned staging buffers, filled by several host threads (page-cache
// reads run at a few GB/s per thread) while the DMA engine drains the
// previous buffer over PCIe.  Tensors keep their file offsets inside the
// device copy, so every device pointer has the file's alignment.
#include <hip/hip_runtime.h>
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <ctype.h>
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>
#include "../../include/fastllm_hip.h"
#include "flh_status.h"
#include "flh_internal.h"

using flh::set_error;
using flh::hip_check;

namespace {

// ggml_type ids this reader gives a payload size to (src/model/gguf.h:12-17)
enum : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14,
    T_IQ2_XXS = 16, T_IQ3_XXS = 18,
};

// GGUF KV value type ids (the GGUF file format, version 2 and 3)
enum : uint32_t {
    V_U8 = 0, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL,
    V_STR, V_ARR, V_U64, V_I64, V_F64,
};

uint64_t value_bytes(uint32_t t) {
    switch (t) {
        case V_U8: case V_I8: case V_BOOL: return 1;
        case V_U16: case V_I16: return 2;
        case V_U32: case V_I32: case V_F32: return 4;
        case V_U64: case V_I64: case V_F64: return 8;
        default: return 0;
    }
}

int fmt_of_type(uint32_t t) {
    switch (t) {
        case T_F32: return FLH_FMT_F32;
        case T_Q8_0: return FLH_FMT_Q8_0;
        case T_Q5_0: return FLH_FMT_Q5_0;
        case T_Q4_K: return FLH_FMT_Q4_K;
        case T_Q6_K: return FLH_FMT_Q6_K;
        case T_IQ2_XXS: return FLH_FMT_IQ2_XXS;
        case T_IQ3_XXS: return FLH_FMT_IQ3_XXS;
        default: return -1;
    }
}

// Bounds-checked little-endian reader over one mapped file.  Any overrun is
// a truncated file.
struct Reader {
    const uint8_t * p;
    const uint8_t * end;
    bool bad = false;
    bool take(uint64_t n) {
        if (bad || (uint64_t)(end - p) < n) { bad = true; return false; }
        return true;
    }
    template <class T> T get() {
        T v{};
        if (take(sizeof(T))) { memcpy(&v, p, sizeof(T)); p += sizeof(T); }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!take(n)) return std::string();
        std::string s((const char *)p, (size_t)n);
        p += n;
        return s;
    }
    void skip(uint64_t n) { if (take(n)) p += n; }
};

struct Shard {
    const uint8_t * base = nullptr;
    size_t size = 0;
    uint64_t data_off = 0;
    int fd = -1;
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    int n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
    int shard = 0;
};

}  // namespace

struct flh_gguf {
    std::vector<Shard> shards;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, uint64_t> index;   // first tensor of a name
    std::map<std::string, int64_t> kv_i;
    std::map<std::string, double> kv_f;
    std::map<std::string, std::string> kv_s;
    std::map<std::string, std::vector<std::string>> kv_sa;
    uint32_t align = 32;

    ~flh_gguf() {
        for (Shard & s : shards) {
            if (s.base) munmap((void *)s.base, s.size);
            if (s.fd >= 0) close(s.fd);
        }
    }
};

namespace {

int fmt_error(const std::string & path, const char * what) {
    return set_error(FLH_ERR_FORMAT, ("gguf " + path + ": " + what).c_str());
}

// Skips one array value (element type, count, elements).  False on a
// truncated file (r.bad) or an element type with no defined size.
bool skip_array(Reader & r) {
    const uint32_t et = r.get<uint32_t>();
    const uint64_t n = r.get<uint64_t>();
    if (r.bad) return false;
    if (et == V_STR) {
        for (uint64_t i = 0; i < n && !r.bad; ++i) r.str();
    } else if (et == V_ARR) {
        for (uint64_t i = 0; i < n && !r.bad; ++i)
            if (!skip_array(r)) return false;
    } else {
        const uint64_t eb = value_bytes(et);
        if (!eb) return false;
        if (n > (uint64_t)(r.end - r.p) / eb) { r.bad = true; return false; }
        r.skip(n * eb);
    }
    return !r.bad;
}

// The tensor payload size for known types (src/model/gguf.cpp:248-256):
// row bytes of ne[0] times the other dims; 2 bytes an element for F16; 0
// (metadata only) for anything else.
// The products are checked (a crafted header could make them wrap and slip
// past the end-of-file check): kOverflow marks a size that does not fit, a
// quantized row wider than 2^32 - 1 elements or not a whole number of blocks.
constexpr uint64_t kOverflow = ~0ull;
uint64_t payload_bytes(const Tensor & t) {
    uint64_t outer = 1;
    for (int d = 1; d < 4; ++d)
        if (__builtin_mul_overflow(outer, t.ne[d], &outer)) return kOverflow;
    const int f = fmt_of_type(t.type);
    uint64_t n = 0;
    if (f >= 0) {
        const uint64_t be = f == FLH_FMT_F32 ? 1 : f == FLH_FMT_Q8_0 || f == FLH_FMT_Q5_0 ? 32 : 256;
        if (t.ne[0] > 0xFFFFFFFFull || t.ne[0] % be) return kOverflow;
        if (__builtin_mul_overflow(flh_row_bytes(f, (uint32_t)t.ne[0]), outer, &n)) return kOverflow;
        return n;
    }
    if (t.type == T_F16) {
        if ((t.ne[0] >> 62) || __builtin_mul_overflow(2 * t.ne[0], outer, &n)) return kOverflow;
        return n;
    }
    return 0;
}

// Maps one file and appends its tensors under shard index `idx`; only when
// keep_kv does its metadata land in g (src/model/gguf.cpp:159-265).
int map_file(flh_gguf * g, const std::string & path, bool keep_kv) {
    Shard sh;
    sh.fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (sh.fd < 0) return set_error(FLH_ERR_IO, ("gguf: cannot open " + path).c_str());
    struct stat st{};
    if (fstat(sh.fd, &st) != 0 || st.st_size < 24) {
        close(sh.fd);
        return fmt_error(path, "truncated file");
    }
    sh.size = (size_t)st.st_size;
    void * m = mmap(nullptr, sh.size, PROT_READ, MAP_PRIVATE, sh.fd, 0);
    if (m == MAP_FAILED) {
        close(sh.fd);
        return set_error(FLH_ERR_IO, ("gguf: mmap failed for " + path).c_str());
    }
    sh.base = (const uint8_t *)m;
    const int idx = (int)g->shards.size();
    g->shards.push_back(sh);            // owned by g from here on (unmapped by its destructor)

    Reader r{sh.base, sh.base + sh.size};
    if (r.get<uint32_t>() != 0x46554747u) return fmt_error(path, "bad magic");
    const uint32_t version = r.get<uint32_t>();
    if (version < 2 || version > 3) return fmt_error(path, "unsupported version");
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kv = r.get<uint64_t>();

    flh_gguf scratch;                   // metadata of shards the caller did not name
    flh_gguf & kv = keep_kv ? *g : scratch;
    uint32_t align = 32;
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = r.str();
        const uint32_t t = r.get<uint32_t>();
        if (r.bad) break;
        switch (t) {
            case V_U8: kv.kv_i[key] = r.get<uint8_t>(); break;
            case V_I8: kv.kv_i[key] = r.get<int8_t>(); break;
            case V_BOOL: kv.kv_i[key] = r.get<uint8_t>() != 0; break;
            case V_U16: kv.kv_i[key] = r.get<uint16_t>(); break;
            case V_I16: kv.kv_i[key] = r.get<int16_t>(); break;
            case V_U32: kv.kv_i[key] = r.get<uint32_t>(); break;
            case V_I32: kv.kv_i[key] = r.get<int32_t>(); break;
            case V_U64: kv.kv_i[key] = (int64_t)r.get<uint64_t>(); break;
            case V_I64: kv.kv_i[key] = r.get<int64_t>(); break;
            case V_F32: kv.kv_f[key] = r.get<float>(); break;
            case V_F64: kv.kv_f[key] = r.get<double>(); break;
            case V_STR: kv.kv_s[key] = r.str(); break;
            case V_ARR: {
                // string arrays are kept (tokenizer vocabularies); others skipped
                const uint8_t * at = r.p;
                const uint32_t et = r.get<uint32_t>();
                if (et == V_STR) {
                    const uint64_t n = r.get<uint64_t>();
                    // a repeated key appends, as the reference's capture does
                    // (src/model/gguf.cpp:220-223)
                    std::vector<std::string> & v = kv.kv_sa[key];
                    for (uint64_t j = 0; j < n && !r.bad; ++j) v.push_back(r.str());
                } else {
                    r.p = at;
                    if (!skip_array(r) && !r.bad) return fmt_error(path, "bad array element type");
                }
                break;
            }
            default:
                return fmt_error(path, "bad kv type");
        }
        if (key == "general.alignment") {
            auto it = kv.kv_i.find(key);
            if (it != kv.kv_i.end() && it->second > 0) {
                if (it->second & (it->second - 1))
                    return fmt_error(path, "general.alignment is not a power of two");
                align = (uint32_t)it->second;
            }
        }
    }
    if (r.bad) return fmt_error(path, "truncated file");
    if (keep_kv) g->align = align;

    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        t.name = r.str();
        t.n_dims = (int)r.get<uint32_t>();
        if (r.bad) break;
        if (t.n_dims < 1 || t.n_dims > 4) return fmt_error(path, "bad n_dims");
        for (int d = 0; d < t.n_dims; ++d) t.ne[d] = r.get<uint64_t>();
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (r.bad) break;
        t.nbytes = payload_bytes(t);
        if (t.nbytes == kOverflow) return fmt_error(path, ("tensor " + t.name + " has an impossible size").c_str());
        t.shard = idx;
        g->tensors.push_back(std::move(t));
    }
    if (r.bad) return fmt_error(path, "truncated file");
    const uint64_t hdr = (uint64_t)(r.p - sh.base);
    const uint64_t data_off = (hdr + align - 1) & ~(uint64_t)(align - 1);
    g->shards[idx].data_off = data_off;
    // the reference trusts the offsets; a payload past the end of the file
    // is rejected here instead of being read out of the mapping's bounds
    for (size_t i = g->tensors.size() - (size_t)n_tensors; i < g->tensors.size(); ++i) {
        const Tensor & t = g->tensors[i];
        if (data_off > sh.size || t.offset > sh.size - data_off ||
            t.nbytes > sh.size - data_off - t.offset)
            return fmt_error(path, ("tensor " + t.name + " extends past the end of the file").c_str());
    }
    madvise((void *)sh.base, sh.size, MADV_WILLNEED);
    return FLH_OK;
}

// "<stem>-NNNNN-of-MMMMM.gguf" -> MMMMM and a printf pattern for the shard
// names; 0 when the name is not a split name (src/model/gguf.cpp:112-131).
int split_count(const std::string & path, std::string * pattern) {
    static const char ext[] = ".gguf";
    const size_t ne = sizeof(ext) - 1;
    if (path.size() < ne + 14 || path.compare(path.size() - ne, ne, ext) != 0) return 0;
    const size_t tail = path.size() - ne;
    const size_t of = tail - 9;          // "-of-" then 5 digits
    if (path.compare(of, 4, "-of-") != 0 || of < 6) return 0;
    const size_t dash = of - 6;          // "-" then 5 digits of the shard number
    if (path[dash] != '-') return 0;
    for (size_t i = dash + 1; i < tail; ++i)
        if (i < of || i >= of + 4)
            if (!isdigit((unsigned char)path[i])) return 0;
    const int total = atoi(path.c_str() + of + 4);
    if (total < 1 || total > 999) return 0;
    *pattern = path.substr(0, dash) + "-%05d-of-" + path.substr(of + 4, 5) + ext;
    return total;
}

// ------------------------------------------------------------- upload ----
// Pinned staging ring shared by every upload of the process.
constexpr size_t kStageBytes = 64u << 20;
constexpr int kStages = 4;

struct Stager {
    std::mutex mu;
    int device = -1;
    void * buf[kStages] = {};
    hipEvent_t done[kStages] = {};
    bool used[kStages] = {};
};
Stager g_stage;

// host threads copying a tensor into the pinned staging ring (FLH_GGUF_THREADS,
// read at flh_init; 0: the hardware's, at most 16)
unsigned copy_threads() {
    const unsigned v = flh::tune().gguf_threads ? flh::tune().gguf_threads : std::thread::hardware_concurrency();
    return std::max(1u, std::min(v, 16u));
}

// memcpy of n bytes split over the copy threads (each part faults its own
// pages of the mapping in)
void parallel_copy(void * dst, const void * src, size_t n) {
    const unsigned nt = n < (4u << 20) ? 1u : copy_threads();
    if (nt == 1) { memcpy(dst, src, n); return; }
    const size_t part = ((n + nt - 1) / nt + 4095) & ~(size_t)4095;
    std::vector<std::thread> th;
    for (unsigned i = 1; i < nt; ++i) {
        const size_t lo = i * part;
        if (lo >= n) break;
        const size_t len = std::min(part, n - lo);
        th.emplace_back([=] { memcpy((uint8_t *)dst + lo, (const uint8_t *)src + lo, len); });
    }
    memcpy(dst, src, std::min(part, n));
    for (auto & t : th) t.join();
}

int stager_ready() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(FLH_ERR_STATE, "no current device");
    if (g_stage.device == dev) return FLH_OK;
    if (g_stage.device >= 0) {
        for (int i = 0; i < kStages; ++i) {
            if (g_stage.used[i]) (void)hipEventSynchronize(g_stage.done[i]);
            (void)hipEventDestroy(g_stage.done[i]);
            (void)hipHostFree(g_stage.buf[i]);
            g_stage.buf[i] = nullptr;
            g_stage.used[i] = false;
        }
        g_stage.device = -1;
    }
    for (int i = 0; i < kStages; ++i) {
        if (int rc = hip_check(hipHostMalloc(&g_stage.buf[i], kStageBytes, hipHostMallocDefault),
                               "gguf staging hipHostMalloc"))
            return rc;
        if (int rc = hip_check(hipEventCreateWithFlags(&g_stage.done[i], hipEventDisableTiming),
                               "gguf staging event"))
            return rc;
    }
    g_stage.device = dev;
    return FLH_OK;
}

// Copies n host bytes to dst on `s` through the staging ring; returns once
// every byte is on the device.
int staged_h2d(uint8_t * dst, const uint8_t * src, size_t n, hipStream_t s) {
    int k = 0;
    for (size_t done = 0; done < n; done += kStageBytes, k = (k + 1) % kStages) {
        const size_t len = std::min(kStageBytes, n - done);
        if (g_stage.used[k])
            if (int rc = hip_check(hipEventSynchronize(g_stage.done[k]), "gguf staging wait")) return rc;
        parallel_copy(g_stage.buf[k], src + done, len);
        if (int rc = hip_check(hipMemcpyAsync(dst + done, g_stage.buf[k], len, hipMemcpyHostToDevice, s),
                               "gguf upload hipMemcpyAsync"))
            return rc;
        if (int rc = hip_check(hipEventRecord(g_stage.done[k], s), "gguf staging record")) return rc;
        g_stage.used[k] = true;
    }
    for (int i = 0; i < kStages; ++i)
        if (g_stage.used[i]) {
            if (int rc = hip_check(hipEventSynchronize(g_stage.done[i]), "gguf staging wait")) return rc;
            g_stage.used[i] = false;
        }
    return FLH_OK;
}

}  // namespace

extern "C" {

int flh_gguf_open(const char * path, flh_gguf ** out) {
    if (!path || !out) return set_error(FLH_ERR_ARG, "null path / out");
    *out = nullptr;
    flh_gguf * g = new flh_gguf;
    const std::string p(path);
    std::string pattern;
    const int total = split_count(p, &pattern);
    int rc = FLH_OK;
    if (total <= 1) {
        rc = map_file(g, p, true);
    } else {
        char name[4096];
        for (int i = 1; i <= total && rc == FLH_OK; ++i) {
            snprintf(name, sizeof name, pattern.c_str(), i);
            rc = map_file(g, name, p == name);
            if (rc == FLH_ERR_IO)
                set_error(rc, (std::string("gguf: missing shard ") + name).c_str());
        }
        if (rc == FLH_OK) {
            auto it = g->kv_i.find("split.tensors.count");
            int64_t want = it != g->kv_i.end() ? it->second : 0;
            if (it == g->kv_i.end()) {
                auto itf = g->kv_f.find("split.tensors.count");
                if (itf != g->kv_f.end()) want = (int64_t)itf->second;
            }
            if (want > 0 && (uint64_t)want != g->tensors.size())
                rc = fmt_error(p, "split.tensors.count does not match the tensors mapped");
        }
    }
    if (rc != FLH_OK) { delete g; return rc; }
    for (uint64_t i = 0; i < g->tensors.size(); ++i) g->index.emplace(g->tensors[i].name, i);
    *out = g;
    return FLH_OK;
}

int flh_gguf_close(flh_gguf * g) {
    delete g;
    return FLH_OK;
}

uint32_t flh_gguf_alignment(const flh_gguf * g) { return g ? g->align : 0; }
int flh_gguf_n_shards(const flh_gguf * g) { return g ? (int)g->shards.size() : 0; }
uint64_t flh_gguf_n_tensors(const flh_gguf * g) { return g ? g->tensors.size() : 0; }

int flh_gguf_tensor_info(const flh_gguf * g, uint64_t i, flh_gguf_tensor * out) {
    if (!g || !out) return set_error(FLH_ERR_ARG, "null gguf / out");
    if (i >= g->tensors.size()) return set_error(FLH_ERR_ARG, "tensor index out of range");
    const Tensor & t = g->tensors[i];
    const Shard & s = g->shards[t.shard];
    out->name = t.name.c_str();
    out->name_len = t.name.size();
    out->type = t.type;
    out->fmt = fmt_of_type(t.type);
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->shard = t.shard;
    out->data = s.base + s.data_off + t.offset;
    return FLH_OK;
}

int64_t flh_gguf_find(const flh_gguf * g, const char * name) {
    if (!g || !name) return -1;
    auto it = g->index.find(name);
    return it == g->index.end() ? -1 : (int64_t)it->second;
}

int flh_gguf_fmt_of(uint32_t ggml_type) { return fmt_of_type(ggml_type); }

const char * flh_gguf_type_name(uint32_t t) {
    switch (t) {
        case T_F32: return "F32"; case T_F16: return "F16"; case T_Q5_0: return "Q5_0";
        case T_Q8_0: return "Q8_0"; case T_Q4_K: return "Q4_K"; case T_Q6_K: return "Q6_K";
        case T_IQ2_XXS: return "IQ2_XXS"; case T_IQ3_XXS: return "IQ3_XXS";
    }
    static thread_local char buf[16];
    snprintf(buf, sizeof buf, "type%u", t);
    return buf;
}

int flh_gguf_has(const flh_gguf * g, const char * k) {
    if (!g || !k) return 0;
    return g->kv_i.count(k) || g->kv_f.count(k) || g->kv_s.count(k) || g->kv_sa.count(k);
}

int64_t flh_gguf_kv_i(const flh_gguf * g, const char * k, int64_t dflt) {
    if (!g || !k) return dflt;
    auto it = g->kv_i.find(k);
    if (it != g->kv_i.end()) return it->second;
    auto itf = g->kv_f.find(k);
    return itf != g->kv_f.end() ? (int64_t)itf->second : dflt;
}

double flh_gguf_kv_f(const flh_gguf * g, const char * k, double dflt) {
    if (!g || !k) return dflt;
    auto it = g->kv_f.find(k);
    if (it != g->kv_f.end()) return it->second;
    auto iti = g->kv_i.find(k);
    return iti != g->kv_i.end() ? (double)iti->second : dflt;
}

const char * flh_gguf_kv_s(const flh_gguf * g, const char * k, const char * dflt,
                           size_t * len) {
    const char * v = dflt;
    size_t n = dflt ? strlen(dflt) : 0;
    if (g && k) {
        auto it = g->kv_s.find(k);
        if (it != g->kv_s.end()) { v = it->second.c_str(); n = it->second.size(); }
    }
    if (len) *len = n;
    return v;
}

int64_t flh_gguf_kv_sarr_len(const flh_gguf * g, const char * k) {
    if (!g || !k) return -1;
    auto it = g->kv_sa.find(k);
    return it == g->kv_sa.end() ? -1 : (int64_t)it->second.size();
}

const char * flh_gguf_kv_sarr_at(const flh_gguf * g, const char * k, uint64_t i, size_t * len) {
    if (!g || !k) return nullptr;
    auto it = g->kv_sa.find(k);
    if (it == g->kv_sa.end() || i >= it->second.size()) return nullptr;
    if (len) *len = it->second[i].size();
    return it->second[i].c_str();
}

int flh_gguf_weight(const flh_gguf * g, const char * name, flh_weight * out) {
    if (!g || !name || !out) return set_error(FLH_ERR_ARG, "null gguf / name / out");
    const int64_t i = flh_gguf_find(g, name);
    if (i < 0) return set_error(FLH_ERR_ARG, (std::string("gguf: missing tensor ") + name).c_str());
    const Tensor & t = g->tensors[(size_t)i];
    const int f = fmt_of_type(t.type);
    if (f < 0)
        return set_error(FLH_ERR_UNSUPPORTED, (std::string("gguf: ") + name + " unsupported type " +
                                               flh_gguf_type_name(t.type)).c_str());
    const Shard & s = g->shards[t.shard];
    if (t.ne[0] > 0xFFFFFFFFull || t.ne[1] > 0xFFFFFFFFull || (t.n_dims >= 3 && t.ne[2] > 0xFFFFFFFFull) ||
        (t.n_dims == 4 && t.ne[3] != 1))
        return set_error(FLH_ERR_UNSUPPORTED, (std::string("gguf: ") + name + " has dimensions a weight cannot take").c_str());
    out->fmt = f;
    out->cols = (uint32_t)t.ne[0];
    out->rows = (uint32_t)t.ne[1];
    out->nexp = (uint32_t)(t.n_dims >= 3 ? t.ne[2] : 1);
    out->row_bytes = flh_row_bytes(f, out->cols);
    out->w_bytes = out->row_bytes * out->rows;
    out->estride = out->nexp > 1 ? out->w_bytes : 0;
    uint64_t all = 0;                                     // every expert lies inside the payload
    if (__builtin_mul_overflow(out->w_bytes, (uint64_t)out->nexp, &all) || all > t.nbytes)
        return set_error(FLH_ERR_UNSUPPORTED, (std::string("gguf: ") + name + " payload smaller than its experts").c_str());
    out->host = s.base + s.data_off + t.offset;
    out->tensor = (uint64_t)i;
    return FLH_OK;
}

int flh_gguf_upload(const flh_gguf * g, uint64_t i, void * dst, uint64_t dst_bytes, void * stream) {
    if (!g || !dst) return set_error(FLH_ERR_ARG, "null gguf / destination");
    if (i >= g->tensors.size()) return set_error(FLH_ERR_ARG, "tensor index out of range");
    const Tensor & t = g->tensors[i];
    if (t.nbytes == 0) return set_error(FLH_ERR_UNSUPPORTED, "tensor type has no known payload size");
    if (dst_bytes < t.nbytes) return set_error(FLH_ERR_ARG, "destination smaller than the tensor");
    if (int rc = flh::need_device()) return rc;
    std::lock_guard<std::mutex> lk(g_stage.mu);
    if (int rc = stager_ready()) return rc;
    const Shard & s = g->shards[t.shard];
    return staged_h2d((uint8_t *)dst, s.base + s.data_off + t.offset, t.nbytes, (hipStream_t)stream);
}

int flh_gguf_upload_all(const flh_gguf * g, flh_arena * arena, void ** dev_ptrs, void * stream) {
    if (!g || !arena || !dev_ptrs) return set_error(FLH_ERR_ARG, "null gguf / arena / dev_ptrs");
    if (int rc = flh::need_device()) return rc;
    std::vector<uint64_t> span(g->shards.size(), 0);
    for (const Tensor & t : g->tensors)
        if (t.nbytes) span[t.shard] = std::max(span[t.shard], t.offset + t.nbytes);
    std::vector<uint8_t *> base(g->shards.size(), nullptr);
    for (size_t s = 0; s < span.size(); ++s) {
        if (!span[s]) continue;
        void * p = nullptr;
        if (int rc = flh_arena_alloc(arena, span[s], 256, &p)) return rc;
        base[s] = (uint8_t *)p;
    }
    {
        std::lock_guard<std::mutex> lk(g_stage.mu);
        if (int rc = stager_ready()) return rc;
        for (size_t s = 0; s < span.size(); ++s)
            if (span[s])
                if (int rc = staged_h2d(base[s], g->shards[s].base + g->shards[s].data_off, span[s],
                                        (hipStream_t)stream))
                    return rc;
    }
    for (size_t i = 0; i < g->tensors.size(); ++i) {
        const Tensor & t = g->tensors[i];
        dev_ptrs[i] = t.nbytes ? base[t.shard] + t.offset : nullptr;
    }
    return FLH_OK;
}

}  // extern "C"
