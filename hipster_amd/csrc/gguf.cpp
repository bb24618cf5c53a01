// gguf.cpp -- the on-disk side of the path: a GGUF v3 reader (mmap, KV header, tensor table, shard
// joining, pread of a tensor) and the engine's load-time choice of the layout the kernels read,
// with the row repacks / requantisation that produce it.  Host code only (no GPU calls).
//
//   qmm_gguf_*             hip::GGUF            engine/src/gguf.h:43-76, gguf.cpp:71-156
//   qmm_gtype_block        gtype_block          gguf.h:20, gguf.cpp:26-42
//   qmm_weight_format,
//   qmm_prepare_weight     to_lin / upload_lin  engine/src/qwen4exp.cpp:34-65, qwen35.cpp:31-58
//
// The file format is GGUF v3 (ggml's): magic "GGUF", version 3, tensor and KV counts, the KV pairs
// (typed values, arrays of typed values), the tensor infos (name, dims, ggml type, offset), then the
// data at the next multiple of general.alignment (default 32).  Split models are named
// <base>-0000i-of-0000N.gguf; opening any shard opens all of them and joins their tensor tables.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <regex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/hipster_qmm.h"

namespace {

// ggml type -> (elements per block, bytes per block); 0 for a type this reader does not size
bool gtype_block(int t, uint32_t& bs, uint32_t& tb) {
    switch (t) {
        case QMM_GGML_F32: bs = 1; tb = 4; return true;
        case QMM_GGML_F16: case QMM_GGML_BF16: bs = 1; tb = 2; return true;
        case QMM_GGML_I8: bs = 1; tb = 1; return true;
        case QMM_GGML_I32: bs = 1; tb = 4; return true;
        case QMM_GGML_Q4_0: bs = 32; tb = 18; return true;
        case QMM_GGML_Q4_1: bs = 32; tb = 20; return true;
        case QMM_GGML_Q5_0: bs = 32; tb = 22; return true;
        case QMM_GGML_Q5_1: bs = 32; tb = 24; return true;
        case QMM_GGML_Q8_0: bs = 32; tb = 34; return true;
        case QMM_GGML_Q8_1: bs = 32; tb = 36; return true;
        case QMM_GGML_Q2_K: bs = 256; tb = 84; return true;
        case QMM_GGML_Q3_K: bs = 256; tb = 110; return true;
        case QMM_GGML_Q4_K: bs = 256; tb = 144; return true;
        case QMM_GGML_Q5_K: bs = 256; tb = 176; return true;
        case QMM_GGML_Q6_K: bs = 256; tb = 210; return true;
        case QMM_GGML_Q8_K: bs = 256; tb = 292; return true;
        case QMM_GGML_IQ4_NL: bs = 32; tb = 18; return true;
        case QMM_GGML_IQ4_XS: bs = 256; tb = 136; return true;
        case QMM_GGML_IQ3_S: bs = 256; tb = 110; return true;
        default: return false;
    }
}

struct Value {
    int kind = 0;            // QMM_GGUF_KV_*
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
    uint64_t arr_len = 0;
};

struct Reader {
    const uint8_t* p;
    const uint8_t* end;
    bool ok = true;
    template <class T>
    T rd() {
        T v{};
        if (!ok || (size_t)(end - p) < sizeof(T)) { ok = false; return v; }
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = rd<uint64_t>();
        if (!ok || (uint64_t)(end - p) < n) { ok = false; return std::string(); }
        std::string s((const char*)p, (size_t)n);
        p += n;
        return s;
    }
};

// one typed value (GGUF value types 0..12); arrays keep their length (their elements are read past)
bool read_value(Reader& c, uint32_t type, Value& v, int depth = 0) {
    switch (type) {
        case 0: v.kind = QMM_GGUF_KV_UINT; v.u = c.rd<uint8_t>(); break;
        case 1: v.kind = QMM_GGUF_KV_INT; v.i = c.rd<int8_t>(); break;
        case 2: v.kind = QMM_GGUF_KV_UINT; v.u = c.rd<uint16_t>(); break;
        case 3: v.kind = QMM_GGUF_KV_INT; v.i = c.rd<int16_t>(); break;
        case 4: v.kind = QMM_GGUF_KV_UINT; v.u = c.rd<uint32_t>(); break;
        case 5: v.kind = QMM_GGUF_KV_INT; v.i = c.rd<int32_t>(); break;
        case 6: v.kind = QMM_GGUF_KV_FLOAT; v.f = c.rd<float>(); break;
        case 7: v.kind = QMM_GGUF_KV_BOOL; v.u = c.rd<uint8_t>(); break;
        case 8: v.kind = QMM_GGUF_KV_STRING; v.s = c.str(); break;
        case 9: {
            if (depth > 4) return false;
            v.kind = QMM_GGUF_KV_ARRAY;
            const uint32_t et = c.rd<uint32_t>();
            v.arr_len = c.rd<uint64_t>();
            for (uint64_t k = 0; k < v.arr_len && c.ok; ++k) {
                Value e;
                if (!read_value(c, et, e, depth + 1)) return false;
            }
            break;
        }
        case 10: v.kind = QMM_GGUF_KV_UINT; v.u = c.rd<uint64_t>(); break;
        case 11: v.kind = QMM_GGUF_KV_INT; v.i = c.rd<int64_t>(); break;
        case 12: v.kind = QMM_GGUF_KV_FLOAT; v.f = c.rd<double>(); break;
        default: return false;
    }
    return c.ok;
}

struct Map { void* p; size_t len; int fd; };

}  // namespace

struct qmm_gguf {
    std::vector<Map> maps;
    std::vector<qmm_gguf_tensor> tensors;
    std::vector<std::string> names;           // storage of the tensor names (tensors[i].name points here)
    std::unordered_map<std::string, size_t> index;
    std::unordered_map<std::string, Value> kv;
    size_t mapped = 0;

    ~qmm_gguf() {
        for (auto& m : maps) {
            munmap(m.p, m.len);
            ::close(m.fd);
        }
    }

    int open_one(const std::string& path) {
        const int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) return QMM_ERR_IO;
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size < 24) { ::close(fd); return QMM_ERR_IO; }
        void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) { ::close(fd); return QMM_ERR_IO; }
        maps.push_back({p, (size_t)st.st_size, fd});
        mapped += (size_t)st.st_size;
        const uint8_t* base = (const uint8_t*)p;
        Reader c{base, base + st.st_size};
        if (c.rd<uint32_t>() != 0x46554747u) return QMM_ERR_IO;          // "GGUF"
        if (c.rd<uint32_t>() != 3u) return QMM_ERR_IO;                   // version 3 only
        const uint64_t n_tensors = c.rd<uint64_t>(), n_kv = c.rd<uint64_t>();
        for (uint64_t k = 0; k < n_kv && c.ok; ++k) {
            std::string key = c.str();
            const uint32_t type = c.rd<uint32_t>();
            Value v;
            if (!read_value(c, type, v)) return QMM_ERR_IO;
            // later shards overwrite a key, except the split.* bookkeeping, which keeps the first
            if (!kv.count(key) || key.rfind("split.", 0) != 0) kv[key] = std::move(v);
        }
        if (!c.ok) return QMM_ERR_IO;
        struct Info { std::string name; uint32_t nd; uint64_t ne[4]; uint32_t type; uint64_t off; };
        std::vector<Info> infos;
        for (uint64_t k = 0; k < n_tensors && c.ok; ++k) {
            Info t;
            t.name = c.str();
            t.nd = c.rd<uint32_t>();
            if (t.nd > 4) return QMM_ERR_IO;
            for (int d = 0; d < 4; ++d) t.ne[d] = 1;
            for (uint32_t d = 0; d < t.nd; ++d) t.ne[d] = c.rd<uint64_t>();
            t.type = c.rd<uint32_t>();
            t.off = c.rd<uint64_t>();
            infos.push_back(std::move(t));
        }
        if (!c.ok) return QMM_ERR_IO;
        uint64_t align = 32;
        auto a = kv.find("general.alignment");
        if (a != kv.end() && a->second.kind == QMM_GGUF_KV_UINT && a->second.u > 0) align = a->second.u;
        const uint64_t data_start = ((uint64_t)(c.p - base) + align - 1) / align * align;
        for (auto& t : infos) {
            uint32_t bs, tb;
            if (!gtype_block((int)t.type, bs, tb)) return QMM_ERR_FORMAT;
            const uint64_t n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
            if (t.ne[0] % bs != 0) return QMM_ERR_IO;
            qmm_gguf_tensor g;
            memset(&g, 0, sizeof g);
            g.type = (int32_t)t.type;
            g.n_dims = t.nd;
            for (int d = 0; d < 4; ++d) g.ne[d] = t.ne[d];
            g.nbytes = (size_t)(n / bs * tb);
            g.file_off = data_start + t.off;
            g.shard = (int32_t)maps.size() - 1;
            if (g.file_off > (uint64_t)st.st_size || g.nbytes > (uint64_t)st.st_size - g.file_off) return QMM_ERR_IO;   // past EOF
            g.data = base + g.file_off;
            index[t.name] = tensors.size();
            names.push_back(t.name);
            tensors.push_back(g);
        }
        return QMM_OK;
    }

    void fix_names() {   // names may have moved while the vector grew
        for (size_t i = 0; i < tensors.size(); ++i) tensors[i].name = names[i].c_str();
    }
};

namespace {

// f32 -> f16 as quant.h:150-155 does it: truncate the mantissa and add one when the first dropped bit
// is set (round half away from zero in magnitude), subnormals alike; tiny values -> signed zero,
// large ones -> infinity
uint16_t f32_to_f16_loadtime(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t s = (x >> 16) & 0x8000u;
    const int e = (int)((x >> 23) & 0xffu) - 127 + 15;
    uint32_t m = x & 0x7fffffu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)s;
        m |= 0x800000u;
        const uint32_t t = (uint32_t)(14 - e);
        uint32_t r = m >> t;
        if ((m >> (t - 1)) & 1u) r++;
        return (uint16_t)(s | r);
    }
    if (e >= 31) return (uint16_t)(s | 0x7c00u);
    uint32_t r = s | ((uint32_t)e << 10) | (m >> 13);
    if (m & 0x1000u) r++;
    return (uint16_t)r;
}
float f16_to_f32_host(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = sign;
        else {
            const float v = ldexpf((float)m, -24);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) bits = sign | 0x7f800000u | (m << 13);
    else bits = sign | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// one row of F32 / F16 / BF16 -> f32 (quant.h:197-199)
void float_row(int type, const uint8_t* src, float* dst, int K) {
    if (type == QMM_GGML_F32) memcpy(dst, src, (size_t)K * 4);
    else if (type == QMM_GGML_F16) for (int i = 0; i < K; ++i) { uint16_t h; memcpy(&h, src + 2 * i, 2); dst[i] = f16_to_f32_host(h); }
    else for (int i = 0; i < K; ++i) { uint16_t b; memcpy(&b, src + 2 * i, 2); const uint32_t u = (uint32_t)b << 16; memcpy(dst + i, &u, 4); }
}

// f32 row -> Q8_0 row-SoA [q K int8][d K/32 f16] (quant.h:174-183): d = f16(amax/127), q = rint(x / d)
void quantize_row_q8_0_soa(const float* x, uint8_t* dst, int K) {
    int8_t* q = (int8_t*)dst;
    uint8_t* dd = dst + K;
    for (int b = 0; b < K / 32; ++b) {
        float amax = 0.f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[b * 32 + j]));
        const uint16_t h = f32_to_f16_loadtime(amax / 127.f);
        memcpy(dd + 2 * b, &h, 2);
        const float dq = f16_to_f32_host(h), idq = dq != 0.f ? 1.f / dq : 0.f;
        for (int j = 0; j < 32; ++j) q[b * 32 + j] = (int8_t)nearbyintf(x[b * 32 + j] * idq);
    }
}

template <class F>
void parallel_rows(int N, int nthreads, F fn) {
    if (nthreads <= 1 || N < 2) {
        for (int r = 0; r < N; ++r) fn(r);
        return;
    }
    std::vector<std::thread> th;
    for (int i = 0; i < nthreads; ++i) th.emplace_back([=] { for (int r = i; r < N; r += nthreads) fn(r); });
    for (auto& t : th) t.join();
}

}  // namespace

extern "C" {

int qmm_gtype_block(int type, uint32_t* block_elems, uint32_t* block_bytes) {
    uint32_t bs, tb;
    if (!gtype_block(type, bs, tb)) return QMM_ERR_FORMAT;
    if (block_elems) *block_elems = bs;
    if (block_bytes) *block_bytes = tb;
    return QMM_OK;
}

int qmm_gguf_open(const char* path, qmm_gguf** out) {
    if (!path || !out) return QMM_ERR_NULL;
    *out = nullptr;
    qmm_gguf* g = new qmm_gguf();
    static const std::regex re(R"(^(.*)-(\d{5})-of-(\d{5})\.gguf$)");
    std::smatch m;
    const std::string p(path);
    int rc = QMM_OK;
    if (std::regex_match(p, m, re)) {
        const int n = std::stoi(m[3].str());
        for (int i = 1; i <= n && rc == QMM_OK; ++i) {
            char buf[32];
            snprintf(buf, sizeof buf, "-%05d-of-%05d.gguf", i, n);
            rc = g->open_one(m[1].str() + buf);
        }
    } else {
        rc = g->open_one(p);
    }
    if (rc != QMM_OK) {
        delete g;
        return rc;
    }
    g->fix_names();
    *out = g;
    return QMM_OK;
}

void qmm_gguf_close(qmm_gguf* g) { delete g; }

int64_t qmm_gguf_n_tensors(const qmm_gguf* g) { return g ? (int64_t)g->tensors.size() : 0; }

size_t qmm_gguf_mapped_bytes(const qmm_gguf* g) { return g ? g->mapped : 0; }

int qmm_gguf_tensor_at(const qmm_gguf* g, int64_t i, qmm_gguf_tensor* out) {
    if (!g || !out) return QMM_ERR_NULL;
    if (i < 0 || i >= (int64_t)g->tensors.size()) return QMM_ERR_ARG;
    *out = g->tensors[(size_t)i];
    return QMM_OK;
}

int qmm_gguf_find(const qmm_gguf* g, const char* name, qmm_gguf_tensor* out) {
    if (!g || !name || !out) return QMM_ERR_NULL;
    auto it = g->index.find(name);
    if (it == g->index.end()) return QMM_ERR_NOT_FOUND;
    *out = g->tensors[it->second];
    return QMM_OK;
}

int qmm_gguf_kv_kind(const qmm_gguf* g, const char* key, int* kind) {
    if (!g || !key || !kind) return QMM_ERR_NULL;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return QMM_ERR_NOT_FOUND;
    *kind = it->second.kind;
    return QMM_OK;
}

int qmm_gguf_kv_u32(const qmm_gguf* g, const char* key, uint32_t* out) {
    if (!g || !key || !out) return QMM_ERR_NULL;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return QMM_ERR_NOT_FOUND;
    const Value& v = it->second;
    if (v.kind == QMM_GGUF_KV_INT) *out = (uint32_t)v.i;         // gguf.cpp:141: signed values reinterpreted
    else if (v.kind == QMM_GGUF_KV_UINT || v.kind == QMM_GGUF_KV_BOOL) *out = (uint32_t)v.u;
    else return QMM_ERR_ARG;
    return QMM_OK;
}

int qmm_gguf_kv_f32(const qmm_gguf* g, const char* key, float* out) {
    if (!g || !key || !out) return QMM_ERR_NULL;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return QMM_ERR_NOT_FOUND;
    if (it->second.kind != QMM_GGUF_KV_FLOAT) return QMM_ERR_ARG;
    *out = (float)it->second.f;
    return QMM_OK;
}

int qmm_gguf_kv_str(const qmm_gguf* g, const char* key, const char** out) {
    if (!g || !key || !out) return QMM_ERR_NULL;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return QMM_ERR_NOT_FOUND;
    if (it->second.kind != QMM_GGUF_KV_STRING) return QMM_ERR_ARG;
    *out = it->second.s.c_str();
    return QMM_OK;
}

int qmm_gguf_kv_array_len(const qmm_gguf* g, const char* key, uint64_t* out) {
    if (!g || !key || !out) return QMM_ERR_NULL;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return QMM_ERR_NOT_FOUND;
    if (it->second.kind != QMM_GGUF_KV_ARRAY) return QMM_ERR_ARG;
    *out = it->second.arr_len;
    return QMM_OK;
}

int qmm_gguf_read_tensor(const qmm_gguf* g, const char* name, void* dst, size_t dst_bytes) {
    if (!g || !name || !dst) return QMM_ERR_NULL;
    auto it = g->index.find(name);
    if (it == g->index.end()) return QMM_ERR_NOT_FOUND;
    const qmm_gguf_tensor& t = g->tensors[it->second];
    if (dst_bytes < t.nbytes) return QMM_ERR_SHAPE;
    const int fd = g->maps[(size_t)t.shard].fd;
    size_t done = 0;
    while (done < t.nbytes) {
        const ssize_t r = pread(fd, (char*)dst + done, t.nbytes - done, (off_t)(t.file_off + done));
        if (r <= 0) return QMM_ERR_IO;
        done += (size_t)r;
    }
    posix_fadvise(fd, (off_t)t.file_off, (off_t)t.nbytes, POSIX_FADV_DONTNEED);   // keep the page cache small
    return QMM_OK;
}

int qmm_weight_format(int gtype, int K, int* wfmt, size_t* row_bytes) {
    if (!wfmt || !row_bytes) return QMM_ERR_NULL;
    int f;
    switch (gtype) {
        case QMM_GGML_Q4_K: f = QMM_Q4_K; break;
        case QMM_GGML_Q5_K: f = QMM_Q5_K; break;
        case QMM_GGML_IQ4_XS: f = QMM_IQ4_XS; break;
        case QMM_GGML_Q6_K: f = QMM_Q6_K_SOA; break;
        case QMM_GGML_Q8_0: f = QMM_Q8_0_SOA; break;
        case QMM_GGML_Q5_0: case QMM_GGML_Q5_1: f = QMM_Q5_1_SOA; break;
        case QMM_GGML_F32: case QMM_GGML_F16: case QMM_GGML_BF16: f = QMM_Q8_0_SOA; break;   // requantised at load
        default: return QMM_ERR_FORMAT;
    }
    const size_t rb = qmm_wfmt_row_bytes(f, K);
    if (rb == 0) return QMM_ERR_SHAPE;
    *wfmt = f;
    *row_bytes = rb;
    return QMM_OK;
}

int qmm_prepare_weight(int gtype, const uint8_t* src, int N, int K, uint8_t* dst, int nthreads) {
    if (!src || !dst) return QMM_ERR_NULL;
    int f;
    size_t rb;
    if (int e = qmm_weight_format(gtype, K, &f, &rb)) return e;
    if (N <= 0) return QMM_ERR_SHAPE;
    uint32_t bs, tb;
    if (!gtype_block(gtype, bs, tb) || K % (int)bs != 0) return QMM_ERR_SHAPE;
    const size_t rs = (size_t)(K / (int)bs) * tb;             // source row bytes
    nthreads = nthreads < 1 ? 1 : (nthreads > 64 ? 64 : nthreads);
    int rc = QMM_OK;
    switch (gtype) {
        case QMM_GGML_Q4_K: case QMM_GGML_Q5_K: case QMM_GGML_IQ4_XS:
            memcpy(dst, src, rs * (size_t)N);
            break;
        case QMM_GGML_Q6_K:
            parallel_rows(N, nthreads, [&](int r) { qmm_repack_row_q6_K(src + (size_t)r * rs, dst + (size_t)r * rb, K); });
            break;
        case QMM_GGML_Q8_0:
            parallel_rows(N, nthreads, [&](int r) { qmm_repack_row_q8_0(src + (size_t)r * rs, dst + (size_t)r * rb, K); });
            break;
        case QMM_GGML_Q5_1:
            parallel_rows(N, nthreads, [&](int r) { qmm_repack_row_q5_1(src + (size_t)r * rs, dst + (size_t)r * rb, K); });
            break;
        case QMM_GGML_Q5_0:
            parallel_rows(N, nthreads, [&](int r) { qmm_repack_row_q5_0(src + (size_t)r * rs, dst + (size_t)r * rb, K); });
            break;
        default:                                               // F32 / F16 / BF16 -> Q8_0_SOA
            parallel_rows(N, nthreads, [&](int r) {
                std::vector<float> row((size_t)K);
                float_row(gtype, src + (size_t)r * rs, row.data(), K);
                quantize_row_q8_0_soa(row.data(), dst + (size_t)r * rb, K);
            });
            break;
    }
    return rc;
}

}  // extern "C"
