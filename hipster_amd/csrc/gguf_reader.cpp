// gguf_reader.cpp -- the on-disk side of the path: a GGUF v3 reader behind the C ABI qmm_gguf_*.
// Host code only (no GPU calls).  It replaces the reference's hip::GGUF (engine/src/gguf.h:43-76,
// gguf.cpp:71-156) and its block table gtype_block (gguf.h:20, gguf.cpp:26-42); what it returns (tensor
// table, KV values, shard numbering, data offsets, the bytes of a tensor) is the reference reader's on the
// same files.
//
// The file format (GGUF v3, ggml's): little-endian
//   u32 magic "GGUF", u32 version = 3, u64 tensor count, u64 KV count,
//   KV pairs:      string key, u32 value type, value
//   tensor infos:  string name, u32 n_dims (<= 4), u64 ne[n_dims], u32 ggml type, u64 offset
//   data:          from the first multiple of general.alignment (default 32) after the infos;
//                  each tensor at data + offset
// with string = u64 length + bytes, and value types 0..12 = u8 i8 u16 i16 u32 i32 f32 bool string array
// u64 i64 f64 (an array: u32 element type, u64 count, the elements).  A model split over N files is named
// <base>-00001-of-0000N.gguf ... <base>-0000N-of-0000N.gguf; naming any one of them opens all N in order.
//
// Structure of this reader:
//   - scalar values are decoded from one table (width, signedness, float or not) instead of one case per
//     type; arrays of fixed-width elements are stepped over in one bounds-checked skip;
//   - each shard is parsed completely into a ShardImage and validated (header, KVs, infos, dims without
//     overflow, every tensor inside the file) before anything of it is merged into the model, so a bad
//     shard leaves no partial state behind;
//   - shard names come from rewriting the five index digits of the given name in place;
//   - a tensor read is chunked: each chunk is read with pread and its page-cache range dropped at once,
//     so reading a large tensor never holds more than one chunk of it in the page cache.
#include <errno.h>
#include <fcntl.h>
#include <limits.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <stdint.h>
#include <string.h>

#include <deque>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/hipster_qmm.h"

namespace {

// ---------------------------------------------------------------------------------- block shapes
// elements and bytes per block, indexed by ggml type number; {0, 0} = a type this library does not size
struct BlockShape { uint16_t elems, bytes; };
constexpr int kMaxGType = 31;
constexpr BlockShape kBlockShape[kMaxGType] = {
    /* 0 F32    */ {1, 4},    /* 1 F16   */ {1, 2},    /* 2 Q4_0  */ {32, 18},   /* 3 Q4_1   */ {32, 20},
    /* 4        */ {0, 0},    /* 5       */ {0, 0},    /* 6 Q5_0  */ {32, 22},   /* 7 Q5_1   */ {32, 24},
    /* 8 Q8_0   */ {32, 34},  /* 9 Q8_1  */ {32, 36},  /* 10 Q2_K */ {256, 84},  /* 11 Q3_K  */ {256, 110},
    /* 12 Q4_K  */ {256, 144},/* 13 Q5_K */ {256, 176},/* 14 Q6_K */ {256, 210}, /* 15 Q8_K  */ {256, 292},
    /* 16..19   */ {0, 0}, {0, 0}, {0, 0}, {0, 0},
    /* 20 IQ4_NL*/ {32, 18},  /* 21 IQ3_S*/ {256, 110},/* 22      */ {0, 0},     /* 23 IQ4_XS*/ {256, 136},
    /* 24 I8    */ {1, 1},    /* 25      */ {0, 0},    /* 26 I32  */ {1, 4},     /* 27..29   */ {0, 0}, {0, 0}, {0, 0},
    /* 30 BF16  */ {1, 2},
};

BlockShape block_shape(uint32_t t) { return t < (uint32_t)kMaxGType ? kBlockShape[t] : BlockShape{0, 0}; }

// ---------------------------------------------------------------------------------- KV value decoding
// GGUF value type -> how its bytes read.  width 0 = variable length (string 8, array 9).
struct ValueType { uint8_t width; uint8_t kind; bool is_signed; bool is_real; };
constexpr uint32_t kTypeString = 8, kTypeArray = 9, kNumValueTypes = 13;
constexpr ValueType kValueType[kNumValueTypes] = {
    {1, QMM_GGUF_KV_UINT, false, false},  {1, QMM_GGUF_KV_INT, true, false},     // u8, i8
    {2, QMM_GGUF_KV_UINT, false, false},  {2, QMM_GGUF_KV_INT, true, false},     // u16, i16
    {4, QMM_GGUF_KV_UINT, false, false},  {4, QMM_GGUF_KV_INT, true, false},     // u32, i32
    {4, QMM_GGUF_KV_FLOAT, false, true},  {1, QMM_GGUF_KV_BOOL, false, false},   // f32, bool
    {0, QMM_GGUF_KV_STRING, false, false}, {0, QMM_GGUF_KV_ARRAY, false, false}, // string, array
    {8, QMM_GGUF_KV_UINT, false, false},  {8, QMM_GGUF_KV_INT, true, false},     // u64, i64
    {8, QMM_GGUF_KV_FLOAT, false, true},                                          // f64
};

// One KV value as the C ABI exposes it: integers widened (unsigned in u, signed in i), reals in f,
// strings in s, arrays by their element count only.
struct KvValue {
    int kind = QMM_GGUF_KV_UINT;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
    uint64_t count = 0;
};

// A bounds-checked forward scan over one mapped file.  Every read either succeeds completely or marks
// the scan failed; after a failure every further read fails too, so callers check once per record.
class Scan {
public:
    Scan(const uint8_t* begin, const uint8_t* end) : pos_(begin), end_(end), begin_(begin) {}
    bool failed() const { return failed_; }
    size_t offset() const { return (size_t)(pos_ - begin_); }

    // little-endian unsigned integer of `width` bytes (1, 2, 4 or 8)
    uint64_t uint(unsigned width) {
        const uint8_t* p = take(width);
        uint64_t v = 0;
        if (p) for (unsigned b = 0; b < width; ++b) v |= (uint64_t)p[b] << (8 * b);
        return v;
    }
    uint32_t u32() { return (uint32_t)uint(4); }
    uint64_t u64() { return uint(8); }

    std::string string() {
        const uint64_t n = u64();
        const uint8_t* p = take(n);
        return p ? std::string((const char*)p, (size_t)n) : std::string();
    }
    void skip_string() { take(u64()); }

    // one value of GGUF type `type`; arrays are counted and stepped over, nested at most kMaxNest deep
    bool value(uint32_t type, KvValue& out, int nest = 0) {
        if (type >= kNumValueTypes) return fail();
        const ValueType& vt = kValueType[type];
        out.kind = vt.kind;
        if (type == kTypeString) {
            out.s = string();
        } else if (type == kTypeArray) {
            const uint32_t elem = u32();
            out.count = u64();
            if (!skip_array(elem, out.count, nest + 1)) return fail();
        } else {
            const uint64_t raw = uint(vt.width);
            if (vt.is_real) {
                if (vt.width == 4) { float x; const uint32_t b = (uint32_t)raw; memcpy(&x, &b, 4); out.f = x; }
                else memcpy(&out.f, &raw, 8);
            } else if (vt.is_signed) {
                const unsigned drop = 64 - 8 * vt.width;                 // sign-extend from the value's width
                out.i = (int64_t)(raw << drop) >> drop;
            } else {
                out.u = raw;
            }
        }
        return !failed_;
    }

private:
    static constexpr int kMaxNest = 4;

    const uint8_t* take(uint64_t n) {
        if (failed_ || n > (uint64_t)(end_ - pos_)) { failed_ = true; return nullptr; }
        const uint8_t* p = pos_;
        pos_ += n;
        return p;
    }
    bool fail() { failed_ = true; return false; }

    bool skip_array(uint32_t elem, uint64_t count, int nest) {
        if (elem >= kNumValueTypes || nest > kMaxNest) return fail();
        const unsigned w = kValueType[elem].width;
        if (w > 0) {                                                   // fixed width: one skip
            uint64_t bytes;
            if (__builtin_mul_overflow(count, (uint64_t)w, &bytes)) return fail();
            return take(bytes) != nullptr;
        }
        for (uint64_t k = 0; k < count && !failed_; ++k) {
            if (elem == kTypeString) skip_string();
            else {
                KvValue inner;
                value(elem, inner, nest);
            }
        }
        return !failed_;
    }

    const uint8_t* pos_;
    const uint8_t* end_;
    const uint8_t* begin_;
    bool failed_ = false;
};

// ---------------------------------------------------------------------------------- one mapped shard
// A shard file held open (the descriptor is kept for pread and page-cache advice) and mapped read-only.
class MappedFile {
public:
    MappedFile() = default;
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
    MappedFile(MappedFile&& o) noexcept { *this = std::move(o); }
    MappedFile& operator=(MappedFile&& o) noexcept {
        std::swap(fd_, o.fd_);
        std::swap(base_, o.base_);
        std::swap(size_, o.size_);
        return *this;
    }
    ~MappedFile() {
        if (base_) munmap((void*)base_, size_);
        if (fd_ >= 0) ::close(fd_);
    }

    int open(const std::string& path) {
        fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd_ < 0) return QMM_ERR_IO;
        struct stat st;
        if (fstat(fd_, &st) != 0 || st.st_size < 24) return QMM_ERR_IO;  // shorter than the fixed header
        void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd_, 0);
        if (p == MAP_FAILED) return QMM_ERR_IO;
        base_ = (const uint8_t*)p;
        size_ = (size_t)st.st_size;
        return QMM_OK;
    }
    int fd() const { return fd_; }
    const uint8_t* base() const { return base_; }
    size_t size() const { return size_; }

private:
    int fd_ = -1;
    const uint8_t* base_ = nullptr;
    size_t size_ = 0;
};

// Everything one shard contributes, parsed and checked before it is merged into the model.
struct ShardImage {
    struct Tensor { std::string name; uint32_t n_dims; uint64_t ne[4]; uint32_t type; uint64_t rel_off; };
    std::vector<std::pair<std::string, KvValue>> kvs;      // in file order
    std::vector<Tensor> tensors;                           // in file order
    size_t header_end = 0;                                 // offset of the first byte after the infos
};

int parse_shard(const MappedFile& f, ShardImage& img) {
    Scan sc(f.base(), f.base() + f.size());
    const uint32_t magic = sc.u32(), version = sc.u32();
    if (sc.failed() || magic != 0x46554747u || version != 3u) return QMM_ERR_IO;   // "GGUF", v3 only
    const uint64_t n_tensors = sc.u64(), n_kv = sc.u64();
    for (uint64_t k = 0; k < n_kv; ++k) {
        std::string key = sc.string();
        KvValue v;
        if (!sc.value(sc.u32(), v)) return QMM_ERR_IO;
        img.kvs.emplace_back(std::move(key), std::move(v));
    }
    for (uint64_t k = 0; k < n_tensors; ++k) {
        ShardImage::Tensor t;
        t.name = sc.string();
        t.n_dims = sc.u32();
        if (sc.failed() || t.n_dims > 4) return QMM_ERR_IO;
        for (int d = 0; d < 4; ++d) t.ne[d] = d < (int)t.n_dims ? sc.u64() : 1;
        t.type = sc.u32();
        t.rel_off = sc.u64();
        if (sc.failed()) return QMM_ERR_IO;
        img.tensors.push_back(std::move(t));
    }
    img.header_end = sc.offset();
    return QMM_OK;
}

// If `path` ends in -IIIII-of-NNNNN.gguf (five decimal digits each), return N and the position of the
// first index digit; otherwise 0.
int split_count(const std::string& path, size_t* index_pos) {
    static const char kTail[] = "-#####-of-#####.gguf";            // # = a decimal digit
    const size_t L = sizeof kTail - 1;
    if (path.size() < L) return 0;
    const size_t at = path.size() - L;
    int count = 0;
    for (size_t k = 0; k < L; ++k) {
        const char c = path[at + k];
        if (kTail[k] != '#') {
            if (c != kTail[k]) return 0;
        } else {
            if (c < '0' || c > '9') return 0;
            if (k >= 10) count = count * 10 + (c - '0');           // the second digit group is N
        }
    }
    *index_pos = at + 1;
    return count;
}

std::string shard_name(std::string path, size_t index_pos, int i) {
    for (int k = 4; k >= 0; --k, i /= 10) path[index_pos + (size_t)k] = (char)('0' + i % 10);
    return path;
}

bool has_prefix(const std::string& s, const char* p) { return s.compare(0, strlen(p), p) == 0; }

}  // namespace

// ---------------------------------------------------------------------------------- the model
struct qmm_gguf {
    std::vector<MappedFile> files;
    std::deque<std::string> names;                 // a deque: tensor name pointers stay valid as it grows
    std::vector<qmm_gguf_tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
    std::unordered_map<std::string, KvValue> kv;
    size_t mapped = 0;

    const KvValue* find_kv(const char* key) const {
        auto it = kv.find(key);
        return it == kv.end() ? nullptr : &it->second;
    }

    // Opens, parses and validates one shard, then merges it: its tensors are appended (a name seen before
    // now resolves to the later tensor) and its KVs replace earlier values, except split.* keys, which
    // keep the value of the shard that first had them.
    int add_shard(const std::string& path) {
        MappedFile f;
        if (int e = f.open(path)) return e;
        ShardImage img;
        if (int e = parse_shard(f, img)) return e;

        // the data alignment: this shard's own general.alignment, else the one merged so far, else 32
        uint64_t align = 32;
        auto pick = [&](const KvValue& v) { if (v.kind == QMM_GGUF_KV_UINT && v.u > 0) align = v.u; };
        if (const KvValue* prev = find_kv("general.alignment")) pick(*prev);
        for (auto& e : img.kvs) if (e.first == "general.alignment") pick(e.second);
        const uint64_t data_start = img.header_end + (align - img.header_end % align) % align;

        const int shard = (int)files.size();
        std::vector<qmm_gguf_tensor> add;
        add.reserve(img.tensors.size());
        for (const auto& t : img.tensors) {
            const BlockShape bs = block_shape(t.type);
            if (bs.elems == 0) return QMM_ERR_FORMAT;
            uint64_t elems = 1;
            for (int d = 0; d < 4; ++d)
                if (__builtin_mul_overflow(elems, t.ne[d], &elems)) return QMM_ERR_IO;
            if (t.ne[0] > (uint64_t)INT_MAX || t.ne[0] % bs.elems != 0) return QMM_ERR_IO;
            uint64_t nbytes, off;
            if (__builtin_mul_overflow(elems / bs.elems, (uint64_t)bs.bytes, &nbytes)) return QMM_ERR_IO;
            if (__builtin_add_overflow(data_start, t.rel_off, &off)) return QMM_ERR_IO;
            if (off > f.size() || nbytes > f.size() - off) return QMM_ERR_IO;      // past the end of the file
            qmm_gguf_tensor g;
            memset(&g, 0, sizeof g);
            g.type = (int32_t)t.type;
            g.n_dims = t.n_dims;
            for (int d = 0; d < 4; ++d) g.ne[d] = t.ne[d];
            g.nbytes = (size_t)nbytes;
            g.file_off = off;
            g.data = f.base() + off;
            g.shard = shard;
            add.push_back(g);
        }

        // the shard is valid: merge it
        for (size_t k = 0; k < add.size(); ++k) {
            names.push_back(img.tensors[k].name);
            add[k].name = names.back().c_str();
            by_name[names.back()] = tensors.size();
            tensors.push_back(add[k]);
        }
        for (auto& e : img.kvs) {
            auto slot = kv.find(e.first);
            if (slot == kv.end()) kv.emplace(std::move(e.first), std::move(e.second));
            else if (!has_prefix(e.first, "split.")) slot->second = std::move(e.second);
        }
        mapped += f.size();
        files.push_back(std::move(f));
        return QMM_OK;
    }
};

namespace {

template <class Fn>
int with_kv(const qmm_gguf* g, const char* key, Fn fn) {
    if (!g || !key) return QMM_ERR_NULL;
    const KvValue* v = g->find_kv(key);
    return v ? fn(*v) : QMM_ERR_NOT_FOUND;
}

}  // namespace

extern "C" {

int qmm_gtype_block(int type, uint32_t* block_elems, uint32_t* block_bytes) {
    const BlockShape bs = block_shape((uint32_t)type);
    if (type < 0 || bs.elems == 0) return QMM_ERR_FORMAT;
    if (block_elems) *block_elems = bs.elems;
    if (block_bytes) *block_bytes = bs.bytes;
    return QMM_OK;
}

int qmm_gguf_open(const char* path, qmm_gguf** out) {
    if (!path || !out) return QMM_ERR_NULL;
    *out = nullptr;
    auto* g = new qmm_gguf();
    const std::string p(path);
    size_t index_pos = 0;
    const int n = split_count(p, &index_pos);
    int rc = QMM_OK;
    if (n > 0)
        for (int i = 1; i <= n && rc == QMM_OK; ++i) rc = g->add_shard(shard_name(p, index_pos, i));
    else
        rc = g->add_shard(p);                      // one file (a name like -00001-of-00000.gguf included)
    if (rc != QMM_OK) {
        delete g;
        return rc;
    }
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
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return QMM_ERR_NOT_FOUND;
    *out = g->tensors[it->second];
    return QMM_OK;
}

int qmm_gguf_kv_kind(const qmm_gguf* g, const char* key, int* kind) {
    if (!kind) return QMM_ERR_NULL;
    return with_kv(g, key, [&](const KvValue& v) { *kind = v.kind; return (int)QMM_OK; });
}

// signed values are reinterpreted as their low 32 bits, as the reference's kv_u32 does (gguf.cpp:141)
int qmm_gguf_kv_u32(const qmm_gguf* g, const char* key, uint32_t* out) {
    if (!out) return QMM_ERR_NULL;
    return with_kv(g, key, [&](const KvValue& v) {
        switch (v.kind) {
            case QMM_GGUF_KV_INT: *out = (uint32_t)v.i; return (int)QMM_OK;
            case QMM_GGUF_KV_UINT: case QMM_GGUF_KV_BOOL: *out = (uint32_t)v.u; return (int)QMM_OK;
            default: return (int)QMM_ERR_ARG;
        }
    });
}

int qmm_gguf_kv_f32(const qmm_gguf* g, const char* key, float* out) {
    if (!out) return QMM_ERR_NULL;
    return with_kv(g, key, [&](const KvValue& v) {
        if (v.kind != QMM_GGUF_KV_FLOAT) return (int)QMM_ERR_ARG;
        *out = (float)v.f;
        return (int)QMM_OK;
    });
}

int qmm_gguf_kv_str(const qmm_gguf* g, const char* key, const char** out) {
    if (!out) return QMM_ERR_NULL;
    return with_kv(g, key, [&](const KvValue& v) {
        if (v.kind != QMM_GGUF_KV_STRING) return (int)QMM_ERR_ARG;
        *out = v.s.c_str();
        return (int)QMM_OK;
    });
}

int qmm_gguf_kv_array_len(const qmm_gguf* g, const char* key, uint64_t* out) {
    if (!out) return QMM_ERR_NULL;
    return with_kv(g, key, [&](const KvValue& v) {
        if (v.kind != QMM_GGUF_KV_ARRAY) return (int)QMM_ERR_ARG;
        *out = v.count;
        return (int)QMM_OK;
    });
}

// The bytes of one tensor into a host buffer, without growing the page cache: the tensor is read in
// chunks, and each chunk's file range is dropped from the cache as soon as it has been copied.
int qmm_gguf_read_tensor(const qmm_gguf* g, const char* name, void* dst, size_t dst_bytes) {
    if (!g || !name || !dst) return QMM_ERR_NULL;
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return QMM_ERR_NOT_FOUND;
    const qmm_gguf_tensor& t = g->tensors[it->second];
    if (dst_bytes < t.nbytes) return QMM_ERR_SHAPE;
    const int fd = g->files[(size_t)t.shard].fd();
    constexpr size_t kChunk = (size_t)32 << 20;
    uint8_t* out = (uint8_t*)dst;
    for (size_t at = 0; at < t.nbytes;) {
        const size_t want = t.nbytes - at < kChunk ? t.nbytes - at : kChunk;
        const off_t chunk_off = (off_t)(t.file_off + at);
        size_t got = 0;
        while (got < want) {
            const ssize_t r = pread(fd, out + at + got, want - got, chunk_off + (off_t)got);
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) return QMM_ERR_IO;
            got += (size_t)r;
        }
        posix_fadvise(fd, chunk_off, (off_t)want, POSIX_FADV_DONTNEED);
        at += want;
    }
    return QMM_OK;
}

}  // extern "C"
