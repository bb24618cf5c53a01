// ref_gguf_shim.cpp -- exposes the reference's own GGUF v3 reader (engine/src/gguf.cpp, compiled from
// where it lies in the reference checkout) through a C ABI, so the library's reader
// (hipster_amd/csrc/gguf_reader.cpp) can be checked against it on the same files.  TEST INFRASTRUCTURE
// ONLY: built into oracle/_ref/ (git-ignored) by oracle/Makefile, loaded only by tests/.
#include <cstring>
#include <exception>

#include "gguf.h"

extern "C" {
// NULL when the reference reader throws (bad magic, version, truncation, missing shard, ...)
void* refgg_open(const char* path) {
    try { return new hip::GGUF(path); } catch (const std::exception&) { return nullptr; }
}
void refgg_close(void* g) { delete (hip::GGUF*)g; }
long refgg_n_tensors(void* g) { return (long)((hip::GGUF*)g)->tensors().size(); }
// tensor i: name copied into name (cap bytes), ne[4], type, nbytes, shard and file offset
int refgg_tensor(void* g, long i, char* name, int cap, uint64_t* ne, int* type, uint64_t* nbytes, int* shard, uint64_t* off) {
    const auto& ts = ((hip::GGUF*)g)->tensors();
    if (i < 0 || i >= (long)ts.size()) return -1;
    const auto& t = ts[(size_t)i];
    std::strncpy(name, t.name.c_str(), (size_t)cap - 1);
    name[cap - 1] = 0;
    for (int d = 0; d < 4; ++d) ne[d] = t.ne[d];
    *type = (int)t.type; *nbytes = t.nbytes; *shard = t.map_index; *off = t.file_off;
    return 0;
}
// the tensor's bytes through read_tensor (pread)
int refgg_read(void* g, const char* name, void* dst) {
    try { auto* gg = (hip::GGUF*)g; gg->read_tensor(gg->get(name), dst); return 0; } catch (const std::exception&) { return -1; }
}
int refgg_kv_u32(void* g, const char* key, uint32_t* out) {
    try { *out = ((hip::GGUF*)g)->kv_u32(key); return 0; } catch (const std::exception&) { return -1; }
}
int refgg_kv_f32(void* g, const char* key, float* out) {
    try { *out = ((hip::GGUF*)g)->kv_f32(key); return 0; } catch (const std::exception&) { return -1; }
}
int refgg_kv_str(void* g, const char* key, char* out, int cap) {
    try { std::strncpy(out, ((hip::GGUF*)g)->kv_str(key).c_str(), (size_t)cap - 1); out[cap - 1] = 0; return 0; }
    catch (const std::exception&) { return -1; }
}
}
