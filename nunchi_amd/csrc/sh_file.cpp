// imi_file's surface (imi/model.h:12-36, imi/model.cpp:48-170) as a C ABI over the GGUF reader: load, get, key_i,
// key_f, keep, drop_data, and the tensors' ggml fields (type, ne, nb, data, name). The C++ imi_file of
// include/seoul_gpu.hpp wraps these for imi's callers.
#include <new>
#include <string>

#include "gguf_file.h"
#include "sh_ctx.h"

struct sh_file {
    sh::gg_file f;
};

namespace {
void describe(const sh::gg_tensor& t, sh_tensor* out) {
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) {
        out->ne[d] = t.ne[d];
        out->nb[d] = t.nb[d];
    }
    out->data = const_cast<void*>(t.data);
}
}  // namespace

extern "C" {

int sh_file_load(const char* path, sh_file** out) {
    if (!path || !out) return sh::set_error(SH_E_ARG, "sh_file_load: bad argument");
    *out = nullptr;
    sh_file* h = new (std::nothrow) sh_file;
    if (!h) return sh::set_error(SH_E_NOMEM, "sh_file_load: out of memory");
    if (!h->f.load(path)) {
        const std::string e = h->f.error;
        delete h;
        return sh::set_error(SH_E_FILE, "sh_file_load: " + e);
    }
    *out = h;
    return SH_OK;
}

int sh_file_free(sh_file* f) {
    delete f;
    return SH_OK;
}

int sh_file_get(const sh_file* f, const char* name, sh_tensor* out) {
    if (!f || !name || !out) return sh::set_error(SH_E_ARG, "sh_file_get: bad argument");
    const sh::gg_tensor* t = f->f.get(name, false);
    if (!t) return sh::set_error(SH_E_ARG, std::string("missing tensor ") + name);
    describe(*t, out);
    return SH_OK;
}

// imi_file::key_i (model.cpp:117-126): the value of a u32, i32 or u64 key, else def
int64_t sh_file_key_i(const sh_file* f, const char* key, int64_t def) {
    if (!f || !key) return def;
    const int ty = f->f.key_type(key);
    return ty == 4 || ty == 5 || ty == 10 ? f->f.key_i(key, def) : def;
}

// imi_file::key_f (model.cpp:128-131): the value of an f32 key, else def (imi stops on a key of another type)
float sh_file_key_f(const sh_file* f, const char* key, float def) {
    if (!f || !key) return def;
    return f->f.key_type(key) == 6 ? f->f.key_f(key, def) : def;
}

int sh_file_keep(sh_file* f, const char* name, sh_tensor* out) {
    if (!f || !name || !out) return sh::set_error(SH_E_ARG, "sh_file_keep: bad argument");
    if (!f->f.get(name, false)) return sh::set_error(SH_E_ARG, std::string("missing tensor ") + name);
    const sh::gg_tensor* t = f->f.keep(name, false);
    if (!t) return sh::set_error(SH_E_NOMEM, "sh_file_keep: " + f->f.error);
    describe(*t, out);
    return SH_OK;
}

int sh_file_drop_data(sh_file* f) {
    if (!f) return sh::set_error(SH_E_ARG, "sh_file_drop_data: bad argument");
    f->f.drop_data();
    return SH_OK;
}

int sh_file_n_tensors(const sh_file* f) { return f ? (int)f->f.tensors.size() : 0; }

int sh_file_tensor(const sh_file* f, int i, sh_tensor* out) {
    if (!f || !out || i < 0 || i >= (int)f->f.tensors.size()) return sh::set_error(SH_E_ARG, "sh_file_tensor: bad argument");
    describe(f->f.tensors[(size_t)i], out);
    return SH_OK;
}

int sh_file_key_arr(const sh_file* f, const char* key, int64_t* out, int cap) {
    if (!f || !key || (cap > 0 && !out)) return sh::set_error(SH_E_ARG, "sh_file_key_arr: bad argument");
    if (f->f.key_type(key) != 9) return 0;
    const std::vector<int64_t> a = f->f.key_arr(key);
    for (int i = 0; i < cap && i < (int)a.size(); i++) out[i] = a[(size_t)i];
    return (int)a.size();
}

int sh_file_block(const sh_file* f, const void** data, size_t* size) {
    if (!f || !data || !size) return sh::set_error(SH_E_ARG, "sh_file_block: bad argument");
    *data = f->f.block;
    *size = f->f.block_size;
    return SH_OK;
}

}  // extern "C"
