#include "gguf_file.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdlib>
#include <cstring>

namespace sh {

namespace {
// bounds-checked cursor over the mapped header
struct cursor {
    const uint8_t* base;
    size_t size, at = 0;
    bool ok = true;
    bool take(void* dst, size_t n) {
        if (!ok || at + n > size) { ok = false; return false; }
        memcpy(dst, base + at, n);
        at += n;
        return true;
    }
    template <class T> T num() { T v{}; take(&v, sizeof v); return v; }
    std::string str() {
        const uint64_t n = num<uint64_t>();
        if (!ok || n > size - at) { ok = false; return {}; }
        std::string s(reinterpret_cast<const char*>(base + at), n);
        at += n;
        return s;
    }
};
// bytes of one element (F32, F16) or one block (quantized types) and the values a block holds (ggml's type size
// and block size)
bool type_block(int type, size_t* bytes, int64_t* values) {
    switch (type) {
        case GT_F32: *bytes = 4; *values = 1; return true;
        case GT_F16: *bytes = 2; *values = 1; return true;
        case GT_Q4_0: *bytes = 18; *values = 32; return true;
        case GT_Q4_1: *bytes = 20; *values = 32; return true;
        case GT_Q8_0: *bytes = 34; *values = 32; return true;
        case GT_Q6_K: *bytes = 210; *values = 256; return true;
        default: return false;
    }
}
}  // namespace

bool gg_file::load(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) { error = "cannot read " + path; return false; }
    struct stat st {};
    if (fstat(fd, &st) != 0 || st.st_size < 24) { ::close(fd); error = "cannot read " + path; return false; }
    map_size = (size_t)st.st_size;
    void* m = mmap(nullptr, map_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) { error = "cannot map " + path; return false; }
    map = m;
    cursor c{static_cast<const uint8_t*>(map), map_size};
    const uint32_t magic = c.num<uint32_t>(), version = c.num<uint32_t>();
    if (magic != 0x46554747u || version < 2) { error = path + " is not a GGUF file"; return false; }
    const uint64_t n_tensors = c.num<uint64_t>(), n_kv = c.num<uint64_t>();
    size_t alignment = 32;
    auto scalar = [&](int type, kv& k) {
        switch (type) {
            case 0: k.i = c.num<uint8_t>(); break;
            case 1: k.i = c.num<int8_t>(); break;
            case 2: k.i = c.num<uint16_t>(); break;
            case 3: k.i = c.num<int16_t>(); break;
            case 4: k.i = c.num<uint32_t>(); break;
            case 5: k.i = c.num<int32_t>(); break;
            case 6: k.f = c.num<float>(); k.i = (int64_t)k.f; return;
            case 7: k.i = c.num<uint8_t>(); break;
            case 8: c.str(); break;
            case 10: k.i = (int64_t)c.num<uint64_t>(); break;
            case 11: k.i = c.num<int64_t>(); break;
            case 12: k.f = c.num<double>(); k.i = (int64_t)k.f; return;
            default: c.ok = false;
        }
        k.f = (double)k.i;
    };
    for (uint64_t i = 0; i < n_kv && c.ok; i++) {
        kv k;
        k.key = c.str();
        k.type = (int)c.num<uint32_t>();
        if (k.type == 9) {
            const int et = (int)c.num<uint32_t>();
            const uint64_t n = c.num<uint64_t>();
            if (n > c.size - c.at) c.ok = false;   // every element takes at least one byte
            for (uint64_t e = 0; e < n && c.ok; e++) { kv tmp; scalar(et, tmp); k.arr.push_back(tmp.i); }
        } else {
            scalar(k.type, k);
        }
        if (k.key == "general.alignment") {
            // a power of two no larger than the file (ggml's gguf reader refuses any other)
            if (k.type == 9 || k.type == 8 || k.i <= 0 || (uint64_t)k.i > map_size || (k.i & (k.i - 1)) != 0) {
                error = path + ": bad general.alignment";
                return false;
            }
            alignment = (size_t)k.i;
        }
        kvs.push_back(std::move(k));
    }
    for (uint64_t i = 0; i < n_tensors && c.ok; i++) {
        gg_tensor t;
        t.name = c.str();
        const uint32_t nd = c.num<uint32_t>();
        if (!c.ok || nd < 1 || nd > 4) { c.ok = false; break; }
        t.n_dims = (int)nd;
        for (int d = 0; d < t.n_dims; d++) t.ne[d] = (int64_t)c.num<uint64_t>();
        t.type = (int)c.num<uint32_t>();
        t.offset = c.num<uint64_t>();
        if (!c.ok) break;
        for (int d = 0; d < 4; d++)
            if (t.ne[d] < 0) { error = "tensor " + t.name + " has a negative dimension"; return false; }
        size_t blk = 0;
        int64_t per = 1;
        if (!type_block(t.type, &blk, &per)) { error = "tensor " + t.name + " has a type this engine does not read"; return false; }
        if (t.ne[0] % per) { error = "tensor " + t.name + " has rows that are not whole blocks"; return false; }
        // byte strides and size, refused when any product overflows
        size_t row = 0, n2 = 0, n3 = 0, all = 0;
        if (__builtin_mul_overflow((size_t)(t.ne[0] / per), blk, &row) || __builtin_mul_overflow(row, (size_t)t.ne[1], &n2) ||
            __builtin_mul_overflow(n2, (size_t)t.ne[2], &n3) || __builtin_mul_overflow(n3, (size_t)t.ne[3], &all)) {
            error = "tensor " + t.name + " is too large";
            return false;
        }
        t.nb[0] = blk;
        t.nb[1] = row;
        t.nb[2] = n2;
        t.nb[3] = n3;
        t.nbytes = all;
        tensors.push_back(std::move(t));
    }
    if (!c.ok) { error = path + ": malformed GGUF header"; return false; }
    // (c.at <= map_size and alignment <= map_size, so the sum does not wrap)
    const size_t data0 = (c.at + alignment - 1) / alignment * alignment;
    if (data0 > map_size) { error = path + ": no data block"; return false; }
    block = static_cast<const uint8_t*>(map) + data0;
    block_size = map_size - data0;
    for (auto& t : tensors) {
        // offset and size each within the block, compared without sums that could wrap
        if (t.offset > block_size || t.nbytes > block_size - t.offset) { error = "short read on " + t.name; return false; }
        t.data = static_cast<const uint8_t*>(map) + data0 + t.offset;
    }
    return true;
}

const gg_tensor* gg_file::get(const std::string& name, bool required) const {
    for (const auto& t : tensors)
        if (t.name == name) return &t;
    if (required) const_cast<gg_file*>(this)->error = "missing tensor " + name;
    return nullptr;
}
int64_t gg_file::key_i(const std::string& name, int64_t def) const {
    for (const auto& k : kvs) if (k.key == name && k.type != 9 && k.type != 8) return k.i;
    return def;
}
float gg_file::key_f(const std::string& name, float def) const {
    for (const auto& k : kvs) if (k.key == name && k.type != 9 && k.type != 8) return (float)k.f;
    return def;
}
int gg_file::key_type(const std::string& name) const {
    for (const auto& k : kvs) if (k.key == name) return k.type;
    return -1;
}
std::vector<int64_t> gg_file::key_arr(const std::string& name) const {
    for (const auto& k : kvs) if (k.key == name && k.type == 9) return k.arr;
    return {};
}
const gg_tensor* gg_file::keep(const std::string& name, bool required) {
    const gg_tensor* t = get(name, required);
    if (!t || !t->data) return t;
    const char* b = static_cast<const char*>(map);
    const char* p = static_cast<const char*>(t->data);
    if (!map || p < b || p >= b + map_size) return t;   // already its own
    void* own = nullptr;
    if (posix_memalign(&own, 64, (t->nbytes + 63) / 64 * 64) != 0) { error = "out of memory keeping " + name; return nullptr; }
    memcpy(own, t->data, t->nbytes);
    kept.push_back(own);
    const_cast<gg_tensor*>(t)->data = own;
    return t;
}
void gg_file::drop_data() {
    if (!map) return;
    const char* b = static_cast<const char*>(map);
    for (auto& t : tensors) {
        const char* p = static_cast<const char*>(t.data);
        if (p >= b && p < b + map_size) t.data = nullptr;
    }
    munmap(map, map_size);
    map = nullptr;
    map_size = 0;
    block = nullptr;
    block_size = 0;
}
gg_file::~gg_file() {
    if (map) munmap(map, map_size);
    for (void* p : kept) free(p);
}

}  // namespace sh
