// GGUF v3 reader with the surface of imi's imi_file (imi/model.h:12-36): load, get, key_i, key_f, keep, drop_data.
// ggml is not part of this build, so tensors are described by a small struct with ggml's fields (type, ne, nb,
// data, name) instead of ggml_tensor.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace sh {

enum ggml_type_id : int { GT_F32 = 0, GT_F16 = 1, GT_Q4_0 = 2, GT_Q4_1 = 3, GT_Q8_0 = 8, GT_Q6_K = 14 };

struct gg_tensor {
    std::string name;
    int type = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};   // ne[0] innermost
    size_t nb[4] = {0, 0, 0, 0};    // ggml's byte strides: nb[0] = one element or block, nb[1] = one row
    size_t offset = 0, nbytes = 0;
    const void* data = nullptr;     // null once the file's block is dropped and the tensor was not kept
};

struct gg_file {
    std::vector<gg_tensor> tensors;
    bool load(const std::string& path);                                  // imi/model.cpp:48-106
    const gg_tensor* get(const std::string& name, bool required = true) const;   // null + error if missing
    int64_t key_i(const std::string& name, int64_t def) const;
    float key_f(const std::string& name, float def) const;
    std::vector<int64_t> key_arr(const std::string& name) const;
    int key_type(const std::string& name) const;                         // GGUF value type, -1 if absent
    const gg_tensor* keep(const std::string& name, bool required = true); // own copy of the bytes (model.cpp:138-150)
    void drop_data();                                                     // let the file's block go (model.cpp:152-163)
    std::string error;
    const void* block = nullptr;   // every tensor's bytes (the mapped file from the data offset on), until drop_data
    size_t block_size = 0;
    ~gg_file();

private:
    struct kv { std::string key; int type = 0; int64_t i = 0; double f = 0; std::vector<int64_t> arr; };
    std::vector<kv> kvs;
    void* map = nullptr;
    size_t map_size = 0;
    std::vector<void*> kept;
};

}  // namespace sh
