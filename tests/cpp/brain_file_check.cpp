// imi's file and brain APIs (imi/model.h:12-36, imi/brain.h:20-65) from include/seoul_gpu.hpp, used the way imi's
// own callers use them (imi/brain.cpp:11-64, imi/core/seoul.cpp:94-165, imi/core/words_check.cpp:16-18).
//   brain_file_check MODEL.gguf           -> the file part only (no device)
//   brain_file_check MODEL.gguf --step    -> also imi_brain on the device: a prompt, then a greedy loop
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "seoul_gpu.hpp"

using seoul_hip::imi_brain;
using seoul_hip::imi_file;
using seoul_hip::imi_tensor;

static int top(const std::vector<float>& a) {   // imi/core/seoul_check.cpp:15
    int t = 0;
    for (int i = 1; i < (int)a.size(); i++)
        if (a[i] > a[t]) t = i;
    return t;
}

static double fsum(const imi_tensor* t) {
    double s = 0;
    const float* p = (const float*)t->data;
    for (int64_t i = 0; i < t->ne[0]; i++) s += p[i];
    return s;
}

int main(int argc, char** argv) {
    if (argc < 2) { fprintf(stderr, "usage: brain_file_check MODEL.gguf [--step]\n"); return 1; }
    imi_file f;
    if (!f.load(argv[1], false)) return 1;
    printf("keys block_count %lld head_count %lld key_length %lld eps %.9g missing %lld\n",
           (long long)f.key_i("lfm3.block_count", -1), (long long)f.key_i("lfm3.attention.head_count", -1),
           (long long)f.key_i("lfm3.attention.key_length", -1), f.key_f("lfm3.attention.layer_norm_rms_epsilon", -1.0f),
           (long long)f.key_i("no.such.key", -7));
    const imi_tensor* te = f.get("token_embd.weight");
    printf("token_embd %s type %d ne %lld %lld nb %zu %zu bytes %zu\n", te->name, te->type, (long long)te->ne[0],
           (long long)te->ne[1], te->nb[0], te->nb[1], seoul_hip::imi_nbytes(te));
    printf("optional missing %d block %d\n", f.get("no.such.tensor", false) == nullptr, f.data != nullptr && f.size > 0);
    const imi_tensor* up = f.get("blk.0.ffn_up.weight");
    const double s0 = fsum(f.get("output_norm.weight"));
    const imi_tensor* on = f.keep("output_norm.weight");
    printf("kept aligned %d same %d\n", (int)((uintptr_t)on->data % 64 == 0), fsum(on) == s0);
    f.drop_data();
    printf("dropped table %d kept %d same %d block %d\n", up->data == nullptr, on->data != nullptr, fsum(on) == s0,
           f.data == nullptr && f.size == 0);
    if (argc > 2 && !strcmp(argv[2], "--step")) {
        imi_brain br;
        if (!br.load(argv[1], 4, 64)) return 1;
        int n_attn = 0;
        for (const auto& L : br.layers) n_attn += L.attn_index >= 0;
        printf("brain n_embd %d n_vocab %d n_head %d n_head_kv %d head_dim %d d_conv %d layers %zu attn %d\n", br.n_embd,
               br.n_vocab, br.n_head, br.n_head_kv, br.head_dim, br.d_conv, br.layers.size(), n_attn);
        const int prompt[4] = {3, 141, 59, 26};
        std::vector<int> first;
        for (int run = 0; run < 2; run++) {   // the second run after reset() must repeat the first
            br.reset();
            for (int i = 0; i < 4; i++) br.step(prompt[i], nullptr, i == 3);
            int tok = top(br.logits);
            std::vector<int> ids;
            for (int i = 0; i < 8; i++) {
                ids.push_back(tok);
                br.step(tok, nullptr, true);
                tok = top(br.logits);
            }
            if (run == 0) {
                first = ids;
                printf("ids:");
                for (int v : ids) printf(" %d", v);
                printf("\npos %d\n", br.pos);
            } else {
                printf("reset repeats %d\n", ids == first);
            }
        }
    }
    return 0;
}
