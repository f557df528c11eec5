// Drives the GPU engine through imi's own API (include/seoul_gpu.hpp) the way imi's callers do
// (imi/core/seoul_check.cpp, imi/core/hear.cpp:58-72): prompt, greedy loop on the host, step2 riding.
//   seoul_gpu_check MODEL.gguf [VOICE.gguf]  -> prints the greedy ids and hidden checksums; with a voice generator,
//   one voice frame (imi/core/talk.cpp:127-187 with the first maximum in place of sampling) and its codes
#include <cmath>
#include <cstdio>
#include <vector>

#include "seoul_gpu.hpp"

using seoul_hip::imi_seoul;
using seoul_hip::imi_seoul_state;
using seoul_hip::imi_voice;

static int top(const std::vector<float>& a) {   // imi/core/seoul_check.cpp:15
    int t = 0;
    for (int i = 1; i < (int)a.size(); i++)
        if (a[i] > a[t]) t = i;
    return t;
}

int main(int argc, char** argv) {
    if (argc < 2) { fprintf(stderr, "usage: seoul_gpu_check MODEL.gguf\n"); return 1; }
    imi_seoul br;
    if (!br.load(argv[1], 4, 128)) return 1;
    const int prompt[4] = {3, 141, 59, 26};
    for (int i = 0; i < 4; i++) br.step(prompt[i], nullptr, i == 3);
    int tok = top(br.logits);
    printf("ids:");
    for (int i = 0; i < 8; i++) {   // greedy loop as imi/core/hear.cpp:66-72
        printf(" %d", tok);
        br.step(tok, nullptr, true);
        tok = top(br.logits);
    }
    printf("\n");
    // a second conversation riding the first one's table reads (imi/core/flow.cpp:118)
    imi_seoul_state b = br.new_state();
    br.step2(tok, nullptr, true, b, 7, nullptr, true);
    double hs = 0, hb = 0;
    for (float v : br.hidden) hs += v;
    for (float v : b.hidden) hb += v;
    printf("pos %d/%d hidden sums %.9g %.9g best %d %d\n", br.pos, b.pos, hs, hb, top(br.logits), top(b.logits));
    br.swap_state(b);
    printf("swapped pos %d/%d\n", br.pos, b.pos);
    if (argc > 2) {
        imi_voice vo;
        if (!vo.load(argv[2], 4)) return 1;
        std::vector<float> h(vo.n_in);
        for (int i = 0; i < vo.n_in; i++) h[i] = (float)(i % 17 - 8) * 0.125f;   // exact values
        vo.begin_frame(h.data());
        std::vector<int32_t> codes(vo.n_cb, -1);
        std::vector<float> sc;
        const int half = vo.n_cb / 2;
        for (int pass = 0; pass < 2; pass++) {
            std::vector<int> need;
            for (int c = pass * half; c < (pass ? vo.n_cb : half); c++) need.push_back(c);
            vo.pass(codes.data(), need, sc);
            for (size_t j = 0; j < need.size(); j++) {
                std::vector<float> row(sc.begin() + j * vo.n_vocab, sc.begin() + (j + 1) * vo.n_vocab);
                codes[need[j]] = top(row);
            }
        }
        std::vector<float> fb(vo.n_in);
        vo.feedback(codes.data(), fb.data());
        double fs = 0;
        for (float v : fb) fs += v;
        printf("codes:");
        for (int c : codes) printf(" %d", c);
        printf("\nfeedback sum %.9g\n", fs);
    }
    return 0;
}
