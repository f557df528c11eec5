// Drives the GPU engine through imi's own API (include/seoul_gpu.hpp) the way imi's callers do
// (imi/core/seoul_check.cpp, imi/core/hear.cpp:58-72): prompt, greedy loop on the host, step2 riding.
//   seoul_gpu_check MODEL.gguf  -> prints the greedy ids and hidden checksums
#include <cmath>
#include <cstdio>
#include <vector>

#include "seoul_gpu.hpp"

using seoul_hip::imi_seoul;
using seoul_hip::imi_seoul_state;

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
    return 0;
}
