// imi's ears and codec APIs (imi/core/ears.h:17-51, imi/core/codec.h:17-65) from include/seoul_gpu.hpp, used the way
// imi's hearing and talk loops use them (imi/core/hear.cpp: encode a clip, then step_batch the rows;
// imi/core/talk.cpp:178-180: one codec frame per voice frame, flush at the end of speech).
//   sound_check EARS.gguf CLIP.f32 ROWS.out CODEC.gguf CODES.i32 PCM.out
// CLIP.f32: 16 kHz samples; CODES.i32: [frames][12] int32. Writes the ears' rows and the codec's samples as raw
// float32 and prints their shapes.
#include <cstdint>
#include <cstdio>
#include <vector>

#include "seoul_gpu.hpp"

using seoul_hip::imi_codec;
using seoul_hip::imi_ears;

template <class T> static std::vector<T> read_all(const char* path) {
    std::vector<T> v;
    FILE* f = fopen(path, "rb");
    if (!f) return v;
    T x;
    while (fread(&x, sizeof x, 1, f) == 1) v.push_back(x);
    fclose(f);
    return v;
}
static bool write_all(const char* path, const std::vector<float>& v) {
    FILE* f = fopen(path, "wb");
    if (!f) return false;
    const bool ok = fwrite(v.data(), 4, v.size(), f) == v.size();
    fclose(f);
    return ok;
}

int main(int argc, char** argv) {
    if (argc < 7) { fprintf(stderr, "usage: sound_check EARS.gguf CLIP.f32 ROWS.out CODEC.gguf CODES.i32 PCM.out\n"); return 1; }
    imi_ears ears;
    if (!ears.load(argv[1], 4)) return 1;
    const std::vector<float> pcm = read_all<float>(argv[2]);
    std::vector<float> rows;
    const int P = ears.encode(pcm.data(), (int)pcm.size(), rows);
    printf("ears n_pos %d n_out %d n_embd %d n_mel %d window %d mel_frames %zu\n", P, ears.n_out, ears.n_embd, ears.n_mel,
           ears.window, ears.last_mel.size() / (size_t)ears.n_mel);
    if (P <= 0 || !write_all(argv[3], rows)) return 1;

    imi_codec codec;
    if (!codec.load(argv[4], 4)) return 1;
    const std::vector<int32_t> codes = read_all<int32_t>(argv[5]);
    std::vector<float> out;
    for (size_t i = 0; i + 12 <= codes.size(); i += 12) codec.frame(codes.data() + i, out);
    codec.flush(out);
    printf("codec frames %zu samples %zu n_embd %d n_bins %d\n", codes.size() / 12, out.size(), codec.n_embd, codec.n_bins);
    return write_all(argv[6], out) ? 0 : 1;
}
