// TEST INFRASTRUCTURE ONLY. A driver around the reference's f32 softmax (the per-token work of `ygg time`,
// cpu/ygg.cpp:46-72, 545-553), compiled from the reference source where it lies (YGG_REF_SOURCE) by oracle/Makefile
// into oracle/_ref/. Nothing of the reference is copied here: this file includes it and calls its own softmax().
//
//   ygg_softmax rows V logits.f32 probs.f32 lse.f32
//
// For each of `rows` rows of V logits: the probabilities the reference writes and the log-sum-exp it returns.
#define main ygg_reference_main
#ifndef YGG_REF_SOURCE
#define YGG_REF_SOURCE "/root/reference/cpu/ygg.cpp"
#endif
#include YGG_REF_SOURCE
#undef main

int main(int argc, char **argv) {
    if (argc != 6) {
        fputs("usage: ygg_softmax rows V logits.f32 probs.f32 lse.f32\n", stderr);
        return 1;
    }
    const long rows = atol(argv[1]);
    const int V = atoi(argv[2]);
    if (rows <= 0 || V <= 0) die("bad rows or V");
    const int VP = (V + 15) / 16 * 16;
    std::vector<float> lg((size_t)rows * V), pr((size_t)rows * V), ls((size_t)rows);
    FILE *f = fopen(argv[3], "rb");
    if (!f || fread(lg.data(), 4, lg.size(), f) != lg.size()) die("%s: short read", argv[3]);
    fclose(f);
    // the reference reads and writes whole 16-float vectors under masks: rows padded to VP, as st.lg and prob are
    float *in, *out;
    if (posix_memalign((void **)&in, 64, (size_t)VP * 4 + 64) || posix_memalign((void **)&out, 64, (size_t)VP * 4 + 64))
        die("out of memory");
    for (long r = 0; r < rows; r++) {
        memset(in, 0, (size_t)VP * 4);
        memcpy(in, &lg[(size_t)r * V], (size_t)V * 4);
        ls[r] = softmax(in, out, V);
        memcpy(&pr[(size_t)r * V], out, (size_t)V * 4);
    }
    auto put = [](const char *path, const void *p, size_t bytes) {
        FILE *o = fopen(path, "wb");
        if (!o || fwrite(p, 1, bytes, o) != bytes) { perror(path); exit(1); }
        fclose(o);
    };
    put(argv[4], pr.data(), pr.size() * 4);
    put(argv[5], ls.data(), ls.size() * 4);
    free(in);
    free(out);
    return 0;
}
