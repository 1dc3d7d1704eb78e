// TEST INFRASTRUCTURE ONLY. A driver around the reference kernel, compiled from the reference source where it lies
// (YGG_REF_SOURCE, default /root/reference/cpu/ygg.cpp) by oracle/Makefile into oracle/_ref/. Nothing of the
// reference is copied here: this file includes it and calls its own load, dispatch_state, rms_rho and route.
//
//   ygg_dump model.bin x.i32 nwin T logits.f32 leaves.i32 states.i8
//
// Same windows as `ygg logits` (zero state at every window, cpu/ygg.cpp:500-525), plus per token the expert of every
// layer (layer 0: the token) and the int8 state of every layer after the token. The routed layer's expert is
// recomputed after the step from the updated state of the layer below, which is what route() read during the step
// (cpu/ygg.cpp:447-450).
#define main ygg_reference_main
#ifndef YGG_REF_SOURCE
#define YGG_REF_SOURCE "/root/reference/cpu/ygg.cpp"
#endif
#include YGG_REF_SOURCE
#undef main

template <int N> static int leaf_of(const Model &m, int l, int x, const int8_t *q) {
    const Layer &y = m.layers[l];
    const int8_t *qb = q + (l - 1) * N;
    const float rho = y.group.state_r2 ? rms_rho_group<N>(qb, y.group.state_r2, y.rms_eps) : rms_rho<N>(qb, y.rms_eps);
    return route<N>(m, y, x, qb, rho);
}

int main(int argc, char **argv) {
    if (argc != 8) {
        fputs("usage: ygg_dump model.bin x.i32 nwin T logits.f32 leaves.i32 states.i8\n", stderr);
        return 1;
    }
    const Model m = load(argv[1]);
    const StepFn fn = dispatch_state(m);
    State st = make_state(m);
    const int nw = atoi(argv[3]), T = atoi(argv[4]), V = m.vocab, L = m.n_layers, n = m.n;
    const std::vector<int32_t> tok = read_i32(argv[2], (size_t)nw * T);
    check_tokens(tok, V);
    std::vector<float> lg((size_t)nw * T * V);
    std::vector<int32_t> lv((size_t)nw * T * L);
    std::vector<int8_t> sv((size_t)nw * T * L * n);
    for (int s = 0; s < nw; s++) {
        reset(m, st);
        for (int t = 0; t < T; t++) {
            const size_t i = (size_t)s * T + t;
            const int x = tok[i];
            fn(m, st, x);
            memcpy(&lg[i * V], st.lg, 4 * (size_t)V);
            memcpy(&sv[i * L * n], st.q, (size_t)L * n);
            lv[i * L] = x;
            for (int l = 1; l < L; l++)
                lv[i * L + l] = n == 256 ? leaf_of<256>(m, l, x, st.q) : n == 128 ? leaf_of<128>(m, l, x, st.q)
                                                                        : leaf_of<64>(m, l, x, st.q);
        }
    }
    auto put = [](const char *path, const void *p, size_t bytes) {
        FILE *o = fopen(path, "wb");
        if (!o || fwrite(p, 1, bytes, o) != bytes) { perror(path); exit(1); }
        fclose(o);
    };
    put(argv[5], lg.data(), lg.size() * 4);
    put(argv[6], lv.data(), lv.size() * 4);
    put(argv[7], sv.data(), sv.size());
    return 0;
}
