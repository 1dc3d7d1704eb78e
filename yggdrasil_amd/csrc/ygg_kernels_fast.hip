// Instantiations of fast_kernel with the round-by-round descent (4 streams per workgroup), for the common shape, in
// two builds: capped at 128 VGPRs (4 wavefronts per SIMD) and uncapped.
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int L, bool CAP>
hipError_t launch_fast(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    const dim3 grid((B + kFastWaves - 1) / kFastWaves), block(64 * kFastWaves);
    if (io.gen)
        hipLaunchKernelGGL((fast_kernel<N, L, true, false, CAP>), grid, block, 0, stream, m, tokens, B, T, state, io);
    else
        hipLaunchKernelGGL((fast_kernel<N, L, false, false, CAP>), grid, block, 0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int L, bool CAP> Kernel fast_k() {
    return make_kernel(launch_fast<N, L, CAP>, "ygg::fast_kernel<%d, %d, %%s, false, %s>", N, L, CAP ? "true" : "false");
}

// workgroups (4 streams each) of one build resident per CU on the current device, for steps (gen false) or
// generation
template <int N, int L, bool CAP> int fast_blocks(bool gen) {
    int nb = 0;
    const void *f = gen ? reinterpret_cast<const void *>(&fast_kernel<N, L, true, false, CAP>)
                        : reinterpret_cast<const void *>(&fast_kernel<N, L, false, false, CAP>);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, 64 * kFastWaves, 0) != hipSuccess) return 0;
    return nb;
}

template <bool CAP> Kernel fast_for(int n, int L) {
#define YGG_L(N) \
    if (L == 1) return fast_k<N, 1, CAP>(); if (L == 2) return fast_k<N, 2, CAP>(); \
    if (L == 3) return fast_k<N, 3, CAP>(); if (L == 4) return fast_k<N, 4, CAP>();
    if (n == 64) { YGG_L(64) }
    if (n == 96) { YGG_L(96) }
    if (n == 128) { YGG_L(128) }
#undef YGG_L
    return Kernel();
}

template <bool CAP> int fast_occ(int n, int L, bool gen) {
#define YGG_O(N) \
    if (L == 1) return fast_blocks<N, 1, CAP>(gen); if (L == 2) return fast_blocks<N, 2, CAP>(gen); \
    if (L == 3) return fast_blocks<N, 3, CAP>(gen); if (L == 4) return fast_blocks<N, 4, CAP>(gen);
    if (n == 64) { YGG_O(64) }
    if (n == 96) { YGG_O(96) }
    if (n == 128) { YGG_O(128) }
#undef YGG_O
    return 0;
}

// the specialised kernel: readout rank 8, block 16, layer-input rank <= 16, table storage, tensor scales, L <= 4
Kernel find_fast_launcher(int n, int L, bool cap) { return cap ? fast_for<true>(n, L) : fast_for<false>(n, L); }

int fast_blocks_per_cu(int n, int L, bool cap, bool gen) {
    return cap ? fast_occ<true>(n, L, gen) : fast_occ<false>(n, L, gen);
}

}  // namespace ygg
