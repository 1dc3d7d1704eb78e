// Instantiations of fast_kernel with the round-by-round descent (many streams), for the common shape.
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int L>
hipError_t launch_fast(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    const dim3 grid((B + kFastWaves - 1) / kFastWaves), block(64 * kFastWaves);
    if (io.gen)
        hipLaunchKernelGGL((fast_kernel<N, L, true, false>), grid, block, 0, stream, m, tokens, B, T, state, io);
    else
        hipLaunchKernelGGL((fast_kernel<N, L, false, false>), grid, block, 0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int L> Kernel kernel() {
    return make_kernel(launch_fast<N, L>, "ygg::fast_kernel<%d, %d, %%s, false>", N, L);
}

#define YGG_L(N) \
    if (L == 1) return kernel<N, 1>(); if (L == 2) return kernel<N, 2>(); \
    if (L == 3) return kernel<N, 3>(); if (L == 4) return kernel<N, 4>();

// the specialised kernel: readout rank 8, block 16, layer-input rank <= 16, table storage, tensor scales, L <= 4
Kernel find_fast_launcher(int n, int L) {
    if (n == 64) { YGG_L(64) }
    if (n == 96) { YGG_L(96) }
    if (n == 128) { YGG_L(128) }
    return Kernel();
}

}  // namespace ygg
