// Instantiations of the general step kernel for every supported (d_state, block, readout rank), and the lookup the
// C-ABI dispatches through. The specialised kernels are instantiated in ygg_kernels_fast.hip and
// ygg_kernels_deep.hip.
#include "ygg_kernel.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int BLK, int R>
hipError_t launch(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    if (io.gen)
        hipLaunchKernelGGL((run_kernel<N, BLK, R, true>), dim3(B), dim3(64), 0, stream, m, tokens, T, state, io);
    else
        hipLaunchKernelGGL((run_kernel<N, BLK, R, false>), dim3(B), dim3(64), 0, stream, m, tokens, T, state, io);
    return hipGetLastError();
}

template <int N, int BLK, int R> Kernel kernel() {
    return make_kernel(launch<N, BLK, R>, "ygg::run_kernel<%d, %d, %d, %%s>", N, BLK, R);
}

#define YGG_R(N, BLK) \
    if (R == 8) return kernel<N, BLK, 8>(); if (R == 16) return kernel<N, BLK, 16>(); \
    if (R == 32) return kernel<N, BLK, 32>();
#define YGG_B(N) \
    if (blk == 8) { YGG_R(N, 8) } if (blk == 16) { YGG_R(N, 16) }

Kernel find_launcher(int n, int blk, int R) {
    if (n == 64) { YGG_B(64) }
    if (n == 96) { YGG_B(96) }
    if (n == 128) { YGG_B(128) }
    if (n == 256) { YGG_B(256) }
    return Kernel();
}

}  // namespace ygg
