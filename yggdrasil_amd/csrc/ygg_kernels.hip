// Instantiations of the fused step kernel for every supported (d_state, block, readout rank), and the lookup the
// C-ABI dispatches through.
#include "ygg_kernel.h"
#include "ygg_kernel_fast.h"

namespace ygg {

typedef hipError_t (*Launcher)(const YggDevModel &, const int32_t *, int, int, int8_t *, const YggIO &, hipStream_t);

template <int N, int BLK, int R>
hipError_t launch(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    if (io.gen)
        hipLaunchKernelGGL((run_kernel<N, BLK, R, true>), dim3(B), dim3(64), 0, stream, m, tokens, T, state, io);
    else
        hipLaunchKernelGGL((run_kernel<N, BLK, R, false>), dim3(B), dim3(64), 0, stream, m, tokens, T, state, io);
    return hipGetLastError();
}

#define YGG_R(N, BLK) \
    if (R == 8) return launch<N, BLK, 8>; if (R == 16) return launch<N, BLK, 16>; if (R == 32) return launch<N, BLK, 32>;
#define YGG_B(N) \
    if (blk == 8) { YGG_R(N, 8) } if (blk == 16) { YGG_R(N, 16) }

template <int N, int L>
hipError_t launch_fast(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    const dim3 grid((B + kFastWaves - 1) / kFastWaves), block(64 * kFastWaves);
    if (io.gen)
        hipLaunchKernelGGL((fast_kernel<N, L, true>), grid, block, 0, stream, m, tokens, B, T, state, io);
    else
        hipLaunchKernelGGL((fast_kernel<N, L, false>), grid, block, 0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

#define YGG_L(N) \
    if (L == 1) return launch_fast<N, 1>; if (L == 2) return launch_fast<N, 2>; \
    if (L == 3) return launch_fast<N, 3>; if (L == 4) return launch_fast<N, 4>;

template <int N, int L>
hipError_t launch_pipe(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    hipLaunchKernelGGL((pipe_kernel<N, L>), dim3(B), dim3(64 * L), 0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

#define YGG_P(N) \
    if (L == 1) return launch_pipe<N, 1>; if (L == 2) return launch_pipe<N, 2>; \
    if (L == 3) return launch_pipe<N, 3>; if (L == 4) return launch_pipe<N, 4>;

// the layer-pipelined kernel for few streams (same shapes as the specialised one)
Launcher find_pipe_launcher(int n, int L) {
    if (n == 64) { YGG_P(64) }
    if (n == 96) { YGG_P(96) }
    if (n == 128) { YGG_P(128) }
    return nullptr;
}

template <int N, int L> int pipe_blocks() {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(&pipe_kernel<N, L>), 64 * L,
                                                     0) != hipSuccess)
        return 0;
    return nb;
}

#define YGG_O(N) \
    if (L == 1) return pipe_blocks<N, 1>(); if (L == 2) return pipe_blocks<N, 2>(); \
    if (L == 3) return pipe_blocks<N, 3>(); if (L == 4) return pipe_blocks<N, 4>();

// workgroups of the layer-pipelined kernel (one stream each) resident per CU on the current device
int pipe_blocks_per_cu(int n, int L) {
    if (n == 64) { YGG_O(64) }
    if (n == 96) { YGG_O(96) }
    if (n == 128) { YGG_O(128) }
    return 0;
}

// the specialised kernel: readout rank 8, block 16, layer-input rank <= 16, table storage, tensor scales, L <= 4
Launcher find_fast_launcher(int n, int L) {
    if (n == 64) { YGG_L(64) }
    if (n == 96) { YGG_L(96) }
    if (n == 128) { YGG_L(128) }
    return nullptr;
}

Launcher find_launcher(int n, int blk, int R) {
    if (n == 64) { YGG_B(64) }
    if (n == 96) { YGG_B(96) }
    if (n == 128) { YGG_B(128) }
    if (n == 256) { YGG_B(256) }
    return nullptr;
}

}  // namespace ygg
