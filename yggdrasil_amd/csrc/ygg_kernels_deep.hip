// Instantiations of the few-stream kernels for the common shape: pipe_kernel (one workgroup per stream, one
// wavefront per layer) and fast_kernel with the deep router descent (one stream per workgroup; routed models only).
#include "ygg_kernel_fast.h"

namespace ygg {

typedef hipError_t (*Launcher)(const YggDevModel &, const int32_t *, int, int, int8_t *, const YggIO &, hipStream_t);

template <int N, int L>
hipError_t launch_deep(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    // one stream per workgroup of 4 wavefronts (all stage the LDS tables, one runs the stream)
    const dim3 grid(B), block(64 * kFastWaves);
    if (io.gen)
        hipLaunchKernelGGL((fast_kernel<N, L, true, true>), grid, block, 0, stream, m, tokens, B, T, state, io);
    else
        hipLaunchKernelGGL((fast_kernel<N, L, false, true>), grid, block, 0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int L>
hipError_t launch_pipe(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    hipLaunchKernelGGL((pipe_kernel<N, L>), dim3(B), dim3(64 * L), 0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int L> int pipe_blocks() {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(&pipe_kernel<N, L>), 64 * L,
                                                     0) != hipSuccess)
        return 0;
    return nb;
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

#define YGG_D(N) \
    if (L == 2) return launch_deep<N, 2>; if (L == 3) return launch_deep<N, 3>; if (L == 4) return launch_deep<N, 4>;

// fast_kernel with the deep descent (2 <= L <= 4)
Launcher find_deep_launcher(int n, int L) {
    if (n == 64) { YGG_D(64) }
    if (n == 96) { YGG_D(96) }
    if (n == 128) { YGG_D(128) }
    return nullptr;
}

}  // namespace ygg
