// Instantiations of the few-stream kernels for the common shape: pipe_kernel (one workgroup per stream, one
// wavefront per layer), with the 128-VGPR cap (more resident workgroups) or without (no spills, for fewer streams),
// and fast_kernel with the deep router descent (one stream per workgroup; routed models only).
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int L>
hipError_t launch_deep(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    // one stream per workgroup of 4 wavefronts (all stage the LDS tables, one runs the stream)
    const dim3 grid(B), block(64 * kFastWaves);
    if (io.gen)
        hipLaunchKernelGGL((fast_kernel<N, L, true, true, false>), grid, block, 0, stream, m, tokens, B, T, state, io);
    else
        hipLaunchKernelGGL((fast_kernel<N, L, false, true, false>), grid, block, 0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int L, bool CAP>
hipError_t launch_pipe(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    hipLaunchKernelGGL((pipe_kernel<N, L, CAP>), dim3(B), dim3(64 * L), 0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int L, bool CAP> int pipe_blocks() {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(&pipe_kernel<N, L, CAP>),
                                                     64 * L, 0) != hipSuccess)
        return 0;
    return nb;
}

template <int N, int L, bool CAP> Kernel pipe_k() {
    return make_kernel(launch_pipe<N, L, CAP>, "ygg::pipe_kernel<%d, %d, %s>", N, L, CAP ? "true" : "false");
}

template <bool CAP> Kernel pipe_for(int n, int L) {
#define YGG_P(N) \
    if (L == 1) return pipe_k<N, 1, CAP>(); if (L == 2) return pipe_k<N, 2, CAP>(); \
    if (L == 3) return pipe_k<N, 3, CAP>(); if (L == 4) return pipe_k<N, 4, CAP>();
    if (n == 64) { YGG_P(64) }
    if (n == 96) { YGG_P(96) }
    if (n == 128) { YGG_P(128) }
#undef YGG_P
    return Kernel();
}

template <bool CAP> int occ_for(int n, int L) {
#define YGG_O(N) \
    if (L == 1) return pipe_blocks<N, 1, CAP>(); if (L == 2) return pipe_blocks<N, 2, CAP>(); \
    if (L == 3) return pipe_blocks<N, 3, CAP>(); if (L == 4) return pipe_blocks<N, 4, CAP>();
    if (n == 64) { YGG_O(64) }
    if (n == 96) { YGG_O(96) }
    if (n == 128) { YGG_O(128) }
#undef YGG_O
    return 0;
}

// the layer-pipelined kernel for few streams (same shapes as the specialised one)
Kernel find_pipe_launcher(int n, int L, bool cap) { return cap ? pipe_for<true>(n, L) : pipe_for<false>(n, L); }

// workgroups of that kernel (one stream each) resident per CU on the current device
int pipe_blocks_per_cu(int n, int L, bool cap) { return cap ? occ_for<true>(n, L) : occ_for<false>(n, L); }

template <int N, int L> Kernel deep_k() {
    return make_kernel(launch_deep<N, L>, "ygg::fast_kernel<%d, %d, %%s, true, false>", N, L);
}

// fast_kernel with the deep descent (2 <= L <= 4)
Kernel find_deep_launcher(int n, int L) {
#define YGG_D(N) \
    if (L == 2) return deep_k<N, 2>(); if (L == 3) return deep_k<N, 3>(); if (L == 4) return deep_k<N, 4>();
    if (n == 64) { YGG_D(64) }
    if (n == 96) { YGG_D(96) }
    if (n == 128) { YGG_D(128) }
#undef YGG_D
    return Kernel();
}

}  // namespace ygg
