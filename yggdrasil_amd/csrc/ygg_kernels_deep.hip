// Instantiations of the few-stream kernels for the specialised shapes (YGG_SHAPES): pipe_kernel (one workgroup per
// stream, one wavefront per layer), with the 128-VGPR cap (more resident workgroups) or without (no spills, for
// fewer streams), and fast_kernel with the deep router descent (one stream per workgroup; routed models whose LDS
// tables and second-round rows fit in a workgroup's 160 KiB).
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int R, int R2> constexpr bool kHasCap = N * R2 < 256 * 64;

// LDS of the deep kernel: tables, the second round's rows of every routed layer, the stream's buffers
template <int N, int R, int R2, int L>
constexpr bool kDeepFits = kTablesBytes<Shape<N, R, R2>, L> + (L - 1) * kR2Slots<N> * N + L * N + 128 <= 160 * 1024;

template <int N, int R, int R2, int L>
hipError_t launch_deep(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    // one stream per workgroup of 4 wavefronts (all stage the LDS tables, one runs the stream)
    const dim3 grid(B), block(64 * kFastWaves);
    if (io.gen)
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, true, true, false>), grid, block, 0, stream, m, tokens, B, T,
                           state, io);
    else
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, false, true, false>), grid, block, 0, stream, m, tokens, B, T,
                           state, io);
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool CAP>
hipError_t launch_pipe(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    hipLaunchKernelGGL((pipe_kernel<N, R, R2, L, CAP>), dim3(B), dim3(64 * L), 0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool CAP> Kernel pipe_k() {
    if constexpr (CAP && !kHasCap<N, R, R2>) {
        return pipe_k<N, R, R2, L, false>();
    } else {
        return make_kernel(launch_pipe<N, R, R2, L, CAP>, "ygg::pipe_kernel<%d, %d, %d, %d, %s>", N, R, R2, L,
                           CAP ? "true" : "false");
    }
}

template <int N, int R, int R2, int L, bool CAP> int pipe_blocks() {
    if constexpr (CAP && !kHasCap<N, R, R2>) {
        return pipe_blocks<N, R, R2, L, false>();
    } else {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, reinterpret_cast<const void *>(&pipe_kernel<N, R, R2, L, CAP>), 64 * L, 0) != hipSuccess)
            return 0;
        return nb;
    }
}

template <int N, int R, int R2, int L> Kernel deep_k() {
    if constexpr (L >= 2 && kDeepFits<N, R, R2, L>)
        return make_kernel(launch_deep<N, R, R2, L>, "ygg::fast_kernel<%d, %d, %d, %d, %%s, true, false>", N, R, R2,
                           L);
    else
        return Kernel();
}

template <int N, int R, int R2, bool CAP> Kernel pipe_for(int L) {
    if (L == 1) {
        if constexpr (R == 8) return pipe_k<N, R, R2, 1, CAP>();
        return Kernel();
    }
    if (L == 2) return pipe_k<N, R, R2, 2, CAP>();
    if (L == 3) return pipe_k<N, R, R2, 3, CAP>();
    if (L == 4) return pipe_k<N, R, R2, 4, CAP>();
    if (L == 5) return pipe_k<N, R, R2, 5, CAP>();
    return Kernel();
}

template <int N, int R, int R2, bool CAP> int pipe_occ(int L) {
    if (L == 1) {
        if constexpr (R == 8) return pipe_blocks<N, R, R2, 1, CAP>();
        return 0;
    }
    if (L == 2) return pipe_blocks<N, R, R2, 2, CAP>();
    if (L == 3) return pipe_blocks<N, R, R2, 3, CAP>();
    if (L == 4) return pipe_blocks<N, R, R2, 4, CAP>();
    if (L == 5) return pipe_blocks<N, R, R2, 5, CAP>();
    return 0;
}

template <int N, int R, int R2> Kernel deep_for(int L) {
    if (L == 2) return deep_k<N, R, R2, 2>();
    if (L == 3) return deep_k<N, R, R2, 3>();
    if (L == 4) return deep_k<N, R, R2, 4>();
    if (L == 5) return deep_k<N, R, R2, 5>();
    return Kernel();
}

// the layer-pipelined kernel for few streams
Kernel find_pipe_launcher(int n, int R, int R2, int L, bool cap) {
#define YGG_P(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) return cap ? pipe_for<N_, R_, R2_, true>(L) : pipe_for<N_, R_, R2_, false>(L);
    YGG_SHAPES(YGG_P)
#undef YGG_P
    return Kernel();
}

// workgroups of that kernel (one stream each) resident per CU on the current device
int pipe_blocks_per_cu(int n, int R, int R2, int L, bool cap) {
#define YGG_P(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) return cap ? pipe_occ<N_, R_, R2_, true>(L) : pipe_occ<N_, R_, R2_, false>(L);
    YGG_SHAPES(YGG_P)
#undef YGG_P
    return 0;
}

// fast_kernel with the deep descent (2 <= L <= 5, where its LDS fits)
Kernel find_deep_launcher(int n, int R, int R2, int L) {
#define YGG_D(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) return deep_for<N_, R_, R2_>(L);
    YGG_SHAPES(YGG_D)
#undef YGG_D
    return Kernel();
}

}  // namespace ygg
