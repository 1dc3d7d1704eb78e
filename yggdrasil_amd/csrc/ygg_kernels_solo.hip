// Instantiations of solo_kernel (one stream per workgroup, all four wavefronts on it: one-token steps and generation
// for few streams) for the specialised shapes (YGG_SHAPES, 2 to 5 layers) whose round-A router rows fit a lane's
// registers ((L - 1) n <= 512). Models with group scales have builds of their own for n of 64, 128 and 256.
#include "ygg_kernel_solo.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int R, int R2, int L, bool GROUP>
hipError_t launch_solo(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    if (io_mode(io) == kModeGenerate)
        hipLaunchKernelGGL((solo_kernel<N, R, R2, L, kModeGenerate, GROUP>), dim3(B), dim3(kSoloThreads), 0, stream, m,
                           tokens, B, T, state, io);
    else
        hipLaunchKernelGGL((solo_kernel<N, R, R2, L, kModeRun, GROUP>), dim3(B), dim3(kSoloThreads), 0, stream, m,
                           tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool GROUP> Kernel solo_k() {
    if constexpr (L >= 2 && kSoloRowsFit<N, L> && (!GROUP || N != 96))
        return modal(make_kernel(launch_solo<N, R, R2, L, GROUP>, "ygg::solo_kernel<%d, %d, %d, %d, %%s, %s>", N, R,
                                 R2, L, GROUP ? "true" : "false"));
    else
        return Kernel();
}

template <int N, int R, int R2, bool GROUP> Kernel solo_for(int L) {
    if (L == 2) return solo_k<N, R, R2, 2, GROUP>();
    if (L == 3) return solo_k<N, R, R2, 3, GROUP>();
    if (L == 4) return solo_k<N, R, R2, 4, GROUP>();
    if (L == 5) return solo_k<N, R, R2, 5, GROUP>();
    return Kernel();
}

Kernel find_solo_launcher(int n, int R, int R2, int L, bool group) {
#define YGG_W(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) return group ? solo_for<N_, R_, R2_, true>(L) : solo_for<N_, R_, R2_, false>(L);
    YGG_SHAPES(YGG_W)
#undef YGG_W
    return Kernel();
}

}  // namespace ygg
