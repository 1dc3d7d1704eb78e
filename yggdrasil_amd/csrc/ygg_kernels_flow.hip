// Instantiations of flow_kernel (scoring with the tokens known, one workgroup per stream, the layers' router rounds
// and updates as a software pipeline over ticks) for the specialised shapes (YGG_SHAPES, 2 to 5 layers, router plans
// of 3 or 4 rounds: depths 9 to 16) whose LDS (tables, state and logit rings) fits a workgroup's 160 KiB. Models with
// group scales have builds of their own for n of 64 and 128.
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N> constexpr bool kGroupOk = N != 96;          // group scales need whole 16-coordinate groups per lane

template <int N, int R, int R2, int L, int P, bool GROUP>
hipError_t launch_flow(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    using SH = Shape<N, R, R2>;
    if (io_mode(io) == kModeScore)
        hipLaunchKernelGGL((flow_kernel<N, R, R2, L, P, kModeScore, GROUP>), dim3(B),
                           dim3(kFlowThreads<SH, L, kModeScore>), 0, stream, m, tokens, B, T, state, io);
    else
        hipLaunchKernelGGL((flow_kernel<N, R, R2, L, P, kModeRun, GROUP>), dim3(B), dim3(kFlowThreads<SH, L, kModeRun>),
                           0, stream, m, tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int R, int R2, int L, int P, bool GROUP> constexpr bool kFlowBuilt =
    kFlowFits<N, R, R2, L, P, GROUP> && (!GROUP || kGroupOk<N>);

template <int N, int R, int R2, int L, int P, bool GROUP> Kernel flow_k() {
    if constexpr (kFlowBuilt<N, R, R2, L, P, GROUP>)
        return modal(make_kernel(launch_flow<N, R, R2, L, P, GROUP>, "ygg::flow_kernel<%d, %d, %d, %d, %d, %%s, %s>",
                                 N, R, R2, L, P, GROUP ? "true" : "false"));
    else
        return Kernel();
}

// resident workgroups per CU of the build of a mode (kModeRun or kModeScore: the score build of the largest shape has
// a wavefront more, for the NLL, and may fit fewer workgroups)
template <int N, int R, int R2, int L, int P, int MODE, bool GROUP> int flow_blocks_mode() {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &nb, reinterpret_cast<const void *>(&flow_kernel<N, R, R2, L, P, MODE, GROUP>),
            kFlowThreads<Shape<N, R, R2>, L, MODE>, 0) != hipSuccess)
        return 0;
    return nb;
}

template <int N, int R, int R2, int L, int P, bool GROUP> int flow_blocks(int mode) {
    if constexpr (kFlowBuilt<N, R, R2, L, P, GROUP>) {
        return mode == kModeScore ? flow_blocks_mode<N, R, R2, L, P, kModeScore, GROUP>()
                                  : flow_blocks_mode<N, R, R2, L, P, kModeRun, GROUP>();
    } else {
        return 0;
    }
}

template <int N, int R, int R2, int P, bool GROUP> Kernel flow_for(int L) {
    if (L == 2) return flow_k<N, R, R2, 2, P, GROUP>();
    if (L == 3) return flow_k<N, R, R2, 3, P, GROUP>();
    if (L == 4) return flow_k<N, R, R2, 4, P, GROUP>();
    if (L == 5) return flow_k<N, R, R2, 5, P, GROUP>();
    return Kernel();
}

template <int N, int R, int R2, int P, bool GROUP> int flow_occ(int L, int mode) {
    if (L == 2) return flow_blocks<N, R, R2, 2, P, GROUP>(mode);
    if (L == 3) return flow_blocks<N, R, R2, 3, P, GROUP>(mode);
    if (L == 4) return flow_blocks<N, R, R2, 4, P, GROUP>(mode);
    if (L == 5) return flow_blocks<N, R, R2, 5, P, GROUP>(mode);
    return 0;
}

template <int N, int R, int R2, bool GROUP> Kernel flow_plan(int L, int P) {
    if (P == 3) return flow_for<N, R, R2, 3, GROUP>(L);
    if (P == 4) return flow_for<N, R, R2, 4, GROUP>(L);
    return Kernel();
}

template <int N, int R, int R2, bool GROUP> int flow_plan_occ(int L, int P, int mode) {
    if (P == 3) return flow_occ<N, R, R2, 3, GROUP>(L, mode);
    if (P == 4) return flow_occ<N, R, R2, 4, GROUP>(L, mode);
    return 0;
}

Kernel find_flow_launcher(int n, int R, int R2, int L, int P, bool group) {
#define YGG_W(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) \
        return group ? flow_plan<N_, R_, R2_, true>(L, P) : flow_plan<N_, R_, R2_, false>(L, P);
    YGG_SHAPES(YGG_W)
#undef YGG_W
    return Kernel();
}

// whether the build of this shape, layer count and mode splits the descent (kFlowSplit)
bool flow_split_build(int n, int R, int R2, int L, int mode) {
#define YGG_W(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) return !kFlowBig<Shape<N_, R_, R2_>> && (L <= 4 || mode != kModeScore);
    YGG_SHAPES(YGG_W)
#undef YGG_W
    return false;
}

int flow_blocks_per_cu(int n, int R, int R2, int L, int P, bool group, int mode) {
#define YGG_W(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) \
        return group ? flow_plan_occ<N_, R_, R2_, true>(L, P, mode) : flow_plan_occ<N_, R_, R2_, false>(L, P, mode);
    YGG_SHAPES(YGG_W)
#undef YGG_W
    return 0;
}

}  // namespace ygg
