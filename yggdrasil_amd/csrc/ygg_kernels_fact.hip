// Instantiations of fact_kernel (fast_kernel for models with factored routed inputs, 4 streams per workgroup) for the
// specialised shapes (YGG_SHAPES, 2 to 5 layers: a factored model has at least one routed layer), capped at 128 VGPRs
// and uncapped as fast_kernel is (the largest shape uncapped only). Group scales have builds of their own for n of
// 64, 128 and 256.
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int R, int R2> constexpr bool kHasCapF = N * R2 < 256 * 64;
template <int N> constexpr bool kGroupOkF = N != 96;

template <int N, int R, int R2, int L, bool CAP, bool GROUP>
hipError_t launch_fact(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    const dim3 grid((B + kFastWaves - 1) / kFastWaves), block(64 * kFastWaves);
    switch (io_mode(io)) {
    case kModeGenerate:
        hipLaunchKernelGGL((fact_kernel<N, R, R2, L, kModeGenerate, CAP, GROUP>), grid, block, 0, stream, m, tokens,
                           B, T, state, io);
        break;
    case kModeScore:
        hipLaunchKernelGGL((fact_kernel<N, R, R2, L, kModeScore, CAP, GROUP>), grid, block, 0, stream, m, tokens, B,
                           T, state, io);
        break;
    default:
        hipLaunchKernelGGL((fact_kernel<N, R, R2, L, kModeRun, CAP, GROUP>), grid, block, 0, stream, m, tokens, B, T,
                           state, io);
    }
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool CAP, bool GROUP> Kernel fact_k() {
    if constexpr (GROUP && !kGroupOkF<N>) {
        return Kernel();
    } else if constexpr (CAP && !kHasCapF<N, R, R2>) {
        return fact_k<N, R, R2, L, false, GROUP>();
    } else {
        return modal(make_kernel(launch_fact<N, R, R2, L, CAP, GROUP>, "ygg::fact_kernel<%d, %d, %d, %d, %%s, %s, %s>",
                                 N, R, R2, L, CAP ? "true" : "false", GROUP ? "true" : "false"));
    }
}

template <int N, int R, int R2, int L, bool CAP, bool GROUP> int fact_blocks(int mode) {
    if constexpr (GROUP && !kGroupOkF<N>) {
        return 0;
    } else if constexpr (CAP && !kHasCapF<N, R, R2>) {
        return fact_blocks<N, R, R2, L, false, GROUP>(mode);
    } else {
        int nb = 0;
        const void *f =
            mode == kModeGenerate ? reinterpret_cast<const void *>(&fact_kernel<N, R, R2, L, kModeGenerate, CAP, GROUP>)
            : mode == kModeScore  ? reinterpret_cast<const void *>(&fact_kernel<N, R, R2, L, kModeScore, CAP, GROUP>)
                                  : reinterpret_cast<const void *>(&fact_kernel<N, R, R2, L, kModeRun, CAP, GROUP>);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, 64 * kFastWaves, 0) != hipSuccess) return 0;
        return nb;
    }
}

template <int N, int R, int R2, bool CAP, bool GROUP> Kernel fact_for(int L) {
    if (L == 2) return fact_k<N, R, R2, 2, CAP, GROUP>();
    if (L == 3) return fact_k<N, R, R2, 3, CAP, GROUP>();
    if (L == 4) return fact_k<N, R, R2, 4, CAP, GROUP>();
    if (L == 5) return fact_k<N, R, R2, 5, CAP, GROUP>();
    return Kernel();
}

template <int N, int R, int R2, bool CAP, bool GROUP> int fact_occ(int L, int mode) {
    if (L == 2) return fact_blocks<N, R, R2, 2, CAP, GROUP>(mode);
    if (L == 3) return fact_blocks<N, R, R2, 3, CAP, GROUP>(mode);
    if (L == 4) return fact_blocks<N, R, R2, 4, CAP, GROUP>(mode);
    if (L == 5) return fact_blocks<N, R, R2, 5, CAP, GROUP>(mode);
    return 0;
}

Kernel find_fact_launcher(int n, int R, int R2, int L, bool cap, bool group) {
#define YGG_F(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) { \
        if (group) return cap ? fact_for<N_, R_, R2_, true, true>(L) : fact_for<N_, R_, R2_, false, true>(L); \
        return cap ? fact_for<N_, R_, R2_, true, false>(L) : fact_for<N_, R_, R2_, false, false>(L); \
    }
    YGG_SHAPES(YGG_F)
#undef YGG_F
    return Kernel();
}

int fact_blocks_per_cu(int n, int R, int R2, int L, bool cap, bool group, int mode) {
#define YGG_F(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) { \
        if (group) return cap ? fact_occ<N_, R_, R2_, true, true>(L, mode) : fact_occ<N_, R_, R2_, false, true>(L, mode); \
        return cap ? fact_occ<N_, R_, R2_, true, false>(L, mode) : fact_occ<N_, R_, R2_, false, false>(L, mode); \
    }
    YGG_SHAPES(YGG_F)
#undef YGG_F
    return 0;
}

}  // namespace ygg
