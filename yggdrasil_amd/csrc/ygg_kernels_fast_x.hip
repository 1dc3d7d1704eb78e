// Instantiations of the per-stream kernel for the fast-only shapes (YGG_FAST_EXTRA: the (state width, readout rank,
// layer-input rank, block) combinations of the reference's kernel-test matrix that no benchmark configuration or
// trained model uses): fast_kernel for blocks of 16, fast8_kernel for blocks of 8; routed models (2 to 5 layers),
// the uncapped build only (these shapes serve correctness, not the batch-4096 benchmark), group-scale builds for n of
// 64, 128 and 256. The other kernel families (deep descent, layer pipeline, tick pipeline) keep to YGG_SHAPES.
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int R, int R2, int BLK, int L, int MODE, bool GROUP> const void *fastx_fn() {
    if constexpr (BLK == 8)
        return reinterpret_cast<const void *>(&fast8_kernel<N, R, R2, L, MODE, false, GROUP>);
    else
        return reinterpret_cast<const void *>(&fast_kernel<N, R, R2, L, MODE, false, false, GROUP>);
}

template <int N, int R, int R2, int BLK, int L, bool GROUP>
hipError_t launch_fastx(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                        hipStream_t stream) {
    const dim3 grid((B + kFastWaves - 1) / kFastWaves), block(64 * kFastWaves);
    switch (io_mode(io)) {
    case kModeGenerate:
        if constexpr (BLK == 8)
            hipLaunchKernelGGL((fast8_kernel<N, R, R2, L, kModeGenerate, false, GROUP>), grid, block, 0, stream, m,
                               tokens, B, T, state, io);
        else
            hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeGenerate, false, false, GROUP>), grid, block, 0,
                               stream, m, tokens, B, T, state, io);
        break;
    case kModeScore:
        if constexpr (BLK == 8)
            hipLaunchKernelGGL((fast8_kernel<N, R, R2, L, kModeScore, false, GROUP>), grid, block, 0, stream, m,
                               tokens, B, T, state, io);
        else
            hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeScore, false, false, GROUP>), grid, block, 0, stream,
                               m, tokens, B, T, state, io);
        break;
    default:
        if constexpr (BLK == 8)
            hipLaunchKernelGGL((fast8_kernel<N, R, R2, L, kModeRun, false, GROUP>), grid, block, 0, stream, m,
                               tokens, B, T, state, io);
        else
            hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeRun, false, false, GROUP>), grid, block, 0, stream, m,
                               tokens, B, T, state, io);
    }
    return hipGetLastError();
}

template <int N, int R, int R2, int BLK, int L, bool GROUP> Kernel fastx_k() {
    if constexpr (GROUP && N == 96) {
        return Kernel();
    } else if constexpr (BLK == 8) {
        return modal(make_kernel(launch_fastx<N, R, R2, BLK, L, GROUP>,
                                 "ygg::fast8_kernel<%d, %d, %d, %d, %%s, false, %s>", N, R, R2, L,
                                 GROUP ? "true" : "false"));
    } else {
        return modal(make_kernel(launch_fastx<N, R, R2, BLK, L, GROUP>,
                                 "ygg::fast_kernel<%d, %d, %d, %d, %%s, false, false, %s>", N, R, R2, L,
                                 GROUP ? "true" : "false"));
    }
}

template <int N, int R, int R2, int BLK, int L, bool GROUP> int fastx_blocks(int mode) {
    if constexpr (GROUP && N == 96) {
        return 0;
    } else {
        const void *f = mode == kModeGenerate ? fastx_fn<N, R, R2, BLK, L, kModeGenerate, GROUP>()
                        : mode == kModeScore  ? fastx_fn<N, R, R2, BLK, L, kModeScore, GROUP>()
                                              : fastx_fn<N, R, R2, BLK, L, kModeRun, GROUP>();
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, 64 * kFastWaves, 0) != hipSuccess) return 0;
        return nb;
    }
}

template <int N, int R, int R2, int BLK, bool GROUP> Kernel fastx_for(int L) {
    if (L == 2) return fastx_k<N, R, R2, BLK, 2, GROUP>();
    if (L == 3) return fastx_k<N, R, R2, BLK, 3, GROUP>();
    if (L == 4) return fastx_k<N, R, R2, BLK, 4, GROUP>();
    if (L == 5) return fastx_k<N, R, R2, BLK, 5, GROUP>();
    return Kernel();
}

template <int N, int R, int R2, int BLK, bool GROUP> int fastx_occ(int L, int mode) {
    if (L == 2) return fastx_blocks<N, R, R2, BLK, 2, GROUP>(mode);
    if (L == 3) return fastx_blocks<N, R, R2, BLK, 3, GROUP>(mode);
    if (L == 4) return fastx_blocks<N, R, R2, BLK, 4, GROUP>(mode);
    if (L == 5) return fastx_blocks<N, R, R2, BLK, 5, GROUP>(mode);
    return 0;
}

Kernel find_fast_extra_launcher(int n, int R, int R2, int blk, int L, bool group) {
#define YGG_X(N_, R_, R2_, B_) \
    if (n == N_ && R == R_ && R2 == R2_ && blk == B_) \
        return group ? fastx_for<N_, R_, R2_, B_, true>(L) : fastx_for<N_, R_, R2_, B_, false>(L);
    YGG_FAST_EXTRA(YGG_X)
#undef YGG_X
    return Kernel();
}

int fast_extra_blocks_per_cu(int n, int R, int R2, int blk, int L, bool group, int mode) {
#define YGG_X(N_, R_, R2_, B_) \
    if (n == N_ && R == R_ && R2 == R2_ && blk == B_) \
        return group ? fastx_occ<N_, R_, R2_, B_, true>(L, mode) : fastx_occ<N_, R_, R2_, B_, false>(L, mode);
    YGG_FAST_EXTRA(YGG_X)
#undef YGG_X
    return 0;
}

}  // namespace ygg
