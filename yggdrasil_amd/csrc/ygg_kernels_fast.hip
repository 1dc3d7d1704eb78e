// Instantiations of fast_kernel with the round-by-round descent (4 streams per workgroup) for the specialised shapes
// (YGG_SHAPES, 1 to 5 layers; one-layer models at readout rank 8 only), in two builds: capped at 128 VGPRs
// (4 wavefronts per SIMD) and uncapped. The largest shape's record alone takes about 130 VGPRs per lane, so it has
// the uncapped build only. Models with group scales have builds of their own for n of 64, 128 and 256.
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int R, int R2> constexpr bool kHasCap = N * R2 < 256 * 64;
template <int N> constexpr bool kGroupOk = N != 96;          // group scales need whole 16-coordinate groups per lane

template <int N, int R, int R2, int L, bool CAP, bool GROUP>
hipError_t launch_fast(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    const dim3 grid((B + kFastWaves - 1) / kFastWaves), block(64 * kFastWaves);
    switch (io_mode(io)) {
    case kModeGenerate:
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeGenerate, false, CAP, GROUP>), grid, block, 0, stream, m,
                           tokens, B, T, state, io);
        break;
    case kModeScore:
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeScore, false, CAP, GROUP>), grid, block, 0, stream, m,
                           tokens, B, T, state, io);
        break;
    default:
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeRun, false, CAP, GROUP>), grid, block, 0, stream, m, tokens,
                           B, T, state, io);
    }
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool CAP, bool GROUP> Kernel fast_k() {
    if constexpr (GROUP && !kGroupOk<N>) {
        return Kernel();
    } else if constexpr (CAP && !kHasCap<N, R, R2>) {
        return fast_k<N, R, R2, L, false, GROUP>();
    } else {
        return modal(make_kernel(launch_fast<N, R, R2, L, CAP, GROUP>,
                                 "ygg::fast_kernel<%d, %d, %d, %d, %%s, false, %s, %s>", N, R, R2, L,
                                 CAP ? "true" : "false", GROUP ? "true" : "false"));
    }
}

template <int N, int R, int R2, int L, bool CAP, bool GROUP> int fast_blocks(int mode) {
    if constexpr (GROUP && !kGroupOk<N>) {
        return 0;
    } else if constexpr (CAP && !kHasCap<N, R, R2>) {
        return fast_blocks<N, R, R2, L, false, GROUP>(mode);
    } else {
        int nb = 0;
        const void *f =
            mode == kModeGenerate ? reinterpret_cast<const void *>(&fast_kernel<N, R, R2, L, kModeGenerate, false, CAP, GROUP>)
            : mode == kModeScore  ? reinterpret_cast<const void *>(&fast_kernel<N, R, R2, L, kModeScore, false, CAP, GROUP>)
                                  : reinterpret_cast<const void *>(&fast_kernel<N, R, R2, L, kModeRun, false, CAP, GROUP>);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, 64 * kFastWaves, 0) != hipSuccess) return 0;
        return nb;
    }
}

template <int N, int R, int R2, bool CAP, bool GROUP> Kernel fast_for(int L) {
    if (L == 1) {
        if constexpr (R == 8) return fast_k<N, R, R2, 1, CAP, GROUP>();
        return Kernel();
    }
    if (L == 2) return fast_k<N, R, R2, 2, CAP, GROUP>();
    if (L == 3) return fast_k<N, R, R2, 3, CAP, GROUP>();
    if (L == 4) return fast_k<N, R, R2, 4, CAP, GROUP>();
    if (L == 5) return fast_k<N, R, R2, 5, CAP, GROUP>();
    return Kernel();
}

template <int N, int R, int R2, bool CAP, bool GROUP> int fast_occ(int L, int mode) {
    if (L == 1) {
        if constexpr (R == 8) return fast_blocks<N, R, R2, 1, CAP, GROUP>(mode);
        return 0;
    }
    if (L == 2) return fast_blocks<N, R, R2, 2, CAP, GROUP>(mode);
    if (L == 3) return fast_blocks<N, R, R2, 3, CAP, GROUP>(mode);
    if (L == 4) return fast_blocks<N, R, R2, 4, CAP, GROUP>(mode);
    if (L == 5) return fast_blocks<N, R, R2, 5, CAP, GROUP>(mode);
    return 0;
}

Kernel find_fast_launcher(int n, int R, int R2, int L, bool cap, bool group) {
#define YGG_F(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) { \
        if (group) return cap ? fast_for<N_, R_, R2_, true, true>(L) : fast_for<N_, R_, R2_, false, true>(L); \
        return cap ? fast_for<N_, R_, R2_, true, false>(L) : fast_for<N_, R_, R2_, false, false>(L); \
    }
    YGG_SHAPES(YGG_F)
#undef YGG_F
    return Kernel();
}

int fast_blocks_per_cu(int n, int R, int R2, int L, bool cap, bool group, int mode) {
#define YGG_F(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) { \
        if (group) return cap ? fast_occ<N_, R_, R2_, true, true>(L, mode) : fast_occ<N_, R_, R2_, false, true>(L, mode); \
        return cap ? fast_occ<N_, R_, R2_, true, false>(L, mode) : fast_occ<N_, R_, R2_, false, false>(L, mode); \
    }
    YGG_SHAPES(YGG_F)
#undef YGG_F
    return 0;
}

}  // namespace ygg
