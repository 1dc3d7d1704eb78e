// Instantiations of fast_kernel with the round-by-round descent (4 streams per workgroup) for the specialised shapes
// (YGG_SHAPES, 1 to 5 layers; one-layer models at readout rank 8 only), in two builds: capped at 128 VGPRs
// (4 wavefronts per SIMD) and uncapped. The largest shape's record alone takes about 130 VGPRs per lane, so it has
// the uncapped build only.
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int R, int R2> constexpr bool kHasCap = N * R2 < 256 * 64;

template <int N, int R, int R2, int L, bool CAP>
hipError_t launch_fast(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    const dim3 grid((B + kFastWaves - 1) / kFastWaves), block(64 * kFastWaves);
    if (io.gen)
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, true, false, CAP>), grid, block, 0, stream, m, tokens, B, T,
                           state, io);
    else
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, false, false, CAP>), grid, block, 0, stream, m, tokens, B, T,
                           state, io);
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool CAP> Kernel fast_k() {
    if constexpr (CAP && !kHasCap<N, R, R2>) {
        return fast_k<N, R, R2, L, false>();
    } else {
        return make_kernel(launch_fast<N, R, R2, L, CAP>, "ygg::fast_kernel<%d, %d, %d, %d, %%s, false, %s>", N, R, R2,
                           L, CAP ? "true" : "false");
    }
}

template <int N, int R, int R2, int L, bool CAP> int fast_blocks(bool gen) {
    if constexpr (CAP && !kHasCap<N, R, R2>) {
        return fast_blocks<N, R, R2, L, false>(gen);
    } else {
        int nb = 0;
        const void *f = gen ? reinterpret_cast<const void *>(&fast_kernel<N, R, R2, L, true, false, CAP>)
                            : reinterpret_cast<const void *>(&fast_kernel<N, R, R2, L, false, false, CAP>);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, 64 * kFastWaves, 0) != hipSuccess) return 0;
        return nb;
    }
}

template <int N, int R, int R2, bool CAP> Kernel fast_for(int L) {
    if (L == 1) {
        if constexpr (R == 8) return fast_k<N, R, R2, 1, CAP>();
        return Kernel();
    }
    if (L == 2) return fast_k<N, R, R2, 2, CAP>();
    if (L == 3) return fast_k<N, R, R2, 3, CAP>();
    if (L == 4) return fast_k<N, R, R2, 4, CAP>();
    if (L == 5) return fast_k<N, R, R2, 5, CAP>();
    return Kernel();
}

template <int N, int R, int R2, bool CAP> int fast_occ(int L, bool gen) {
    if (L == 1) {
        if constexpr (R == 8) return fast_blocks<N, R, R2, 1, CAP>(gen);
        return 0;
    }
    if (L == 2) return fast_blocks<N, R, R2, 2, CAP>(gen);
    if (L == 3) return fast_blocks<N, R, R2, 3, CAP>(gen);
    if (L == 4) return fast_blocks<N, R, R2, 4, CAP>(gen);
    if (L == 5) return fast_blocks<N, R, R2, 5, CAP>(gen);
    return 0;
}

Kernel find_fast_launcher(int n, int R, int R2, int L, bool cap) {
#define YGG_F(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) return cap ? fast_for<N_, R_, R2_, true>(L) : fast_for<N_, R_, R2_, false>(L);
    YGG_SHAPES(YGG_F)
#undef YGG_F
    return Kernel();
}

int fast_blocks_per_cu(int n, int R, int R2, int L, bool cap, bool gen) {
#define YGG_F(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) \
        return cap ? fast_occ<N_, R_, R2_, true>(L, gen) : fast_occ<N_, R_, R2_, false>(L, gen);
    YGG_SHAPES(YGG_F)
#undef YGG_F
    return 0;
}

}  // namespace ygg
