// Instantiations of the per-stream kernel for the fast-only shapes (YGG_FAST_EXTRA and, with factored routed inputs,
// YGG_FACT_EXTRA: the (state width, readout rank, layer-input rank, block) combinations of the reference's
// kernel-test matrix that no benchmark configuration or trained model uses): fast_kernel / fact_kernel for blocks of
// 16, fast8_kernel / fact8_kernel for blocks of 8; routed models (2 to 5 layers), the uncapped build only (these
// shapes serve correctness, not the batch-4096 benchmark), group-scale builds for n of 64, 128 and 256. The other
// kernel families (deep descent, layer pipeline, tick pipeline) keep to YGG_SHAPES.
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

// the kernel of a fast-only shape: FACT picks the factored-input form, BLK the block
template <int N, int R, int R2, int BLK, bool FACT, int L, int MODE, bool GROUP> const void *fastx_fn() {
    if constexpr (FACT && BLK == 8)
        return reinterpret_cast<const void *>(&fact8_kernel<N, R, R2, L, MODE, false, GROUP>);
    else if constexpr (FACT)
        return reinterpret_cast<const void *>(&fact_kernel<N, R, R2, L, MODE, false, GROUP>);
    else if constexpr (BLK == 8)
        return reinterpret_cast<const void *>(&fast8_kernel<N, R, R2, L, MODE, false, GROUP>);
    else
        return reinterpret_cast<const void *>(&fast_kernel<N, R, R2, L, MODE, false, false, GROUP>);
}

template <int N, int R, int R2, int BLK, bool FACT, int L, bool GROUP>
hipError_t launch_fastx(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                        hipStream_t stream) {
    const int mode = io_mode(io);
    const void *f = mode == kModeGenerate ? fastx_fn<N, R, R2, BLK, FACT, L, kModeGenerate, GROUP>()
                    : mode == kModeScore  ? fastx_fn<N, R, R2, BLK, FACT, L, kModeScore, GROUP>()
                                          : fastx_fn<N, R, R2, BLK, FACT, L, kModeRun, GROUP>();
    YggDevModel mm = m;
    YggIO ii = io;
    const int32_t *tk = tokens;
    int8_t *sp = state;
    void *args[] = {&mm, &tk, &B, &T, &sp, &ii};
    return hipLaunchKernel(f, dim3((B + kFastWaves - 1) / kFastWaves), dim3(64 * kFastWaves), args, 0, stream);
}

template <int N, int R, int R2, int BLK, bool FACT, int L, bool GROUP> Kernel fastx_k() {
    if constexpr (GROUP && N == 96) {
        return Kernel();
    } else if constexpr (FACT) {
        return modal(make_kernel(launch_fastx<N, R, R2, BLK, FACT, L, GROUP>,
                                 BLK == 8 ? "ygg::fact8_kernel<%d, %d, %d, %d, %%s, false, %s>"
                                          : "ygg::fact_kernel<%d, %d, %d, %d, %%s, false, %s>",
                                 N, R, R2, L, GROUP ? "true" : "false"));
    } else if constexpr (BLK == 8) {
        return modal(make_kernel(launch_fastx<N, R, R2, BLK, FACT, L, GROUP>,
                                 "ygg::fast8_kernel<%d, %d, %d, %d, %%s, false, %s>", N, R, R2, L,
                                 GROUP ? "true" : "false"));
    } else {
        return modal(make_kernel(launch_fastx<N, R, R2, BLK, FACT, L, GROUP>,
                                 "ygg::fast_kernel<%d, %d, %d, %d, %%s, false, false, %s>", N, R, R2, L,
                                 GROUP ? "true" : "false"));
    }
}

template <int N, int R, int R2, int BLK, bool FACT, int L, bool GROUP> int fastx_blocks(int mode) {
    if constexpr (GROUP && N == 96) {
        return 0;
    } else {
        const void *f = mode == kModeGenerate ? fastx_fn<N, R, R2, BLK, FACT, L, kModeGenerate, GROUP>()
                        : mode == kModeScore  ? fastx_fn<N, R, R2, BLK, FACT, L, kModeScore, GROUP>()
                                              : fastx_fn<N, R, R2, BLK, FACT, L, kModeRun, GROUP>();
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, 64 * kFastWaves, 0) != hipSuccess) return 0;
        return nb;
    }
}

template <int N, int R, int R2, int BLK, bool FACT, bool GROUP> Kernel fastx_for(int L) {
    if (L == 2) return fastx_k<N, R, R2, BLK, FACT, 2, GROUP>();
    if (L == 3) return fastx_k<N, R, R2, BLK, FACT, 3, GROUP>();
    if (L == 4) return fastx_k<N, R, R2, BLK, FACT, 4, GROUP>();
    if (L == 5) return fastx_k<N, R, R2, BLK, FACT, 5, GROUP>();
    return Kernel();
}

template <int N, int R, int R2, int BLK, bool FACT, bool GROUP> int fastx_occ(int L, int mode) {
    if (L == 2) return fastx_blocks<N, R, R2, BLK, FACT, 2, GROUP>(mode);
    if (L == 3) return fastx_blocks<N, R, R2, BLK, FACT, 3, GROUP>(mode);
    if (L == 4) return fastx_blocks<N, R, R2, BLK, FACT, 4, GROUP>(mode);
    if (L == 5) return fastx_blocks<N, R, R2, BLK, FACT, 5, GROUP>(mode);
    return 0;
}

Kernel find_fast_extra_launcher(int n, int R, int R2, int blk, int L, bool group, bool factored) {
#define YGG_X(N_, R_, R2_, B_) \
    if (!factored && n == N_ && R == R_ && R2 == R2_ && blk == B_) \
        return group ? fastx_for<N_, R_, R2_, B_, false, true>(L) : fastx_for<N_, R_, R2_, B_, false, false>(L);
    YGG_FAST_EXTRA(YGG_X)
#undef YGG_X
#define YGG_X(N_, R_, R2_, B_) \
    if (factored && n == N_ && R == R_ && R2 == R2_ && blk == B_) \
        return group ? fastx_for<N_, R_, R2_, B_, true, true>(L) : fastx_for<N_, R_, R2_, B_, true, false>(L);
    YGG_FACT_EXTRA(YGG_X)
#undef YGG_X
    return Kernel();
}

int fast_extra_blocks_per_cu(int n, int R, int R2, int blk, int L, bool group, bool factored, int mode) {
#define YGG_X(N_, R_, R2_, B_) \
    if (!factored && n == N_ && R == R_ && R2 == R2_ && blk == B_) \
        return group ? fastx_occ<N_, R_, R2_, B_, false, true>(L, mode) \
                     : fastx_occ<N_, R_, R2_, B_, false, false>(L, mode);
    YGG_FAST_EXTRA(YGG_X)
#undef YGG_X
#define YGG_X(N_, R_, R2_, B_) \
    if (factored && n == N_ && R == R_ && R2 == R2_ && blk == B_) \
        return group ? fastx_occ<N_, R_, R2_, B_, true, true>(L, mode) : fastx_occ<N_, R_, R2_, B_, true, false>(L, mode);
    YGG_FACT_EXTRA(YGG_X)
#undef YGG_X
    return 0;
}

}  // namespace ygg
