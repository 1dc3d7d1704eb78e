// Instantiations of the few-stream kernels for the specialised shapes (YGG_SHAPES): pipe_kernel (one workgroup per
// stream, one wavefront per layer), with the 128-VGPR cap (more resident workgroups) or without (no spills, for
// fewer streams), and fast_kernel with the deep router descent (one stream per workgroup; routed models whose LDS
// tables and second-round rows fit in a workgroup's 160 KiB). Models with group scales have builds of their own for n
// of 64, 128 and 256.
#include "ygg_kernel_fast.h"
#include "ygg_launch.h"

namespace ygg {

template <int N, int R, int R2> constexpr bool kHasCap = N * R2 < 256 * 64;
template <int N> constexpr bool kGroupOk = N != 96;          // group scales need whole 16-coordinate groups per lane

// LDS of the deep kernel: tables, group-scale tables, the second round's rows of every routed layer, the stream's
// buffers
template <int N, int R, int R2, int L, bool GROUP>
constexpr bool kDeepFits = kTablesBytes<Shape<N, R, R2>, L> + sizeof(GroupTablesOf<Shape<N, R, R2>, L, GROUP>) +
                               (L - 1) * kR2Slots<N> * N + L * N + 128 <=
                           160 * 1024;

template <int N, int R, int R2, int L, bool GROUP>
hipError_t launch_deep(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    // one stream per workgroup of 4 wavefronts (three stage the LDS tables, one runs the stream)
    const dim3 grid(B), block(64 * kFastWaves);
    switch (io_mode(io)) {
    case kModeGenerate:
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeGenerate, true, false, GROUP>), grid, block, 0, stream, m,
                           tokens, B, T, state, io);
        break;
    case kModeScore:
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeScore, true, false, GROUP>), grid, block, 0, stream, m,
                           tokens, B, T, state, io);
        break;
    default:
        hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeRun, true, false, GROUP>), grid, block, 0, stream, m, tokens,
                           B, T, state, io);
    }
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool CAP, bool GROUP>
hipError_t launch_pipe(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    if (io_mode(io) == kModeScore)
        hipLaunchKernelGGL((pipe_kernel<N, R, R2, L, kModeScore, CAP, GROUP>), dim3(B), dim3(64 * L), 0, stream, m,
                           tokens, B, T, state, io);
    else
        hipLaunchKernelGGL((pipe_kernel<N, R, R2, L, kModeRun, CAP, GROUP>), dim3(B), dim3(64 * L), 0, stream, m,
                           tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool CAP, bool GROUP> Kernel pipe_k() {
    if constexpr (GROUP && !kGroupOk<N>) {
        return Kernel();
    } else if constexpr (CAP && !kHasCap<N, R, R2>) {
        return pipe_k<N, R, R2, L, false, GROUP>();
    } else {
        return modal(make_kernel(launch_pipe<N, R, R2, L, CAP, GROUP>, "ygg::pipe_kernel<%d, %d, %d, %d, %%s, %s, %s>",
                                 N, R, R2, L, CAP ? "true" : "false", GROUP ? "true" : "false"));
    }
}

template <int N, int R, int R2, int L, bool CAP, bool GROUP> int pipe_blocks(int mode) {
    if constexpr (GROUP && !kGroupOk<N>) {
        return 0;
    } else if constexpr (CAP && !kHasCap<N, R, R2>) {
        return pipe_blocks<N, R, R2, L, false, GROUP>(mode);
    } else {
        int nb = 0;
        const void *f = mode == kModeScore
                            ? reinterpret_cast<const void *>(&pipe_kernel<N, R, R2, L, kModeScore, CAP, GROUP>)
                            : reinterpret_cast<const void *>(&pipe_kernel<N, R, R2, L, kModeRun, CAP, GROUP>);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, 64 * L, 0) != hipSuccess) return 0;
        return nb;
    }
}

template <int N, int R, int R2, int L, bool GROUP> Kernel deep_k() {
    if constexpr (L >= 2 && kDeepFits<N, R, R2, L, GROUP> && (!GROUP || kGroupOk<N>))
        return modal(make_kernel(launch_deep<N, R, R2, L, GROUP>,
                                 "ygg::fast_kernel<%d, %d, %d, %d, %%s, true, false, %s>", N, R, R2, L,
                                 GROUP ? "true" : "false"));
    else
        return Kernel();
}

// fast_kernel's one-token build (kModeOne: the deep descent with the second round from global memory or folded into
// the tail, one stream per workgroup; at the largest shape 324 VGPRs, one wavefront per SIMD as its run build)
template <int N, int R, int R2, int L, bool GROUP>
hipError_t launch_one(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                      hipStream_t stream) {
    if (io_mode(io) != kModeRun || T != 1) return hipErrorInvalidValue;     // (the dispatch gives it no other call)
    // one stream per workgroup of 4 wavefronts (three stage the LDS tables, one runs the stream)
    const dim3 grid(B), block(64 * kFastWaves);
    hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeOne, false, false, GROUP>), grid, block, 0, stream, m, tokens, B,
                       T, state, io);
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool GROUP> Kernel one_k() {
    if constexpr (L >= 2 && (!GROUP || kGroupOk<N>))
        return make_kernel(launch_one<N, R, R2, L, GROUP>, "ygg::fast_kernel<%d, %d, %d, %d, 3, false, false, %s>", N,
                           R, R2, L, GROUP ? "true" : "false");
    else
        return Kernel();
}

// generation with the one-token build's descent (kModeGenOne), for more streams than the deep build takes and for
// models with no deep build: the second round from global memory or folded into the tail instead of staged in LDS
template <int N, int R, int R2, int L, bool GROUP>
hipError_t launch_gen_one(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                          hipStream_t stream) {
    if (io_mode(io) != kModeGenerate) return hipErrorInvalidValue;     // (the dispatch gives it no other call)
    // one stream per workgroup of 4 wavefronts (three stage the LDS tables, one runs the stream)
    const dim3 grid(B), block(64 * kFastWaves);
    hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeGenOne, false, false, GROUP>), grid, block, 0, stream, m,
                       tokens, B, T, state, io);
    return hipGetLastError();
}

template <int N, int R, int R2, int L, bool GROUP> Kernel gen_one_k() {
    if constexpr (L >= 2 && (!GROUP || kGroupOk<N>))
        return make_kernel(launch_gen_one<N, R, R2, L, GROUP>, "ygg::fast_kernel<%d, %d, %d, %d, 4, false, false, %s>",
                           N, R, R2, L, GROUP ? "true" : "false");
    else
        return Kernel();
}

// generation of one stream with speculating helper workgroups (kModeGenSpec, ygg_kernel_spec.h): workgroup 0 runs the
// stream, workgroups 1 .. io.spec_helpers help (spec_k below)
template <int N, int R, int R2, int L, bool GROUP, bool DEEP>
hipError_t launch_spec(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                       hipStream_t stream) {
    if (io_mode(io) != kModeGenerate || B != 1 || !io.spec || io.spec_helpers < 0 ||
        io.spec_helpers > kSpecMaxHelpers)
        return hipErrorInvalidValue;   // (the dispatch's rule)
    const dim3 grid(1 + io.spec_helpers), block(64 * kFastWaves);
    hipLaunchKernelGGL((fast_kernel<N, R, R2, L, kModeGenSpec, DEEP, false, GROUP>), grid, block, 0, stream, m,
                       tokens, B, T, state, io);
    return hipGetLastError();
}

// the speculating build's LDS with the deep descent: the deep kernel's, with every wavefront's states and slot tail
template <int N, int R, int R2, int L, bool GROUP>
constexpr bool kSpecDeepFits = kTablesBytes<Shape<N, R, R2>, L> + sizeof(GroupTablesOf<Shape<N, R, R2>, L, GROUP>) +
                                   (L - 1) * kR2Slots<N> * N +
                                   kFastWaves * ((2 * kSpecDepth<L> > L ? 2 * kSpecDepth<L> : L) * N +
                                                 kSpecDepth<L> * R + 4 + 64) +
                                   256 <=
                               160 * 1024;

// (with the deep descent where its LDS fits, else with the one-token build's descent)
template <int N, int R, int R2, int L, bool GROUP> Kernel spec_k() {
    if constexpr (L >= 2 && (!GROUP || kGroupOk<N>)) {
        constexpr bool D = kSpecDeepFits<N, R, R2, L, GROUP>;
        return make_kernel(launch_spec<N, R, R2, L, GROUP, D>, "ygg::fast_kernel<%d, %d, %d, %d, 5, %s, false, %s>",
                           N, R, R2, L, D ? "true" : "false", GROUP ? "true" : "false");
    } else {
        return Kernel();
    }
}

template <int N, int R, int R2, bool GROUP> Kernel spec_for(int L) {
    if (L == 2) return spec_k<N, R, R2, 2, GROUP>();
    if (L == 3) return spec_k<N, R, R2, 3, GROUP>();
    if (L == 4) return spec_k<N, R, R2, 4, GROUP>();
    if (L == 5) return spec_k<N, R, R2, 5, GROUP>();
    return Kernel();
}

template <int N, int R, int R2, bool GROUP> Kernel gen_one_for(int L) {
    if (L == 2) return gen_one_k<N, R, R2, 2, GROUP>();
    if (L == 3) return gen_one_k<N, R, R2, 3, GROUP>();
    if (L == 4) return gen_one_k<N, R, R2, 4, GROUP>();
    if (L == 5) return gen_one_k<N, R, R2, 5, GROUP>();
    return Kernel();
}

// the one-token build's (BUILD = kModeOne) or the generation build's (kModeGenOne) resident workgroups (one stream
// each) per CU on the current device
template <int N, int R, int R2, int L, bool GROUP, int BUILD> int one_blocks() {
    if constexpr (L >= 2 && (!GROUP || kGroupOk<N>)) {
        int nb = 0;
        const void *f = reinterpret_cast<const void *>(&fast_kernel<N, R, R2, L, BUILD, false, false, GROUP>);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, 64 * kFastWaves, 0) != hipSuccess) return 0;
        return nb;
    } else {
        return 0;
    }
}

template <int N, int R, int R2, bool GROUP, int BUILD> int one_occ(int L) {
    if (L == 2) return one_blocks<N, R, R2, 2, GROUP, BUILD>();
    if (L == 3) return one_blocks<N, R, R2, 3, GROUP, BUILD>();
    if (L == 4) return one_blocks<N, R, R2, 4, GROUP, BUILD>();
    if (L == 5) return one_blocks<N, R, R2, 5, GROUP, BUILD>();
    return 0;
}

template <int N, int R, int R2, bool GROUP> Kernel one_for(int L) {
    if (L == 2) return one_k<N, R, R2, 2, GROUP>();
    if (L == 3) return one_k<N, R, R2, 3, GROUP>();
    if (L == 4) return one_k<N, R, R2, 4, GROUP>();
    if (L == 5) return one_k<N, R, R2, 5, GROUP>();
    return Kernel();
}

template <int N, int R, int R2, bool CAP, bool GROUP> Kernel pipe_for(int L) {
    if (L == 1) {
        if constexpr (R == 8) return pipe_k<N, R, R2, 1, CAP, GROUP>();
        return Kernel();
    }
    if (L == 2) return pipe_k<N, R, R2, 2, CAP, GROUP>();
    if (L == 3) return pipe_k<N, R, R2, 3, CAP, GROUP>();
    if (L == 4) return pipe_k<N, R, R2, 4, CAP, GROUP>();
    if (L == 5) return pipe_k<N, R, R2, 5, CAP, GROUP>();
    return Kernel();
}

template <int N, int R, int R2, bool CAP, bool GROUP> int pipe_occ(int L, int mode) {
    if (L == 1) {
        if constexpr (R == 8) return pipe_blocks<N, R, R2, 1, CAP, GROUP>(mode);
        return 0;
    }
    if (L == 2) return pipe_blocks<N, R, R2, 2, CAP, GROUP>(mode);
    if (L == 3) return pipe_blocks<N, R, R2, 3, CAP, GROUP>(mode);
    if (L == 4) return pipe_blocks<N, R, R2, 4, CAP, GROUP>(mode);
    if (L == 5) return pipe_blocks<N, R, R2, 5, CAP, GROUP>(mode);
    return 0;
}

template <int N, int R, int R2, bool GROUP> Kernel deep_for(int L) {
    if (L == 2) return deep_k<N, R, R2, 2, GROUP>();
    if (L == 3) return deep_k<N, R, R2, 3, GROUP>();
    if (L == 4) return deep_k<N, R, R2, 4, GROUP>();
    if (L == 5) return deep_k<N, R, R2, 5, GROUP>();
    return Kernel();
}

// the layer-pipelined kernel for few streams
Kernel find_pipe_launcher(int n, int R, int R2, int L, bool cap, bool group) {
#define YGG_P(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) { \
        if (group) return cap ? pipe_for<N_, R_, R2_, true, true>(L) : pipe_for<N_, R_, R2_, false, true>(L); \
        return cap ? pipe_for<N_, R_, R2_, true, false>(L) : pipe_for<N_, R_, R2_, false, false>(L); \
    }
    YGG_SHAPES(YGG_P)
#undef YGG_P
    return Kernel();
}

// workgroups of that kernel (one stream each) resident per CU on the current device
int pipe_blocks_per_cu(int n, int R, int R2, int L, bool cap, bool group, int mode) {
#define YGG_P(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) { \
        if (group) return cap ? pipe_occ<N_, R_, R2_, true, true>(L, mode) : pipe_occ<N_, R_, R2_, false, true>(L, mode); \
        return cap ? pipe_occ<N_, R_, R2_, true, false>(L, mode) : pipe_occ<N_, R_, R2_, false, false>(L, mode); \
    }
    YGG_SHAPES(YGG_P)
#undef YGG_P
    return 0;
}

// fast_kernel's one-token build (2 <= L <= 5)
Kernel find_one_launcher(int n, int R, int R2, int L, bool group) {
#define YGG_D(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) return group ? one_for<N_, R_, R2_, true>(L) : one_for<N_, R_, R2_, false>(L);
    YGG_SHAPES(YGG_D)
#undef YGG_D
    return Kernel();
}

int one_blocks_per_cu(int n, int R, int R2, int L, bool group, bool gen) {
#define YGG_D(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) { \
        if (gen) return group ? one_occ<N_, R_, R2_, true, kModeGenOne>(L) : one_occ<N_, R_, R2_, false, kModeGenOne>(L); \
        return group ? one_occ<N_, R_, R2_, true, kModeOne>(L) : one_occ<N_, R_, R2_, false, kModeOne>(L); \
    }
    YGG_SHAPES(YGG_D)
#undef YGG_D
    return 0;
}

// fast_kernel's generation build with the one-token build's descent (2 <= L <= 5)
Kernel find_gen_one_launcher(int n, int R, int R2, int L, bool group) {
#define YGG_D(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) \
        return group ? gen_one_for<N_, R_, R2_, true>(L) : gen_one_for<N_, R_, R2_, false>(L);
    YGG_SHAPES(YGG_D)
#undef YGG_D
    return Kernel();
}

// fast_kernel's generation build for one stream with speculating helpers (2 <= L <= 5, d_state <= 128)
Kernel find_spec_launcher(int n, int R, int R2, int L, bool group) {
#define YGG_D(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) return group ? spec_for<N_, R_, R2_, true>(L) : spec_for<N_, R_, R2_, false>(L);
    YGG_SHAPES(YGG_D)
#undef YGG_D
    return Kernel();
}

// fast_kernel with the deep descent (2 <= L <= 5, where its LDS fits)
Kernel find_deep_launcher(int n, int R, int R2, int L, bool group) {
#define YGG_D(N_, R_, R2_) \
    if (n == N_ && R == R_ && R2 == R2_) return group ? deep_for<N_, R_, R2_, true>(L) : deep_for<N_, R_, R2_, false>(L);
    YGG_SHAPES(YGG_D)
#undef YGG_D
    return Kernel();
}

}  // namespace ygg
