// The kernels the C-ABI launches: one launcher per instantiation (or per set of mode builds), found by shape, with
// the name a profiler shows for it. A "%s" in the name stands for the call's mode: the GEN argument of run_kernel
// ("true" in ygg_generate, else "false") or, for a modal kernel, the MODE argument (kModeRun, kModeGenerate,
// kModeScore).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "ygg_layout.h"

namespace ygg {

typedef hipError_t (*Launcher)(const YggDevModel &, const int32_t *, int, int, int8_t *, const YggIO &, hipStream_t);

struct Kernel {
    Launcher fn = nullptr;
    char name[96] = {0};
    bool modal = false;     // the launcher picks a build by io_mode(io), the name's "%s" is that mode
    explicit operator bool() const { return fn != nullptr; }
    // the name of the build a call of this mode runs
    void name_for(int mode, char *out, size_t len) const {
        static const char *const modes[3] = {"0", "1", "2"};
        snprintf(out, len, name, modal ? modes[mode] : (mode == kModeGenerate ? "true" : "false"));
    }
};

inline Kernel make_kernel(Launcher fn, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
inline Kernel make_kernel(Launcher fn, const char *fmt, ...) {
    Kernel k;
    k.fn = fn;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(k.name, sizeof k.name, fmt, ap);
    va_end(ap);
    return k;
}

// k, whose launcher picks a build per mode
inline Kernel modal(Kernel k) {
    k.modal = true;
    return k;
}

// The shapes of the specialised kernels (block 16, table storage, tensor or group scales): state width, readout rank,
// layer-input rank, and the most layers. The first three are the benchmark configurations' (and the reference's
// small models), the last two its medium and large models (configs/{enwik8,hg38}/{medium,large}.yaml).
#define YGG_SHAPES(X) X(64, 8, 16) X(96, 8, 16) X(128, 8, 16) X(128, 16, 32) X(256, 32, 64)
constexpr int kMaxFastLayers = 5;
// The fast-only shapes (state width, readout rank, layer-input rank, block): the reference's kernel-test shapes
// (cpu/tests/test_kernel.py:22-33) outside YGG_SHAPES or at block 8, with table storage; routed models only. Only
// the per-stream kernel has builds for them (ygg_kernels_fast_x.hip).
#define YGG_FAST_EXTRA(X) X(128, 16, 32, 8) X(64, 8, 0, 8) X(256, 16, 48, 8) X(128, 16, 4, 16) X(256, 8, 20, 16) \
    X(64, 8, 0, 16) X(64, 32, 20, 16)
// the same for factored routed inputs (fact_kernel, fact8_kernel)
#define YGG_FACT_EXTRA(X) X(128, 16, 16, 16) X(64, 8, 0, 8)

Kernel find_launcher(int n, int blk, int R);                            // run_kernel (ygg_kernels.hip)
// group: the model has group scales (builds for n of 64, 128 and 256 only)
// fast_kernel, 4 streams per workgroup, 128-VGPR cap or none (ygg_kernels_fast.hip); its resident workgroups per CU
Kernel find_fast_launcher(int n, int R, int R2, int L, bool cap, bool group);
int fast_blocks_per_cu(int n, int R, int R2, int L, bool cap, bool group, int mode);
// the fast-only shapes' per-stream kernel (uncapped; fast8_kernel at block 8; fact_kernel / fact8_kernel for factored
// inputs) and its resident workgroups per CU
Kernel find_fast_extra_launcher(int n, int R, int R2, int blk, int L, bool group, bool factored);
int fast_extra_blocks_per_cu(int n, int R, int R2, int blk, int L, bool group, bool factored, int mode);
// fact_kernel: fast_kernel for factored routed inputs (ygg_kernels_fact.hip), 2 to 5 layers
Kernel find_fact_launcher(int n, int R, int R2, int L, bool cap, bool group);
int fact_blocks_per_cu(int n, int R, int R2, int L, bool cap, bool group, int mode);
// fast_kernel with the deep descent, one stream per workgroup; pipe_kernel, 128-VGPR cap or none
// (ygg_kernels_deep.hip)
Kernel find_deep_launcher(int n, int R, int R2, int L, bool group);
Kernel find_one_launcher(int n, int R, int R2, int L, bool group);
// resident workgroups per CU of the one-token build, or (gen) of the generation build with its descent
int one_blocks_per_cu(int n, int R, int R2, int L, bool group, bool gen);
Kernel find_gen_one_launcher(int n, int R, int R2, int L, bool group);
// generation of one stream with speculating helper workgroups (2 <= L <= 5, d_state <= 128): io.spec, io.spec_epoch
Kernel find_spec_launcher(int n, int R, int R2, int L, bool group);
Kernel find_pipe_launcher(int n, int R, int R2, int L, bool cap, bool group);
int pipe_blocks_per_cu(int n, int R, int R2, int L, bool cap, bool group, int mode);
// flow_kernel, one workgroup per stream, for scoring with the tokens known, router plans of P = 3 or 4 rounds
// (ygg_kernels_flow.hip); the resident workgroups per CU of its build for a mode (kModeRun or kModeScore)
Kernel find_flow_launcher(int n, int R, int R2, int L, int P, bool group);
int flow_blocks_per_cu(int n, int R, int R2, int L, int P, bool group, int mode);
bool flow_split_build(int n, int R, int R2, int L, int mode);
// the leaf-grouped step (ygg_kernels_group.hip; n 128, readout rank 8, layer-input rank 16, table storage, tensor
// scales, at most 16384 experts a layer): every (token, layer) of the call as route, plan and update launches on
// the stream, in a workspace of grouped_ws_bytes(B, L) bytes at ws
hipError_t launch_grouped(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                          void *ws, int mfma_min, hipStream_t stream);
size_t grouped_ws_bytes(int B, int L);
// the f32 softmax of the reference's time mode over rows of V <= 256 logits (ygg_softmax.hip)
hipError_t launch_softmax(const float *logits, int64_t rows, int V, float *probs, float *lse, hipStream_t stream);

}  // namespace ygg
