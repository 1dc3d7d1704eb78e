// The kernels the C-ABI launches: one launcher per instantiation, found by shape, with the name a profiler shows for
// it (a "%s" in the name stands for the GEN argument, "true" in ygg_generate, else "false").
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "ygg_layout.h"

namespace ygg {

typedef hipError_t (*Launcher)(const YggDevModel &, const int32_t *, int, int, int8_t *, const YggIO &, hipStream_t);

struct Kernel {
    Launcher fn = nullptr;
    char name[80] = {0};
    explicit operator bool() const { return fn != nullptr; }
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

// The shapes of the specialised kernels (block 16, table storage, tensor scales): state width, readout rank,
// layer-input rank, and the most layers. The first three are the benchmark configurations' (and the reference's
// small models), the last two its medium and large models (configs/{enwik8,hg38}/{medium,large}.yaml).
#define YGG_SHAPES(X) X(64, 8, 16) X(96, 8, 16) X(128, 8, 16) X(128, 16, 32) X(256, 32, 64)
constexpr int kMaxFastLayers = 5;

Kernel find_launcher(int n, int blk, int R);                            // run_kernel (ygg_kernels.hip)
// fast_kernel, 4 streams per workgroup, 128-VGPR cap or none (ygg_kernels_fast.hip); its resident workgroups per CU
Kernel find_fast_launcher(int n, int R, int R2, int L, bool cap);
int fast_blocks_per_cu(int n, int R, int R2, int L, bool cap, bool gen);
// fast_kernel with the deep descent, one stream per workgroup; pipe_kernel, 128-VGPR cap or none
// (ygg_kernels_deep.hip)
Kernel find_deep_launcher(int n, int R, int R2, int L);
Kernel find_pipe_launcher(int n, int R, int R2, int L, bool cap);
int pipe_blocks_per_cu(int n, int R, int R2, int L, bool cap);

}  // namespace ygg
