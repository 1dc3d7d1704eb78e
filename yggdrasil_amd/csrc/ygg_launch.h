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
    char name[64] = {0};
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

Kernel find_launcher(int n, int blk, int R);                // run_kernel (ygg_kernels.hip)
Kernel find_fast_launcher(int n, int L, bool cap);          // fast_kernel, 128-VGPR cap or none (ygg_kernels_fast.hip)
int fast_blocks_per_cu(int n, int L, bool cap, bool gen);   // its resident workgroups (4 streams each) per CU
Kernel find_deep_launcher(int n, int L);                    // fast_kernel, deep descent (ygg_kernels_deep.hip)
Kernel find_pipe_launcher(int n, int L, bool cap);          // pipe_kernel, 128-VGPR cap or none (ygg_kernels_deep.hip)
int pipe_blocks_per_cu(int n, int L, bool cap);             // its resident workgroups per CU

}  // namespace ygg
