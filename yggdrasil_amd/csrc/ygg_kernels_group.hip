// The leaf-grouped step's launches (ygg_kernel_group.h): per (token, layer) of a call, grp_route, grp_plan and
// grp_update on the caller's stream, after one grp_init. For the benchmark shape only (n 128, readout rank 8,
// layer-input rank 16, block 16, table storage, tensor scales).
#include "ygg_kernel_group.h"
#include "ygg_launch.h"

namespace ygg {

hipError_t launch_grouped(const YggDevModel &m, const int32_t *tokens, int B, int T, int8_t *state, const YggIO &io,
                          void *ws_mem, int mfma_min, hipStream_t stream) {
    if (B <= 0 || T <= 0) return hipSuccess;
    if (m.V > kGrpMaxExperts || (m.L > 1 && m.E > kGrpMaxExperts)) return hipErrorInvalidValue;
    // (the MFMA tile stages a whole record in LDS)
    for (int l = 0; l < m.L; l++)
        if (m.layers[l].gath_bytes > kGrpRec) return hipErrorInvalidValue;
    const GroupWS ws = group_ws_carve(ws_mem, B, m.L);
    hipLaunchKernelGGL(grp_init, dim3((B + 255) / 256), dim3(256), 0, stream, B, T, ws);
    // update workgroups: about one wavefront per tile of the worst case (every stream alone at its expert)
    const int emax = m.L > 1 && m.E > m.V ? m.E : m.V;
    const int tiles_max = B / kGrpTile + (B < emax ? B : emax) + 1;
    int gu = (tiles_max + 3) / 4;
    if (gu > 4096) gu = 4096;
    for (int t = 0; t < T; t++)
        for (int l = 0; l < m.L; l++) {
            hipLaunchKernelGGL((grp_route<128, 8, 16>), dim3((B + 3) / 4), dim3(256), 0, stream, m, tokens, B, T, t, l,
                               state, io.leaves, ws);
            hipLaunchKernelGGL(grp_plan, dim3(1), dim3(1024), 0, stream, B, l == 0 ? m.V : m.E, ws);
            hipLaunchKernelGGL((grp_update<128, 8, 16>), dim3(gu), dim3(256), 0, stream, m, tokens, B, T, t, l, state,
                               io.states, io.logits, io.digest, ws, mfma_min);
        }
    return hipGetLastError();
}

size_t grouped_ws_bytes(int B, int L) { return group_ws_bytes(B, L); }

}  // namespace ygg
