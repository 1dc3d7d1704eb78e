// Device layout of a loaded model: what the host relayout writes and the kernels read.
//
// The file layout (YGG1) is the interface; the device layout is this library's own. At load every expert's weights
// that one stream reads at one step (transition A16, layer-input projection U', readout P, factored input U) are
// rewritten into one contiguous "gather record", with every part signed (the file's u8 = w + 128 storage is undone,
// so no 128 * sum corrections remain in the kernels) and interleaved by lane, so that each load instruction of a
// wavefront reads one contiguous span. Shared arrays (router rows, layer-input down-projection, unembedding) become
// plain signed row-major arrays.
//
// Lane mapping (one 64-lane wavefront per stream):
//   state rows      lane l < NL owns the C consecutive coordinates [C l, C l + C), C = 1 (n <= 64), 2 (n <= 128),
//                   4 (n <= 256), NL = n / C (n = 96: 48 lanes)
//   router / V'     quad j = l / 4 takes one row (a tree node, a V' row), quad lane k = l % 4 the n/4 coordinates
//                   [k n/4, (k + 1) n/4)
//   readout P       RL = 64 / R lanes per readout row: row j = l / RL, coordinates [(l % RL) SP, (l % RL + 1) SP),
//                   SP = n / RL bytes
//   unembedding     lane l owns classes [4 l, 4 l + 4) of the padded class count VP
//
// Gather record of one expert (gath_bytes, a multiple of 128):
//   A   at 0:      16-byte chunks, chunk c of lane l at (c NL + l) 16. A lane's bytes are its C rows in order, each
//                  row the b int16 of that row inside its diagonal block (columns in block order). Models run by
//                  the specialised kernels (ygg_kernel_fast.h) store each row instead as b signed bytes hi followed
//                  by b signed bytes lo with A16 = 256 hi + lo, so the transition is two v_dot4 on the int8 state.
//   P   at off_P:  granules of GP bytes (16, 8 or 4: the largest dividing SP), granule g of lane l at
//                  off_P + (g 64 + l) GP. A lane's bytes are P[j][i] (s8) for its row j and coordinates i in order.
//   U'  at off_U:  for k4 < R2/4: lane l's C dwords at off_U + ((k4 NL + l) C + c) 4; dword c holds
//                  U'[C l + c][4 k4 .. 4 k4 + 3] (s8).
//   U   at off_F:  the same for the factored input projection with input_rank in place of R2.
//   Cb  at off_FB: int16[n] factored bias.  S at off_FS: f32 factored input scale.
//
// Router descent plan: the D levels are taken in rounds of h_k levels (round_h), the first of min(4, D) levels, the
// rest split as evenly as possible into ceil((D - h_0) / 4) rounds, larger first (D = 14: 4, 4, 3, 3). A round of h
// levels evaluates the 2^h - 1 nodes of one subtree in parallel.
//
// Router rows and thresholds (file: w[node][n], thr[x][node], heap order) are regrouped by round. Round k covers
// depths [d0, d0 + h); each subtree root ix at depth d0 owns one block of 2^h slots holding its 2^h - 1 nodes in
// breadth-first order (slot j: depth dj = floor(log2(j + 1)), heap index (ix << dj) + j + 1 - 2^dj), the last slot
// unused. Blocks of round k start at base_k = sum over earlier rounds of 2^(d0 + h); the block of root ix is at
// base_k + (ix - 2^d0) 2^h. w holds one n-byte row per slot, thr one float per slot and token; one round of one stream
// reads one contiguous block of rows and one block of thresholds (64 bytes for h = 4).
#pragma once
#include <stdint.h>

#define YGG_MAX_LAYERS 8
#define YGG_MAX_RANK 64
#define YGG_MAX_FACT_RANK 64      // factored input ranks the specialised kernels take

struct YggDevLayer {
    const uint8_t *gath;     // E gather records
    const int16_t *table;    // token layer [V][n] (expert x = its own row); routed table storage [E][V][n]
    const int8_t *w;         // routed: [thr_stride][n] router rows, blocked by round (see below)
    const float *thr;        // routed: [V][thr_stride] thresholds, blocked by router round (see below)
    const int8_t *vl;        // routed, R2 > 0: [16 RG][n] layer-input down-projection V' (rows >= R2 zero)
    const float *mv;         // routed, R2 > 0: [16 RG]
    const float *mulv;       // [n] per-coordinate layer-input scale, or null
    const float *r2b;        // [n/16] squared group scales of the layer below, or null
    const float *mz;         // [E][R] per expert and row readout scale, or null
    const float *sqv;        // [VP] per class unembedding scale, or null
    const int8_t *Q;         // [VP][R] unembedding, class-major
    const int8_t *vt;        // factored: [V][k] token codes, or null
    const float *mT;         // factored: [n] token scale
    int64_t gath_bytes;
    int64_t table_sr;        // table elements per expert (token layer: n; routed: V n)
    int32_t table_sx;        // table elements per token (token layer: 0; routed: n)
    int32_t off_P, off_U, off_F, off_FB, off_FS;  // byte offsets in the gather record, -1 absent
    int32_t thr_stride;      // slots per token: floats per token row of thr, rows of w
    float readout_scale, unembed_scale, rms_eps, layer_input_scale;
};

#define YGG_MAX_ROUNDS 16

struct YggDevModel {
    int32_t L, N, BLK, V, VP, D, E, R, R2, K, shift;
    int32_t n_rounds, round_h[YGG_MAX_ROUNDS];   // router descent plan
    uint64_t round_pack;        // round_h[r] in bits 4 r .. 4 r + 3 (rounds 0 .. 15)
    const float *output_bias;   // [VP]
    uint32_t *err;              // error word (bit 0: token out of range)
    YggDevLayer layers[YGG_MAX_LAYERS];
};

// Optional inputs and outputs of one launch of a step kernel (null: not read or written).
struct YggIO {
    float *logits;                  // (B, T, V) f32
    int32_t *leaves;                // (B, T, L)
    int8_t *states;                 // (B, T, L, n) after every token
    unsigned long long *digest;     // (B) in and out
    const int32_t *targets;         // score: (B, T) targets
    double *nll;                    // score: (B) in and out
    int32_t *gen;                   // generate: (B, T) the token sampled after every step, which is the next input;
                                    // the launch's tokens are then one first token per stream
    float temperature;              // generate: 0 = greedy (first maximal class)
    int32_t top_k;                  // generate: keep classes at least the k-th largest logit (0: all)
    unsigned long long seed;        // generate
    uint64_t *spec;                 // generate, kModeGenSpec: the model's speculation area (tagged 8-byte units)
    uint32_t spec_epoch;            // generate, kModeGenSpec: the call's first epoch; token t's tag is spec_epoch + t
    int32_t spec_helpers;           // generate, kModeGenSpec: helper workgroups (workgroups 8 .. 8 spec_helpers)
};

// What a launch computes, from its outputs: the specialised per-stream kernel has a build per mode (the digest and
// NLL terms cost registers that plain runs keep for streams). Also the mode argument of ygg_kernel_name.
constexpr int kModeRun = 0;         // logits, leaves, states after every token
constexpr int kModeGenerate = 1;    // io.gen: each token sampled from the step before
constexpr int kModeScore = 2;       // io.digest or io.nll
// a build of the per-stream kernel, not a mode argument: kModeRun for calls of one token with the deep descent, its
// second round's rows read from global memory instead of staged in LDS
constexpr int kModeOne = 3;
// a build of the per-stream kernel, not a mode argument: kModeGenerate with the same descent as kModeOne, one stream
// per workgroup, for more streams than the deep build takes, or for models with no deep build (their second-round rows
// do not fit LDS beside the tables)
constexpr int kModeGenOne = 4;
// a build of the per-stream kernel, not a mode argument: kModeGenerate for one stream, with helper workgroups on the
// stream's XCD that compute the next token's first layers for every candidate token while the stream finishes the
// current one (ygg_kernel_spec.h)
constexpr int kModeGenSpec = 5;

// The speculation area of a model (kModeGenSpec), in 8-byte units (a 32-bit tag in the low half, a 32-bit word in the
// high half): counters at kSpecStats, the token units at kSpecTok (kSpecCopies copies kSpecCopyUnits apart: their
// readers spread over as many memory channels), then one slot of kSpecSlotUnits units per candidate token: copy 0 of
// its states and the rest of its words at its start, copies 1 .. kSpecCopies - 1 of its states kSpecCopyUnits apart.
constexpr int kSpecStats = 8;           // 5 counters (uint64): hits, misses, helper waves served, started, timed out
constexpr int kSpecNStats = 5;
constexpr int kSpecTok = 64;
constexpr int kSpecCopyUnits = 256, kSpecCopies = 8;
constexpr int kSpecSlots = kSpecTok + kSpecCopyUnits * kSpecCopies;
constexpr int kSpecSlotUnits = kSpecCopyUnits * kSpecCopies;
// helper workgroups (workgroups 1 .. h of the launch, one CU each): at most kSpecMaxHelpers of them
constexpr int kSpecMaxHelpers = 255;
inline size_t spec_area_units(int V) { return (size_t)kSpecSlots + (size_t)V * kSpecSlotUnits; }
inline int io_mode(const YggIO &io) {
    return io.gen ? kModeGenerate : ((io.digest || io.nll) ? kModeScore : kModeRun);
}

// Compile-time lane constants of a d_state N, readout rank R.
template <int N> struct Lanes {
    static constexpr int C = N <= 64 ? 1 : (N <= 128 ? 2 : 4);
    static constexpr int NL = N / C;
};
template <int N, int R> struct ReadoutLanes {
    static constexpr int RL = 64 / R;
    static constexpr int SP = N / RL;
    static constexpr int GP = SP % 16 == 0 ? 16 : (SP % 8 == 0 ? 8 : 4);
};

// Runtime versions for the host relayout.
static inline int lanes_c(int n) { return n <= 64 ? 1 : (n <= 128 ? 2 : 4); }
static inline int readout_gp(int sp) { return sp % 16 == 0 ? 16 : (sp % 8 == 0 ? 8 : 4); }
