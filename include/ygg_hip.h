/*
 * ygg_hip: the int8 streaming step of Yggdrasil on AMD Instinct MI355X (gfx950), as a C-ABI shared library
 * (yggdrasil_amd/libygg_hip.so).
 *
 * The reference runs this step in cpu/ygg.cpp (one stream per process, one core, AVX-512 VNNI) and exposes it only as
 * a CLI with files in and out (cpu/ygg.cpp:25-29, 500-574). This library keeps the same model file (YGG1, written by
 * cpu/export.py:444-468) and the same arithmetic bit for bit, and runs B independent streams per launch on the GPU.
 *
 * Conventions:
 *   - Every pointer named d_* is device memory on the model's device. Every call is ordered on the caller's HIP
 *     stream (`stream`, a hipStream_t passed as void*; NULL is the default stream) and returns without waiting.
 *   - Errors are returned as YGG_* status codes; the message of the last error on the calling thread is
 *     ygg_last_error(). Nothing exits the process (the reference's die(), cpu/ygg.cpp:41-43, exits).
 *   - State is int8 (B, L, n) row-major: the L layer states of one stream are contiguous, as State.q in
 *     cpu/ygg.cpp:439, 474-481. A zero state is the reference's reset() (cpu/ygg.cpp:481).
 *   - Tokens must lie in [0, vocab). The kernels never read out of bounds for a bad token: the stream stops at that
 *     token (its state keeps the value before it, its later outputs are left unwritten) and the model's error word
 *     records it; ygg_take_errors() reports it (the reference checks the whole token file first, cpu/ygg.cpp:493-495).
 */
#ifndef YGG_HIP_H
#define YGG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    YGG_OK = 0,
    YGG_ERR_IO = 1,        /* file cannot be opened or read */
    YGG_ERR_FORMAT = 2,    /* not a YGG1 file, short file, missing array (cpu/ygg.cpp:139-140, 153, 163, 176) */
    YGG_ERR_LIMITS = 3,    /* outside the supported LIMITS (cpu/ygg.cpp:141-146, 183-184) */
    YGG_ERR_NOMEM = 4,     /* host or device allocation failed (cpu/ygg.cpp:120, 476-477) */
    YGG_ERR_ARG = 5,       /* bad argument (null pointer, negative size) */
    YGG_ERR_TOKEN = 6,     /* a token outside [0, vocab) reached a kernel (cpu/ygg.cpp:493-495) */
    YGG_ERR_DEVICE = 7     /* a HIP runtime call failed */
};

typedef struct ygg_model ygg_model;

typedef struct {
    int32_t n_layers, d_state, block_size, vocab, vocab_pad, router_depth, n_experts;
    int32_t readout_rank, layer_input_rank, input_rank, shift;
    int32_t factored;          /* routed layers use factored input storage */
    int32_t group;             /* group scales present */
    int32_t device;            /* HIP device holding the weights */
    int32_t kernel;            /* step kernel in use: 0 general, 1 specialised (d_state, readout rank, layer-input
                                  rank one of (64, 8, 16), (96, 8, 16), (128, 8, 16), (128, 16, 32), (256, 32, 64),
                                  block 16, table storage, tensor scales or group scales (group: d_state 64, 128
                                  or 256), <= 5 layers, A16 entries <= 32639, each layer's tables and records under
                                  4 GiB); YGG_KERNEL=generic at load time forces 0 */
    int32_t pipe_max_streams;  /* ygg_run/ygg_score calls with B at most this and T > 1 use the layer-pipelined kernel
                                  (one wavefront per layer, for latency): its resident workgroups (one per stream)
                                  per CU times the CUs; 0: never. YGG_KERNEL=fast or =deep at load time disables
                                  it, =pipe uses it for every call */
    int32_t deep;              /* 1: the model's router plan allows the deep descent (2 to 4 rounds, the first of at
                                  least 2 levels, the third and fourth at most 6 levels together) and it is on
                                  (YGG_DEEP=0 at load time turns it off) */
    int32_t deep_max_streams;  /* ygg_generate calls of at least 8 tokens with B at most this (the CUs) use the
                                  one-stream-per-workgroup kernel with the deep descent; 0: never. YGG_KERNEL=deep
                                  uses it for every call */
    int32_t flow_max_streams;  /* ygg_run calls of at least 32 tokens with B at most this use the tick-pipelined
                                  kernel (one workgroup per stream, router rounds and updates of consecutive tokens
                                  overlapped): 8 streams per CU, or for the largest shape twice its resident
                                  workgroups, or its resident workgroups if more (score calls: the same rule for
                                  the score build); 0: never (plans other than 3 or 4 rounds, YGG_FLOW=0 or another
                                  YGG_KERNEL at load time). YGG_KERNEL=flow uses it for every call but
                                  ygg_generate */
    int32_t router_rounds;     /* rounds of the router plan (levels read per dependent step of the descent) */
    int32_t spec_max_streams;  /* 1: ygg_generate calls of one stream (B = 1) and at least 8 tokens run with helper
                                  workgroups that compute the next token's first layers for every candidate token
                                  (2 to 5 layers, a router plan the deep descent takes; YGG_SPEC=0 at load time:
                                  off); 0: never */
    int32_t grouped;           /* 1: ygg_run_grouped takes the model (d_state 128, readout rank 8, layer-input rank 16,
                                  block 16, table storage, tensor scales, router depth <= 14); 0: it reports
                                  YGG_ERR_LIMITS */
    int64_t file_array_bytes;  /* bytes of the file's arrays (the reference's Model::bytes, cpu/ygg.cpp:158, 167) */
    int64_t device_bytes;      /* device memory held by the model */
    int64_t gather_bytes[8];   /* per layer: bytes of one expert's transition, layer-input and readout weights */
} ygg_info;

/* Load a YGG1 model file onto `device`, relaying the weights out for the kernels.
   Replaces load() and read_header() of cpu/ygg.cpp:137-220. d_state may be 64, 96, 128 or 256. */
int ygg_load(const char *path, int device, ygg_model **out);

/* The same from a model file already in host memory (`bytes` bytes at `data`). */
int ygg_load_blob(const void *data, size_t bytes, int device, ygg_model **out);

/* Shape of a loaded model (the Model fields of cpu/ygg.cpp:112-116). */
int ygg_model_info(const ygg_model *m, ygg_info *info);

/* Release a model's device and host memory. Safe on NULL. */
void ygg_free(ygg_model *m);

/* One token for each of B streams: step<>() of cpu/ygg.cpp:441-459 applied to B independent streams.
   d_tokens (B) int32; d_state_in, d_state_out (B, L, n) int8, which may be the same buffer; d_logits (B, vocab) f32;
   d_leaves (B, L) int32 or NULL: the expert of every layer (layer 0: the token), as the Triton step's expert_out
   (yggdrasil/inference_triton.py:45, 86). */
int ygg_step(const ygg_model *m, const int32_t *d_tokens, const int8_t *d_state_in, int8_t *d_state_out,
             float *d_logits, int32_t *d_leaves, int B, void *stream);

/* T tokens for each of B streams in one launch, the state carried from token to token and left in d_state: the hot
   loop of cmd_logits_score (cpu/ygg.cpp:507-517) for B streams at once.
   d_tokens (B, T) int32; d_state (B, L, n) int8 in and out; optional outputs (NULL: not written):
   d_logits (B, T, vocab) f32, d_leaves (B, T, L) int32, d_states (B, T, L, n) int8 (the state after every token),
   d_digest (B) uint64 in and out: d = d * 0x100000001B3 + (leaf * 0xD6E8FEB86659FD93
   + sum_i (u8(q_i) + 1) * ((2 i + 1) * 0x9E3779B97F4A7C15) + l) for every token and layer in order (mod 2^64). */
int ygg_run(const ygg_model *m, const int32_t *d_tokens, int B, int T, int8_t *d_state, float *d_logits,
            int32_t *d_leaves, int8_t *d_states, uint64_t *d_digest, void *stream);

/* ygg_run computed leaf-grouped (the north_star's grouped path; no counterpart in the reference, whose step is one
   stream at a time): every (token, layer) of the call is a phase of three launches on the stream, which groups the
   streams that take the same expert at that phase, reads the expert's record once per group and contracts groups of
   at least YGG_GROUP_MFMA_MIN streams (default 8, read at load) on int8 MFMA. Same arguments, results and error
   behaviour as ygg_run (digest included). Models of d_state 128, readout rank 8, layer-input rank 16, block 16, table
   storage, tensor scales and router depth at most 14 only (else YGG_ERR_LIMITS). The first call, and any call with more streams than an earlier
   one, allocates its workspace with hipMalloc (and waits for the stream): under graph capture, make a call of at
   least that many streams first. Calls on one model must not overlap (they share the workspace). */
int ygg_run_grouped(ygg_model *m, const int32_t *d_tokens, int B, int T, int8_t *d_state, float *d_logits,
                    int32_t *d_leaves, int8_t *d_states, uint64_t *d_digest, void *stream);

/* ygg_run_grouped without any allocation, for callers that cannot allocate device memory (code under HIP graph
   capture, tight serving loops, harnesses that forbid hipMalloc); no counterpart in the reference. Same arguments,
   results and errors as ygg_run_grouped; its workspace is a static device array of YGG_SCRATCH_BYTES on each GPU
   (held until the process ends), so B is limited to what fits: the workspace takes 16 + 32 + 16 + 8 L bytes per
   stream plus 16 (each of its 8 pieces rounded up to 256 bytes): up to 10 912 streams of a 4-layer model, 10 071 of
   a 5-layer one; more give YGG_ERR_LIMITS. Every call on one GPU shares that array: calls that overlap on one GPU (other streams, other
   threads, other models) race and must not be made. Nothing in the array needs clearing between calls. */
#define YGG_SCRATCH_BYTES (1 << 20)
int ygg_run_grouped_noalloc(const ygg_model *m, const int32_t *d_tokens, int B, int T, int8_t *d_state,
                            float *d_logits, int32_t *d_leaves, int8_t *d_states, uint64_t *d_digest, void *stream);

/* The f32 softmax of the reference's time mode, softmax() at cpu/ygg.cpp:59-72 (which `ygg time` applies to every
   token's logits, cpu/ygg.cpp:545-553): for each of `rows` rows of V (1..256) logits at d_logits, the probabilities
   into d_probs (bit-identical to the reference's; may be d_logits itself) and, unless d_lse is NULL, the row's
   log-sum-exp (the value softmax() returns; the device's logf) into d_lse. On the caller's current device and stream. */
int ygg_softmax(const float *d_logits, int64_t rows, int V, float *d_probs, float *d_lse, void *stream);

/* Score T tokens of each of B streams without writing logits: the reference's `ygg score` (cpu/ygg.cpp:500-519) for
   B streams at once. Per token, in double: mx = max_c lg[c], se = sum_c exp(lg[c] - mx), and
   d_nll[b] += log(se) + mx - lg[target] (cpu/ygg.cpp:514-516; se is summed as a tree over classes, not in class
   order). d_tokens, d_targets (B, T) int32; d_state (B, L, n) int8 in and out; d_nll (B) double in and out. A
   target outside [0, vocab) adds nothing and sets bit 1 of the error word. */
int ygg_score(const ygg_model *m, const int32_t *d_tokens, const int32_t *d_targets, int B, int T, int8_t *d_state,
              double *d_nll, void *stream);

/* Sample n tokens for each of B streams in one launch, every sampled token fed straight back as the next input: the
   generate loop of yggdrasil/inference.py:190-202 (and yggdrasil/inference_triton.py:229-248) after its prompt.
   Step t consumes x_t (x_0 = d_first[b], then x_t = d_out[b, t-1]) from d_state and samples d_out[b, t] from its
   logits: temperature 0 takes the first class of maximal logit (argmax); otherwise classes whose logit is below the
   top_k-th largest are dropped (top_k 0: none) and class c is drawn with probability proportional to
   exp((lg[c] - max) / temperature), by inverse CDF over classes in order with a 24-bit uniform that depends only on
   (seed, b, t). d_first (B) int32; d_state (B, L, n) int8 in and out (left after consuming x_0 .. x_{n-1});
   d_out (B, n) int32; d_logits (B, n, vocab) f32 or NULL. A first token outside [0, vocab) sets bit 0 of the error
   word and leaves that stream's d_out unwritten.
   One stream (B = 1) and n >= 8 on a model with info.spec_max_streams = 1: the launch also runs helper workgroups
   (up to one per CU but the stream's) that compute step t + 1's first layers for every candidate token while step t
   finishes, in the model's speculation area; results are the same bit for bit. Calls of this kind that overlap on one model (other
   streams, other threads) share that area: each one's results stay correct, but they take each other's slots and
   run slower. */
int ygg_generate(const ygg_model *m, const int32_t *d_first, int B, int n, int8_t *d_state, float temperature,
                 int top_k, uint64_t seed, int32_t *d_out, float *d_logits, void *stream);

/* Counters of the speculating generation since the last reset (no counterpart in the reference; for tests and
   benchmarks): out[0] steps whose first layers came from a helper, out[1] steps the stream computed itself (after
   the first of each call), out[2] helper wavefronts that served a step, out[3] helper wavefronts that started (one
   per candidate token they cover), out[4] helper wavefronts that stopped waiting (no step's states for 200 us).
   Synchronous: call after the generating stream has finished. reset != 0 sets them to zero. All zero for a model
   without the speculating build. */
int ygg_spec_stats(const ygg_model *m, uint64_t out[5], int reset);

/* Wait for `stream`, then return and clear the model's error word: bit 0 set when a kernel met a token outside
   [0, vocab), bit 1 when ygg_score met a target outside it, bit 2 when a one-token launch's wait for its LDS tables
   passed 1 ms (a safety bound that a working device never reaches; that launch's results are then undefined), since
   the last call. */
int ygg_take_errors(const ygg_model *m, void *stream, uint32_t *errors);

/* ---- The float step (yggdrasil/inference.py:42-74): the inference model of a float checkpoint (.npz), in f32 (the
   serving precision of the Triton backend, yggdrasil/inference_triton.py) or f64 (the precision cpu/export.py
   calibrates in). The host (Python) reads the checkpoint and precomputes T_r[x] and A_r as yggdrasil/inference.py:
   145-155 does; every array below is row-major float64 on the host. */
typedef struct ygg_fmodel ygg_fmodel;

typedef struct {
    const double *table;            /* token layer [V][n], row x = T_x[x]; routed [E][V][n] */
    const double *transition;       /* [E][n/b][b][b] A_r, or NULL (experts without transitions) */
    const double *readout;          /* [E][R][n] P_r */
    const double *unembed;          /* [classes][R] Q */
    const double *router_embed;     /* routed: [V][F] */
    const double *router_weight;    /* routed: [2^D - 1][F + n] (router_state) or [2^D - 1][F] */
    const double *router_bias;      /* routed: [2^D - 1] */
    const double *layer_input_down; /* routed, R2 > 0: [R2][n] V' */
    const double *layer_input_proj; /* routed, R2 > 0: [E][n][R2] U'_r */
} ygg_float_layer;

typedef struct {
    int32_t n_layers, d_state, block_size, vocab, classes, router_depth, readout_rank, layer_input_rank;
    int32_t router_token_dim;       /* F */
    int32_t router_state;           /* 1: the router also reads rms(h_below) */
    const double *output_bias;      /* [classes] */
    ygg_float_layer layers[8];
} ygg_float_desc;

/* Copy a float model to `device` in `precision` 32 (f32) or 64 (f64). Limits: n <= 256 and a multiple of 16,
   classes <= 256, R and R2 <= 64, F <= 256, D <= 20, <= 8 layers. */
int ygg_float_load(const ygg_float_desc *desc, int precision, int device, ygg_fmodel **out);

/* T tokens for each of B streams: d_state (B, L, n) in and out and d_logits (B, T, classes) in the model's precision
   (float or double); d_leaves (B, T, L) int32 or NULL; d_stats (L x (3 + n/16 + R)) double or NULL, zero-filled by
   the caller: per layer the running maxima of |h|, |V' rms(h_below)|, |P_r h|, |h| per 16 coordinates and |P_r h|
   per row, the calibration statistics of cpu/export.py:117-153. A token outside [0, vocab) stops its stream and sets
   bit 0 of the model's error word. */
int ygg_float_run(const ygg_fmodel *m, const int32_t *d_tokens, int B, int T, void *d_state, void *d_logits,
                  int32_t *d_leaves, double *d_stats, void *stream);

/* Wait for `stream`, then return and clear the float model's error word (bit 0: a token outside [0, vocab)). */
int ygg_float_take_errors(const ygg_fmodel *m, void *stream, uint32_t *errors);

void ygg_float_free(ygg_fmodel *m);

/* Message of the last failed call on this thread ("" if none). */
const char *ygg_last_error(void);

/* The kernel a call would launch, by the name profilers show for it (e.g.
   "ygg::fast_kernel<128, 8, 16, 4, 0, false, true, false>"): mode = 0 for ygg_run without a digest and ygg_step
   (T = 1), 1 for ygg_generate (T = its n), 2 for ygg_score and ygg_run with a digest (the specialised per-stream
   kernel has a build per mode); written NUL-terminated into name (len bytes). No counterpart in the reference (its one
   kernel is the CPU step); for profiles and tests. */
int ygg_kernel_name(const ygg_model *m, int B, int T, int mode, char *name, size_t len);

/* Library ABI version (bumped when a signature above changes). */
int ygg_version(void);

#ifdef __cplusplus
}
#endif
#endif /* YGG_HIP_H */
