/*
 * TEST INFRASTRUCTURE ONLY. A plain-C, scalar restatement of the reference's int8 streaming step, used as the
 * checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg. The product path (yggdrasil_amd)
 * never links, loads or calls this file.
 *
 * It follows cpu/ygg.cpp:222-459 (the AVX-512 VNNI step) and its bit-exact NumPy twin cpu/export.py:268-316
 * (int_forward), reading the YGG1 file exactly as cpu/ygg.cpp:137-220 does. Every f32 operation is one IEEE
 * rounded operation in the reference's order (built with -ffp-contract=off, as cpu/Makefile:5). Unlike ygg.cpp it
 * takes any d_state that is a multiple of 16 (so d = 96 too), and it can emit the leaf of every layer, the int8
 * state after every token, and a per-stream digest of both.
 *
 * Pinning: the logits, leaves and states are compared against the reference kernel compiled from
 * /root/reference/cpu/ygg.cpp (oracle/Makefile, outputs in oracle/_ref/) on every kernel-test shape of
 * cpu/tests/test_kernel.py:22-33 and on the benchmark configurations with d in {64, 128, 256}, live where the
 * reference builds and through committed digests in tests/golden/ elsewhere. d = 96 is pinned by embedding checks
 * described in tests/test_oracle.py.
 */
#define _GNU_SOURCE 1
#include "ygg_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define MAX_LAYERS 8
#define MAX_RANK 64

typedef struct {
    const uint8_t *rec;               /* expert r at rec + r * record_bytes */
    int record_bytes, off_A, off_U2, off_P, off_T, off_F, off_C, off_S;
    int table_stride;                 /* bytes per token row of T_r; 0 for the token layer (cpu/ygg.cpp:188) */
    const uint8_t *Q;                 /* u8 [R/4][VP][4] */
    float readout_scale, unembed_scale, rms_eps, layer_input_scale;
    const uint8_t *w;                 /* u8 [E][n] */
    const float *thr;                 /* [V][E] */
    const uint8_t *vl;                /* u8 [RG][n/4][16][4] */
    const float *mv;                  /* [16 RG] */
    const float *mulv, *r2b, *mzl, *sqv;
    const int8_t *vt;                 /* [V][k] */
    const float *mT;                  /* [n] */
} yo_layer;

struct yo_model {
    int n_layers, n, block, vocab, depth, R, R2, input_rank, shift, E, VP;
    const float *output_bias;
    yo_layer layers[MAX_LAYERS];
    uint8_t *blob;
    size_t bytes;
};

static void set_err(char *err, int errlen, const char *fmt, ...) {
    if (!err || errlen <= 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, (size_t)errlen, fmt, ap);
    va_end(ap);
}

typedef struct { char name[32]; int64_t offset, bytes; } entry_t;

static const uint8_t *find(const entry_t *tab, int na, const uint8_t *base, const char *name, int64_t *nb) {
    for (int i = 0; i < na; i++)
        if (!strncmp(tab[i].name, name, 32)) { if (nb) *nb = tab[i].bytes; return base + tab[i].offset; }
    return NULL;
}

int yo_load(const char *path, yo_model **out, char *err, int errlen) {
    *out = NULL;
    FILE *f = fopen(path, "rb");
    if (!f) { set_err(err, errlen, "%s: cannot open", path); return YO_ERR_IO; }
    char magic[4];
    int32_t h[12];
    if (fread(magic, 1, 4, f) != 4 || memcmp(magic, "YGG1", 4) || fread(h, 4, 12, f) != 12) {
        fclose(f); set_err(err, errlen, "%s: not a model file", path); return YO_ERR_FORMAT;
    }
    const int nl = h[0], n = h[1], blk = h[2], V = h[3], D = h[4], R = h[5], R2 = h[6], reserved = h[7];
    const int kin = h[9], shift = h[10], na = h[11];
    const int ok = n >= 16 && n <= 256 && n % 16 == 0 && (blk == 8 || blk == 16) && (R == 8 || R == 16 || R == 32) &&
                   R2 >= 0 && R2 <= MAX_RANK && R2 % 4 == 0 && nl >= 1 && nl <= MAX_LAYERS && V >= 1 && V <= 256 &&
                   D >= 0 && D <= 16 && (nl == 1 || D >= 1) && reserved == 0 && shift >= 1 && shift <= 30 && na > 0;
    if (!ok) { fclose(f); set_err(err, errlen, "%s: unsupported model (LIMITS)", path); return YO_ERR_LIMITS; }
    entry_t *tab = (entry_t *)calloc((size_t)na, sizeof(entry_t));
    if (fread(tab, sizeof(entry_t), (size_t)na, f) != (size_t)na) {
        free(tab); fclose(f); set_err(err, errlen, "%s: short array table", path); return YO_ERR_FORMAT;
    }
    long pos = ftell(f);
    pos += (64 - pos % 64) % 64;
    fseek(f, 0, SEEK_END);
    const long end = ftell(f);
    fseek(f, pos, SEEK_SET);
    const size_t sz = end > pos ? (size_t)(end - pos) : 0;
    uint8_t *blob = (uint8_t *)malloc(sz + 128);
    if (!blob) { free(tab); fclose(f); set_err(err, errlen, "out of memory"); return YO_ERR_NOMEM; }
    memset(blob + sz, 0, 128);
    if (fread(blob, 1, sz, f) != sz) {
        free(blob); free(tab); fclose(f); set_err(err, errlen, "%s: short model file", path); return YO_ERR_FORMAT;
    }
    fclose(f);
    for (int i = 0; i < na; i++)
        if (tab[i].offset < 0 || tab[i].bytes < 0 || (size_t)(tab[i].offset + tab[i].bytes) > sz) {
            free(blob); free(tab); set_err(err, errlen, "%s: array %.32s out of the file", path, tab[i].name);
            return YO_ERR_FORMAT;
        }
    yo_model *m = (yo_model *)calloc(1, sizeof(yo_model));
    m->n_layers = nl; m->n = n; m->block = blk; m->vocab = V; m->depth = D; m->R = R; m->R2 = R2;
    m->input_rank = kin; m->shift = shift; m->E = 1 << D; m->VP = (V + 31) / 32 * 32;
    m->blob = blob; m->bytes = sz;
    int rc = YO_OK;
    m->output_bias = (const float *)find(tab, na, blob, "head_b", NULL);
    if (!m->output_bias) { set_err(err, errlen, "%s: missing head_b", path); rc = YO_ERR_FORMAT; }
    for (int l = 0; l < nl && rc == YO_OK; l++) {
        yo_layer *y = &m->layers[l];
        char nm[40];
#define GET(tag) (snprintf(nm, sizeof nm, "l%d_%s", l, tag), find(tab, na, blob, nm, NULL))
#define NEED(dst, type, tag)                                                                           \
    do {                                                                                               \
        dst = (type)GET(tag);                                                                          \
        if (!dst) { set_err(err, errlen, "model file: missing l%d_%s", l, tag); rc = YO_ERR_FORMAT; } \
    } while (0)
        const int32_t *meta;
        NEED(meta, const int32_t *, "meta");
        if (rc) break;
        y->record_bytes = meta[0]; y->off_A = meta[1]; y->off_U2 = meta[2]; y->off_P = meta[3]; y->off_T = meta[4];
        y->off_F = y->off_C = y->off_S = -1;
        y->vt = (const int8_t *)GET("vt");
        if (y->vt) {
            if (kin % 4 || kin > MAX_RANK || kin < 4) {
                set_err(err, errlen, "model file: factored input_rank %d", kin); rc = YO_ERR_LIMITS; break;
            }
            y->off_F = meta[5]; y->off_C = meta[6]; y->off_S = meta[7];
            NEED(y->mT, const float *, "mT");
        }
        y->table_stride = l == 0 ? 0 : 2 * n;
        NEED(y->rec, const uint8_t *, "rec");
        NEED(y->Q, const uint8_t *, "Q");
        y->mzl = (const float *)GET("mzl");
        y->sqv = (const float *)GET("sqv");
        const float *sc;
        NEED(sc, const float *, "scal");
        if (rc) break;
        y->readout_scale = sc[0]; y->unembed_scale = sc[1]; y->rms_eps = sc[2]; y->layer_input_scale = sc[3];
        if (l > 0) {
            NEED(y->w, const uint8_t *, "w");
            NEED(y->thr, const float *, "thr");
            if (R2) {
                NEED(y->vl, const uint8_t *, "vl");
                NEED(y->mv, const float *, "mv");
            }
            y->mulv = (const float *)GET("mulv");
            y->r2b = (const float *)GET("r2b");
        }
#undef GET
#undef NEED
    }
    free(tab);
    if (rc) { free(blob); free(m); return rc; }
    *out = m;
    return YO_OK;
}

void yo_free(yo_model *m) {
    if (!m) return;
    free(m->blob);
    free(m);
}

int yo_info(const yo_model *m, int32_t *out12) {
    const int32_t v[12] = {m->n_layers, m->n, m->block, m->vocab, m->depth, m->R, m->R2, m->input_rank, m->shift,
                           m->E, m->VP, m->layers[1 < m->n_layers ? 1 : 0].vt != NULL};
    memcpy(out12, v, sizeof v);
    return YO_OK;
}

/* ---------------------------------------------------------------------------------------------- arithmetic */

/* _mm512_cvtps_epi32 in the default rounding mode: round half to even; NaN and |x| >= 2^31 give INT32_MIN
   (cpu/ygg.cpp:292, 355, 372, 375, 410, 416). */
static inline int32_t cvt_rne(float x) {
    if (!(x >= -2147483648.0f && x < 2147483648.0f)) return INT32_MIN;
    return (int32_t)rintf(x);
}
static inline int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
static inline int32_t clamp127(int32_t v) { return v > 127 ? 127 : v < -127 ? -127 : v; }
static inline int8_t sat8(int32_t v) { return (int8_t)(v > 127 ? 127 : v < -128 ? -128 : v); }

/* rho = 1 / sqrt(f32(sum q^2) * f32(1/n) + eps), or with group scales the f32 sum over 16-coordinate groups in
   order of r2[g] * f32(S_g) (cpu/ygg.cpp:248-266, cpu/export.py:282-289) */
static float rms_rho(const int8_t *qb, int n, const float *r2, float eps) {
    const float inv_n = 1.0f / (float)n;
    if (r2) {
        float s = 0.0f;
        for (int g = 0; g < n / 16; g++) {
            int32_t sg = 0;
            for (int i = 16 * g; i < 16 * g + 16; i++) sg += (int32_t)qb[i] * qb[i];
            s = s + r2[g] * (float)sg;
        }
        return 1.0f / sqrtf(s * inv_n + eps);
    }
    int32_t ss = 0;
    for (int i = 0; i < n; i++) ss += (int32_t)qb[i] * qb[i];
    return 1.0f / sqrtf((float)ss * inv_n + eps);
}

/* heap descent from node 1: right iff f32(w_ix . qb) rho > thr[x][ix] (cpu/ygg.cpp:271-280) */
static int route(const yo_model *m, const yo_layer *y, int x, const int8_t *qb, float rho) {
    const int n = m->n;
    const float *th = y->thr + (size_t)x * m->E;
    int ix = 1;
    for (int d = 0; d < m->depth; d++) {
        const uint8_t *w = y->w + (size_t)ix * n;
        int32_t dot = 0;
        for (int i = 0; i < n; i++) dot += ((int32_t)w[i] - 128) * qb[i];
        ix = 2 * ix + ((float)dot * rho > th[ix]);
    }
    return ix - m->E;
}

/* zl[k] = clamp(rint((f32(V'_k . qb) * mv[k]) * rho), +-127) for k < 16 RG (cpu/ygg.cpp:285-296) */
static void layer_input(const yo_model *m, const yo_layer *y, const int8_t *qb, float rho, int8_t *zl) {
    const int n = m->n, RG = (m->R2 + 15) / 16;
    for (int k = 0; k < 16 * RG; k++) {
        const int gi = k / 16, lane = k % 16;
        int32_t a = 0;
        for (int i = 0; i < n; i++) {
            const size_t o = (((size_t)gi * (n / 4) + i / 4) * 16 + lane) * 4 + i % 4;
            a += ((int32_t)y->vl[o] - 128) * qb[i];
        }
        float zf = (float)a * y->mv[k];
        zf = zf * rho;
        zl[k] = (int8_t)clamp127(cvt_rne(zf));
    }
}

/* q <- sat8(((A16_r q + 2^(shift-1)) >> shift) + input + layer input) (cpu/ygg.cpp:311-389) */
static void update(const yo_model *m, const yo_layer *y, int l, int r, int x, int8_t *q, const int8_t *zl) {
    const int n = m->n, b = m->block;
    const uint8_t *rec = y->rec + (size_t)r * y->record_bytes;
    int32_t acc[256];
    /* transition: A16 [n/16][b/2][16][2] int16 */
    const int16_t *A = (const int16_t *)(rec + y->off_A);
    for (int i = 0; i < n; i++) {
        const int g = i / 16, rr = i % 16, c0 = (i / b) * b;
        int32_t s = 0;
        for (int j = 0; j < b; j++) s += (int32_t)A[((g * (b / 2) + j / 2) * 16 + rr) * 2 + (j & 1)] * q[c0 + j];
        acc[i] = (s + (1 << (m->shift - 1))) >> m->shift;
    }
    if (y->vt) {
        /* factored: acc += rint(f32(U_r v[x]) * f32(su_r * mT_i)) + c_r (cpu/ygg.cpp:339-358) */
        const int k = m->input_rank;
        const uint8_t *U = rec + y->off_F;
        const int8_t *v = y->vt + (size_t)x * k;
        const int16_t *C = (const int16_t *)(rec + y->off_C);
        float su;
        memcpy(&su, rec + y->off_S, 4);
        for (int i = 0; i < n; i++) {
            int32_t d = 0;
            for (int j = 0; j < k; j++) d += ((int32_t)U[((size_t)(j / 4) * n + i) * 4 + j % 4] - 128) * v[j];
            const float mul = su * y->mT[i];
            acc[i] = wadd(acc[i], wadd(cvt_rne((float)d * mul), C[i]));
        }
    } else {
        const int16_t *T = (const int16_t *)(rec + y->off_T + (size_t)x * y->table_stride);
        for (int i = 0; i < n; i++) acc[i] = wadd(acc[i], T[i]);
    }
    if (l > 0 && m->R2) {
        /* acc += rint(f32(U'_r zl) * m_ul) (cpu/ygg.cpp:360-377) */
        const uint8_t *U2 = rec + y->off_U2;
        for (int i = 0; i < n; i++) {
            int32_t d = 0;
            for (int j = 0; j < m->R2; j++) d += ((int32_t)U2[((size_t)(j / 4) * n + i) * 4 + j % 4] - 128) * zl[j];
            const float mu = y->mulv ? y->mulv[i] : y->layer_input_scale;
            acc[i] = wadd(acc[i], cvt_rne((float)d * mu));
        }
    }
    for (int i = 0; i < n; i++) q[i] = sat8(acc[i]);
}

/* lg = base + f32(Q zq) * sq, zq = clamp(rint(f32(P_r q) * m_z), +-127) (cpu/ygg.cpp:395-435) */
static void readout(const yo_model *m, const yo_layer *y, int r, const int8_t *q, float *lg, const float *base) {
    const int n = m->n, R = m->R, VP = m->VP;
    const uint8_t *P = y->rec + (size_t)r * y->record_bytes + y->off_P;
    int32_t zq[32];
    for (int j = 0; j < R; j++) {
        int32_t z = 0;
        for (int i = 0; i < n; i++) {
            size_t o;
            if (R == 8) o = ((size_t)(i / 8) * 16 + 2 * j + (i % 8) / 4) * 4 + i % 4;
            else o = (((size_t)(j / 16) * (n / 4) + i / 4) * 16 + j % 16) * 4 + i % 4;
            z += ((int32_t)P[o] - 128) * q[i];
        }
        const float mz = y->mzl ? y->mzl[(size_t)r * (R == 8 ? 16 : R) + (R == 8 ? 2 * j : j)] : y->readout_scale;
        zq[j] = clamp127(cvt_rne((float)z * mz));
    }
    for (int c = 0; c < VP; c++) {
        int32_t d = 0;
        for (int j = 0; j < R; j++) d += ((int32_t)y->Q[((size_t)(j / 4) * VP + c) * 4 + j % 4] - 128) * zq[j];
        const float s = y->sqv ? y->sqv[c] : y->unembed_scale;
        lg[c] = base[c] + (float)d * s;
    }
}

/* digest of (layer, leaf, state) at every token and layer; the GPU kernel computes the same value */
static inline uint64_t digest_term(int l, int leaf, const int8_t *q, int n) {
    uint64_t f = (uint64_t)(uint32_t)leaf * YO_DIGEST_LEAF;
    for (int i = 0; i < n; i++) f += (uint64_t)((uint8_t)q[i] + 1u) * ((uint64_t)(2 * i + 1) * YO_DIGEST_COORD);
    return f + (uint64_t)l;
}

/* one token of one stream through every layer (cpu/ygg.cpp:441-459) */
static void step(const yo_model *m, int8_t *q, int x, float *lg, int32_t *leaf, uint64_t *dg) {
    const int n = m->n;
    for (int l = 0; l < m->n_layers; l++) {
        const yo_layer *y = &m->layers[l];
        int8_t *ql = q + (size_t)l * n;
        int r = x;
        int8_t zl[MAX_RANK];
        if (l > 0) {
            const int8_t *qb = ql - n;
            const float rho = rms_rho(qb, n, y->r2b, y->rms_eps);
            r = route(m, y, x, qb, rho);
            if (m->R2) layer_input(m, y, qb, rho, zl);
        }
        update(m, y, l, r, x, ql, zl);
        readout(m, y, r, ql, lg, l == 0 ? m->output_bias : lg);
        if (leaf) leaf[l] = r;
        if (dg) *dg = *dg * YO_DIGEST_MUL + digest_term(l, r, ql, n);
    }
}

typedef struct {
    const yo_model *m;
    const int32_t *tokens;
    int B, T, s0, s1;
    int8_t *state;
    float *logits;
    int32_t *leaves;
    int8_t *states;
    uint64_t *digest;
    uint64_t *lgsum;
} job_t;

static void *run_job(void *p) {
    job_t *j = (job_t *)p;
    const yo_model *m = j->m;
    const int L = m->n_layers, n = m->n, V = m->vocab;
    float lg[256];
    for (int s = j->s0; s < j->s1; s++) {
        int8_t *q = j->state + (size_t)s * L * n;
        uint64_t dg = j->digest ? j->digest[s] : 0;
        for (int t = 0; t < j->T; t++) {
            const size_t i = (size_t)s * j->T + t;
            step(m, q, j->tokens[i], lg, j->leaves ? j->leaves + i * L : NULL, j->digest ? &dg : NULL);
            if (j->logits) memcpy(j->logits + i * V, lg, sizeof(float) * V);
            if (j->lgsum) {
                uint64_t acc = 0;
                for (int c = 0; c < V; c++) {
                    uint32_t b;
                    memcpy(&b, &lg[c], 4);
                    acc += b;
                }
                j->lgsum[s] += acc;
            }
            if (j->states) memcpy(j->states + i * L * n, q, (size_t)L * n);
        }
        if (j->digest) j->digest[s] = dg;
    }
    return NULL;
}

static int run_all(const yo_model *m, const int32_t *tokens, int B, int T, int8_t *state, float *logits,
                   int32_t *leaves, int8_t *states, uint64_t *digest, uint64_t *lgsum, int threads, char *err,
                   int errlen) {
    if (B < 0 || T < 0) { set_err(err, errlen, "negative B or T"); return YO_ERR_ARG; }
    for (size_t i = 0; i < (size_t)B * T; i++)
        if (tokens[i] < 0 || tokens[i] >= m->vocab) {
            set_err(err, errlen, "token %d out of range [0, %d)", tokens[i], m->vocab);
            return YO_ERR_TOKEN;
        }
    if (threads < 1) threads = 1;
    if (threads > B) threads = B > 0 ? B : 1;
    job_t *jobs = (job_t *)calloc((size_t)threads, sizeof(job_t));
    pthread_t *th = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
    for (int k = 0; k < threads; k++) {
        jobs[k] = (job_t){m, tokens, B, T, (int)((long)B * k / threads), (int)((long)B * (k + 1) / threads),
                          state, logits, leaves, states, digest, lgsum};
        if (threads > 1) pthread_create(&th[k], NULL, run_job, &jobs[k]);
        else run_job(&jobs[k]);
    }
    if (threads > 1)
        for (int k = 0; k < threads; k++) pthread_join(th[k], NULL);
    free(jobs);
    free(th);
    return YO_OK;
}

int yo_run(const yo_model *m, const int32_t *tokens, int B, int T, int8_t *state, float *logits, int32_t *leaves,
           int8_t *states, uint64_t *digest, int threads, char *err, int errlen) {
    return run_all(m, tokens, B, T, state, logits, leaves, states, digest, NULL, threads, err, errlen);
}

int yo_run_sums(const yo_model *m, const int32_t *tokens, int B, int T, int8_t *state, uint64_t *digest,
                uint64_t *lgsum, int threads, char *err, int errlen) {
    return run_all(m, tokens, B, T, state, NULL, NULL, NULL, digest, lgsum, threads, err, errlen);
}

uint64_t yo_digest_init(void) { return YO_DIGEST_INIT; }

/* ------------------------------------------------------------------------------------------- f32 softmax
 * The per-token softmax of the reference's `time` mode, softmax() and vexp() at cpu/ygg.cpp:44-72, as scalar C:
 *   mx = max_i lg[i];  e_i = exp2(clamp(lg[i] - mx, -87, 88))  (vexp below);
 *   tot = the 16 lane sums s_j = sum over k of e[16 k + j] (k ascending), joined as ((s_j + s_(8+j)), then + the
 *         element 4 apart, then 2 apart, then 1 apart) -- the 16-lane accumulator and the halving reduction of the
 *         reference's vector code (checked bit for bit against the reference build in tests/test_oracle.py);
 *   probs_i = e_i * (1 / tot);  lse = mx + logf(tot).
 * vexp(x): t = x * f32(log2 e), n = t rounded to nearest even, f = t - n, p = the reference's degree-6 polynomial for
 * 2^f in Horner form with fused multiply-adds (cpu/ygg.cpp:48-55), result p * 2^n. */
static float vexp1(float x) {
    x = fminf(fmaxf(x, -87.f), 88.f);
    const float t = x * 1.4426950408889634f;
    const float n = rintf(t);
    const float f = t - n;
    float p = 1.5353362e-4f;
    p = fmaf(p, f, 1.3398874e-3f);
    p = fmaf(p, f, 9.6181291e-3f);
    p = fmaf(p, f, 5.5504109e-2f);
    p = fmaf(p, f, 2.4022651e-1f);
    p = fmaf(p, f, 6.9314718e-1f);
    p = fmaf(p, f, 1.0f);
    return ldexpf(p, (int)n);
}

void yo_softmax(const float *logits, long rows, int V, float *probs, float *lse) {
    for (long r = 0; r < rows; r++) {
        const float *lg = logits + (size_t)r * V;
        float *pr = probs + (size_t)r * V;
        float mx = -INFINITY;
        for (int i = 0; i < V; i++) mx = lg[i] > mx ? lg[i] : mx;
        float s[16];
        for (int j = 0; j < 16; j++) s[j] = 0.0f;
        for (int i = 0; i < V; i++) {
            const float e = vexp1(lg[i] - mx);
            pr[i] = e;
            s[i & 15] = s[i & 15] + e;
        }
        float h[8], q[4];
        for (int j = 0; j < 8; j++) h[j] = s[j] + s[8 + j];
        for (int j = 0; j < 4; j++) q[j] = h[j] + h[4 + j];
        const float tot = (q[0] + q[2]) + (q[1] + q[3]);
        const float inv = 1.0f / tot;
        for (int i = 0; i < V; i++) pr[i] = pr[i] * inv;
        lse[r] = mx + logf(tot);
    }
}
