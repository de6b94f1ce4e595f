/* The Needle-3 decode step on the CPU, restated from the reference's
 * native engine (crates/needle-engine/src/infer/step.rs:171-760 and the
 * helpers of crates/needle-engine/src/infer.rs), x86-64 portable branches,
 * in the same float-operation order (fmaf where Rust has mul_add).
 *
 * TEST INFRASTRUCTURE: the parity checker (and CPU baseline) for a GPU
 * forward; nothing in the product links it.
 *
 * Scope: Model::forward_native (infer.rs:1105-1132) over step_native and
 * chunk_job with every Outputs mode (model.rs:150-160, chunk.rs:331-353),
 * Model::prefill_native's stale-slot re-feed (infer.rs:1078-1101), the
 * session attention span (sink, ring) with its KV slot ring and slot map
 * (model.rs:62-66, infer.rs:1749-1826), Session::rollback / rewind_zeroed /
 * clone (model.rs:81-121, infer.rs:1039-1071), the head functions
 * (infer.rs:1135-1166) and the per-depth cells of Model::forward_cells and
 * a tracking session (model.rs:60-62,330-345; infer/step.rs:240-243,
 * 672-714; infer/chunk.rs:69-70,310,353-356; infer.rs:1105-1130).
 *
 * libm: off Apple targets the reference computes its f32 functions in f64
 * with the Rust `libm` crate (0.2.16, Cargo.lock:647-650) and rounds once
 * (infer.rs:76-101): lexpf = (f32)exp((f64)x), lpowf = (f32)pow, sincosf =
 * the f64 sincos rounded; lexp = exp.  Here the f64 functions are glibc's.
 * Both are accurate to under an f64 ulp, so the f32 results agree unless an
 * f32 rounding boundary falls between the two f64 results (about 2^-29 of
 * calls): the step is parity unpinned at that boundary only.
 */
#define _GNU_SOURCE /* sincos */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "cq_oracle.h"
#include "forward.h"

/* ------------------------------------------------------------- constants */
/* infer.rs:30-38 */
static float bits_f(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}
#define INV_SQRT_QK bits_f(0x3e13cd3au)
#define Q21 bits_f(0x49fffff8u)
#define C21 bits_f(0x35000004u)
#define NATIVE_TEAM 4
/* crates/needle-core/src/config.rs:10-13 */
#define ENGRAM_CONV_TAPS 4
#define ENGRAM_SEED 0x9E3779B9u
#define ENGRAM_PRIME 0x01000193u
#define HADA_COND_RANK 8
#define NB 32
#define HN (NB * NB)

/* ---------------------------------------------------------------- helpers */

/* lexpf / lpowf / sincosf off Apple targets (infer.rs:84-101). */
static float lexpf(float x) { return (float)exp((double)x); }
static float lpowf(float x, float y) { return (float)pow((double)x, (double)y); }
static void lsincosf(float x, float* s, float* c) {
    double sd, cd;
    sincos((double)x, &sd, &cd);
    *s = (float)sd;
    *c = (float)cd;
}

/* nexp (infer.rs:353-367). */
float nf_nexp(float x) {
    x = fminf(fmaxf(x, bits_f(0xc2b0c0a5u)), bits_f(0x42b0c0a5u));
    const float k = rintf(x * bits_f(0x3fb8aa3bu));
    float r = fmaf(k, bits_f(0xbf318000u), x);
    r = fmaf(k, bits_f(0x395e8083u), r);
    float p = fmaf(bits_f(0x39506967u), r, bits_f(0x3ab743ceu));
    p = fmaf(r, p, bits_f(0x3c088908u));
    p = fmaf(r, p, bits_f(0x3d2aa9c1u));
    p = fmaf(r, p, bits_f(0x3e2aaaaau));
    p = fmaf(r, p, 0.5f);
    const float y = fmaf(r * r, p, r);
    const uint32_t sb = (uint32_t)((int32_t)k << 23) + 0x3f800000u;
    const float s = bits_f(sb);
    return fmaf(s, y, s);
}

/* zcn (infer.rs:426-444) with an f32 scale. */
static void zcn(const float* x, const float* s, size_t n, float* out) {
    const float r = cq_rinv(cq_dot16(x, x, n), n);
    for (size_t i = 0; i < n; ++i) {
        const float t = x[i] * r;
        out[i] = fmaf(t, s[i], t);
    }
}

/* zcn16_inplace (infer.rs:475-494). */
static void zcn16_inplace(float* x, const uint16_t* s, size_t n) {
    const float r = cq_rinv(cq_dot16(x, x, n), n);
    for (size_t i = 0; i < n; ++i) {
        const float t = x[i] * r;
        x[i] = fmaf(t, cq_f16_to_f32(s[i]), t);
    }
}

/* rope_rotate (infer.rs:637-665). */
void nf_rope_rotate(float* x, size_t n, const float* cs, const float* sn) {
    const size_t half = n / 2;
    for (size_t f = 0; f < half; ++f) {
        const float a = x[f], b = x[f + half];
        x[f] = fmaf(-sn[f], b, cs[f] * a);
        x[f + half] = fmaf(sn[f], a, cs[f] * b);
    }
}

/* idot (infer.rs:769-775). */
static int32_t idot(const int8_t* a, const int8_t* b, size_t n) {
    int32_t s = 0;
    for (size_t i = 0; i < n; ++i) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

/* cond_weights (infer.rs:1640-1656), portable branch. */
void nf_cond_weights(const float* h2, size_t d, const uint16_t* cond_v, float out[8]) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    for (size_t j = 0; j < d; ++j) {
        float* a = acc[j % 4];
        for (int k = 0; k < 8; ++k) a[k] = fmaf(h2[j], cq_f16_to_f32(cond_v[j * 8 + k]), a[k]);
    }
    float lg[8], e[8], m = -INFINITY;
    for (int k = 0; k < 8; ++k) {
        lg[k] = ((acc[2][k] + acc[3][k]) + acc[1][k]) + acc[0][k];
        m = fmaxf(m, lg[k]);
    }
    for (int k = 0; k < 8; ++k) e[k] = lexpf(lg[k] - m);
    const float sum = e[7] + ((e[6] + (e[5] + e[4])) + ((e[3] + e[2]) + (e[1] + e[0])));
    const float inv = 1.0f / sum;
    for (int k = 0; k < 8; ++k) out[k] = e[k] * inv;
}

/* mix8 (infer.rs:2343-2380), portable branch, all 16 tiles or the first
 * `tiles`: out[r][c] = sum_j ct[j][r] * rows[j][c] (fma chain from j = 0);
 * transposed, out[c][r].  ct / rows are f16 (`h` set) or f32. */
static inline float at(const void* p, int half, size_t i) {
    return half ? cq_f16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

void nf_mix8(int transpose, const void* ct, int ct_half, const void* rows, int rows_half, float* out, int tiles) {
    for (int t = 0; t < tiles; ++t) {
        const int r0 = (t / 4) * 8, c0 = (t % 4) * 8;
        for (int r = r0; r < r0 + 8; ++r) {
            float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int j = 0; j < NB; ++j) {
                const float c = at(ct, ct_half, (size_t)j * NB + r);
                for (int k = 0; k < 8; ++k) o[k] = fmaf(c, at(rows, rows_half, (size_t)j * NB + c0 + k), o[k]);
            }
            for (int k = 0; k < 8; ++k) {
                const int cc = c0 + k;
                out[transpose ? cc * NB + r : r * NB + cc] = o[k];
            }
        }
    }
}

/* sinkhorn64 (infer.rs:2501-2528). */
void nf_sinkhorn64(const float z[16], float out[16]) {
    double e[16];
    for (int r = 0; r < 4; ++r) {
        const double m = (double)fmaxf(fmaxf(z[r * 4], z[r * 4 + 1]), fmaxf(z[r * 4 + 2], z[r * 4 + 3]));
        for (int c = 0; c < 4; ++c) e[r * 4 + c] = exp((double)z[r * 4 + c] - m);
    }
    for (int it = 0; it < 20; ++it) {
        for (int r = 0; r < 4; ++r) {
            const double inv = 1.0 / ((e[r * 4] + e[r * 4 + 1]) + (e[r * 4 + 2] + e[r * 4 + 3]));
            for (int c = 0; c < 4; ++c) e[r * 4 + c] *= inv;
        }
        for (int c = 0; c < 4; ++c) {
            const double inv = 1.0 / ((e[c] + e[4 + c]) + (e[8 + c] + e[12 + c]));
            for (int r = 0; r < 4; ++r) e[r * 4 + c] *= inv;
        }
    }
    for (int i = 0; i < 16; ++i) out[i] = (float)e[i];
}

/* chunk_exp (infer.rs:2222-2279), x86-64 branch: numerators in place and
 * their sum in the engine's order. */
float nf_chunk_exp(float* s, size_t l, float m) {
    size_t i = 0;
    float a[4] = {0, 0, 0, 0}, b[4] = {0, 0, 0, 0};
    while (i + 8 <= l) {
        for (int k = 0; k < 4; ++k) {
            const float e = nf_nexp(s[i + k] - m);
            s[i + k] = e;
            a[k] += e;
        }
        for (int k = 0; k < 4; ++k) {
            const float e = nf_nexp(s[i + 4 + k] - m);
            s[i + 4 + k] = e;
            b[k] += e;
        }
        i += 8;
    }
    while (i + 4 <= l) {
        for (int k = 0; k < 4; ++k) {
            const float e = nf_nexp(s[i + k] - m);
            s[i + k] = e;
            a[k] += e;
        }
        i += 4;
    }
    float t[4];
    for (int k = 0; k < 4; ++k) t[k] = a[k] + b[k];
    float sum = (t[0] + t[1]) + (t[2] + t[3]);
    if (l - i >= 2) {
        const float e0 = lexpf(s[i] - m), e1 = lexpf(s[i + 1] - m);
        s[i] = e0;
        s[i + 1] = e1;
        sum = (e0 + sum) + e1;
        i += 2;
    }
    if (l - i == 1) {
        const float e = lexpf(s[i] - m);
        s[i] = e;
        sum += e;
    }
    return sum;
}

/* digits21 (infer.rs:2171-2220), portable branch: round half away. */
void nf_digits21(const float* w, size_t n, float qw, int8_t* hi, int8_t* mid, int8_t* lo) {
    for (size_t i = 0; i < n; ++i) {
        const int32_t wq = (int32_t)roundf(w[i] * qw);
        hi[i] = (int8_t)(wq >> 14);
        mid[i] = (int8_t)((wq >> 7) & 127);
        lo[i] = (int8_t)(wq & 127);
    }
}

/* key_chunks (infer.rs:2093-2101) with the minimum chunk count k: (count,
 * size).  attend_head_ref uses k = max(1, 2 NATIVE_TEAM / nkv), or 1 when
 * nested (infer.rs:1888). */
static void key_chunks_k(size_t n, size_t k, size_t* count, size_t* size) {
    size_t c = (n + 255) / 256;
    if (k * 64 <= n && c < k) c = k;
    if (c < 1) c = 1;
    const size_t chunk = ((n + c - 1) / c + 15) / 16 * 16;
    *size = chunk;
    *count = chunk ? (n + chunk - 1) / chunk : 0;
}

void nf_key_chunks(size_t n, size_t nkv, size_t* count, size_t* size) {
    size_t k = 2 * NATIVE_TEAM / nkv;
    if (k < 1) k = 1;
    key_chunks_k(n, k, count, size);
}

/* ------------------------------------------------------------------ model */
/* (nf_engram_rows, nf_mhc_read, nf_post_gates and nf_mhc_write are defined
 * after the model; nf_rows calls each of them once per row.) */

struct nf_layer16 {
    uint16_t *kron[6], *cond_v, *cond_u, *d1, *d2, *b2, *d3, *d4, *norm_in, *post_norm, *pre_hada, *q_taps, *k_taps,
        *v_taps, *q_norm, *k_norm;
    float a_pre, a_post, a_res, attn_gate, b_pre[4], b_post[4], b_res[16];
    int8_t* phi_q;  /* Phi8 (infer.rs:850-867): ncols x nc */
    float* phi_s;
};

struct nf_model {
    nf_config c;
    struct nf_layer16* L;
    const cq_qmat* embedding;
    const cq_qlinear** qkvg;
    const cq_qlinear** out;
    const cq_qmat** etables;
    const cq_qlinear** ekv;
    float** etaps;       /* per site [4][d] */
    float* final_norm;   /* [d] */
    int32_t *perm1, *perm2;
    float *freq, *sd, *cd;  /* RoPE tables (Tables::new, infer.rs:935-947) */
    int site_of_layer[64];
};

/* ROLLBACK (model.rs:181-183): the conv history and the RoPE list keep
 * this many extra rows. */
#define NF_ROLLBACK 32
#define NF_KEY_RUNS 16 /* KEY_RUNS (infer.rs:1760) */
#define NF_MAX_TAPS 16

struct nf_session {
    size_t cap;     /* positions */
    size_t len;     /* tokens fed */
    uint32_t* tokens;
    /* per layer, by KV slot: k8 [slot][nkv][qk], ks [slot][nkv], v8t [nkv][vd][cap], vs [slot][nkv] */
    int8_t** k8;
    float** ks;
    int8_t** v8t;
    float** vs;
    /* per layer: the pre-tap q|k|v row of every position [pos][width]; of
     * them LayerState::hist holds the last `hrows` (infer.rs:968-980): the
     * conv reads a row only from there (newest last, trimmed as
     * step.rs:706-712 and chunk.rs:319-329 trim it) */
    float** hist;
    size_t hrows;
    /* engram value history per site: [pos][d] int8 + [pos][d/32] */
    int8_t** ev8;
    float** evs;
    /* RoPE rows of every position fed [pos][32]; NatState::rope holds the
     * last `rope_n` of them, ending at position len - 1 (infer.rs:1716-1747) */
    float *rope_c, *rope_s;
    size_t rope_n;
    /* Session::attend (model.rs:62-66): sink, ring (ring 0: None), and the
     * slot map NatState::slot_pos (infer.rs:1000-1006) with its length */
    size_t sink, ring;
    int64_t* slot_pos;
    size_t nslot;
    /* NatState::last_hidden (infer.rs:996-998) */
    float* last_hidden;
    int have_hidden;
    /* Session::cells (model.rs:60-62): when tracked, the cell rows
     * [ncells][L+1][d] the feeds appended (room for cap rows) */
    int track_cells;
    float* cells;
    size_t ncells;
};

static uint16_t* dup16(const uint16_t* p, size_t n) {
    uint16_t* q = (uint16_t*)malloc(n * 2);
    memcpy(q, p, n * 2);
    return q;
}

nf_model* nf_model_new(const nf_config* c) {
    nf_model* m = (nf_model*)calloc(1, sizeof *m);
    m->c = *c;
    m->L = (struct nf_layer16*)calloc((size_t)c->layers, sizeof *m->L);
    m->qkvg = (const cq_qlinear**)calloc((size_t)c->layers, sizeof(void*));
    m->out = (const cq_qlinear**)calloc((size_t)c->layers, sizeof(void*));
    m->etables = (const cq_qmat**)calloc((size_t)c->sites + 1, sizeof(void*));
    m->ekv = (const cq_qlinear**)calloc((size_t)c->sites + 1, sizeof(void*));
    m->etaps = (float**)calloc((size_t)c->sites + 1, sizeof(float*));
    for (int l = 0; l < 64; ++l) m->site_of_layer[l] = -1;
    for (int s = 0; s < c->sites; ++s) m->site_of_layer[c->site_layers[s]] = s;
    /* Tables::new (infer.rs:942-947): freq = lpowf(theta, i * (-2 / qk)), then sincosf. */
    const int half = c->qk / 2;
    m->freq = (float*)malloc(sizeof(float) * half);
    m->sd = (float*)malloc(sizeof(float) * half);
    m->cd = (float*)malloc(sizeof(float) * half);
    const float coef = -2.0f / (float)c->qk;
    for (int i = 0; i < half; ++i) {
        m->freq[i] = lpowf(c->rope_theta, (float)i * coef);
        lsincosf(m->freq[i], &m->sd[i], &m->cd[i]);
    }
    return m;
}

void nf_model_free(nf_model* m) {
    if (!m) return;
    for (int l = 0; l < m->c.layers; ++l) {
        struct nf_layer16* L = &m->L[l];
        for (int k = 0; k < 6; ++k) free(L->kron[k]);
        free(L->cond_v), free(L->cond_u), free(L->d1), free(L->d2), free(L->b2), free(L->d3), free(L->d4);
        free(L->norm_in), free(L->post_norm), free(L->pre_hada), free(L->q_taps), free(L->k_taps), free(L->v_taps);
        free(L->q_norm), free(L->k_norm), free(L->phi_q), free(L->phi_s);
    }
    for (int s = 0; s < m->c.sites; ++s) free(m->etaps[s]);
    free(m->L), free(m->qkvg), free(m->out), free(m->etables), free(m->ekv), free(m->etaps);
    free(m->final_norm), free(m->perm1), free(m->perm2), free(m->freq), free(m->sd), free(m->cd);
    free(m);
}

void nf_set_layer_f16(nf_model* m, int l, int which, const uint16_t* v, size_t n) {
    struct nf_layer16* L = &m->L[l];
    uint16_t** slot = NULL;
    switch (which) {
        case NF_KRON0: case NF_KRON1: case NF_KRON2: case NF_KRON3: case NF_KRON4: case NF_KRON5:
            slot = &L->kron[which - NF_KRON0]; break;
        case NF_COND_V: slot = &L->cond_v; break;
        case NF_COND_U: slot = &L->cond_u; break;
        case NF_D1: slot = &L->d1; break;
        case NF_D2: slot = &L->d2; break;
        case NF_B2: slot = &L->b2; break;
        case NF_D3: slot = &L->d3; break;
        case NF_D4: slot = &L->d4; break;
        case NF_NORM_IN: slot = &L->norm_in; break;
        case NF_POST_NORM: slot = &L->post_norm; break;
        case NF_PRE_HADA: slot = &L->pre_hada; break;
        case NF_Q_TAPS: slot = &L->q_taps; break;
        case NF_K_TAPS: slot = &L->k_taps; break;
        case NF_V_TAPS: slot = &L->v_taps; break;
        case NF_Q_NORM: slot = &L->q_norm; break;
        case NF_K_NORM: slot = &L->k_norm; break;
        default: return;
    }
    free(*slot);
    *slot = dup16(v, n);
}

void nf_set_layer_scalars(nf_model* m, int l, float a_pre, float a_post, float a_res, float attn_gate,
                          const float* b_pre, const float* b_post, const float* b_res) {
    struct nf_layer16* L = &m->L[l];
    L->a_pre = a_pre, L->a_post = a_post, L->a_res = a_res, L->attn_gate = attn_gate;
    memcpy(L->b_pre, b_pre, 4 * sizeof(float));
    memcpy(L->b_post, b_post, 4 * sizeof(float));
    memcpy(L->b_res, b_res, 16 * sizeof(float));
}

/* Phi8::new over the dequantized fused pre|post|res rows of a layer. */
void nf_set_phi(nf_model* m, int l, const float* w, size_t rows, size_t width) {
    struct nf_layer16* L = &m->L[l];
    free(L->phi_q), free(L->phi_s);
    L->phi_q = (int8_t*)malloc(rows * width);
    L->phi_s = (float*)malloc(rows * sizeof(float));
    for (size_t r = 0; r < rows; ++r) L->phi_s[r] = cq_quant_i8(w + r * width, width, L->phi_q + r * width);
}

void nf_set_matrices(nf_model* m, const cq_qmat* embedding, const cq_qlinear* const* qkvg, const cq_qlinear* const* out,
                     const cq_qmat* const* etables, const cq_qlinear* const* ekv) {
    m->embedding = embedding;
    for (int l = 0; l < m->c.layers; ++l) m->qkvg[l] = qkvg[l], m->out[l] = out[l];
    for (int s = 0; s < m->c.sites; ++s) m->etables[s] = etables[s], m->ekv[s] = ekv[s];
}

void nf_set_engram_taps(nf_model* m, int site, const float* taps, size_t n) {
    free(m->etaps[site]);
    m->etaps[site] = (float*)malloc(n * sizeof(float));
    memcpy(m->etaps[site], taps, n * sizeof(float));
}

void nf_set_globals(nf_model* m, const float* final_norm, const int32_t* perm1, const int32_t* perm2) {
    const int d = m->c.d;
    free(m->final_norm), free(m->perm1), free(m->perm2);
    m->final_norm = (float*)malloc(d * sizeof(float));
    memcpy(m->final_norm, final_norm, d * sizeof(float));
    m->perm1 = (int32_t*)malloc(HN * sizeof(int32_t));
    m->perm2 = (int32_t*)malloc(HN * sizeof(int32_t));
    memcpy(m->perm1, perm1, HN * sizeof(int32_t));
    memcpy(m->perm2, perm2, HN * sizeof(int32_t));
}

/* ---------------------------------------------------------------- session */

static int width_of(const nf_config* c) { return (c->nh + c->nkv) * c->qk + c->nkv * c->vd; }

nf_session* nf_session_new(const nf_model* m, size_t cap) {
    const nf_config* c = &m->c;
    nf_session* s = (nf_session*)calloc(1, sizeof *s);
    s->cap = cap;
    s->tokens = (uint32_t*)calloc(cap, sizeof(uint32_t));
    s->k8 = (int8_t**)calloc((size_t)c->layers, sizeof(void*));
    s->ks = (float**)calloc((size_t)c->layers, sizeof(void*));
    s->v8t = (int8_t**)calloc((size_t)c->layers, sizeof(void*));
    s->vs = (float**)calloc((size_t)c->layers, sizeof(void*));
    s->hist = (float**)calloc((size_t)c->layers, sizeof(void*));
    const int W = width_of(c);
    for (int l = 0; l < c->layers; ++l) {
        s->k8[l] = (int8_t*)calloc(cap * c->nkv * c->qk, 1);
        s->ks[l] = (float*)calloc(cap * c->nkv, sizeof(float));
        s->v8t[l] = (int8_t*)calloc((size_t)c->nkv * c->vd * cap, 1);
        s->vs[l] = (float*)calloc(cap * c->nkv, sizeof(float));
        s->hist[l] = (float*)calloc(cap * (size_t)W, sizeof(float));
    }
    s->ev8 = (int8_t**)calloc((size_t)c->sites + 1, sizeof(void*));
    s->evs = (float**)calloc((size_t)c->sites + 1, sizeof(void*));
    for (int e = 0; e < c->sites; ++e) {
        s->ev8[e] = (int8_t*)calloc(cap * c->d, 1);
        s->evs[e] = (float*)calloc(cap * (c->d / 32), sizeof(float));
    }
    s->rope_c = (float*)calloc(cap * 32, sizeof(float));
    s->rope_s = (float*)calloc(cap * 32, sizeof(float));
    s->slot_pos = (int64_t*)malloc(cap * sizeof(int64_t));
    for (size_t i = 0; i < cap; ++i) s->slot_pos[i] = -1;
    s->last_hidden = (float*)calloc((size_t)c->d, sizeof(float));
    return s;
}

void nf_session_free(const nf_model* m, nf_session* s) {
    if (!s) return;
    for (int l = 0; l < m->c.layers; ++l) free(s->k8[l]), free(s->ks[l]), free(s->v8t[l]), free(s->vs[l]), free(s->hist[l]);
    for (int e = 0; e < m->c.sites; ++e) free(s->ev8[e]), free(s->evs[e]);
    free(s->k8), free(s->ks), free(s->v8t), free(s->vs), free(s->hist), free(s->ev8), free(s->evs);
    free(s->tokens), free(s->rope_c), free(s->rope_s), free(s->slot_pos), free(s->last_hidden), free(s->cells);
    free(s);
}

static void* dupb(const void* p, size_t n) {
    void* q = malloc(n ? n : 1);
    if (n) memcpy(q, p, n);
    return q;
}

/* Session::clone (#[derive(Clone)], model.rs:53-55): every cache copied. */
nf_session* nf_session_clone(const nf_model* m, const nf_session* s) {
    const nf_config* c = &m->c;
    const size_t cap = s->cap, W = (size_t)width_of(c);
    nf_session* o = (nf_session*)malloc(sizeof *o);
    *o = *s;
    o->tokens = (uint32_t*)dupb(s->tokens, cap * 4);
    o->k8 = (int8_t**)calloc((size_t)c->layers, sizeof(void*));
    o->ks = (float**)calloc((size_t)c->layers, sizeof(void*));
    o->v8t = (int8_t**)calloc((size_t)c->layers, sizeof(void*));
    o->vs = (float**)calloc((size_t)c->layers, sizeof(void*));
    o->hist = (float**)calloc((size_t)c->layers, sizeof(void*));
    for (int l = 0; l < c->layers; ++l) {
        o->k8[l] = (int8_t*)dupb(s->k8[l], cap * c->nkv * c->qk);
        o->ks[l] = (float*)dupb(s->ks[l], cap * c->nkv * 4);
        o->v8t[l] = (int8_t*)dupb(s->v8t[l], (size_t)c->nkv * c->vd * cap);
        o->vs[l] = (float*)dupb(s->vs[l], cap * c->nkv * 4);
        o->hist[l] = (float*)dupb(s->hist[l], cap * W * 4);
    }
    o->ev8 = (int8_t**)calloc((size_t)c->sites + 1, sizeof(void*));
    o->evs = (float**)calloc((size_t)c->sites + 1, sizeof(void*));
    for (int e = 0; e < c->sites; ++e) {
        o->ev8[e] = (int8_t*)dupb(s->ev8[e], cap * c->d);
        o->evs[e] = (float*)dupb(s->evs[e], cap * (c->d / 32) * 4);
    }
    o->rope_c = (float*)dupb(s->rope_c, cap * 32 * 4);
    o->rope_s = (float*)dupb(s->rope_s, cap * 32 * 4);
    o->slot_pos = (int64_t*)dupb(s->slot_pos, cap * 8);
    o->last_hidden = (float*)dupb(s->last_hidden, (size_t)c->d * 4);
    o->cells = s->cells ? (float*)dupb(s->cells, cap * (size_t)(c->layers + 1) * c->d * 4) : NULL;
    return o;
}

size_t nf_session_len(const nf_session* s) { return s->len; }

/* Session::attend (model.rs:62-66): ring 0 is None.  Any ring is taken; a
 * feed with a chunk longer than a ring shorter than 32 is refused
 * (nf_forward): two rows of that chunk would share a KV slot (the
 * reference's members race on it) and a row could see no key at all
 * (attend_head_ref's step_by(0) panics). */
int nf_session_set_attend(nf_session* s, size_t sink, size_t ring) {
    s->sink = sink;
    s->ring = ring;
    return 0;
}

/* Session::rollback (model.rs:81-113) with NatState::rollback
 * (infer.rs:1053-1071): drop the last n <= ROLLBACK positions; the KV slots
 * and the slot map keep what they hold. */
int nf_session_rollback(const nf_model* m, nf_session* s, size_t n) {
    (void)m;
    if (n > NF_ROLLBACK || n > s->len) return -1;
    if (n == 0) return 0;
    s->len -= n;
    s->hrows = s->hrows > n ? s->hrows - n : 0;
    s->rope_n = s->rope_n > n ? s->rope_n - n : 0; /* rope.retain(p < len) */
    if (s->ncells > s->len) s->ncells = s->len;  /* cells.truncate(len (L+1) d) */
    return 0;
}

/* Session::rewind_zeroed (model.rs:115-121), NatState::rewind_zeroed
 * (infer.rs:1039-1051): positions len.. forgotten, the conv history emptied
 * and the RoPE list dropped; the KV slots and slot map stay. */
int nf_session_rewind_zeroed(const nf_model* m, nf_session* s, size_t len) {
    (void)m;
    if (len < s->len) s->len = len;
    s->hrows = 0;
    s->rope_n = 0;
    if (s->ncells > len) s->ncells = len;  /* cells.truncate(len (L+1) d) */
    return 0;
}

/* Session::cells = Some(vec![]) (on) or None (off).  Tracking starts at an
 * empty session: the store's truncations (rollback, rewind_zeroed, prefill's
 * re-feed) index it by position. */
int nf_session_track_cells(const nf_model* m, nf_session* s, int on) {
    if (on && s->len != 0) return -1;
    s->track_cells = on != 0;
    s->ncells = 0;
    if (on && !s->cells) s->cells = (float*)calloc(s->cap * (size_t)(m->c.layers + 1) * m->c.d, sizeof(float));
    return 0;
}

/* The tracked cell rows [row0, row0 + n) into dst[n][L+1][d]; the count of
 * rows held, or -1 (not tracking, or past the end). */
int nf_session_cells(const nf_model* m, const nf_session* s, size_t row0, size_t n, float* dst) {
    if (!s->track_cells || row0 + n > s->ncells) return -1;
    const size_t w = (size_t)(m->c.layers + 1) * m->c.d;
    if (n) memcpy(dst, s->cells + row0 * w, n * w * sizeof(float));
    return (int)s->ncells;
}

/* NatState::last_hidden into out[d]; 0, or -1 when no feed has set it. */
int nf_session_last_hidden(const nf_model* m, const nf_session* s, float* out) {
    if (!s->have_hidden) return -1;
    memcpy(out, s->last_hidden, sizeof(float) * m->c.d);
    return 0;
}

/* slot_of (infer.rs:1749-1756). */
static size_t slot_of(size_t p, const nf_session* s) {
    return (s->ring > 0 && p >= s->sink) ? (p - s->sink) % s->ring + s->sink : p;
}

/* mark_slots (infer.rs:1770-1779). */
static void mark_slots(nf_session* s, size_t p0, size_t end) {
    for (size_t p = p0; p < end; ++p) {
        const size_t sl = slot_of(p, s);
        if (s->nslot <= sl) {
            for (size_t i = s->nslot; i <= sl; ++i) s->slot_pos[i] = -1;
            s->nslot = sl + 1;
        }
        s->slot_pos[sl] = (int64_t)p;
    }
}

/* key_ranges (infer.rs:1781-1826) over the slot map snapshot `sp` (nsp
 * entries): up to 16 ascending position ranges [lo, hi); returns how many,
 * or -1 past KEY_RUNS (the reference asserts). */
static int key_ranges(size_t pos, size_t chunk_end, size_t window, const nf_session* s, const int64_t* sp, size_t nsp,
                      size_t* lo_out, size_t* hi_out) {
    const size_t lo = window ? (pos + 1 > window ? pos + 1 - window : 0) : 0;
    size_t clo[2], chi[2];
    if (s->ring == 0) {
        clo[0] = lo, chi[0] = pos + 1, clo[1] = chi[1] = 0;
    } else {
        const size_t sink = s->sink, ring = s->ring;
        size_t ae = sink < pos + 1 ? sink : pos + 1;
        if (ae < lo) ae = lo;
        clo[0] = lo, chi[0] = ae;
        size_t b0 = chunk_end > ring ? chunk_end - ring : 0;
        if (b0 < sink) b0 = sink;
        if (b0 > pos + 1) b0 = pos + 1;
        clo[1] = b0, chi[1] = pos + 1;
    }
    int k = 0;
    for (int r = 0; r < 2; ++r) {
        if (s->ring == 0) {
            if (chi[r] > clo[r]) {
                if (k >= NF_KEY_RUNS) return -1;
                lo_out[k] = clo[r], hi_out[k] = chi[r], ++k;
            }
            continue;
        }
        int open = 0;
        size_t a = 0;
        for (size_t p = clo[r]; p < chi[r]; ++p) {
            const size_t sl = slot_of(p, s);
            const int ok = sl < nsp && sp[sl] == (int64_t)p;
            if (ok && !open) {
                open = 1, a = p;
            } else if (!ok && open) {
                if (k >= NF_KEY_RUNS) return -1;
                lo_out[k] = a, hi_out[k] = p, ++k, open = 0;
            }
        }
        if (open) {
            if (k >= NF_KEY_RUNS) return -1;
            lo_out[k] = a, hi_out[k] = chi[r], ++k;
        }
    }
    return k;
}

/* attend_head_ref (infer.rs:1871-2007) over the keys in `nr` ascending
 * position ranges [klo, khi), each key read from its KV slot (slot_of).
 * `nested` (a chunk's rows, infer/chunk.rs:263) drops the minimum chunk
 * count (infer.rs:1888).  The P.V sums are integers, so summing per key
 * gives the reference's per-run sums (infer.rs:1966-1985). */
static void attend_head(const nf_model* m, const nf_session* s, int l, const float* qh, int kvh, const size_t* klo,
                        const size_t* khi, int nr, int nested, float* out) {
    const nf_config* c = &m->c;
    const size_t qk = c->qk, vd = c->vd, nkv = c->nkv, cap = s->cap;
    int8_t q8[64];
    const float qs = cq_quant_i8(qh, qk, q8) * INV_SQRT_QK;
    size_t n = 0;
    for (int r = 0; r < nr; ++r) n += khi[r] - klo[r];
    size_t* slots = (size_t*)malloc((n ? n : 1) * sizeof(size_t));
    n = 0;
    for (int r = 0; r < nr; ++r)
        for (size_t p = klo[r]; p < khi[r]; ++p) slots[n++] = slot_of(p, s);
    size_t count, chunk;
    size_t kmin = 2 * NATIVE_TEAM / nkv;
    if (kmin < 1 || nested) kmin = 1;
    key_chunks_k(n, kmin, &count, &chunk);
    float* sc = (float*)malloc(chunk * sizeof(float));
    float* scale = (float*)malloc(chunk * sizeof(float));
    int32_t* dots = (int32_t*)malloc(chunk * sizeof(int32_t));
    int8_t* dig = (int8_t*)malloc(3 * chunk);
    float pm[8], psum[8], po[8][64];
    int np = 0;
    for (size_t c0 = 0; c0 < n; c0 += chunk) {
        const size_t len = chunk < n - c0 ? chunk : n - c0;
        const size_t blocked = len / 4 * 4;
        const size_t* sl = slots + c0;
        for (size_t i = 0; i < len; ++i) dots[i] = idot(q8, s->k8[l] + (sl[i] * nkv + kvh) * qk, qk);
        for (size_t i = 0; i < len; ++i) scale[i] = s->ks[l][sl[i] * nkv + kvh];
        for (size_t i = 0; i < blocked; ++i) sc[i] = (scale[i] * (float)dots[i]) * qs;
        for (size_t i = blocked; i < len; ++i) sc[i] = (scale[i] * qs) * (float)dots[i];
        float mx = -INFINITY;
        for (size_t i = 0; i < len; ++i) mx = fmaxf(mx, sc[i]);
        const float sum = nf_chunk_exp(sc, len, mx);
        for (size_t i = 0; i < len; ++i) scale[i] = s->vs[l][sl[i] * nkv + kvh];
        float wmax = 0.0f;
        for (size_t i = 0; i < len; ++i) {
            sc[i] *= scale[i];
            wmax = fmaxf(wmax, sc[i]);
        }
        const float qw = Q21 / wmax;
        int8_t *hi = dig, *mid = dig + chunk, *lo8 = dig + 2 * chunk;
        nf_digits21(sc, len, qw, hi, mid, lo8);
        const float cw = wmax * C21;
        for (size_t dm = 0; dm < vd; ++dm) {
            const int8_t* row = s->v8t[l] + ((size_t)kvh * vd + dm) * cap;
            int32_t a = 0, b = 0, cc = 0;
            for (size_t i = 0; i < len; ++i) {
                const int32_t v = row[sl[i]];
                a += (int32_t)hi[i] * v, b += (int32_t)mid[i] * v, cc += (int32_t)lo8[i] * v;
            }
            po[np][dm] = fmaf(16384.0f, (float)a, fmaf(128.0f, (float)b, (float)cc)) * cw;
        }
        pm[np] = mx;
        psum[np] = sum;
        ++np;
    }
    if (np == 1) {
        const float inv = 1.0f / psum[0];
        for (size_t i = 0; i < vd; ++i) out[i] = po[0][i] * inv;
    } else {
        float big = -1e30f;
        for (int p = 0; p < np; ++p) big = fmaxf(big, pm[p]);
        float acc[64] = {0}, total = 0.0f;
        for (int p = 0; p < np; ++p) {
            const float w = lexpf(pm[p] - big);
            for (size_t i = 0; i < vd; ++i) acc[i] = fmaf(po[p][i], w, acc[i]);
            total = fmaf(w, psum[p], total);
        }
        const float inv = 1.0f / total;
        for (size_t i = 0; i < vd; ++i) out[i] = acc[i] * inv;
    }
    free(sc), free(scale), free(dots), free(dig), free(slots);
}

/* The test hook for attend_head: one head against keys written straight
 * into layer 0's cache slots.  k8 [n][qk] / ks [n] / v8 [n][vd] / vs [n]
 * fill slots 0 .. n-1 of kv head 0; the query attends to positions
 * 0 .. n-1 (no attention span) in one chunk list as a step would. */
int nf_attend_test(const nf_model* m, nf_session* s, const int8_t* k8, const float* ks, const int8_t* v8,
                   const float* vs, size_t n, const float* q, int nested, float* out) {
    const nf_config* c = &m->c;
    if (n == 0 || n > s->cap) return -1;
    const size_t qk = c->qk, vd = c->vd, nkv = c->nkv;
    for (size_t i = 0; i < n; ++i) {
        memcpy(s->k8[0] + i * nkv * qk, k8 + i * qk, qk);
        s->ks[0][i * nkv] = ks[i];
        s->vs[0][i * nkv] = vs[i];
        for (size_t dm = 0; dm < vd; ++dm) s->v8t[0][dm * s->cap + i] = v8[i * vd + dm];
    }
    const size_t lo = 0, hi = n;
    attend_head(m, s, 0, q, 0, &lo, &hi, 1, nested, out);
    return 0;
}

/* The hashed engram rows of position `pos` (engram_native,
 * infer.rs:1256-1275): for order oi and head h, table tbl = oi * heads + h
 * takes row tbl * slots + (hash % slots), the hash seeded with
 * ENGRAM_SEED * (oi * stride + h + 1) and folded over the last `order`
 * tokens (token 0 before the start) with xor then * ENGRAM_PRIME, then
 * acc ^= acc >> 15; -1 where pos + 1 < order.  rows[16]. */
void nf_engram_rows(const nf_model* m, const uint32_t* tokens, size_t pos, long* rows) {
    const nf_config* c = &m->c;
    const int stride = c->seed_heads > 0 ? c->seed_heads : c->eheads;
    for (int k = 0; k < 16; ++k) rows[k] = -1;
    for (int oi = 0; oi < c->norders; ++oi)
        for (int h = 0; h < c->eheads; ++h) {
            const int order = c->orders[oi], tbl = oi * c->eheads + h;
            if (pos + 1 < (size_t)order) continue;
            uint32_t acc = ENGRAM_SEED * (uint32_t)(oi * stride + h + 1);
            for (int j = 0; j < order; ++j) {
                const uint32_t tk = pos >= (size_t)j ? tokens[pos - j] : 0;
                acc = (acc ^ tk) * ENGRAM_PRIME;
            }
            acc ^= acc >> 15;
            rows[tbl] = (long)tbl * c->engram_slots + (long)(acc % (uint32_t)c->engram_slots);
        }
}

/* The engram input row of position `pos` at one site: each hashed table
 * row (QMat::row) at its table's sub-width slot, zeros where no row
 * (infer.rs:1261-1275).  out[d]. */
void nf_engram_input(const nf_model* m, int site, const uint32_t* tokens, size_t pos, float* out) {
    const nf_config* c = &m->c;
    long rows[16];
    nf_engram_rows(m, tokens, pos, rows);
    memset(out, 0, sizeof(float) * c->d);
    for (int tbl = 0; tbl < c->norders * c->eheads; ++tbl)
        if (rows[tbl] >= 0) cq_qmat_row(m->etables[site], (size_t)rows[tbl], out + (size_t)tbl * c->engram_sub);
}

/* The mHC read of one row (infer.rs:1359-1393): the 4 lanes x[4d]
 * normalized by rinv over all of them, int8 with one scale, projected on
 * the Phi8 rows (p[k] = (sx * phi_s[k]) * idot), the pre gates
 * hp[j] = 1 / (lexpf(-z) + 1) with z = ((p[j] * a_pre) + (+4 own lane,
 * -4 others)) + b_pre[j], then u = x0 hp0 and fma(x_b, hp_b, u) for
 * b = 1..3.  Scratch nx[4d], nx8[4d]. */
void nf_mhc_read(const int8_t* phi_q, const float* phi_s, int ncols, int d, float a_pre, const float* b_pre, int lane,
                 const float* x, float* p, float* u, float* nx, int8_t* nx8) {
    const int nc = 4 * d;
    const float r = cq_rinv(cq_dot16(x, x, nc), nc);
    for (int k = 0; k < nc; ++k) nx[k] = x[k] * r;
    const float sx = cq_quant_scale(nx, nc);
    cq_quant_with(nx, nc, 1.0f / sx, nx8);
    for (int k = 0; k < ncols; ++k) p[k] = (sx * phi_s[k]) * (float)idot(phi_q + (size_t)k * nc, nx8, nc);
    float hp[4];
    for (int j = 0; j < 4; ++j) {
        const float off = j == lane ? 4.0f : -4.0f;
        const float zz = ((p[j] * a_pre) + off) + b_pre[j];
        hp[j] = 1.0f / (lexpf(-zz) + 1.0f);
    }
    for (int k = 0; k < d; ++k) u[k] = x[k] * hp[0];
    for (int b = 1; b < 4; ++b)
        for (int k = 0; k < d; ++k) u[k] = fmaf(x[b * d + k], hp[b], u[k]);
}

/* The post and residual gates of one row (infer.rs:1577-1583): hpost[j] =
 * 2 / (lexpf(-z) + 1) with z = ((p[4 + j] * a_post) + (0 own lane, -4
 * others)) + b_post[j]; zres[k] = fma(p[8 + k], a_res, b_res[k]) and
 * hres = sinkhorn64(zres). */
void nf_post_gates(const float* p, float a_post, const float* b_post, float a_res, const float* b_res, int lane,
                   float hpost[4], float hres[16]) {
    float zres[16];
    for (int j = 0; j < 4; ++j) {
        const float off = j == lane ? 0.0f : -4.0f;
        const float zz = ((p[4 + j] * a_post) + off) + b_post[j];
        hpost[j] = 2.0f / (lexpf(-zz) + 1.0f);
    }
    for (int k = 0; k < 16; ++k) zres[k] = fmaf(p[8 + k], a_res, b_res[k]);
    nf_sinkhorn64(zres, hres);
}

/* The mHC write of one row (infer.rs:1584-1605): lane a becomes
 * y hpost[a], then fma(old_b, hres[a * 4 + b], .) for b = 0..3, with the
 * lanes as they were before the write.  x[4d] in place. */
void nf_mhc_write(int d, const float* y, const float hpost[4], const float hres[16], float* x) {
    for (int ch = 0; ch < d; ++ch) {
        float old[4];
        for (int b = 0; b < 4; ++b) old[b] = x[b * d + ch];
        for (int a = 0; a < 4; ++a) {
            float v = y[ch] * hpost[a];
            for (int b = 0; b < 4; ++b) v = fmaf(old[b], hres[a * 4 + b], v);
            x[a * d + ch] = v;
        }
    }
}

/* Model::head_logits (infer.rs:1135-1141): the tied head over the final
 * normed hidden state h[d] with the decode combine, out_rows logits. */
void nf_head_logits(const nf_model* m, const float* h, float* logits, int nthreads) {
    cq_qact* a = cq_qact_new(h, 1, m->c.d, m->embedding->bits, 1);
    float* full = (float*)malloc(sizeof(float) * m->embedding->out);
    cq_matmul_into(m->embedding, a, full, m->embedding->out, 0, nthreads);
    memcpy(logits, full, sizeof(float) * m->c.out_rows);
    free(full);
    cq_qact_free(a);
}

/* Model::head_logits_sparse (infer.rs:1145-1166): NEG (infer.rs:36)
 * everywhere but the ids, scored with QMat::single_row.  0, or -1 for an id
 * past out_rows. */
int nf_head_logits_sparse(const nf_model* m, const float* h, const uint32_t* ids, size_t n, float* logits) {
    for (size_t i = 0; i < n; ++i)
        if (ids[i] >= (uint32_t)m->c.out_rows) return -1;
    cq_qact* a = cq_qact_new(h, 1, m->c.d, m->embedding->bits, 1);
    for (int i = 0; i < m->c.out_rows; ++i) logits[i] = bits_f(0xf149f2cau);
    for (size_t i = 0; i < n; ++i) logits[ids[i]] = cq_single_row(m->embedding, ids[i], a);
    cq_qact_free(a);
    return 0;
}

/* The rows p0 .. p0 + t - 1 of one feed: Model::step_native
 * (infer/step.rs:171-760) for t = 1, Model::chunk_job (infer/chunk.rs:32-358)
 * for a chunk of t > 1 tokens.  The two share the per-row arithmetic; a chunk
 * differs in its projections (the prefill combine over its t rows), its RoPE
 * rows (sincosf per position, rope_rows, infer.rs:1716-1747) and its
 * attention chunking (nested, infer.rs:1888).  `outputs` (NF_OUT_*) picks
 * what goes to `out` (chunk.rs:331-353, step.rs:715-729): logits [rows]
 * [out_rows] or hidden states [rows][d]; returns the rows written, or -1. */
/* The qkv conv of one row part (infer/step.rs:502-516): out[k] = w_0[k]
 * cur[k], then for taps j = 1 .. taps - 1, out[k] = fma(w_j[k], prev_j[k],
 * out[k]), where rows[j] is the part's pre-tap row of position pos - j, or
 * NULL when the history no longer holds it (a zero row: fma_w16s(.., 0.0)).
 * w is the tap tensor [taps][cw]. */
void nf_conv_taps(const float* const* rows, int taps, const uint16_t* w, int cw, float* out) {
    for (int k = 0; k < cw; ++k) out[k] = cq_f16_to_f32(w[k]) * rows[0][k];
    for (int j = 1; j < taps; ++j) {
        const uint16_t* wj = w + (size_t)j * cw;
        for (int k = 0; k < cw; ++k) out[k] = fmaf(cq_f16_to_f32(wj[k]), rows[j] ? rows[j][k] : 0.0f, out[k]);
    }
}

/* The engram conv of site e at pos (engram_native, infer.rs:1310-1325,
 * engram_tap 667-689): out[k] = sum over taps j < 4 with pos >= j dil of
 * fma(taps_j[k], vs[pos - j dil][k / 32] * v8[pos - j dil][k], out[k]), from
 * zero, over the session's int8 value history. */
void nf_engram_conv(const nf_model* m, const nf_session* s, int e, size_t pos, float* out) {
    const int d = m->c.d, dil = m->c.dilation;
    for (int k = 0; k < d; ++k) out[k] = 0.0f;
    for (int j = 0; j < ENGRAM_CONV_TAPS; ++j) {
        if (pos < (size_t)(j * dil)) break;
        const size_t pj = pos - (size_t)j * dil;
        const int8_t* q8 = s->ev8[e] + pj * d;
        const float* qs = s->evs[e] + pj * (d / 32);
        const float* tw = m->etaps[e] + (size_t)j * d;
        for (int k = 0; k < d; ++k) out[k] = fmaf(tw[k], qs[k / 32] * (float)q8[k], out[k]);
    }
}

/* The engram gate (infer.rs:1409-1412): alpha = 1 / (lexpf(-dot16(x r_x,
 * k r_k) / sqrtf(d)) + 1), r = rinv(dot16(v, v), d). */
float nf_engram_gate(const float* x, const float* k, int d) {
    const float rx = cq_rinv(cq_dot16(x, x, d), d), rk = cq_rinv(cq_dot16(k, k, d), d);
    float* ea = (float*)malloc(sizeof(float) * d);
    float* eb = (float*)malloc(sizeof(float) * d);
    for (int i = 0; i < d; ++i) ea[i] = x[i] * rx, eb[i] = k[i] * rk;
    const float alpha = 1.0f / (lexpf((-cq_dot16(ea, eb, d)) / sqrtf((float)d)) + 1.0f);
    free(ea), free(eb);
    return alpha;
}

/* The Hadamard MLP of layer l for one pre-MLP row h2[d] (mlp_native,
 * infer.rs:1610-1637): the conditioning weights, z = h2 d1 zero-padded,
 * t = kron(z, A0, B0) = A0^T Z B0 (kron_native 2322-2330 as two mix8
 * passes), cond = 1 + sum_k u_k w_k, z = fma(t[perm1], cond d2, b2), SiLU,
 * t = kron(z, A1, B1), z = t[perm2] d3, t = kron(z, A2, B2); mlp[j] =
 * t[j] d4[j] for j < d. */
void nf_hada_mlp(const nf_model* m, int l, const float* h2, float* mlp) {
    const struct nf_layer16* Lw = &m->L[l];
    const int d = m->c.d;
    float* z = (float*)malloc(sizeof(float) * HN);
    float* mt = (float*)malloc(sizeof(float) * HN);
    float* bt = (float*)malloc(sizeof(float) * HN);
    float* cond = (float*)malloc(sizeof(float) * HN);
    float* zs = (float*)malloc(sizeof(float) * HN);
    float* t3 = (float*)malloc(sizeof(float) * HN);
    float wk[8];
    nf_cond_weights(h2, d, Lw->cond_v, wk);
    for (int k = 0; k < d; ++k) z[k] = h2[k] * cq_f16_to_f32(Lw->d1[k]);
    for (int k = d; k < HN; ++k) z[k] = 0.0f;
    nf_mix8(1, Lw->kron[0], 1, z, 0, mt, 16);
    nf_mix8(0, mt, 0, Lw->kron[1], 1, bt, 16);
    for (int j = 0; j < HN; ++j) cond[j] = 1.0f;
    for (int k = 0; k < HADA_COND_RANK; ++k)
        for (int j = 0; j < HN; ++j) cond[j] = fmaf(cq_f16_to_f32(Lw->cond_u[(size_t)k * HN + j]), wk[k], cond[j]);
    for (int j = 0; j < HN; ++j)
        zs[j] = fmaf(bt[m->perm1[j]], cond[j] * cq_f16_to_f32(Lw->d2[j]), cq_f16_to_f32(Lw->b2[j]));
    for (int j = 0; j < HN; ++j) zs[j] /= nf_nexp(-zs[j]) + 1.0f;
    nf_mix8(1, Lw->kron[2], 1, zs, 0, mt, 16);
    nf_mix8(0, mt, 0, Lw->kron[3], 1, bt, 16);
    for (int j = 0; j < HN; ++j) zs[j] = bt[m->perm2[j]] * cq_f16_to_f32(Lw->d3[j]);
    nf_mix8(1, Lw->kron[4], 1, zs, 0, mt, 16);
    nf_mix8(0, mt, 0, Lw->kron[5], 1, t3, d / NB / 8 * 4);
    for (int j = 0; j < d; ++j) mlp[j] = t3[j] * cq_f16_to_f32(Lw->d4[j]);
    free(z), free(mt), free(bt), free(cond), free(zs), free(t3);
}

/* RoPE rows (rope_rows, infer.rs:1716-1747) for positions p0 .. p0 + t - 1
 * into cs / sn [t][32]: for a single token right after the newest known
 * row (c0, s0: its cos and sin, or NULL) the angle-addition recurrence
 * cos = fma(-sd, s0, cd c0), sin = fma(sd, c0, cd s0); else sincosf(freq
 * (p0 + i)) with the product in f32. */
void nf_rope_rows(const nf_model* m, size_t p0, size_t t, const float* c0, const float* s0, float* cs, float* sn) {
    const int half = m->c.qk / 2;
    if (t == 1 && c0 && s0) {
        for (int f = 0; f < half; ++f) {
            cs[f] = fmaf(-m->sd[f], s0[f], m->cd[f] * c0[f]);
            sn[f] = fmaf(m->sd[f], c0[f], m->cd[f] * s0[f]);
        }
    } else {
        for (size_t i = 0; i < t; ++i)
            for (int f = 0; f < half; ++f) lsincosf(m->freq[f] * (float)(p0 + i), &sn[i * 32 + f], &cs[i * 32 + f]);
    }
}

/* The RoPE tables (Tables::new, infer.rs:942-947) into freq, sd, cd [qk/2]. */
void nf_rope_tables(const nf_model* m, float* freq, float* sd, float* cd) {
    const int half = m->c.qk / 2;
    memcpy(freq, m->freq, half * sizeof(float));
    memcpy(sd, m->sd, half * sizeof(float));
    memcpy(cd, m->cd, half * sizeof(float));
}

/* Read-only views of a session for the checks: the RoPE row of a position
 * fed; the KV slot contents of a layer (k8 [nkv][qk], ks [nkv], v8
 * [nkv][vd], vs [nkv]); the int8 engram value history of a site at a
 * position (v8 [d], vs [d / 32]).  0, or -1 out of range. */
int nf_session_rope(const nf_session* s, size_t pos, float* c, float* sn, int half) {
    if (pos >= s->len) return -1;
    memcpy(c, s->rope_c + pos * 32, half * sizeof(float));
    memcpy(sn, s->rope_s + pos * 32, half * sizeof(float));
    return 0;
}

int nf_session_kv(const nf_model* m, const nf_session* s, int l, size_t slot, int8_t* k8, float* ks, int8_t* v8,
                  float* vs) {
    const nf_config* c = &m->c;
    if (l < 0 || l >= c->layers || slot >= s->cap) return -1;
    memcpy(k8, s->k8[l] + slot * c->nkv * c->qk, (size_t)c->nkv * c->qk);
    memcpy(ks, s->ks[l] + slot * c->nkv, (size_t)c->nkv * sizeof(float));
    memcpy(vs, s->vs[l] + slot * c->nkv, (size_t)c->nkv * sizeof(float));
    for (int h = 0; h < c->nkv; ++h)
        for (int i = 0; i < c->vd; ++i) v8[h * c->vd + i] = s->v8t[l][((size_t)h * c->vd + i) * s->cap + slot];
    return 0;
}

int nf_session_engram_hist(const nf_model* m, const nf_session* s, int e, size_t pos, int8_t* v8, float* vs) {
    const int d = m->c.d;
    if (e < 0 || e >= m->c.sites || pos >= s->len) return -1;
    memcpy(v8, s->ev8[e] + pos * d, d);
    memcpy(vs, s->evs[e] + pos * (d / 32), (d / 32) * sizeof(float));
    return 0;
}

/* One feed of t tokens (step_native for one, chunk_job for a chunk).
 * `cells` (or NULL): the feed's cells [t][L+1][d], the lane mean
 * (((x0 + x1) + x2) + x3) * 0.25 of every row after the embedding and after
 * each layer's mHC write (step.rs:240-243,672-714; chunk.rs:69-70,310;
 * lane_mean, infer.rs:1707-1711). */
static int nf_rows(const nf_model* m, nf_session* s, const uint32_t* toks, size_t t, int outputs, float* outbuf,
                   float* cells, int nthreads) {
    const nf_config* c = &m->c;
    const int n = c->lanes, d = c->d, nc = n * d, L = c->layers;
    const int qk = c->qk, vd = c->vd, nh = c->nh, nkv = c->nkv;
    const int qd = nh * qk, kd = nkv * qk, vdim = nkv * vd, W = qd + kd + vdim, taps = c->taps;
    const int group = nh / nkv, sites = c->sites;
    const size_t p0 = s->len;
    int rc = 0;
    if (t == 0 || p0 + t > s->cap || n != 4 || qk > 64 || vd > 64 || c->norders * c->eheads > 16 || L > 64 ||
        taps > NF_MAX_TAPS)
        return -1;
    const int nested = t > 1;
    for (size_t i = 0; i < t; ++i) s->tokens[p0 + i] = toks[i];
    s->len = p0 + t;
    /* the slot map with this feed's positions, and its snapshot
     * (step.rs:193,229-231, chunk.rs:54,81) */
    mark_slots(s, p0, p0 + t);
    int64_t* sp = (int64_t*)dupb(s->slot_pos, s->nslot * 8);
    const size_t nsp = s->nslot;
    /* the first position LayerState::hist still holds */
    const size_t hist_lo = p0 - s->hrows;

    /* embedding row * sqrt(d) into every lane (step.rs:228-235, chunk.rs:58-66) */
    float* xs = (float*)malloc(sizeof(float) * t * nc);
    float* row = (float*)malloc(sizeof(float) * d);
    const float scale = sqrtf((float)d);
    for (size_t i = 0; i < t; ++i) {
        cq_qmat_row(m->embedding, toks[i], row);
        for (int lane = 0; lane < n; ++lane)
            for (int k = 0; k < d; ++k) xs[i * nc + lane * d + k] = row[k] * scale;
    }
    const size_t depths = (size_t)L + 1;
#define NF_CELLS(depth)                                                                                  \
    if (cells)                                                                                           \
        for (size_t i = 0; i < t; ++i) {                                                                 \
            const float* x = xs + i * nc;                                                                \
            float* cr = cells + (i * depths + (depth)) * d;                                              \
            for (int ch = 0; ch < d; ++ch) cr[ch] = (((x[ch] + x[d + ch]) + x[2 * d + ch]) + x[3 * d + ch]) * 0.25f; \
        }
    NF_CELLS(0)

    /* engram rows and their key|value products over the t rows, value
     * history and conv (engram_native, infer.rs:1244-1335) */
    const int norders = c->norders, eheads = c->eheads, ntab = norders * eheads, sub = c->engram_sub;
    float* ekv = (float*)calloc((size_t)sites * t * 2 * d + 1, sizeof(float));
    float* evals = (float*)calloc((size_t)sites * t * d + 1, sizeof(float));
    if (sites > 0) {
        long* erow = (long*)malloc(sizeof(long) * t * 16);
        for (size_t i = 0; i < t; ++i) nf_engram_rows(m, s->tokens, p0 + i, erow + i * 16);
        float* er = (float*)malloc(sizeof(float) * t * d);
        float* trow = (float*)malloc(sizeof(float) * sub);
        for (int e = 0; e < sites; ++e) {
            memset(er, 0, sizeof(float) * t * d);
            for (size_t i = 0; i < t; ++i)
                for (int tbl = 0; tbl < ntab; ++tbl)
                    if (erow[i * 16 + tbl] >= 0) {
                        cq_qmat_row(m->etables[e], (size_t)erow[i * 16 + tbl], trow);
                        memcpy(er + i * d + tbl * sub, trow, sizeof(float) * sub);
                    }
            cq_qact* a = cq_qact_new(er, t, d, m->ekv[e]->parts[0]->bits, 1);
            float* kv = ekv + (size_t)e * t * 2 * d;
            cq_qlinear_matmul(m->ekv[e], a, kv, nthreads);
            cq_qact_free(a);
            /* int8 value history, groups of 32 */
            for (size_t i = 0; i < t; ++i)
                for (int g = 0; g < d / 32; ++g)
                    s->evs[e][(p0 + i) * (d / 32) + g] =
                        cq_quant_i8(kv + i * 2 * d + d + g * 32, 32, s->ev8[e] + (p0 + i) * d + g * 32);
        }
        free(er), free(trow), free(erow);
        for (int e = 0; e < sites; ++e)
            for (size_t i = 0; i < t; ++i) nf_engram_conv(m, s, e, p0 + i, evals + ((size_t)e * t + i) * d);
    }

    /* RoPE rows (rope_rows, infer.rs:1716-1747): the recurrence for a single
     * token right after the newest known position, sincosf otherwise. */
    float* cs = s->rope_c + p0 * 32;
    float* sn = s->rope_s + p0 * 32;
    /* with a RoPE list, it ends at position p0 - 1 */
    const int prev = t == 1 && s->rope_n > 0;
    nf_rope_rows(m, p0, t, prev ? s->rope_c + (p0 - 1) * 32 : NULL, prev ? s->rope_s + (p0 - 1) * 32 : NULL, cs, sn);
    /* push the rows, then trim to ROLLBACK + 1 past twice that */
    s->rope_n += t;
    if (s->rope_n > 2 * (NF_ROLLBACK + 1)) s->rope_n = NF_ROLLBACK + 1;

    const int nq = W + nh * vd;  /* the fused projection: q | k | v | gate */
    const int ncols = 2 * n + n * n;
    float* nx = (float*)malloc(sizeof(float) * nc);
    int8_t* nx8 = (int8_t*)malloc(nc);
    float *u = (float*)malloc(sizeof(float) * t * d), *x1 = (float*)malloc(sizeof(float) * t * d);
    float* p = (float*)malloc(sizeof(float) * t * ncols);
    float *hloc = (float*)malloc(sizeof(float) * t * d), *proj = (float*)malloc(sizeof(float) * t * nq);
    float *qkv = (float*)malloc(sizeof(float) * t * W), *att = (float*)malloc(sizeof(float) * t * nh * vd);
    float *o = (float*)malloc(sizeof(float) * t * d), *on = (float*)malloc(sizeof(float) * d);
    float *x2 = (float*)malloc(sizeof(float) * d), *h2 = (float*)malloc(sizeof(float) * d);
    float *z = (float*)malloc(sizeof(float) * d), *t3 = (float*)malloc(sizeof(float) * d);

    for (int l = 0; l < L; ++l) {
        const struct nf_layer16* Lw = &m->L[l];
        const int lane = l % n;
        const int site = l < 64 ? m->site_of_layer[l] : -1;
        /* (a) mHC read, (b) engram gate, (c) input norm, per row */
        for (size_t i = 0; i < t; ++i) {
            const float* x = xs + i * nc;
            float* pr = p + i * ncols;
            float* ur = u + i * d;
            float* xr = x1 + i * d;
            nf_mhc_read(Lw->phi_q, Lw->phi_s, ncols, d, Lw->a_pre, Lw->b_pre, lane, x, pr, ur, nx, nx8);
            memcpy(xr, ur, sizeof(float) * d);
            if (site >= 0) {
                const float* kr = ekv + ((size_t)site * t + i) * 2 * d;  /* the key half */
                const float alpha = nf_engram_gate(xr, kr, d);
                const float* ev = evals + ((size_t)site * t + i) * d;
                for (int k = 0; k < d; ++k) xr[k] = fmaf(ev[k], alpha, xr[k]);
            }
            const float rh = cq_rinv(cq_dot16(xr, xr, d), d);
            cq_norm_apply16(hloc + i * d, xr, rh, Lw->norm_in, d);
        }
        /* (d) A8 of the rows and q|k|v|gate over all of them */
        {
            cq_qact* a = cq_qact_new(hloc, t, d, m->qkvg[l]->parts[0]->bits, 1);
            cq_qlinear_matmul(m->qkvg[l], a, proj, nthreads);
            cq_qact_free(a);
        }
        /* (e)-(g) the rows' pre-tap history, then per row the conv taps,
         * head norms, RoPE and the KV cache */
        float* hist = s->hist[l];
        for (size_t i = 0; i < t; ++i) memcpy(hist + (p0 + i) * (size_t)W, proj + i * nq, sizeof(float) * W);
        for (size_t i = 0; i < t; ++i) {
            const size_t pos = p0 + i;
            float* out = qkv + i * W;
            for (int part = 0; part < 3; ++part) {
                const int start = part == 0 ? 0 : part == 1 ? qd : qd + kd;
                const int cw = part == 0 ? qd : part == 1 ? kd : vdim;
                const uint16_t* w = part == 0 ? Lw->q_taps : part == 1 ? Lw->k_taps : Lw->v_taps;
                /* tap j reads the row of position pos - j while the history holds it */
                const float* rows[NF_MAX_TAPS];
                for (int j = 0; j < taps; ++j)
                    rows[j] = (j == 0 || pos >= hist_lo + (size_t)j) ? hist + (pos - j) * (size_t)W + start : NULL;
                nf_conv_taps(rows, taps, w, cw, out + start);
            }
            for (int hh = 0; hh < nh + nkv; ++hh) {
                float* v = out + (hh < nh ? hh * qk : qd + (hh - nh) * qk);
                zcn16_inplace(v, hh < nh ? Lw->q_norm : Lw->k_norm, qk);
                nf_rope_rotate(v, qk, cs + i * 32, sn + i * 32);
            }
            const size_t slot = slot_of(pos, s);
            for (int kvh = 0; kvh < nkv; ++kvh) {
                s->ks[l][slot * nkv + kvh] = cq_quant_i8(out + qd + kvh * qk, qk, s->k8[l] + (slot * nkv + kvh) * qk);
                int8_t vq[64];
                s->vs[l][slot * nkv + kvh] = cq_quant_i8(out + qd + kd + kvh * vd, vd, vq);
                for (int dm = 0; dm < vd; ++dm) s->v8t[l][((size_t)kvh * vd + dm) * s->cap + slot] = vq[dm];
            }
        }
        /* (h) attention per (row, head), (i) its gate, (j) A8 and out */
        {
            const int window = (c->sliding_window > 0 && !((c->global_mask >> l) & 1)) ? c->sliding_window : 0;
            for (size_t i = 0; i < t; ++i) {
                const size_t pos = p0 + i;
                size_t klo[NF_KEY_RUNS], khi[NF_KEY_RUNS];
                const int nr = key_ranges(pos, p0 + t, (size_t)window, s, sp, nsp, klo, khi);
                if (nr < 0) {
                    rc = -1;
                    goto done;
                }
                for (int hh = 0; hh < nh; ++hh) {
                    float* ah = att + (i * nh + hh) * vd;
                    attend_head(m, s, l, qkv + i * W + hh * qk, hh / group, klo, khi, nr, nested, ah);
                    const float* gate = proj + i * nq + W + hh * vd;
                    for (int k = 0; k < vd; ++k) ah[k] /= nf_nexp(-gate[k]) + 1.0f;
                }
            }
            cq_qact* a = cq_qact_new(att, t, nh * vd, m->out[l]->parts[0]->bits, 1);
            cq_qlinear_matmul(m->out[l], a, o, nthreads);
            cq_qact_free(a);
        }
        /* (k) post block and the Hadamard MLP, the post and residual gates,
         * the mHC write, per row */
        const float ga = 1.0f / (lexpf(-Lw->attn_gate) + 1.0f);
        for (size_t i = 0; i < t; ++i) {
            const float* pr = p + i * ncols;
            float* x = xs + i * nc;
            cq_zcn16(o + i * d, Lw->post_norm, d, on);
            for (int k = 0; k < d; ++k) x2[k] = fmaf(on[k], ga, x1[i * d + k]);
            cq_zcn16(x2, Lw->pre_hada, d, h2);
            nf_hada_mlp(m, l, h2, t3);
            float hpost[4], hres[16];
            nf_post_gates(pr, Lw->a_post, Lw->b_post, Lw->a_res, Lw->b_res, lane, hpost, hres);
            /* y = (x2 + mlp) - u (step.rs:675-681) */
            for (int ch = 0; ch < d; ++ch) z[ch] = (x2[ch] + t3[ch]) - u[i * d + ch];
            nf_mhc_write(d, z, hpost, hres, x);
        }
        NF_CELLS((size_t)l + 1)
    }
#undef NF_CELLS

    /* the history rows this feed wrote, then the trim (chunk.rs:319-329,
     * step.rs:706-712) */
    {
        const size_t keep = (size_t)taps - 1 + NF_ROLLBACK;
        s->hrows += t;
        if (s->hrows > 2 * keep) s->hrows = keep;
    }
    /* outputs: lane mean, final norm, tied head per chosen row
     * (chunk.rs:331-353, step.rs:715-729); last_hidden is the last chosen
     * row's normed state */
    {
        const size_t first = (outputs == NF_OUT_ALL_LOGITS || outputs == NF_OUT_HIDDEN) ? 0 : t - 1;
        const size_t nrows = outputs == NF_OUT_NONE ? 0 : t - first;
        float* mean = (float*)malloc(sizeof(float) * d);
        for (size_t r = 0; r < nrows; ++r) {
            const float* x = xs + (first + r) * nc;
            for (int ch = 0; ch < d; ++ch) mean[ch] = (((x[ch] + x[d + ch]) + x[2 * d + ch]) + x[3 * d + ch]) * 0.25f;
            zcn(mean, m->final_norm, d, s->last_hidden);
            s->have_hidden = 1;
            if (!outbuf) continue;
            if (outputs == NF_OUT_HIDDEN || outputs == NF_OUT_LAST_HIDDEN)
                memcpy(outbuf + r * d, s->last_hidden, sizeof(float) * d);
            else
                nf_head_logits(m, s->last_hidden, outbuf + r * c->out_rows, nthreads);
        }
        free(mean);
        rc = (int)nrows;
    }
done:
    free(sp);
    free(xs), free(row), free(ekv), free(evals), free(nx), free(nx8), free(u), free(x1), free(p);
    free(hloc), free(proj), free(qkv), free(att), free(o), free(on), free(x2), free(h2), free(z), free(t3);
    return rc;
}

int nf_step(const nf_model* m, nf_session* s, uint32_t tok, float* logits, int nthreads) {
    const int r = nf_rows(m, s, &tok, 1, logits ? NF_OUT_LAST_LOGITS : NF_OUT_NONE, logits, NULL, nthreads);
    return r < 0 ? -1 : 0;
}

int nf_chunk(const nf_model* m, nf_session* s, const uint32_t* toks, size_t t, float* logits, int nthreads) {
    const int r = nf_rows(m, s, toks, t, logits ? NF_OUT_LAST_LOGITS : NF_OUT_NONE, logits, NULL, nthreads);
    return r < 0 ? -1 : 0;
}

/* Model::forward_native (infer.rs:1105-1132): chunks of 32, a one-token
 * chunk as a step; LastLogits / LastHidden only from the last chunk.
 * want_cells: the cells are computed (into `cells` [n][L+1][d] when not
 * NULL, and appended to a tracking session's store, step.rs:730-732,
 * chunk.rs:353-355).  A ring shorter than 32 with a chunk longer than it is
 * refused (nf_session_set_attend).  Returns the rows written to `out`, or -1. */
static int forward_native(const nf_model* m, nf_session* s, const uint32_t* toks, size_t n, int outputs, float* out,
                          int want_cells, float* cells, int nthreads) {
    if (outputs < NF_OUT_NONE || outputs > NF_OUT_LAST_HIDDEN || s->len + n > s->cap) return -1;
    if (s->ring > 0 && s->ring < 32 && n > s->ring) return -1;
    const size_t width = (outputs == NF_OUT_HIDDEN || outputs == NF_OUT_LAST_HIDDEN) ? (size_t)m->c.d
                                                                                    : (size_t)m->c.out_rows;
    const size_t cw = (size_t)(m->c.layers + 1) * m->c.d;
    float* tmp = want_cells ? (float*)malloc(32 * cw * sizeof(float)) : NULL;
    int rows = 0;
    for (size_t i = 0; i < n; i += 32) {
        const size_t t = n - i < 32 ? n - i : 32;
        const int last = i + t == n;
        const int want = (!last && (outputs == NF_OUT_LAST_LOGITS || outputs == NF_OUT_LAST_HIDDEN)) ? NF_OUT_NONE
                                                                                                       : outputs;
        const int r = nf_rows(m, s, toks + i, t, want, out ? out + (size_t)rows * width : NULL, tmp, nthreads);
        if (r < 0) {
            free(tmp);
            return -1;
        }
        if (tmp && cells) memcpy(cells + i * cw, tmp, t * cw * sizeof(float));
        if (tmp && s->track_cells) {
            memcpy(s->cells + s->ncells * cw, tmp, t * cw * sizeof(float));
            s->ncells += t;
        }
        rows += r;
    }
    free(tmp);
    return rows;
}

/* Model::forward (model.rs:304-306): cells when the session tracks them. */
int nf_forward(const nf_model* m, nf_session* s, const uint32_t* toks, size_t n, int outputs, float* out, int nthreads) {
    return forward_native(m, s, toks, n, outputs, out, s->track_cells, NULL, nthreads);
}

/* Model::forward_cells (model.rs:330-345): as nf_forward, with the feed's
 * cells [n][L+1][d] in `cells`. */
int nf_forward_cells(const nf_model* m, nf_session* s, const uint32_t* toks, size_t n, int outputs, float* out,
                     float* cells, int nthreads) {
    return forward_native(m, s, toks, n, outputs, out, 1, cells, nthreads);
}

/* Model::prefill_native (infer.rs:1078-1101): with an attention span and
 * a slot map, the first position in max(end - ring, sink) .. len whose
 * slot another position holds now starts a re-feed with the conv history
 * zeroed (rewind_zeroed, which also truncates tracked cells); else
 * forward_native.  Either way forward_native runs with want_cells = false,
 * so a prefill appends no cells to a tracking session. */
int nf_prefill(const nf_model* m, nf_session* s, const uint32_t* toks, size_t n, int outputs, float* out, int nthreads) {
    const size_t pos = s->len, end = pos + n;
    if (s->ring > 0 && s->nslot > 0) {
        size_t lo = end > s->ring ? end - s->ring : 0;
        if (lo < s->sink) lo = s->sink;
        for (size_t p = lo; p < pos; ++p) {
            const size_t sl = slot_of(p, s);
            if (sl < s->nslot && s->slot_pos[sl] == (int64_t)p) continue;
            const size_t k = pos - p;
            if (end > s->cap) return -1;
            uint32_t* refeed = (uint32_t*)malloc((k + n + 1) * 4);
            memcpy(refeed, s->tokens + p, k * 4);
            if (n) memcpy(refeed + k, toks, n * 4);
            if (s->ring < 32 && k + n > s->ring) {
                free(refeed);
                return -1;
            }
            nf_session_rewind_zeroed(m, s, p);
            const int r = forward_native(m, s, refeed, k + n, outputs, out, 0, NULL, nthreads);
            free(refeed);
            return r;
        }
    }
    return forward_native(m, s, toks, n, outputs, out, 0, NULL, nthreads);
}
