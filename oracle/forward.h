/* The Needle-3 decode step on the CPU (forward.c): test infrastructure. */
#ifndef NEEDLE_FORWARD_ORACLE_H
#define NEEDLE_FORWARD_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "cq_oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The geometry step_native reads (crates/needle-core/src/config.rs). */
typedef struct nf_config {
    int d, nh, nkv, qk, vd, layers, lanes, taps;
    int out_rows;
    int sliding_window;
    uint64_t global_mask;
    int sites, site_layers[16];
    int norders, orders[4], eheads, seed_heads, engram_slots, engram_sub, dilation;
    float rope_theta;
} nf_config;

/* Small per-layer tensors (f16 as the archive stores them). */
enum {
    NF_KRON0 = 0, NF_KRON1, NF_KRON2, NF_KRON3, NF_KRON4, NF_KRON5,
    NF_COND_V, NF_COND_U, NF_D1, NF_D2, NF_B2, NF_D3, NF_D4,
    NF_NORM_IN, NF_POST_NORM, NF_PRE_HADA, NF_Q_TAPS, NF_K_TAPS, NF_V_TAPS, NF_Q_NORM, NF_K_NORM
};

typedef struct nf_model nf_model;
typedef struct nf_session nf_session;

nf_model* nf_model_new(const nf_config* c);
void nf_model_free(nf_model* m);
void nf_set_layer_f16(nf_model* m, int l, int which, const uint16_t* v, size_t n);
void nf_set_layer_scalars(nf_model* m, int l, float a_pre, float a_post, float a_res, float attn_gate,
                          const float* b_pre, const float* b_post, const float* b_res);
void nf_set_phi(nf_model* m, int l, const float* w, size_t rows, size_t width);
void nf_set_matrices(nf_model* m, const cq_qmat* embedding, const cq_qlinear* const* qkvg, const cq_qlinear* const* out,
                     const cq_qmat* const* etables, const cq_qlinear* const* ekv);
void nf_set_engram_taps(nf_model* m, int site, const float* taps, size_t n);
void nf_set_globals(nf_model* m, const float* final_norm, const int32_t* perm1, const int32_t* perm2);

nf_session* nf_session_new(const nf_model* m, size_t cap);
void nf_session_free(const nf_model* m, nf_session* s);
size_t nf_session_len(const nf_session* s);
/* Outputs (crates/needle-engine/src/model.rs:150-160). */
#define NF_OUT_NONE 0
#define NF_OUT_LAST_LOGITS 1
#define NF_OUT_ALL_LOGITS 2
#define NF_OUT_HIDDEN 3
#define NF_OUT_LAST_HIDDEN 4

nf_session* nf_session_clone(const nf_model* m, const nf_session* s);
int nf_session_set_attend(nf_session* s, size_t sink, size_t ring);
int nf_session_rollback(const nf_model* m, nf_session* s, size_t n);
int nf_session_rewind_zeroed(const nf_model* m, nf_session* s, size_t len);
int nf_session_last_hidden(const nf_model* m, const nf_session* s, float* out);
/* Model::forward / Model::prefill on the native path: rows written or -1. */
int nf_forward(const nf_model* m, nf_session* s, const uint32_t* toks, size_t n, int outputs, float* out, int nthreads);
int nf_prefill(const nf_model* m, nf_session* s, const uint32_t* toks, size_t n, int outputs, float* out, int nthreads);
/* Model::forward_cells (model.rs:330-345): also the feed's cells [n][L+1][d]. */
int nf_forward_cells(const nf_model* m, nf_session* s, const uint32_t* toks, size_t n, int outputs, float* out,
                     float* cells, int nthreads);
/* Session::cells = Some(vec![]) / None (at an empty session); the tracked rows. */
int nf_session_track_cells(const nf_model* m, nf_session* s, int on);
int nf_session_cells(const nf_model* m, const nf_session* s, size_t row0, size_t n, float* dst);
void nf_head_logits(const nf_model* m, const float* h, float* logits, int nthreads);
int nf_head_logits_sparse(const nf_model* m, const float* h, const uint32_t* ids, size_t n, float* logits);
int nf_attend_test(const nf_model* m, nf_session* s, const int8_t* k8, const float* ks, const int8_t* v8,
                   const float* vs, size_t n, const float* q, int nested, float* out);
/* One decode step (step_native); logits [out_rows] (NULL: none).  0 or -1. */
int nf_step(const nf_model* m, nf_session* s, uint32_t tok, float* logits, int nthreads);
/* One prompt chunk of t <= 32 tokens (chunk_job; a single token is a step);
 * logits of its last row.  0 or -1. */
int nf_chunk(const nf_model* m, nf_session* s, const uint32_t* toks, size_t t, float* logits, int nthreads);

/* Helpers, exposed for their own checks. */
void nf_conv_taps(const float* const* rows, int taps, const uint16_t* w, int cw, float* out);
void nf_engram_conv(const nf_model* m, const nf_session* s, int e, size_t pos, float* out);
float nf_engram_gate(const float* x, const float* k, int d);
void nf_hada_mlp(const nf_model* m, int l, const float* h2, float* mlp);
void nf_rope_rows(const nf_model* m, size_t p0, size_t t, const float* c0, const float* s0, float* cs, float* sn);
void nf_rope_tables(const nf_model* m, float* freq, float* sd, float* cd);
int nf_session_rope(const nf_session* s, size_t pos, float* c, float* sn, int half);
int nf_session_kv(const nf_model* m, const nf_session* s, int l, size_t slot, int8_t* k8, float* ks, int8_t* v8,
                  float* vs);
int nf_session_engram_hist(const nf_model* m, const nf_session* s, int e, size_t pos, int8_t* v8, float* vs);
void nf_engram_rows(const nf_model* m, const uint32_t* tokens, size_t pos, long* rows);
void nf_engram_input(const nf_model* m, int site, const uint32_t* tokens, size_t pos, float* out);
void nf_mhc_read(const int8_t* phi_q, const float* phi_s, int ncols, int d, float a_pre, const float* b_pre, int lane,
                 const float* x, float* p, float* u, float* nx, int8_t* nx8);
void nf_post_gates(const float* p, float a_post, const float* b_post, float a_res, const float* b_res, int lane,
                   float hpost[4], float hres[16]);
void nf_mhc_write(int d, const float* y, const float hpost[4], const float hres[16], float* x);
float nf_nexp(float x);
void nf_rope_rotate(float* x, size_t n, const float* cs, const float* sn);
void nf_cond_weights(const float* h2, size_t d, const uint16_t* cond_v, float out[8]);
void nf_mix8(int transpose, const void* ct, int ct_half, const void* rows, int rows_half, float* out, int tiles);
void nf_sinkhorn64(const float z[16], float out[16]);
float nf_chunk_exp(float* s, size_t l, float m);
void nf_digits21(const float* w, size_t n, float qw, int8_t* hi, int8_t* mid, int8_t* lo);
void nf_key_chunks(size_t n, size_t nkv, size_t* count, size_t* size);

#ifdef __cplusplus
}
#endif
#endif
