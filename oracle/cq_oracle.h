/*
 * cq_oracle.h -- CPU restatement of needle-rs's packed CQ runtime.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity oracle (and, timed on the
 * host cores, the CPU baseline).  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product library
 * (needle-rs_amd/) never links or calls it.
 *
 * Every function restates one reference function in the same loop order
 * and float-operation order; the citation in each comment is the
 * reference file:line it follows.  Built with -ffp-contract=off: Rust never
 * contracts a*b+c, and fmaf() is used exactly where Rust calls mul_add.
 *
 * Parity pins (what checks each part; see tests/test_oracle_*.py):
 *   codebook / int8 codebook  closed-form KAT (cb8 table, cbs bits)
 *   fwht / rotate             dense Sylvester Hadamard product, n = 16..128
 *   nearest                   the reference's tie cases + brute force
 *   pack_lsb / unpack         round trips (4-bit, 3-bit, 2-bit)
 *   lane_sums                 brute-force integer sums from unpacked codes
 *   decode / prefill combine  reference tests restated (out 37, in 384,
 *                             rows {2,3,5,9,13,17}; the 2-bit matrix) plus
 *                             the tolerance invariant against cq_unpack
 *   threefry / normal         Random123 KAT, JAX split/normal values
 *   numpy streams             SeedSequence words, permutation KATs
 *   f16 conversion            numpy float16 (IEEE RNE), exhaustive f16 set
 *   dot16 / rinv / zcn16      scalar-order restatement vs float64 bound
 */
#ifndef CQ_ORACLE_H
#define CQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CQ_GROUP 128
#define CQ_TERNARY_RECORD_BITS 5

/* ---- scalars ---------------------------------------------------------- */
uint16_t cq_f32_to_f16(float f);
float cq_f16_to_f32(uint16_t h);
float cq_k127(void);
float cq_neg(void);

/* ---- quant.rs --------------------------------------------------------- */
int cq_lloyd_max(uint32_t bits, double* out);
int cq_codebook(uint32_t bits, size_t group, float* out);
float cq_hadamard_scale(size_t n);
void cq_hadamard(size_t n, float* out);
void cq_fwht(float* x, size_t n);
void cq_rotate(float* x, size_t n);
size_t cq_nearest(float x, const float* cb, size_t ncb);
size_t cq_pack_lsb(const uint8_t* idx, size_t n, uint32_t bits, uint8_t* out);
void cq_unpack_lsb_into(const uint8_t* packed, size_t npacked, uint32_t bits, uint8_t* out, size_t nout);
size_t cq_packed_row_bytes(size_t in_pad, uint32_t bits);
void cq_pack(const float* w, size_t rows, size_t d, uint32_t bits, size_t group, uint8_t* packed,
             uint16_t* norms, int nthreads);
void cq_unpack(const uint8_t* packed, const uint16_t* norms, size_t out, size_t in_dim, uint32_t bits,
               size_t group, float* w);

/* ---- qlinear.rs ------------------------------------------------------- */
float cq_quant_i8(const float* x, size_t n, int8_t* q);
float cq_quant_scale(const float* x, size_t n);
void cq_quant_with(const float* x, size_t n, float inv, int8_t* q);
size_t cq_act_pos(size_t p, uint8_t bits);
float cq_prep_group(const float* x, size_t len, size_t g, int8_t* q, uint8_t bits);
void cq_int8_codebook(const float* cb, size_t n, int8_t* cb8, float* scale);

typedef struct cq_qact {
    size_t rows, groups;
    uint8_t bits;
    int8_t* xq; /* [rows][groups][128], act_pos layout */
    float* sx;  /* [rows][groups] */
} cq_qact;

cq_qact* cq_qact_new(const float* x, size_t rows, size_t in_dim, uint8_t bits, int nthreads);
cq_qact* cq_qact_empty_rows(size_t rows, size_t in_dim, uint8_t bits);
void cq_qact_free(cq_qact* a);

typedef struct cq_qmat {
    size_t out, in_dim, groups;
    uint8_t bits;
    uint8_t* codes;  /* out * groups * bytes_per_group, archive layout */
    uint16_t* norms; /* [out][groups] f16 bits */
    int8_t tables[2][16];
    int8_t vals[16];
    float cbs;
    float fvals[16];
} cq_qmat;

cq_qmat* cq_qmat_build(size_t out, size_t in_dim, uint8_t bits, const float* cb, size_t ncb, int ternary,
                       const uint8_t* codes, const uint16_t* norms);
cq_qmat* cq_qmat_from_cq(const uint8_t* packed, const uint16_t* norms, size_t out, size_t in_dim, uint32_t bits,
                         size_t group);
cq_qmat* cq_qmat_from_f32(const float* w, size_t out, size_t in_dim, int nthreads);
void cq_qmat_free(cq_qmat* q);
size_t cq_qmat_bytes(const cq_qmat* q);
void cq_qmat_row(const cq_qmat* q, size_t r, float* out);
void cq_lane_sums(const cq_qmat* q, size_t r, size_t g, const cq_qact* a, size_t t, int32_t s[4]);
float cq_decode_row_ref(const cq_qmat* q, size_t r, const cq_qact* a);
float cq_prefill_row_ref(const cq_qmat* q, size_t r, const cq_qact* a, size_t t, int block);
float cq_single_row(const cq_qmat* q, size_t r, const cq_qact* a);
void cq_matmul_into(const cq_qmat* q, const cq_qact* a, float* y, size_t ldy, size_t col0, int nthreads);
void cq_prefill_rows_flags(const cq_qmat* q, const cq_qact* a, const uint8_t* block, float* y, size_t ldy,
                           size_t col0, int nthreads);
void cq_head_logits_sparse(const cq_qmat* q, const cq_qact* a, const uint32_t* ids, size_t nids, size_t out_rows,
                           float* out);
/* Bulk forms for checks at full size: decode lanes [out][groups][4] of
 * token t; group totals [rows][out][groups]; the matmul_into result for
 * output rows [r0, r1) only. */
void cq_all_lane_sums(const cq_qmat* q, const cq_qact* a, size_t t, int32_t* out, int nthreads);
void cq_all_totals(const cq_qmat* q, const cq_qact* a, int32_t* out, int nthreads);
void cq_matmul_rows(const cq_qmat* q, const cq_qact* a, const uint8_t* block, float* y, size_t ldy, size_t col0,
                    size_t r0, size_t r1, int nthreads);

/* QLinear (qlinear.rs:493-574): parts merged when compatible. */
typedef struct cq_qlinear {
    size_t nparts, out, in_dim;
    cq_qmat** parts;
} cq_qlinear;

cq_qlinear* cq_qlinear_new(cq_qmat* const* parts, size_t n);
void cq_qlinear_free(cq_qlinear* l);
void cq_qlinear_matmul(const cq_qlinear* l, const cq_qact* a, float* y, int nthreads);

/* ---- infer.rs norms --------------------------------------------------- */
float cq_dot16(const float* x, const float* y, size_t n);
float cq_rinv(float ss, size_t n);
void cq_zcn16(const float* x, const uint16_t* s, size_t n, float* out);
void cq_norm_apply16(float* out, const float* x, float r, const uint16_t* s, size_t n);

/* ---- generate.rs ------------------------------------------------------ */
size_t cq_argmax(const float* x, size_t n);

/* ---- needle-train rand.rs -------------------------------------------- */
void cq_threefry2x32(const uint32_t key[2], const uint32_t x[2], uint32_t out[2]);
void cq_prng_key(uint64_t seed, uint32_t out[2]);
void cq_split(const uint32_t key[2], uint32_t out_key[2], uint32_t out_sub[2]);
float cq_erfinv_f32(float x);
void cq_normal(const uint32_t key[2], size_t n, float* out, int nthreads);
void cq_seed_sequence_u64(uint64_t seed, size_t n, uint64_t* out);

typedef struct cq_nprng cq_nprng;
cq_nprng* cq_nprng_new(uint64_t seed);
void cq_nprng_free(cq_nprng* r);
uint64_t cq_nprng_next_u64(cq_nprng* r);
uint32_t cq_nprng_next_u32(cq_nprng* r);
uint64_t cq_nprng_interval(cq_nprng* r, uint64_t max);
void cq_nprng_permutation(cq_nprng* r, size_t n, uint64_t* out);

#ifdef __cplusplus
}
#endif
#endif
