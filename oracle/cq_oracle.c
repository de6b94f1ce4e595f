/*
 * cq_oracle.c -- CPU restatement of needle-rs's packed CQ runtime.
 *
 * TEST INFRASTRUCTURE ONLY (the parity oracle and the timed CPU baseline);
 * the product library never links or calls this file.  Citations are
 * reference file:line.  Build with -ffp-contract=off (see oracle/Makefile):
 * every float operation below is a single IEEE operation in the order the
 * Rust source performs it, and fmaf() stands exactly where Rust has
 * mul_add.
 */
#include "cq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bits_f32(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}
static inline uint32_t f32_bits(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}

/* ------------------------------------------------------------------ f16 */
/* IEEE binary16, round to nearest even: what `half` 2.7.1's f16::from_f32
 * computes (Cargo.lock pin; used at crates/needle-engine/src/qlinear.rs:228
 * and crates/needle-core/src/quant.rs:251).  NaN keeps its top payload bits
 * and is made quiet. */
uint16_t cq_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds past 65504 */
    if (ax < 0x38800000u) {                                     /* f16 subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;          /* below half the least subnormal */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value in units of 2^-24 is m >> shift */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ax - 0x38000000u; /* rebias 127 -> 15 */
    uint32_t q = r >> 13;
    uint32_t rem = r & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float cq_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bits_f32(sign);
        /* subnormal: m * 2^-24, exact in f32 */
        float v = (float)m * bits_f32(0x33800000u);
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* `1/127` as the engine rounds it (crates/needle-engine/src/qlinear.rs:40). */
float cq_k127(void) { return bits_f32(0x3c010204u); }
/* Masked logits (crates/needle-engine/src/infer.rs:36). */
float cq_neg(void) { return bits_f32(0xf149f2cau); }

/* --------------------------------------------------------------- quant.rs */
/* Lloyd-Max centroids as exact f64 bit patterns
 * (crates/needle-core/src/quant.rs:15-47). */
static const uint64_t LM2[4] = {0xbff81b52e4028034ull, 0xbfdce467275b97c2ull, 0x3fdcfd177c54d348ull,
                                0x3ff828af1c856640ull};
static const uint64_t LM3[8] = {0xc00121468f3c6b81ull, 0xbff556e7125deacaull, 0xbfe7f2e0f9d592abull,
                                0xbfce6e4509e1aa2cull, 0x3fd000bb25e4dfa5ull, 0x3fe82dc469b936a5ull,
                                0x3ff568607ac227c5ull, 0x40012e5beccc8fdaull};
static const uint64_t LM4[16] = {0xc005ae0f408928fbull, 0xc0005b0b8a516d54ull, 0xbff9841ff0758fc8ull,
                                 0xbff3bbbebadac679ull, 0xbfed82c6dd21f59eull, 0xbfe47717151708b5ull,
                                 0xbfd7d9b9e4b565faull, 0xbfbd4ca474b8559bull, 0x3fc2683e9154fce2ull,
                                 0x3fd9daf49368793aull, 0x3fe586b43e57d29dull, 0x3feec3d50cbc3b33ull,
                                 0x3ff4688db93b85f1ull, 0x3ffa3164906b428full, 0x4000ace7bbde2442ull,
                                 0x4005ed98d06f2a4aull};

static double bits_f64(uint64_t b) {
    double d;
    memcpy(&d, &b, 8);
    return d;
}

/* lloyd_max (crates/needle-core/src/quant.rs:50-62).  Returns the count. */
int cq_lloyd_max(uint32_t bits, double* out) {
    switch (bits) {
    case 1: {
        double c = sqrt(2.0 / 3.14159265358979323846);
        out[0] = -c;
        out[1] = c;
        return 2;
    }
    case 2:
        for (int i = 0; i < 4; i++) out[i] = bits_f64(LM2[i]);
        return 4;
    case 3:
        for (int i = 0; i < 8; i++) out[i] = bits_f64(LM3[i]);
        return 8;
    case 4:
        for (int i = 0; i < 16; i++) out[i] = bits_f64(LM4[i]);
        return 16;
    case CQ_TERNARY_RECORD_BITS: {
        const double t = 1.2240064; /* TERNARY_C, quant.rs:15 */
        out[0] = -t;
        out[1] = 0.0;
        out[2] = t;
        return 3;
    }
    default:
        return 0;
    }
}

/* codebook (crates/needle-core/src/quant.rs:65-68): centroid / sqrt(group)
 * in f64, then rounded to f32. */
int cq_codebook(uint32_t bits, size_t group, float* out) {
    double c[16];
    int n = cq_lloyd_max(bits, c);
    double s = sqrt((double)group);
    for (int i = 0; i < n; i++) out[i] = (float)(c[i] / s);
    return n;
}

/* hadamard_scale (crates/needle-core/src/quant.rs:71-73). */
float cq_hadamard_scale(size_t n) { return (float)(1.0 / sqrt((double)n)); }

/* hadamard (crates/needle-core/src/quant.rs:76-87). */
void cq_hadamard(size_t n, float* h) {
    float s = cq_hadamard_scale(n);
    for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < n; j++) {
            float sign = (__builtin_popcountll((unsigned long long)(i & j)) % 2 == 0) ? 1.0f : -1.0f;
            h[i * n + j] = sign * s;
        }
}

/* fwht (crates/needle-core/src/quant.rs:91-105): unnormalised, h = 1, 2, 4,
 * ..., a + b then a - b. */
void cq_fwht(float* x, size_t n) {
    for (size_t h = 1; h < n; h *= 2)
        for (size_t i = 0; i < n; i += h * 2)
            for (size_t j = i; j < i + h; j++) {
                float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
}

/* rotate (crates/needle-core/src/quant.rs:109-115). */
void cq_rotate(float* x, size_t n) {
    cq_fwht(x, n);
    float s = cq_hadamard_scale(n);
    for (size_t i = 0; i < n; i++) x[i] *= s;
}

/* nearest (crates/needle-core/src/quant.rs:119-124): searchsorted(left),
 * clamped to 1..len-1, ties to the lower centroid. */
size_t cq_nearest(float x, const float* cb, size_t ncb) {
    size_t pos = 0;
    while (pos < ncb && cb[pos] < x) pos++;
    if (pos < 1) pos = 1;
    if (pos > ncb - 1) pos = ncb - 1;
    float l = cb[pos - 1], r = cb[pos];
    return (fabsf(x - l) <= fabsf(x - r)) ? pos - 1 : pos;
}

/* quantize_group (crates/needle-core/src/quant.rs:127-135): rotate, then the
 * sequential f32 sum of squares, sqrt, and nearest(v / max(norm, 1e-12)). */
static float quantize_group(float* g, size_t group, const float* cb, size_t ncb, uint8_t* idx) {
    cq_rotate(g, group);
    float norm = 0.0f;
    for (size_t i = 0; i < group; i++) {
        float sq = g[i] * g[i];
        norm = norm + sq;
    }
    norm = sqrtf(norm);
    float denom = norm > 1e-12f ? norm : 1e-12f;
    for (size_t i = 0; i < group; i++) idx[i] = (uint8_t)cq_nearest(g[i] / denom, cb, ncb);
    return norm;
}

/* pack_lsb (crates/needle-core/src/quant.rs:185-198).  Returns bytes. */
size_t cq_pack_lsb(const uint8_t* idx, size_t n, uint32_t bits, uint8_t* out) {
    size_t o = 0;
    for (size_t c = 0; c < n; c += 8) {
        uint64_t word = 0;
        for (size_t i = 0; i < 8 && c + i < n; i++) word |= (uint64_t)idx[c + i] << (i * bits);
        for (uint32_t b = 0; b < bits; b++) out[o++] = (uint8_t)(word >> (8 * b));
    }
    return o;
}

/* unpack_lsb_into (crates/needle-core/src/quant.rs:207-224). */
void cq_unpack_lsb_into(const uint8_t* packed, size_t npacked, uint32_t bits, uint8_t* out, size_t nout) {
    uint64_t mask = (1ull << bits) - 1ull;
    size_t k = 0;
    for (size_t c = 0; c < npacked; c += bits) {
        uint64_t word = 0;
        for (size_t b = 0; b < bits && c + b < npacked; b++) word |= (uint64_t)packed[c + b] << (8 * b);
        for (size_t i = 0; i < 8; i++) {
            if (k == nout) return;
            out[k++] = (uint8_t)((word >> (i * bits)) & mask);
        }
    }
}

/* packed_row_bytes (crates/needle-core/src/quant.rs:285-287). */
size_t cq_packed_row_bytes(size_t in_pad, uint32_t bits) {
    return bits == CQ_TERNARY_RECORD_BITS ? in_pad * 2 / 8 : in_pad * bits / 8;
}

/* cq_pack (crates/needle-core/src/quant.rs:233-256): per row, per group,
 * zero-padded, quantize_group, f16 norm; rows are independent (rayon there,
 * OpenMP here; no numeric effect). */
void cq_pack(const float* w, size_t rows, size_t d, uint32_t bits, size_t group, uint8_t* packed, uint16_t* norms,
             int nthreads) {
    float cb[16];
    size_t ncb = (size_t)cq_codebook(bits, group, cb);
    size_t in_pad = (d + group - 1) / group * group;
    size_t per_row = in_pad * bits / 8;
    size_t ng = in_pad / group;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (long long rr = 0; rr < (long long)rows; rr++) {
        size_t r = (size_t)rr;
        const float* src = w + r * d;
        uint8_t* idx = (uint8_t*)malloc(in_pad);
        float* g = (float*)malloc(group * sizeof(float));
        for (size_t gi = 0, start = 0; start < in_pad; start += group, gi++) {
            size_t take = d > start ? (d - start < group ? d - start : group) : 0;
            memcpy(g, src + start, take * sizeof(float));
            for (size_t i = take; i < group; i++) g[i] = 0.0f;
            float norm = quantize_group(g, group, cb, ncb, idx + start);
            norms[r * ng + gi] = cq_f32_to_f16(norm);
        }
        cq_pack_lsb(idx, in_pad, bits, packed + r * per_row);
        free(idx);
        free(g);
    }
}

/* cq_unpack (crates/needle-core/src/quant.rs:259-283). */
void cq_unpack(const uint8_t* packed, const uint16_t* norms, size_t out, size_t in_dim, uint32_t bits, size_t group,
               float* w) {
    size_t in_pad = (in_dim + group - 1) / group * group;
    float cb[16];
    cq_codebook(bits, group, cb);
    size_t row_bytes = cq_packed_row_bytes(in_pad, bits);
    uint8_t* idx = (uint8_t*)malloc(in_pad);
    float* g = (float*)malloc(group * sizeof(float));
    for (size_t r = 0; r < out; r++) {
        const uint8_t* prow = packed + r * row_bytes;
        if (bits == CQ_TERNARY_RECORD_BITS) {
            cq_unpack_lsb_into(prow, row_bytes, 2, idx, in_pad);
            for (size_t i = 0; i < in_pad; i++) idx[i] = idx[i] == 3 ? 0 : (uint8_t)(idx[i] + 1);
        } else {
            cq_unpack_lsb_into(prow, row_bytes, bits, idx, in_pad);
        }
        for (size_t gi = 0, start = 0; start < in_pad; start += group, gi++) {
            float norm = cq_f16_to_f32(norms[r * (in_pad / group) + gi]);
            for (size_t i = 0; i < group; i++) g[i] = cb[idx[start + i]] * norm;
            cq_rotate(g, group);
            size_t take = in_dim > start ? (in_dim - start < group ? in_dim - start : group) : 0;
            memcpy(w + r * in_dim + start, g, take * sizeof(float));
        }
    }
    free(idx);
    free(g);
}

/* ------------------------------------------------------------ qlinear.rs */
static inline float rust_round(float v) { return roundf(v); } /* half away from zero */

static inline int8_t sat_i8(float v) {
    /* `.clamp(-128.0, 127.0) as i8` */
    if (v < -128.0f) v = -128.0f;
    if (v > 127.0f) v = 127.0f;
    return (int8_t)(int)v;
}

static inline float rust_max(float m, float v) {
    /* f32::max: the non-NaN operand when one is NaN. */
    if (isnan(m)) return v;
    if (isnan(v)) return m;
    return m > v ? m : v;
}

/* quant_scale (crates/needle-engine/src/qlinear.rs:92-108). */
float cq_quant_scale(const float* x, size_t n) {
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) m = rust_max(m, fabsf(x[i]));
    return m > 0.0f ? m * cq_k127() : 1.0f;
}

/* quant_with (crates/needle-engine/src/qlinear.rs:113-140). */
void cq_quant_with(const float* x, size_t n, float inv, int8_t* q) {
    for (size_t i = 0; i < n; i++) {
        float v = x[i] * inv;
        q[i] = sat_i8(rust_round(v));
    }
}

/* quant_i8 (crates/needle-engine/src/qlinear.rs:77-88). */
float cq_quant_i8(const float* x, size_t n, int8_t* q) {
    float s = cq_quant_scale(x, n);
    cq_quant_with(x, n, 1.0f / s, q);
    return s;
}

/* act_pos (crates/needle-engine/src/qlinear.rs:145-147). */
size_t cq_act_pos(size_t p, uint8_t bits) { return bits == 2 ? (p % 4) * 32 + p / 4 : (p % 2) * 64 + p / 2; }

/* prep_group (crates/needle-engine/src/qlinear.rs:152-164): the group,
 * zero-padded past the row end, rotated, quantized, stored at act_pos. */
float cq_prep_group(const float* x, size_t len, size_t g, int8_t* q, uint8_t bits) {
    float buf[CQ_GROUP];
    size_t start = g * CQ_GROUP;
    size_t take = len - start < CQ_GROUP ? len - start : CQ_GROUP;
    memset(buf, 0, sizeof buf);
    memcpy(buf, x + start, take * sizeof(float));
    cq_rotate(buf, CQ_GROUP);
    int8_t nat[CQ_GROUP];
    float s = cq_quant_i8(buf, CQ_GROUP, nat);
    for (size_t p = 0; p < CQ_GROUP; p++) q[cq_act_pos(p, bits)] = nat[p];
    return s;
}

/* share (crates/needle-engine/src/team.rs:257-262): member tid's contiguous
 * part of 0..n. */
static void share(size_t n, int tid, int threads, size_t* lo, size_t* hi) {
    size_t per = (n + (size_t)threads - 1) / (size_t)threads;
    size_t a = (size_t)tid * per;
    size_t b = ((size_t)tid + 1) * per;
    *lo = a < n ? a : n;
    *hi = b < n ? b : n;
}

/* QAct::empty_rows (crates/needle-engine/src/qlinear.rs:175-178). */
cq_qact* cq_qact_empty_rows(size_t rows, size_t in_dim, uint8_t bits) {
    cq_qact* a = (cq_qact*)calloc(1, sizeof *a);
    a->rows = rows;
    a->groups = (in_dim + CQ_GROUP - 1) / CQ_GROUP;
    a->bits = bits;
    a->xq = (int8_t*)calloc(rows * a->groups * CQ_GROUP, 1);
    a->sx = (float*)calloc(rows * a->groups, sizeof(float));
    return a;
}

/* QAct::new (crates/needle-engine/src/qlinear.rs:191-207): units split over
 * the team (share) when there are at least 24 of them. */
cq_qact* cq_qact_new(const float* x, size_t rows, size_t in_dim, uint8_t bits, int nthreads) {
    cq_qact* a = cq_qact_empty_rows(rows, in_dim, bits);
    size_t groups = a->groups;
    size_t units = rows * groups;
    int nt = (units >= 24 && nthreads > 1) ? nthreads : 1;
#pragma omp parallel num_threads(nt)
    {
        int tid = 0, n = 1;
#ifdef _OPENMP
        tid = omp_get_thread_num();
        n = omp_get_num_threads();
#endif
        size_t lo, hi;
        share(units, tid, n, &lo, &hi);
        for (size_t u = lo; u < hi; u++) {
            size_t r = u / groups, g = u % groups;
            a->sx[u] = cq_prep_group(x + r * in_dim, in_dim, g, a->xq + u * CQ_GROUP, bits);
        }
    }
    return a;
}

void cq_qact_free(cq_qact* a) {
    if (!a) return;
    free(a->xq);
    free(a->sx);
    free(a);
}

/* int8_codebook (crates/needle-engine/src/qlinear.rs:211-216). */
void cq_int8_codebook(const float* cb, size_t n, int8_t* cb8, float* scale) {
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) m = rust_max(m, fabsf(cb[i]));
    float s = m > 0.0f ? m * cq_k127() : 1.0f;
    float inv = 1.0f / s;
    for (size_t i = 0; i < n; i++) cb8[i] = sat_i8(rust_round(cb[i] * inv));
    *scale = s;
}

/* QMat::build (crates/needle-engine/src/qlinear.rs:244-265); `ternary`
 * selects from_cq's code_of remap (qlinear.rs:227). */
cq_qmat* cq_qmat_build(size_t out, size_t in_dim, uint8_t bits, const float* cb, size_t ncb, int ternary,
                       const uint8_t* codes, const uint16_t* norms) {
    cq_qmat* q = (cq_qmat*)calloc(1, sizeof *q);
    q->out = out;
    q->in_dim = in_dim;
    q->groups = (in_dim + CQ_GROUP - 1) / CQ_GROUP;
    q->bits = bits;
    size_t bpg = CQ_GROUP * bits / 8;
    q->codes = (uint8_t*)malloc(out * q->groups * bpg);
    memcpy(q->codes, codes, out * q->groups * bpg);
    q->norms = (uint16_t*)malloc(out * q->groups * sizeof(uint16_t));
    memcpy(q->norms, norms, out * q->groups * sizeof(uint16_t));
    int8_t cb8[16];
    cq_int8_codebook(cb, ncb, cb8, &q->cbs);
    size_t ncodes = (size_t)1 << bits;
    for (size_t c = 0; c < ncodes; c++) {
        size_t k = ternary ? (c == 3 ? 0 : c + 1) : c;
        q->vals[c] = k < ncb ? cb8[k] : 0;
        q->fvals[c] = k < ncb ? cb[k] : 0.0f;
    }
    for (int n = 0; n < 16; n++) {
        if (bits == 2) {
            q->tables[0][n] = q->vals[n & 3];
            q->tables[1][n] = q->vals[n >> 2];
        } else {
            q->tables[0][n] = q->vals[n];
        }
    }
    return q;
}

/* QMat::from_cq (crates/needle-engine/src/qlinear.rs:220-236): group must be
 * 128 (the reference asserts; NULL here), ternary records read as 2-bit
 * with the code remap, each row's groups*bpg bytes copied. */
cq_qmat* cq_qmat_from_cq(const uint8_t* packed, const uint16_t* norms, size_t out, size_t in_dim, uint32_t bits,
                         size_t group) {
    if (group != CQ_GROUP) return NULL;
    size_t in_pad = (in_dim + group - 1) / group * group;
    size_t groups = in_pad / CQ_GROUP;
    int ternary = bits == CQ_TERNARY_RECORD_BITS;
    float cb[16];
    size_t ncb = (size_t)cq_codebook(bits, group, cb);
    uint8_t b = ternary ? 2 : (uint8_t)bits;
    size_t row_bytes = cq_packed_row_bytes(in_pad, bits);
    size_t bpg = CQ_GROUP * b / 8;
    uint8_t* codes = (uint8_t*)malloc(out * groups * bpg);
    for (size_t r = 0; r < out; r++) memcpy(codes + r * groups * bpg, packed + r * row_bytes, groups * bpg);
    /* norms: f16 -> f32 -> f16 is the identity on finite values. */
    uint16_t* nn = (uint16_t*)malloc(out * groups * sizeof(uint16_t));
    for (size_t i = 0; i < out * groups; i++) nn[i] = cq_f32_to_f16(cq_f16_to_f32(norms[i]));
    cq_qmat* q = cq_qmat_build(out, in_dim, b, cb, ncb, ternary, codes, nn);
    free(codes);
    free(nn);
    return q;
}

/* QMat::from_f32 (crates/needle-engine/src/qlinear.rs:239-242). */
cq_qmat* cq_qmat_from_f32(const float* w, size_t out, size_t in_dim, int nthreads) {
    size_t in_pad = (in_dim + CQ_GROUP - 1) / CQ_GROUP * CQ_GROUP;
    uint8_t* packed = (uint8_t*)malloc(out * in_pad / 2);
    uint16_t* norms = (uint16_t*)malloc(out * (in_pad / CQ_GROUP) * sizeof(uint16_t));
    cq_pack(w, out, in_dim, 4, CQ_GROUP, packed, norms, nthreads);
    float cb[16];
    size_t ncb = (size_t)cq_codebook(4, CQ_GROUP, cb);
    cq_qmat* q = cq_qmat_build(out, in_dim, 4, cb, ncb, 0, packed, norms);
    free(packed);
    free(norms);
    return q;
}

void cq_qmat_free(cq_qmat* q) {
    if (!q) return;
    free(q->codes);
    free(q->norms);
    free(q);
}

/* QMat::bytes (crates/needle-engine/src/qlinear.rs:287-289). */
size_t cq_qmat_bytes(const cq_qmat* q) {
    return q->out * q->groups * (CQ_GROUP * q->bits / 8) + q->out * q->groups * 2;
}

/* group_codes (crates/needle-engine/src/qlinear.rs:301-305). */
static void group_codes(const cq_qmat* q, size_t r, size_t g, uint8_t out[CQ_GROUP]) {
    size_t bpg = CQ_GROUP * q->bits / 8;
    size_t at = (r * q->groups + g) * bpg;
    cq_unpack_lsb_into(q->codes + at, bpg, q->bits, out, CQ_GROUP);
}

/* QMat::row (crates/needle-engine/src/qlinear.rs:309-323). */
void cq_qmat_row(const cq_qmat* q, size_t r, float* out) {
    float buf[CQ_GROUP];
    uint8_t codes[CQ_GROUP];
    for (size_t g = 0; g < q->groups; g++) {
        group_codes(q, r, g, codes);
        float norm = cq_f16_to_f32(q->norms[r * q->groups + g]);
        for (size_t i = 0; i < CQ_GROUP; i++) buf[i] = q->fvals[codes[i]] * norm;
        cq_rotate(buf, CQ_GROUP);
        size_t start = g * CQ_GROUP;
        size_t take = q->in_dim - start < CQ_GROUP ? q->in_dim - start : CQ_GROUP;
        memcpy(out + start, buf, take * sizeof(float));
    }
}

/* lane_sums (crates/needle-engine/src/qlinear.rs:327-337). */
void cq_lane_sums(const cq_qmat* q, size_t r, size_t g, const cq_qact* a, size_t t, int32_t s[4]) {
    uint8_t codes[CQ_GROUP];
    group_codes(q, r, g, codes);
    const int8_t* x = a->xq + (t * a->groups + g) * CQ_GROUP;
    s[0] = s[1] = s[2] = s[3] = 0;
    for (size_t p = 0; p < CQ_GROUP; p++) {
        size_t lane = q->bits == 2 ? (p % 64) / 16 : (p % 32) / 8;
        s[lane] += (int32_t)q->vals[codes[p]] * (int32_t)x[cq_act_pos(p, q->bits)];
    }
}

/* decode_row_ref (crates/needle-engine/src/qlinear.rs:340-350). */
float cq_decode_row_ref(const cq_qmat* q, size_t r, const cq_qact* a) {
    float lanes[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t g = 0; g < q->groups; g++) {
        int32_t s[4];
        cq_lane_sums(q, r, g, a, 0, s);
        float sc = (a->sx[g] * q->cbs) * cq_f16_to_f32(q->norms[r * q->groups + g]);
        for (int l = 0; l < 4; l++) lanes[l] = fmaf((float)s[l], sc, lanes[l]);
    }
    return (lanes[0] + lanes[1]) + (lanes[2] + lanes[3]);
}

/* prefill_row_ref (crates/needle-engine/src/qlinear.rs:353-363). */
float cq_prefill_row_ref(const cq_qmat* q, size_t r, const cq_qact* a, size_t t, int block) {
    float acc = 0.0f;
    for (size_t g = 0; g < q->groups; g++) {
        int32_t s4[4];
        cq_lane_sums(q, r, g, a, t, s4);
        int32_t s = s4[0] + s4[1] + s4[2] + s4[3];
        float sx = a->sx[t * a->groups + g];
        float norm = cq_f16_to_f32(q->norms[r * q->groups + g]);
        float sc = block ? (norm * q->cbs) * sx : norm * (q->cbs * sx);
        acc = fmaf((float)s, sc, acc);
    }
    return acc;
}

/* single_row (crates/needle-engine/src/qlinear.rs:454-456): the block
 * combine for token 0. */
float cq_single_row(const cq_qmat* q, size_t r, const cq_qact* a) { return cq_prefill_row_ref(q, r, a, 0, 1); }

/* decode_rows + prefill_rows on rows [lo, hi) (qlinear.rs:366-419), the
 * portable branch the reference takes on x86-64 (qlinear.rs:387-390,
 * 448-449).  `block` overrides the t < rows/4*4 rule when non-NULL. */
static void rows_range(const cq_qmat* q, const cq_qact* a, const uint8_t* block, float* y, size_t ldy, size_t col0,
                       size_t lo, size_t hi) {
    if (a->rows == 1 && !block) {
        for (size_t r = lo; r < hi; r++) y[col0 + r] = cq_decode_row_ref(q, r, a);
        return;
    }
    size_t blocked = a->rows / 4 * 4;
    for (size_t r = lo; r < hi; r++)
        for (size_t t = 0; t < a->rows; t++) {
            int b = block ? (int)block[t] : (t < blocked);
            y[t * ldy + col0 + r] = cq_prefill_row_ref(q, r, a, t, b);
        }
}

/* matmul_into (crates/needle-engine/src/qlinear.rs:468-487): below 1024
 * group-units on one core, else output rows split with share(). */
static void matmul_impl(const cq_qmat* q, const cq_qact* a, const uint8_t* block, float* y, size_t ldy, size_t col0,
                        int nthreads) {
    size_t work = a->rows * q->out * q->groups;
    int nt = (work < 1024 || nthreads < 1) ? 1 : nthreads;
#pragma omp parallel num_threads(nt)
    {
        int tid = 0, n = 1;
#ifdef _OPENMP
        tid = omp_get_thread_num();
        n = omp_get_num_threads();
#endif
        size_t lo, hi;
        share(q->out, tid, n, &lo, &hi);
        rows_range(q, a, block, y, ldy, col0, lo, hi);
    }
}

void cq_matmul_into(const cq_qmat* q, const cq_qact* a, float* y, size_t ldy, size_t col0, int nthreads) {
    matmul_impl(q, a, NULL, y, ldy, col0, nthreads);
}

/* The prefill combine with an explicit block flag per token: what a chunked
 * prefill (crates/needle-engine/src/infer.rs:1105-1132) gives each token of a
 * batched feed (flag = index within its chunk < chunk_len/4*4). */
void cq_prefill_rows_flags(const cq_qmat* q, const cq_qact* a, const uint8_t* block, float* y, size_t ldy,
                           size_t col0, int nthreads) {
    matmul_impl(q, a, block, y, ldy, col0, nthreads);
}

/* head_logits_sparse (crates/needle-engine/src/infer.rs:1145-1166). */
void cq_head_logits_sparse(const cq_qmat* q, const cq_qact* a, const uint32_t* ids, size_t nids, size_t out_rows,
                           float* out) {
    for (size_t i = 0; i < out_rows; i++) out[i] = cq_neg();
    for (size_t k = 0; k < nids; k++) out[ids[k]] = cq_single_row(q, ids[k], a);
}

void cq_all_lane_sums(const cq_qmat* q, const cq_qact* a, size_t t, int32_t* out, int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (long long rr = 0; rr < (long long)q->out; rr++)
        for (size_t g = 0; g < q->groups; g++) cq_lane_sums(q, (size_t)rr, g, a, t, out + ((size_t)rr * q->groups + g) * 4);
}

void cq_all_totals(const cq_qmat* q, const cq_qact* a, int32_t* out, int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (long long rr = 0; rr < (long long)q->out; rr++)
        for (size_t t = 0; t < a->rows; t++)
            for (size_t g = 0; g < q->groups; g++) {
                int32_t s[4];
                cq_lane_sums(q, (size_t)rr, g, a, t, s);
                out[(t * q->out + (size_t)rr) * q->groups + g] = s[0] + s[1] + s[2] + s[3];
            }
}

/* Output rows [r0, r1) of matmul_into (or of the flagged prefill). */
void cq_matmul_rows(const cq_qmat* q, const cq_qact* a, const uint8_t* block, float* y, size_t ldy, size_t col0,
                    size_t r0, size_t r1, int nthreads) {
    size_t n = r1 - r0;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads)
    {
        int tid = 0, nt = 1;
#ifdef _OPENMP
        tid = omp_get_thread_num();
        nt = omp_get_num_threads();
#endif
        size_t lo, hi;
        share(n, tid, nt, &lo, &hi);
        rows_range(q, a, block, y, ldy, col0, r0 + lo, r0 + hi);
    }
}

/* QLinear::new (crates/needle-engine/src/qlinear.rs:501-519): neighbours
 * with the same width/codebook merged by row concatenation. */
static int compatible(const cq_qmat* a, const cq_qmat* b) {
    return a->in_dim == b->in_dim && a->bits == b->bits && memcmp(a->tables, b->tables, sizeof a->tables) == 0 &&
           memcmp(a->fvals, b->fvals, sizeof a->fvals) == 0 && a->cbs == b->cbs;
}

cq_qlinear* cq_qlinear_new(cq_qmat* const* parts, size_t n) {
    cq_qlinear* l = (cq_qlinear*)calloc(1, sizeof *l);
    l->parts = (cq_qmat**)calloc(n, sizeof(cq_qmat*));
    l->in_dim = parts[0]->in_dim;
    for (size_t i = 0; i < n; i++) {
        const cq_qmat* p = parts[i];
        l->out += p->out;
        cq_qmat* last = l->nparts ? l->parts[l->nparts - 1] : NULL;
        size_t bpg = CQ_GROUP * p->bits / 8;
        if (last && compatible(last, p)) {
            size_t oc = last->out * last->groups * bpg, pc = p->out * p->groups * bpg;
            last->codes = (uint8_t*)realloc(last->codes, oc + pc);
            memcpy(last->codes + oc, p->codes, pc);
            size_t on = last->out * last->groups, pn = p->out * p->groups;
            last->norms = (uint16_t*)realloc(last->norms, (on + pn) * sizeof(uint16_t));
            memcpy(last->norms + on, p->norms, pn * sizeof(uint16_t));
            last->out += p->out;
        } else {
            cq_qmat* c = (cq_qmat*)malloc(sizeof *c);
            *c = *p;
            c->codes = (uint8_t*)malloc(p->out * p->groups * bpg);
            memcpy(c->codes, p->codes, p->out * p->groups * bpg);
            c->norms = (uint16_t*)malloc(p->out * p->groups * sizeof(uint16_t));
            memcpy(c->norms, p->norms, p->out * p->groups * sizeof(uint16_t));
            l->parts[l->nparts++] = c;
        }
    }
    return l;
}

void cq_qlinear_free(cq_qlinear* l) {
    if (!l) return;
    for (size_t i = 0; i < l->nparts; i++) cq_qmat_free(l->parts[i]);
    free(l->parts);
    free(l);
}

/* QLinear::matmul (crates/needle-engine/src/qlinear.rs:526-534). */
void cq_qlinear_matmul(const cq_qlinear* l, const cq_qact* a, float* y, int nthreads) {
    size_t col = 0;
    for (size_t i = 0; i < l->nparts; i++) {
        cq_matmul_into(l->parts[i], a, y, l->out, col, nthreads);
        col += l->parts[i]->out;
    }
}

/* -------------------------------------------------------- infer.rs norms */
/* dot16, portable branch (crates/needle-engine/src/infer.rs:401-418): four
 * 4-lane fma accumulators over 16-element chunks, combined
 * ((A2 + A3) + A1) + A0 per lane, then (l0 + l1) + (l2 + l3). */
float cq_dot16(const float* x, const float* y, size_t n) {
    float a[4][4] = {{0}};
    for (size_t c = 0; c < n / 16; c++)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 4; l++) {
                size_t i = c * 16 + (size_t)j * 4 + (size_t)l;
                a[j][l] = fmaf(x[i], y[i], a[j][l]);
            }
    float t[4];
    for (int l = 0; l < 4; l++) t[l] = ((a[2][l] + a[3][l]) + a[1][l]) + a[0][l];
    return (t[0] + t[1]) + (t[2] + t[3]);
}

/* rinv (crates/needle-engine/src/infer.rs:422-424). */
float cq_rinv(float ss, size_t n) {
    float v = ss / (float)n + 1e-6f;
    return 1.0f / sqrtf(v);
}

/* norm_apply16 (crates/needle-engine/src/infer.rs:614-635). */
void cq_norm_apply16(float* out, const float* x, float r, const uint16_t* s, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float t = x[i] * r;
        out[i] = fmaf(t, cq_f16_to_f32(s[i]), t);
    }
}

/* zcn16 (crates/needle-engine/src/infer.rs:455-473). */
void cq_zcn16(const float* x, const uint16_t* s, size_t n, float* out) {
    float r = cq_rinv(cq_dot16(x, x, n), n);
    cq_norm_apply16(out, x, r, s, n);
}

/* ----------------------------------------------------------- generate.rs */
/* argmax (crates/needle-engine/src/generate.rs:42-50): the first maximum. */
size_t cq_argmax(const float* x, size_t n) {
    size_t best = 0;
    for (size_t i = 0; i < n; i++)
        if (x[i] > x[best]) best = i;
    return best;
}

/* ---------------------------------------------------- needle-train rand.rs */
static inline uint32_t rotl32(uint32_t x, uint32_t r) { return (x << r) | (x >> (32u - r)); }

/* threefry2x32, 20 rounds (crates/needle-train/src/rand.rs:139-153). */
void cq_threefry2x32(const uint32_t key[2], const uint32_t x[2], uint32_t out[2]) {
    static const uint32_t R[2][4] = {{13, 15, 26, 6}, {17, 29, 16, 24}};
    uint32_t ks[3] = {key[0], key[1], key[0] ^ key[1] ^ 0x1BD11BDAu};
    uint32_t x0 = x[0] + ks[0];
    uint32_t x1 = x[1] + ks[1];
    for (uint32_t round = 0; round < 5; round++) {
        for (int i = 0; i < 4; i++) {
            x0 = x0 + x1;
            x1 = rotl32(x1, R[round % 2][i]) ^ x0;
        }
        x0 = x0 + ks[(round + 1) % 3];
        x1 = x1 + ks[(round + 2) % 3] + (round + 1);
    }
    out[0] = x0;
    out[1] = x1;
}

/* prng_key (crates/needle-train/src/rand.rs:156-158). */
void cq_prng_key(uint64_t seed, uint32_t out[2]) {
    out[0] = (uint32_t)(seed >> 32);
    out[1] = (uint32_t)seed;
}

/* split (crates/needle-train/src/rand.rs:161-163). */
void cq_split(const uint32_t key[2], uint32_t out_key[2], uint32_t out_sub[2]) {
    const uint32_t c0[2] = {0, 0}, c1[2] = {0, 1};
    uint32_t k[2], s[2];
    cq_threefry2x32(key, c0, k);
    cq_threefry2x32(key, c1, s);
    out_key[0] = k[0];
    out_key[1] = k[1];
    out_sub[0] = s[0];
    out_sub[1] = s[1];
}

/* erfinv_f32, XLA's Giles approximation (crates/needle-train/src/rand.rs:166-202). */
float cq_erfinv_f32(float x) {
    float w = -logf((1.0f - x) * (1.0f + x));
    float p;
    if (w < 5.0f) {
        static const float c[8] = {3.4327394e-7f,  -3.5233877e-06f, -4.3915065e-6f, 0.00021858087f,
                                   -0.001253725f, -0.0041776816f,  0.24664073f,    1.5014094f};
        w = w - 2.5f;
        p = 2.8102264e-8f;
        for (int i = 0; i < 8; i++) p = c[i] + p * w;
    } else {
        static const float c[8] = {0.00010095056f, 0.0013493432f, -0.0036734284f, 0.0057395077f,
                                   -0.0076224613f, 0.0094388705f, 1.001674f,      2.8329768f};
        w = sqrtf(w) - 3.0f;
        p = -0.00020021426f;
        for (int i = 0; i < 8; i++) p = c[i] + p * w;
    }
    if (fabsf(x) == 1.0f) return x * INFINITY;
    return p * x;
}

/* normal (crates/needle-train/src/rand.rs:205-217): jax.random.normal for
 * float32, element i from threefry(key, (i >> 32, i)). */
void cq_normal(const uint32_t key[2], size_t n, float* out, int nthreads) {
    const float lo = bits_f32(f32_bits(-1.0f) - 1u); /* nextafter(-1, 0) */
    const float hi = 1.0f;
    const float sqrt2 = bits_f32(0x3fb504f3u); /* std::f32::consts::SQRT_2 */
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (long long ii = 0; ii < (long long)n; ii++) {
        uint64_t i = (uint64_t)ii;
        uint32_t xx[2] = {(uint32_t)(i >> 32), (uint32_t)i}, b[2];
        cq_threefry2x32(key, xx, b);
        uint32_t bits = b[0] ^ b[1];
        float f = bits_f32((bits >> 9) | 0x3f800000u) - 1.0f;
        float u = f * (hi - lo);
        u = u + lo;
        u = rust_max(lo, u);
        out[i] = sqrt2 * cq_erfinv_f32(u);
    }
}

/* numpy SeedSequence + PCG64 (crates/needle-train/src/rand.rs:9-130). */
#define INIT_A 0x43b0d7e5u
#define MULT_A 0x931e8875u
#define INIT_B 0x8b51f9ddu
#define MULT_B 0x58f38dedu
#define MIX_MULT_L 0xca01f9ddu
#define MIX_MULT_R 0x4973f715u
#define XSHIFT 16

static uint32_t hashmix(uint32_t value, uint32_t* hc) {
    uint32_t v = value ^ *hc;
    *hc = *hc * MULT_A;
    v = v * *hc;
    return v ^ (v >> XSHIFT);
}

static uint32_t mixf(uint32_t x, uint32_t y) {
    uint32_t r = MIX_MULT_L * x - MIX_MULT_R * y;
    return r ^ (r >> XSHIFT);
}

/* seed_sequence_u64 (crates/needle-train/src/rand.rs:31-63). */
void cq_seed_sequence_u64(uint64_t seed, size_t n, uint64_t* out) {
    uint32_t entropy[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    size_t nent = (seed >> 32) ? 2 : 1;
    uint32_t pool[4];
    uint32_t hc = INIT_A;
    for (size_t i = 0; i < 4; i++) pool[i] = hashmix(i < nent ? entropy[i] : 0, &hc);
    for (size_t src = 0; src < 4; src++)
        for (size_t dst = 0; dst < 4; dst++)
            if (src != dst) pool[dst] = mixf(pool[dst], hashmix(pool[src], &hc));
    uint32_t hb = INIT_B;
    uint32_t* words = (uint32_t*)malloc(n * 2 * sizeof(uint32_t));
    for (size_t i = 0; i < n * 2; i++) {
        uint32_t v = pool[i % 4] ^ hb;
        hb = hb * MULT_B;
        v = v * hb;
        words[i] = v ^ (v >> XSHIFT);
    }
    for (size_t i = 0; i < n; i++) out[i] = (uint64_t)words[2 * i] | ((uint64_t)words[2 * i + 1] << 32);
    free(words);
}

typedef unsigned __int128 u128;
struct cq_nprng {
    u128 state, inc;
    int has_spare;
    uint32_t spare;
};

static const u128 PCG_MULT = ((u128)2549297995355413924ull << 64) | (u128)4865540595714422341ull;

static void np_step(cq_nprng* r) { r->state = r->state * PCG_MULT + r->inc; }

/* NpRng::new (crates/needle-train/src/rand.rs:75-84). */
cq_nprng* cq_nprng_new(uint64_t seed) {
    uint64_t s[4];
    cq_seed_sequence_u64(seed, 4, s);
    cq_nprng* r = (cq_nprng*)calloc(1, sizeof *r);
    u128 initstate = ((u128)s[0] << 64) | (u128)s[1];
    u128 initseq = ((u128)s[2] << 64) | (u128)s[3];
    r->state = 0;
    r->inc = (initseq << 1) | 1u;
    np_step(r);
    r->state += initstate;
    np_step(r);
    return r;
}

void cq_nprng_free(cq_nprng* r) { free(r); }

/* next_u64, XSL-RR (crates/needle-train/src/rand.rs:90-94). */
uint64_t cq_nprng_next_u64(cq_nprng* r) {
    np_step(r);
    u128 s = r->state;
    uint64_t v = (uint64_t)(s >> 64) ^ (uint64_t)s;
    uint32_t rot = (uint32_t)(s >> 122);
    return rot ? (v >> rot) | (v << (64u - rot)) : v;
}

/* next_u32 with numpy's spare half (crates/needle-train/src/rand.rs:96-103). */
uint32_t cq_nprng_next_u32(cq_nprng* r) {
    if (r->has_spare) {
        r->has_spare = 0;
        return r->spare;
    }
    uint64_t n = cq_nprng_next_u64(r);
    r->spare = (uint32_t)(n >> 32);
    r->has_spare = 1;
    return (uint32_t)n;
}

/* interval, masked rejection (crates/needle-train/src/rand.rs:105-119). */
uint64_t cq_nprng_interval(cq_nprng* r, uint64_t max) {
    if (max == 0) return 0;
    uint64_t mask = max;
    for (int s = 1; s <= 32; s *= 2) mask |= mask >> s;
    for (;;) {
        uint64_t v = max <= 0xffffffffull ? ((uint64_t)cq_nprng_next_u32(r) & mask) : (cq_nprng_next_u64(r) & mask);
        if (v <= max) return v;
    }
}

/* permutation (crates/needle-train/src/rand.rs:122-129). */
void cq_nprng_permutation(cq_nprng* r, size_t n, uint64_t* out) {
    for (size_t i = 0; i < n; i++) out[i] = i;
    for (size_t i = n; i-- > 1;) {
        size_t j = (size_t)cq_nprng_interval(r, (uint64_t)i);
        uint64_t t = out[i];
        out[i] = out[j];
        out[j] = t;
    }
}
