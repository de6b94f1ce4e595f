// The Needle-3 decode step (Model::step_native,
// crates/needle-engine/src/infer/step.rs:171-760) on gfx950, one token per
// step, the KV cache and every activation resident in HBM.
//
// Per step: fwd_begin (embedding row, RoPE rows, hashed engram rows as A8),
// one key | value GEMV per engram site, fwd_engram_hist (int8 value history
// and its dilated conv), then per layer
//   fwd_layer   one workgroup: the previous layer's Hadamard MLP and mHC
//               write, then this layer's mHC read, engram gate, input norm
//               and A8;
//   GEMV        q | k | v | gate;
//   fwd_units   one wavefront per head unit: conv taps, head norm, RoPE,
//               int8 KV append, the tap history;
//   fwd_attend  one workgroup per (query head, key chunk): int8 scores,
//               chunk softmax, 21-bit digit P.V;
//   fwd_attn_out one workgroup: chunk merge, head gate, A8;
//   GEMV        out;
// and a last fwd_layer (lane mean, final norm, A8) before the head GEMV.
//
// Every floating-point operation follows the reference's portable branch in
// order and rounding (fma where it has mul_add, no contraction elsewhere):
// the serial dot16 chains, the cond_weights chains and the mix8 fma chains
// run in their reference order; integer sums (idot, P.V digits) are exact
// and order-free.  The reference's f32 exponential off Apple targets is the
// f64 exp rounded once (lexpf, crates/needle-engine/src/infer.rs:84-101);
// here too, with the device library's f64 exp: two f64 exps accurate to an
// ulp give the same f32 unless an f32 rounding boundary falls between them.
#include <algorithm>

#include "nh_device.h"
#include "nh_forward.h"
#include "nh_internal.h"

namespace nh {

namespace {

constexpr int LT = 1024;  // fwd_layer / fwd_attn_out threads
constexpr uint32_t ENGRAM_SEED = 0x9E3779B9u;   // crates/needle-core/src/config.rs:11
constexpr uint32_t ENGRAM_PRIME = 0x01000193u;  // config.rs:12
constexpr int NATIVE_TEAM = 4;                  // infer.rs:38

__device__ __forceinline__ float h2f(uint16_t h) { return f16_bits_to_f32(h); }

// nexp (crates/needle-engine/src/infer.rs:353-367).
__device__ __forceinline__ float nexp(float x) {
    x = fminf(fmaxf(x, bits_f32(0xc2b0c0a5u)), bits_f32(0x42b0c0a5u));
    const float k = __builtin_rintf(x * bits_f32(0x3fb8aa3bu));
    float r = __builtin_fmaf(k, bits_f32(0xbf318000u), x);
    r = __builtin_fmaf(k, bits_f32(0x395e8083u), r);
    float p = __builtin_fmaf(bits_f32(0x39506967u), r, bits_f32(0x3ab743ceu));
    p = __builtin_fmaf(r, p, bits_f32(0x3c088908u));
    p = __builtin_fmaf(r, p, bits_f32(0x3d2aa9c1u));
    p = __builtin_fmaf(r, p, bits_f32(0x3e2aaaaau));
    p = __builtin_fmaf(r, p, 0.5f);
    const float y = __builtin_fmaf(r * r, p, r);
    const float s = __builtin_bit_cast(float, (uint32_t)((int32_t)k << 23) + 0x3f800000u);
    return __builtin_fmaf(s, y, s);
}

// lexpf (infer.rs:84-88): exp in f64, rounded once.
__device__ __forceinline__ float lexpf(float x) { return (float)exp((double)x); }

// rinv (infer.rs:422-424).
__device__ __forceinline__ float rinv(float ss, int n) {
    const float v = ss / (float)n + 1e-6f;
    return 1.0f / __builtin_sqrtf(v);
}

// dot16's combine of its 16 accumulators held by lanes 0..15 (lane
// i16 = 4 j + l holds a[j][l]): t[l] = ((a[2][l] + a[3][l]) + a[1][l]) +
// a[0][l], then (t0 + t1) + (t2 + t3), the result in every lane.  DPP row
// shifts bring lanes l + 4, l + 8, l + 12 to lane l and quad broadcasts
// t0..t3 (no LDS round trips); lanes 0..3 hold the exact value.
__device__ __forceinline__ float dot16_combine(float a) {
    const int ai = __builtin_bit_cast(int, a);
    const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ai, 0x104, 0xF, 0xF, false));
    const float a2 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ai, 0x108, 0xF, 0xF, false));
    const float a3 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ai, 0x10C, 0xF, 0xF, false));
    const float t = ((a2 + a3) + a1) + a;
    const int ti = __builtin_bit_cast(int, t);
    const float t0 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x00, 0xF, 0xF, false));
    const float t1 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x55, 0xF, 0xF, false));
    const float t2 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xAA, 0xF, 0xF, false));
    const float t3 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xFF, 0xF, 0xF, false));
    const float r = (t0 + t1) + (t2 + t3);
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, r)));
}

// dot16 (infer.rs:369-419, portable branch) over a vector held one element
// per lane (n <= 64): lane i16 = 4 j + l carries accumulator a[j][l] over
// 16-element chunks in order; t[l] = ((a[2][l] + a[3][l]) + a[1][l]) +
// a[0][l]; the result (t0 + t1) + (t2 + t3) reaches every lane.
__device__ __forceinline__ float dot16_lanes(float v, int n, int lane) {
    float a = 0.0f;
    const int chunks = n / 16;
    for (int c = 0; c < chunks; ++c) {
        const float x = __shfl(v, c * 16 + (lane & 15), 64);
        a = __builtin_fmaf(x, x, a);
    }
    return dot16_combine(a);
}

// quant_i8's scale (qlinear.rs:92-108) of a value per lane, max over the
// whole wavefront (lanes outside the vector hold 0).
__device__ __forceinline__ float wave_quant_scale(float v) {
    const float m = wave_max_nonneg(fabsf(v));
    return m > 0.0f ? m * bits_f32(0x3c010204u) : 1.0f;
}

// key_chunks (infer.rs:2093-2101): the chunk count and length of n keys,
// at least k = 2 NATIVE_TEAM / nkv chunks past 64 k keys, or 1 for a
// feed's rows (nested, infer.rs:1888).
__host__ __device__ inline void key_chunks(int n, int nkv, bool nested, int& count, int& size) {
    int k = 2 * NATIVE_TEAM / nkv;
    if (k < 1 || nested) k = 1;
    int c = (n + 255) / 256;
    if (k * 64 <= n && c < k) c = k;
    if (c < 1) c = 1;
    const int chunk = ((n + c - 1) / c + 15) / 16 * 16;
    size = chunk;
    count = chunk ? (n + chunk - 1) / chunk : 0;
}

// The attended range of position p0: keys lo..p0.
// slot_of (infer.rs:1749-1756): the KV slot of position p; the sink keeps
// its positions, the rest share the ring.
__device__ __forceinline__ int slot_of(const Dims& D, int p) {
    return (D.ring > 0 && p >= D.sink) ? (p - D.sink) % D.ring + D.sink : p;
}

__host__ __device__ inline int window_lo(int window, int p0) {
    return (window > 0 && p0 + 1 > window) ? p0 + 1 - window : 0;
}

}  // namespace

// argmax (crates/needle-engine/src/generate.rs:42-50): the first maximum.
// The reference's loop keeps index 0 when x[0] is NaN (nothing compares
// greater) and otherwise never moves to a NaN, so NaNs are skipped and a
// NaN first element gives 0.  Each thread keeps the first maximum of its
// strided share (all its loads issued first); a wavefront's first maximum is the smallest index among
// the lanes holding the wavefront's maximum (two DPP reductions; the maximum's sign of zero does not
// matter, the lanes compare equal to it), and the
// same again over the wavefronts' results, by every wavefront (so every
// thread of the NT-thread block returns it; sv / si: NT / 64 entries of LDS).
template <int NT>
__device__ __forceinline__ uint32_t block_argmax(const float* __restrict__ x, int n, float* sv, int* si) {
    constexpr int PER = 16;  // elements per thread read in one batch
    constexpr int NW = NT / 64;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const float x0 = x[0];
    float best = -__builtin_inff();
    int bi = n;
    for (int base = 0; base < n; base += NT * PER) {
        float v[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) v[k] = x[min(base + k * NT + t, n - 1)];
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = base + k * NT + t;
            // a NaN is never greater than the best so far: it never wins
            if (i < n && v[k] == v[k] && (bi == n || v[k] > best)) {
                best = v[k];
                bi = i;
            }
        }
    }
    const float wm = wave_max_ordered(best);
    const int wi = wave_min_i32(best == wm && bi < n ? bi : 0x7fffffff);
    if (lane == 0) {
        sv[wave] = wm;
        si[wave] = wi;
    }
    __syncthreads();
    const float v = lane < NW && si[min(lane, NW - 1)] != 0x7fffffff ? sv[min(lane, NW - 1)] : -__builtin_inff();
    const int ix = lane < NW ? si[min(lane, NW - 1)] : 0x7fffffff;
    const float m = wave_max_ordered(v);
    const int first = wave_min_i32(v == m && ix != 0x7fffffff ? ix : 0x7fffffff);
    return (uint32_t)(first < n && x0 == x0 ? first : 0);
}


// ------------------------------------------------------------------ begin
// Per row i of the feed (position p0 + i): waves for the embedding row
// groups (step.rs:228-235, chunk.rs:58-66: row * sqrt(d) into every lane),
// then per engram site e and group g the hashed row of table g
// (engram_native, infer.rs:1261-1275) dequantized and rotated (QMat::row),
// A8-prepared as group g of the site's activation row i (QAct::new over the
// concatenated rows); missing rows are zeros.  The last t waves: the RoPE
// rows (rope_rows, infer.rs:1716-1747), one row each: for one token right
// after the newest row the reference still keeps (D.rope_prev, the host's
// mirror of its list) the angle-addition recurrence from that row, else
// sincosf(freq * pos); every row also goes to the ring of recent rows.
// PICK (one row, the greedy loop): the row's token is the argmax of the
// previous step's logits (S.logits), worked out by every workgroup (block 0
// stores it at S.tokens[p0]) in place of a launch of its own.
template <bool PICK>
__global__ __launch_bounds__(256) void k_begin(Dims D, Globals G, SessDev S, BeginArgs B, int p0, int t) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    uint32_t pick = 0;
    if constexpr (PICK) {
        __shared__ float sv[4];
        __shared__ int si[4];
        pick = block_argmax<256>(S.logits, D.out_rows, sv, si);
        if (blockIdx.x == 0 && threadIdx.x == 0) S.tokens[p0] = pick;
    }
    // the token at position q of the feed (the picked one at p0)
    auto token = [&](int q) { return PICK && q == p0 ? pick : S.tokens[q]; };
    const int Gd = (D.d + GROUP - 1) / GROUP;
    const int per_row = Gd * (1 + D.sites);
    if (wave < t * per_row) {
        const int i = wave / per_row, r = wave % per_row, pos = p0 + i;
        if (r == 0 && lane == 0) {
            // the block flag of row i: its place in its 32-token chunk below
            // the chunk's length rounded down to 4 (qlinear.rs:397)
            const int tc = min(FWD_ROWS, t - (i & ~(FWD_ROWS - 1)));
            S.flags[i] = (i & (FWD_ROWS - 1)) < tc / 4 * 4;
        }
        if (r < Gd) {
            const uint32_t tok = token(pos);
            float v0, v1;
            if (B.emb.bits == 2)
                row_group<2>(B.emb.codes, B.emb.norms, B.emb.fsel, B.emb.groups, tok, r, lane, v0, v1);
            else
                row_group<4>(B.emb.codes, B.emb.norms, B.emb.fsel, B.emb.groups, tok, r, lane, v0, v1);
            const float scale = __builtin_sqrtf((float)D.d);
            const int i0 = r * GROUP + lane, i1 = i0 + 64;
            float* xs = S.xs + (size_t)i * MHC_LANES * D.d;
            const float e0 = v0 * scale, e1 = v1 * scale;
            for (int b = 0; b < MHC_LANES; ++b) {
                if (i0 < D.d) xs[b * D.d + i0] = e0;
                if (i1 < D.d) xs[b * D.d + i1] = e1;
            }
            if (S.cells) {
                // cell depth 0: the lane mean of the four embedding lanes
                // (step.rs:240-243, chunk.rs:69-70, lane_mean infer.rs:1707-1711)
                float* c = S.cells + (size_t)i * (D.layers + 1) * D.d;
                if (i0 < D.d) c[i0] = (((e0 + e0) + e0) + e0) * 0.25f;
                if (i1 < D.d) c[i1] = (((e1 + e1) + e1) + e1) * 0.25f;
            }
        } else {
            const int e = (r - Gd) / Gd, g = (r - Gd) % Gd;
            float v0 = 0.0f, v1 = 0.0f;
            if (g < D.ntab) {
                const int oi = g / D.eheads, h = g % D.eheads, order = D.orders[oi];
                if (pos + 1 >= order) {
                    uint32_t acc = ENGRAM_SEED * (uint32_t)(oi * D.seed_stride + h + 1);
                    for (int j = 0; j < order; ++j) acc = (acc ^ token(pos - j)) * ENGRAM_PRIME;
                    acc ^= acc >> 15;
                    const uint32_t row = (uint32_t)g * (uint32_t)D.slots + acc % (uint32_t)D.slots;
                    const RowSrc& tb = B.tab[e];
                    if (tb.bits == 2)
                        row_group<2>(tb.codes, tb.norms, tb.fsel, tb.groups, row, 0, lane, v0, v1);
                    else
                        row_group<4>(tb.codes, tb.norms, tb.fsel, tb.groups, row, 0, lane, v0, v1);
                }
            }
            const size_t unit = ((size_t)e * ACT_ROWS + i) * Gd + g;
            a8_group(v0, v1, lane, B.eng_bits[e], S.xq_eng + unit * GROUP, S.sx_eng + unit);
        }
    } else if (wave < t * per_row + t) {
        const int half = D.qk / 2, i = wave - t * per_row;
        if (lane < half) {
            if (t == 1 && D.rope_prev) {
                const size_t prev = (size_t)((p0 + ROPE_RING - 1) % ROPE_RING) * half + lane;
                const float oc = S.rope_rc[prev], os = S.rope_rs[prev];
                const float c = __builtin_fmaf(-G.sd[lane], os, G.cd[lane] * oc);
                const float sn = __builtin_fmaf(G.sd[lane], oc, G.cd[lane] * os);
                S.rope_c[lane] = c;
                S.rope_s[lane] = sn;
                S.rope_rc[(size_t)(p0 % ROPE_RING) * half + lane] = c;
                S.rope_rs[(size_t)(p0 % ROPE_RING) * half + lane] = sn;
            } else {
                double sv, cv;
                sincos((double)(G.freq[lane] * (float)(p0 + i)), &sv, &cv);
                const float c = (float)cv, sn = (float)sv;
                S.rope_c[i * half + lane] = c;
                S.rope_s[i * half + lane] = sn;
                if (i + ROPE_RING >= t) {  // the rows the ring keeps (no two share a slot)
                    S.rope_rc[(size_t)((p0 + i) % ROPE_RING) * half + lane] = c;
                    S.rope_rs[(size_t)((p0 + i) % ROPE_RING) * half + lane] = sn;
                }
            }
        }
    }
}

hipError_t fwd_begin(const Dims& D, const Globals& G, const SessDev& S, const BeginArgs& B, int p0, int t,
                     hipStream_t s, bool pick) {
    const int Gd = (D.d + GROUP - 1) / GROUP;
    const int waves = t * Gd * (1 + D.sites) + t;
    if (pick && t != 1) return hipErrorInvalidValue;
    if (pick)
        hipLaunchKernelGGL(k_begin<true>, dim3((waves + 3) / 4), dim3(256), 0, s, D, G, S, B, p0, t);
    else
        hipLaunchKernelGGL(k_begin<false>, dim3((waves + 3) / 4), dim3(256), 0, s, D, G, S, B, p0, t);
    return hipGetLastError();
}

// ---------------------------------------------------------- engram history
// Per site and row: the value half of key | value as int8 groups of 32
// appended to the site's history, then the dilated causal conv over the
// last ENGRAM_TAPS history rows (infer.rs:1283-1330): dst = fma(tap, s * q,
// dst) from the newest row back, stopping at position 0.  A tap on a row of
// the same feed re-quantizes that row here (the same values its own block
// appends), so no block reads another's writes.
__device__ __forceinline__ int8_t group_quant32(float v, float& s) {
    float m = fabsf(v);
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    s = m > 0.0f ? m * bits_f32(0x3c010204u) : 1.0f;
    return quant_one(v, 1.0f / s);
}

__global__ __launch_bounds__(1024) void k_engram_hist(Dims D, Globals G, SessDev S, int p0) {
    const int e = blockIdx.x, i = blockIdx.y, k = threadIdx.x, d = D.d, pos = p0 + i;
    const bool on = k < d;
    const int kc = on ? k : 0;
    const float* kv = S.ekv + (size_t)e * BATCH_ROWS * 2 * d;
    const int gs = d / 32;
    int8_t* ev8 = S.ev8 + (size_t)e * D.cap * d;
    float* evs = S.evs + (size_t)e * D.cap * gs;
    // Every load first, at clamped in-range addresses: the row's value and,
    // per tap, both sources of its row (the value, for a row of this feed;
    // the int8 history and its scale, for an earlier one) and the tap
    // weight; the taps then pick theirs.
    const float v0 = kv[(size_t)i * 2 * d + d + kc];
    float kvj[ENGRAM_TAPS], hsj[ENGRAM_TAPS], twj[ENGRAM_TAPS];
    int8_t h8j[ENGRAM_TAPS];
#pragma unroll
    for (int j = 0; j < ENGRAM_TAPS; ++j) {
        const int pj = max(pos - j * D.dilation, 0);
        kvj[j] = kv[(size_t)max(pj - p0, 0) * 2 * d + d + kc];
        hsj[j] = evs[(size_t)pj * gs + kc / 32];
        h8j[j] = ev8[(size_t)pj * d + kc];
        twj[j] = G.etaps[((size_t)e * ENGRAM_TAPS + j) * d + kc];
    }
    float s;
    const int8_t q = group_quant32(on ? v0 : 0.0f, s);
    if (on) {
        ev8[(size_t)pos * d + k] = q;
        if ((k & 31) == 0) evs[(size_t)pos * gs + k / 32] = s;
    }
    float dst = 0.0f;
#pragma unroll
    for (int j = 0; j < ENGRAM_TAPS; ++j) {
        if (pos < j * D.dilation) break;
        const int pj = pos - j * D.dilation;
        float qs;
        int8_t q8;
        if (j == 0) {
            qs = s, q8 = q;
        } else if (pj >= p0) {
            q8 = group_quant32(on ? kvj[j] : 0.0f, qs);
        } else {
            qs = on ? hsj[j] : 0.0f;
            q8 = on ? h8j[j] : 0;
        }
        const float tw = on ? twj[j] : 0.0f;
        dst = __builtin_fmaf(tw, qs * (float)q8, dst);
    }
    if (on) S.evals[((size_t)e * BATCH_ROWS + i) * d + k] = dst;
}

hipError_t fwd_engram_hist(const Dims& D, const Globals& G, const SessDev& S, int p0, int t, hipStream_t s) {
    if (D.sites <= 0) return hipSuccess;
    const int threads = (D.d + 63) / 64 * 64;
    hipLaunchKernelGGL(k_engram_hist, dim3(D.sites, t), dim3(threads), 0, s, D, G, S, p0);
    return hipGetLastError();
}

// -------------------------------------------------------------- the layer
// One workgroup of 1024 threads per token row; thread t owns element t of
// every d- and hada_n-long vector (d <= 1024 = hada_n), and element t of each
// of the 4 residual lanes, in registers.  Every global read is issued at the
// start: the Kronecker factors and cond_v land in LDS, the elementwise
// weights, the thread's cond_u column and its wavefront's Phi8 rows in
// registers.  The LDS footprint stays under half a CU's, so two rows of a
// batched feed run on a CU side by side.  The short serial chains (dot16 over d, the gates) run
// in every wavefront that needs their result, so no barrier is spent on
// handing it out.
namespace {

constexpr int BT_STRIDE = HADA_NB + 2;  // padded (even: 8-byte reads) row of a transposed mix8 output
constexpr int MIX_T = 256;              // threads of one mix8 (a 2 x 2 output block each)
constexpr int MIX_STEPS = 4;            // j steps per pipelined batch of a mix8 pass (one 16-byte factor read)
constexpr int KP_PITCH = HADA_NB + 4;   // dwords per pair row of a staged factor (16-byte reads, 2-way banks)
// Transposed copies for the serial chains, so a chain lane reads its
// operands as contiguous 16-byte vectors: a dot16 operand x[16 c + l] at
// l * pitch + c (pitch TP_D for d-long vectors, TP_X for the 4 lanes);
// h2[4 u + jm] at jm * TP_H + u and cond_v[4 u + jm][k] at
// (8 jm + k) * TP_C + u for cond_weights.
constexpr int TP_D = FWD_MAX_D / 16 + 4;
constexpr int TP_X = MHC_LANES * FWD_MAX_D / 16 + 4;
constexpr int TP_H = FWD_MAX_D / 4 + 4;
constexpr int TP_C = FWD_MAX_D / 4 + 8;

struct LayerShared {
    float x2[FWD_MAX_D];
    float h[FWD_MAX_D];
    // The MLP's buffers are dead once its last pass is read; the mHC write
    // then fills the transposed lanes over them.
    union {
        struct {
            alignas(16) float A[HADA_N];
            alignas(16) float B[HADA_NB * BT_STRIDE];
            alignas(16) uint32_t kp[6][HADA_NB / 2 * KP_PITCH];  // Kronecker factors as f16 pairs, pair-major
        };
        alignas(16) float tX[16 * TP_X];
    };
    alignas(16) float C[HADA_N];
    alignas(16) int8_t nx8[MHC_LANES * FWD_MAX_D];
    alignas(16) uint16_t cvT[4 * COND_RANK * TP_C];
    alignas(16) float tA[16 * TP_D];
    alignas(16) float tB[16 * TP_D];
    alignas(16) float hT[4 * TP_H];
    float red[LT / 64];
    float p[64];
    float wk[COND_RANK];
    float r_sx, r_a, r_b, r_c;
    int mix_count;  // the mixer wavefronts' arrivals (mixer_sync)
};

// chain_pipe for a fixed batch count, fully unrolled (batch indices are
// constants, so register arrays indexed by them stay in registers).
template <int NB, int DEPTH, typename Buf, typename Load, typename Chain>
__device__ __forceinline__ void chain_pipe_n(Load load, Chain chain) {
    Buf buf[DEPTH];
#pragma unroll
    for (int i = 0; i < DEPTH - 1 && i < NB; ++i) load(buf[i], i);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (b + DEPTH - 1 < NB) load(buf[(b + DEPTH - 1) % DEPTH], b + DEPTH - 1);
        __builtin_amdgcn_sched_barrier(0);
        chain(buf[b % DEPTH], b);
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int DEPTH, typename Buf, typename Load, typename Chain>
__device__ __forceinline__ void chain_pipe(int nb, Load load, Chain chain);

// chain_pipe with the batch counts of the model's own widths (d = 768: 6
// batches of 8 chunks; 4 d, and cond_weights' 192 steps: 24) fully
// unrolled.  In the loop form the compiler's LDS wait at the loop head
// counts every read in flight, the batch just issued included, so each
// trip through the loop exposes one LDS round trip; unrolled, every wait
// counts exactly and only the reads a batch uses are waited for.
template <int DEPTH, typename Buf, typename Load, typename Chain>
__device__ __forceinline__ void chain_pipe_any(int nb, Load load, Chain chain) {
    auto ch = [&](const Buf& d, int) __attribute__((always_inline)) { chain(d); };
    if (nb == 6)
        chain_pipe_n<6, DEPTH, Buf>(load, ch);
    else if (nb == 24)
        chain_pipe_n<24, DEPTH, Buf>(load, ch);
    else
        chain_pipe<DEPTH, Buf>(nb, load, chain);
}

// mix8 (infer.rs:2343-2380), portable branch: out[r][c] =
// sum_j ct[j][r] * rows[j][c], each output an fma chain from j = 0.  Thread
// u < 256 computes the 2 x 2 block r = 2 (u / 16) + {0, 1}, c = 2 (u % 16) +
// {0, 1}.  The factor operand is read from its pair-major f16 copy (kp[p]
// [j] = the factor's elements [j][2p], [j][2p + 1], p = the thread's pair):
// one 16-byte read per MIX_STEPS steps, beside one 8-byte read of the
// vector operand per step, for four fmas a step.
// Transposed (ct = a factor, rows = [32][32]): stored at out[c * BT_STRIDE + r].
__device__ __forceinline__ void mix8_t(int u, const uint32_t* kp, const float* rows, float* out) {
    const int r = (u >> 4) * 2, c = (u & 15) * 2;
    const uint4* fr = reinterpret_cast<const uint4*>(kp + (u >> 4) * KP_PITCH);
    float o00 = 0.0f, o01 = 0.0f, o10 = 0.0f, o11 = 0.0f;
    struct Buf {
        uint4 f;
        float2 v[MIX_STEPS];
    };
    auto load = [&](Buf& d, int b) {
        d.f = fr[b];
#pragma unroll
        for (int i = 0; i < MIX_STEPS; ++i)
            d.v[i] = *reinterpret_cast<const float2*>(rows + (b * MIX_STEPS + i) * HADA_NB + c);
    };
    auto chain = [&](const Buf& d, int) {
        const uint32_t fw[4] = {d.f.x, d.f.y, d.f.z, d.f.w};
#pragma unroll
        for (int i = 0; i < MIX_STEPS; ++i) {
            const float ax = h2f((uint16_t)(fw[i] & 0xffffu)), ay = h2f((uint16_t)(fw[i] >> 16));
            const float2 b = d.v[i];
            o00 = __builtin_fmaf(ax, b.x, o00);
            o01 = __builtin_fmaf(ax, b.y, o01);
            o10 = __builtin_fmaf(ay, b.x, o10);
            o11 = __builtin_fmaf(ay, b.y, o11);
        }
    };
    chain_pipe_n<HADA_NB / MIX_STEPS, 3, Buf>(load, chain);
    *reinterpret_cast<float2*>(out + c * BT_STRIDE + r) = make_float2(o00, o10);
    *reinterpret_cast<float2*>(out + (c + 1) * BT_STRIDE + r) = make_float2(o01, o11);
}

// Plain (ct = the output of mix8_t, rows = a factor): out[r][c], rows
// r < rows_limit (a multiple of 2).
__device__ __forceinline__ void mix8_n(int u, const float* ct, const uint32_t* kp, float* out, int rows_limit) {
    const int r = (u >> 4) * 2, c = (u & 15) * 2;
    if (r >= rows_limit) return;
    const uint4* fr = reinterpret_cast<const uint4*>(kp + (u & 15) * KP_PITCH);
    float o00 = 0.0f, o01 = 0.0f, o10 = 0.0f, o11 = 0.0f;
    struct Buf {
        uint4 f;
        float2 v[MIX_STEPS];
    };
    auto load = [&](Buf& d, int b) {
        d.f = fr[b];
#pragma unroll
        for (int i = 0; i < MIX_STEPS; ++i)
            d.v[i] = *reinterpret_cast<const float2*>(ct + (b * MIX_STEPS + i) * BT_STRIDE + r);
    };
    auto chain = [&](const Buf& d, int) {
        const uint32_t fw[4] = {d.f.x, d.f.y, d.f.z, d.f.w};
#pragma unroll
        for (int i = 0; i < MIX_STEPS; ++i) {
            const float2 a = d.v[i];
            const float bx = h2f((uint16_t)(fw[i] & 0xffffu)), by = h2f((uint16_t)(fw[i] >> 16));
            o00 = __builtin_fmaf(a.x, bx, o00);
            o01 = __builtin_fmaf(a.x, by, o01);
            o10 = __builtin_fmaf(a.y, bx, o10);
            o11 = __builtin_fmaf(a.y, by, o11);
        }
    };
    chain_pipe_n<HADA_NB / MIX_STEPS, 3, Buf>(load, chain);
    *reinterpret_cast<float2*>(out + r * HADA_NB + c) = make_float2(o00, o01);
    *reinterpret_cast<float2*>(out + (r + 1) * HADA_NB + c) = make_float2(o10, o11);
}

// Element i of a dot16 operand into its transposed copy.
__device__ __forceinline__ void put_t(float* T, int pitch, int i, float v) { T[(i & 15) * pitch + (i >> 4)] = v; }

// A dependent fma chain over nb batches read from LDS: a ring of DEPTH
// batch buffers, batch b + DEPTH - 1's reads issued before batch b's fmas;
// scheduling barriers keep the compiler from sinking the reads back to
// their use (which would leave every batch waiting a full LDS round trip).
// Reads past the last batch are clamped to it (read and ignored).  A chain
// step costs ~13 cycles (the dependent fma's latency) at any depth from 3
// up, so 3 is used.  Requires nb >= 1.
template <int DEPTH, typename Buf, typename Load, typename Chain>
__device__ __forceinline__ void chain_pipe(int nb, Load load, Chain chain) {
    Buf buf[DEPTH];
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i) load(buf[i], min(i, nb - 1));
    int b = 0;
    for (; b + DEPTH <= nb; b += DEPTH) {
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) {
            load(buf[(i + DEPTH - 1) % DEPTH], min(b + i + DEPTH - 1, nb - 1));
            __builtin_amdgcn_sched_barrier(0);
            chain(buf[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i)
        if (b + i < nb) chain(buf[i]);
    if (b + DEPTH - 1 < nb) {
        load(buf[DEPTH - 1], b + DEPTH - 1);
        chain(buf[DEPTH - 1]);
    }
}

// dot16 over operands held transposed (x[16 c + l] at xT[l * pitch + c]),
// the same chains and combine as the reference's dot16: lane l < 16
// carries accumulator l over c in order, in 8-step batches (two 16-byte
// reads per operand) on chain_pipe.
template <bool SELF>
__device__ __forceinline__ float dot16_t(const float* xT, const float* yT, int pitch, int n, int lane) {
    float a = 0.0f;
    if (lane < 16) {
        const int chunks = n / 16, nb = chunks / 8;
        const float4* xr = reinterpret_cast<const float4*>(xT + lane * pitch);
        const float4* yr = reinterpret_cast<const float4*>(yT + lane * pitch);
        struct Buf {
            float4 x[2], y[SELF ? 1 : 2];
        };
        auto load = [&](Buf& d, int b) {
            d.x[0] = xr[2 * b];
            d.x[1] = xr[2 * b + 1];
            if constexpr (!SELF) {
                d.y[0] = yr[2 * b];
                d.y[1] = yr[2 * b + 1];
            }
        };
        auto chain = [&](const Buf& d) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const float4 x = d.x[u];
                float4 y;
                if constexpr (SELF)
                    y = x;
                else
                    y = d.y[u];
                a = __builtin_fmaf(x.x, y.x, a);
                a = __builtin_fmaf(x.y, y.y, a);
                a = __builtin_fmaf(x.z, y.z, a);
                a = __builtin_fmaf(x.w, y.w, a);
            }
        };
        if (nb > 0) chain_pipe_any<3, Buf>(nb, load, chain);
        const float* xs = xT + lane * pitch;
        const float* ys = yT + lane * pitch;
        for (int c = nb * 8; c < chunks; ++c) a = __builtin_fmaf(xs[c], ys[c], a);
    }
    return dot16_combine(a);
}

// A barrier among the mix8 wavefronts only (the other wavefronts go on):
// lane 0 of each adds its arrival to an LDS counter and waits for `target`
// arrivals.  LDS operations of a wavefront complete in order, so the
// wavefront's earlier LDS writes are visible once its arrival is.  The wait
// is bounded: after `limit` polls the wavefront records STATUS_SPIN in the
// session's status word and goes on, so the kernel always ends (the host
// reports the failure at its next synchronization).
__device__ __forceinline__ void mixer_sync(int* count, int target, int limit, int32_t* status) {
    if ((threadIdx.x & 63) == 0) {
        __hip_atomic_fetch_add(count, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        for (int polls = 0; __hip_atomic_load(count, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target;
             ++polls) {
            if (polls >= limit) {
                __hip_atomic_fetch_or(status, STATUS_SPIN, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __builtin_amdgcn_wave_barrier();
}

// rinv(dot16(x, x)) over a transposed operand by wavefront 0, handed to
// the block through LDS.
__device__ __forceinline__ float block_rinv_t(const float* xT, int pitch, int n, float* slot) {
    if ((threadIdx.x >> 6) == 0) {
        const float r = rinv(dot16_t<true>(xT, xT, pitch, n, threadIdx.x & 63), n);
        if (threadIdx.x == 0) *slot = r;
    }
    __syncthreads();
    return *slot;
}

// The same value computed by every wavefront (each runs the 16-lane chain;
// the result is wavefront-uniform and identical in all of them), so no
// barrier hands it over.  The chain is latency-bound (~13 cycles a step),
// so four wavefronts on a SIMD run their copies side by side at about the
// cost of one for d-long operands: the MLP's h2 norm (measured: 0.5 k cycles
// saved).  The other d-long norms (post norm, input norm, the head's norm)
// measured slower this way (decode 501.6 -> 507.5 us per token, prefill
// 1.303 -> 1.332 ms), and for the 4d-long mHC operand the sixteen copies'
// LDS reads cost more than the barrier (0.7 k cycles lost), so those stay on
// wavefront 0.  The phase that follows must not write the operand.
__device__ __forceinline__ float block_rinv_all(const float* xT, int pitch, int n) {
    return rinv(dot16_t<true>(xT, xT, pitch, n, threadIdx.x & 63), n);
}


// The previous layer's inputs and weights a thread needs, read up front.
// The LDS tables go out as one list of 16-byte chunks, up to STAGE_PER per
// thread: [0, 768) the six Kronecker factors (128 each), then cond_v
// (d chunks); cond_u follows them, one 16-byte column per thread.
constexpr int STAGE_PER = 2;

// f16 weights stay raw bits (one per register) until their use:
// converting or packing them on arrival would make the wave wait for each
// load before issuing the next.
struct OutRegs {
    float o, x1, u, pv;
    uint32_t pn, ph, d1, d2, b2, d3, d4;
    int p1, p2;
    uint4 st[STAGE_PER];
    uint4 cu;  // cond_u [k][t], k < 8, as f16 pairs
};

__device__ __forceinline__ OutRegs load_out(int d, const uint4* stage, const uint16_t* pn, const Globals& G,
                                            const SessDev& S, const LayerDev& P) {
    const int t = threadIdx.x;
    OutRegs q{};
    const int kron_n = 6 * HADA_N / 8, cv_n = d * COND_RANK / 8;
    static_assert(STAGE_PER * LT >= 6 * HADA_N / 8 + FWD_MAX_D * COND_RANK / 8, "the stage loads cover the tables");
#pragma unroll
    for (int r = 0; r < STAGE_PER; ++r) {
        const int e = min(t + r * LT, kron_n + cv_n - 1);
        q.st[r] = stage[e];
    }
    q.cu = stage[kron_n + cv_n + t];
    // (unconditional loads: threads past d read element d - 1 and ignore it)
    const int td = min(t, d - 1);
    q.o = S.o[td];
    q.pv = S.p[t & 63];
    q.x1 = S.x1[td];
    q.u = S.u[td];
    // (the loads above take preloaded operands only: none waits for the
    // argument segment, which those below need)
    __builtin_amdgcn_sched_barrier(0);
    q.pn = pn[td];
    q.ph = P.pre_hada[td];
    q.d1 = P.d1[td];
    q.d4 = P.d4[td];
    q.d2 = P.d2[t];
    q.b2 = P.b2[t];
    q.d3 = P.d3[t];
    q.p1 = G.perm1[t];
    q.p2 = G.perm2[t];
    return q;
}

// A raw f16 weight as f32 at its use: the empty asm keeps the conversion
// (and so the wait for the load) from being hoisted up to the load.
__device__ __forceinline__ float h2f_late(uint32_t b) {
    asm volatile("" : "+v"(b));
    return h2f((uint16_t)b);
}

__device__ __forceinline__ void store_out(int d, const OutRegs& q, LayerShared& sh) {
    const int t = threadIdx.x;
    const int kron_n = 6 * HADA_N / 8, cv_n = d * COND_RANK / 8;
#pragma unroll
    for (int r = 0; r < STAGE_PER; ++r) {
        const int e = t + r * LT;
        if (e < kron_n) {
            // 8 f16 of factor row j: pairs 4 (e % 4) + k, stored pair-major
            const int i = e / (HADA_N / 8), ee = e % (HADA_N / 8), j = ee >> 2, p0 = (ee & 3) * 4;
            const uint4 v = q.st[r];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) sh.kp[i][(p0 + k) * KP_PITCH + j] = w[k];
        } else if (e < kron_n + cv_n) {
            // row j of cond_v (8 f16) into column j / 4 of rows 8 (j % 4) + k
            const int j = e - kron_n;
            const uint4 v = q.st[r];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            uint16_t* dst = sh.cvT + (j & 3) * COND_RANK * TP_C + (j >> 2);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                dst[(2 * k) * TP_C] = (uint16_t)(w[k] & 0xffffu);
                dst[(2 * k + 1) * TP_C] = (uint16_t)(w[k] >> 16);
            }
        }
    }
    if (t < d) put_t(sh.tA, TP_D, t, q.o);
    if (t < 64) sh.p[t] = q.pv;
}

// cond_weights (infer.rs:1640-1656) by wavefront 0: lane 8 jm + k carries
// acc[jm][k] = fma(h2[j], cond_v[j][k], .) over j = jm, jm + 4, ...
// (u = j / 4 in order), reading h2 and cond_v from their transposed copies
// in 8-step batches on chain_pipe; then the softmax of the
// combined logits.
__device__ __forceinline__ void cond_weights(const LayerShared& sh, int d, int lane, float* wk) {
    const int k = lane & 7, jm = lane >> 3;
    float a = 0.0f;
    if (lane < 32) {
        const int steps = d / 4, nb = steps / 8;
        const float4* hr = reinterpret_cast<const float4*>(sh.hT + jm * TP_H);
        const uint4* cr = reinterpret_cast<const uint4*>(sh.cvT + (jm * COND_RANK + k) * TP_C);
        struct Buf {
            float4 h[2];
            uint4 c;
        };
        auto load = [&](Buf& d, int b) {
            d.h[0] = hr[2 * b];
            d.h[1] = hr[2 * b + 1];
            d.c = cr[b];
        };
        auto chain = [&](const Buf& d) {
            const float hv[8] = {d.h[0].x, d.h[0].y, d.h[0].z, d.h[0].w, d.h[1].x, d.h[1].y, d.h[1].z, d.h[1].w};
            const uint32_t cw[4] = {d.c.x, d.c.y, d.c.z, d.c.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a = __builtin_fmaf(hv[2 * u], h2f((uint16_t)(cw[u] & 0xffffu)), a);
                a = __builtin_fmaf(hv[2 * u + 1], h2f((uint16_t)(cw[u] >> 16)), a);
            }
        };
        if (nb > 0) chain_pipe_any<3, Buf>(nb, load, chain);
        for (int u = nb * 8; u < steps; ++u)
            a = __builtin_fmaf(sh.hT[jm * TP_H + u], h2f(sh.cvT[(jm * COND_RANK + k) * TP_C + u]), a);
    }
    const float a0 = __shfl(a, k, 64), a1 = __shfl(a, 8 + k, 64), a2 = __shfl(a, 16 + k, 64),
                a3 = __shfl(a, 24 + k, 64);
    const float lg = ((a2 + a3) + a1) + a0;
    float m = lg;
    m = fmaxf(m, quad_xor1(m));
    m = fmaxf(m, quad_xor2(m));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    const float e = lexpf(lg - m);
    float ev[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        ev[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), i));
    const float sum = ev[7] + ((ev[6] + (ev[5] + ev[4])) + ((ev[3] + ev[2]) + (ev[1] + ev[0])));
    const float inv = 1.0f / sum;
    if (lane < 8) wk[lane] = e * inv;
}

// The Hadamard MLP and mHC write of layer P (step.rs:600-705): xl holds the
// thread's element of the 4 lanes (t < d) and gets the new ones; returns
// this thread's max |new lane value| (for the next layer's mHC read).
template <typename BeforeMix, typename AfterMlp>
__device__ float layer_out(const Dims& D, const SessDev& S, const LayerDev& P, const OutRegs& q, LayerShared& sh,
                           float (&xl)[MHC_LANES], BeforeMix before_mix, AfterMlp after_mlp) {
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, d = D.d;
    // mix8 runs on waves 4..7 (threads 256..511), beside cond_weights on wave 0
    const bool mixer = t >= MIX_T && t < 2 * MIX_T;
    const int mu = t - MIX_T;
    // on = zcn16(o, post_norm); x2 = fma(on, sigmoid(attn_gate), x1)
    float x2 = 0.0f;
    {
        const float r = block_rinv_t(sh.tA, TP_D, d, &sh.r_a);
        if (t < d) {
            const float tt = q.o * r;
            const float on = __builtin_fmaf(tt, h2f_late(q.pn), tt);
            x2 = __builtin_fmaf(on, P.ga, q.x1);
            put_t(sh.tB, TP_D, t, x2);
        }
    }
    __syncthreads();
    // h2 = zcn16(x2, pre_hada); z = h2 * d1 zero-padded to hada_n
    float h2 = 0.0f;
    {
        const float r = block_rinv_all(sh.tB, TP_D, d);
        if (t < d) {
            const float tt = x2 * r;
            h2 = __builtin_fmaf(tt, h2f_late(q.ph), tt);
            sh.hT[(t & 3) * TP_H + (t >> 2)] = h2;
        }
        sh.A[t] = t < d ? h2 * h2f_late(q.d1) : 0.0f;
    }
    __syncthreads();
    // cond_weights (wavefront 0) spans both passes of the first mix8; the
    // mixers meet between their passes on their own
    before_mix();
    if (wave == 0) cond_weights(sh, d, lane, sh.wk);
    if (mixer) {
        mix8_t(mu, sh.kp[0], sh.A, sh.B);
        mixer_sync(&sh.mix_count, MIX_T / 64, D.spin_limit, S.status);
        mix8_n(mu, sh.B, sh.kp[1], sh.C, HADA_NB);
    }
    __syncthreads();
    {
        float cond = 1.0f;
        const uint32_t cw[4] = {q.cu.x, q.cu.y, q.cu.z, q.cu.w};
#pragma unroll
        for (int k = 0; k < COND_RANK; ++k)
            cond = __builtin_fmaf(h2f((uint16_t)(cw[k >> 1] >> (16 * (k & 1)))), sh.wk[k], cond);
        float zs = __builtin_fmaf(sh.C[q.p1], cond * h2f_late(q.d2), h2f_late(q.b2));
        zs = zs / (nexp(-zs) + 1.0f);
        sh.A[t] = zs;
    }
    __syncthreads();
    if (mixer) mix8_t(mu, sh.kp[2], sh.A, sh.B);
    __syncthreads();
    if (mixer) mix8_n(mu, sh.B, sh.kp[3], sh.C, HADA_NB);
    __syncthreads();
    sh.A[t] = sh.C[q.p2] * h2f_late(q.d3);
    __syncthreads();
    if (mixer) mix8_t(mu, sh.kp[4], sh.A, sh.B);
    __syncthreads();
    if (mixer) mix8_n(mu, sh.B, sh.kp[5], sh.C, d / HADA_NB / 8 * 8);
    __syncthreads();
    after_mlp();
    // The mHC write: y = (x2 + t3 * d4) - u; lane a = y hpost[a] + sum_b
    // hres[a][b] old[b] as an fma chain over b.
    float m = 0.0f;
    if (t < d) {
        const float* hpost = sh.p + MHC_COLS;
        const float* hres = sh.p + MHC_COLS + MHC_LANES;
        const float y = (x2 + sh.C[t] * h2f_late(q.d4)) - q.u;
        float old[MHC_LANES];
#pragma unroll
        for (int b = 0; b < MHC_LANES; ++b) old[b] = xl[b];
#pragma unroll
        for (int a = 0; a < MHC_LANES; ++a) {
            float v = y * hpost[a];
#pragma unroll
            for (int b = 0; b < MHC_LANES; ++b) v = __builtin_fmaf(old[b], hres[a * MHC_LANES + b], v);
            xl[a] = v;
            put_t(sh.tX, TP_X, a * d + t, v);
            m = fmaxf(m, fabsf(v));
        }
    }
    return m;
}

// The next layer's weights a thread needs, read up front: its norm scale,
// engram key / conv element, and its wavefront's Phi8 rows (16 bytes at
// lane + 64 j of each, j < 4: rows of up to 4096).
constexpr int PHI_CHUNKS = MHC_LANES * FWD_MAX_D / 16 / 64;
constexpr int PHI_B = LT / 64 - 1;  // wavefronts holding Phi8 rows
static_assert(2 * PHI_B >= MHC_COLS, "two Phi8 rows per wavefront cover the 24 rows");
// The one-row kernel issues the rows beside cond_weights, where the mix8
// wavefronts (4-7) are busy: there they are held by the other eleven (MF,
// mixer-free), rows h, h + 11 and, for h < 2, h + 22 on holder h.
constexpr int PHI_MF = PHI_B - MIX_T / 64;
static_assert(3 * PHI_MF >= MHC_COLS && 2 * PHI_MF < MHC_COLS, "holders 0 and 1 take a third row");
__device__ __forceinline__ int phi_holder(int wave) { return wave >= 1 && wave <= 3 ? wave - 1 : wave >= 8 ? wave - 5 : -1; }
// PC: the 1 KB chunks a Phi8 row has (its 4 d int8 / 1024), fixed at compile
// time so a narrower model holds no registers for chunks it never reads (3
// at d = 768: 24 VGPRs instead of 32, which the 64-VGPR batched kernel needs).
template <int PC>
struct InRegs {
    uint32_t norm;
    float kr, ev, ps0, ps1, ps2;
    uint4 r0[PC], r1[PC], r2[PC];
};

template <int PC, bool MF>
__device__ __forceinline__ void load_phi(const Dims& D, const LayerDev& N, InRegs<PC>& q);

// PHI: the Phi8 rows too (else layer_in reads them itself).
template <bool PHI, int PC, bool MF>
__device__ __forceinline__ InRegs<PC> load_in(const Dims& D, const SessDev& S, const LayerDev& N) {
    const int t = threadIdx.x, d = D.d;
    // Unconditional loads at clamped addresses (threads, rows and chunks
    // past the ranges read an in-range element and ignore it; a layer
    // without an engram site reads the projection row instead, which
    // nothing else here reads).
    InRegs<PC> q;
    const int td = min(t, d - 1);
    q.norm = N.norm_in[td];
    const bool site = N.site >= 0;
    const float* kp = site ? S.ekv + (size_t)N.site * BATCH_ROWS * 2 * d : S.proj;
    const float* ep = site ? S.evals + (size_t)N.site * BATCH_ROWS * d : S.proj + d;
    q.kr = kp[td];
    q.ev = ep[td];
    if constexpr (PHI) load_phi<PC, MF>(D, N, q);
    return q;
}

template <int PC, bool MF>
__device__ __forceinline__ void load_phi(const Dims& D, const LayerDev& N, InRegs<PC>& q) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nc = MHC_LANES * D.d;
    if constexpr (MF) {
        const int h = phi_holder(__builtin_amdgcn_readfirstlane(wave));
        if (h >= 0) {
            const int per = nc / 16;
            const bool three = h + 2 * PHI_MF < MHC_COLS;
            const int k2 = min(h + 2 * PHI_MF, MHC_COLS - 1);
            const uint4* row0 = reinterpret_cast<const uint4*>(N.phi_q + (size_t)h * nc);
            const uint4* row1 = reinterpret_cast<const uint4*>(N.phi_q + (size_t)(h + PHI_MF) * nc);
            const uint4* row2 = reinterpret_cast<const uint4*>(N.phi_q + (size_t)k2 * nc);
#pragma unroll
            for (int j = 0; j < PC; ++j) {
                if (64 * j < per) {
                    const int c = min(lane + 64 * j, per - 1);
                    q.r0[j] = row0[c];
                    q.r1[j] = row1[c];
                    if (three) q.r2[j] = row2[c];
                }
            }
            q.ps0 = N.phi_s[h];
            q.ps1 = N.phi_s[h + PHI_MF];
            q.ps2 = N.phi_s[k2];
        }
        return;
    }
    // Phi8 rows: wavefront w >= 1 holds row w - 1, and row w + PHI_B - 1
    // while that is below 24; wavefront 0, which runs the first chain of the
    // MLP right after these loads are issued, holds none, so it never waits
    // behind them in the CU's load queue.  Issuing them takes the CU's
    // address unit ~16 cycles per 1 KB load, so none is issued that is not
    // used: chunk j only while the row has one (a wavefront-uniform test;
    // registers of skipped chunks stay unset and unread).
    const int wu = __builtin_amdgcn_readfirstlane(wave);
    if (wu != 0) {
        const int per = nc / 16;  // uint4 per row
        const int w0 = wu - 1, w1 = min(wu - 1 + PHI_B, MHC_COLS - 1);
        const bool two = wu - 1 + PHI_B < MHC_COLS;
        const uint4* row0 = reinterpret_cast<const uint4*>(N.phi_q + (size_t)w0 * nc);
        const uint4* row1 = reinterpret_cast<const uint4*>(N.phi_q + (size_t)w1 * nc);
#pragma unroll
        for (int j = 0; j < PC; ++j) {
            if (64 * j < per) {
                const int c = min(lane + 64 * j, per - 1);
                q.r0[j] = row0[c];
                if (two) q.r1[j] = row1[c];
            }
        }
        q.ps0 = N.phi_s[w0];
        q.ps1 = N.phi_s[w1];
    }
}

// (The device library's wavefront sum: the DPP form of wave_sum_i32
// measured no faster in the one-row kernel and spilled 8 more bytes in the
// 64-VGPR batched one.)
extern "C" __device__ __attribute__((const)) int __ockl_wfred_add_i32(int);

template <int PC>
__device__ __forceinline__ int dot_row(const uint4* r, const int8_t* x8, int per, int lane) {
    const uint4* xv = reinterpret_cast<const uint4*>(x8);
    int acc = 0;
#pragma unroll
    for (int j = 0; j < PC; ++j) {
        const int i = lane + 64 * j;
        if (i < per) {
            const uint4 b = xv[i];
            acc = __builtin_amdgcn_sdot4((int)r[j].x, (int)b.x, acc, false);
            acc = __builtin_amdgcn_sdot4((int)r[j].y, (int)b.y, acc, false);
            acc = __builtin_amdgcn_sdot4((int)r[j].z, (int)b.z, acc, false);
            acc = __builtin_amdgcn_sdot4((int)r[j].w, (int)b.w, acc, false);
        }
    }
    return __ockl_wfred_add_i32(acc);
}

// The mHC read, engram gate, input norm and A8 of layer N
// (step.rs:400-479).  xl holds the thread's element of the 4 lanes (t < d);
// their transposed copy and the wavefronts' maxima of |xs| are in LDS
// behind a barrier.  The post and residual
// gates of the layer (hpost, the Sinkhorn hres) are computed beside its
// units, off this kernel's path.
template <bool LATE_PHI, int PC, bool MF>
__device__ void layer_in(const Dims& D, const SessDev& S, const LayerDev& N, InRegs<PC> q, int in_bits,
                         LayerShared& sh, const float (&xl)[MHC_LANES]) {
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, d = D.d, nc = MHC_LANES * d;
    // (the Phi8 rows read now land while wavefront 0 runs the norm chain)
    if constexpr (LATE_PHI) load_phi<PC, MF>(D, N, q);
    // every wavefront: r = rinv(dot16(xs)), the amax over the wavefronts'
    // maxima of |xs| (rounding is monotonic, so max_i |xs_i r| =
    // max_i |xs_i| r for r > 0), then the int8 lanes
    {
        const float r = block_rinv_t(sh.tX, TP_X, nc, &sh.r_a);
        float m = sh.red[0];
#pragma unroll
        for (int i = 1; i < LT / 64; ++i) m = fmaxf(m, sh.red[i]);
        m = m * r;
        const float sx = m > 0.0f ? m * bits_f32(0x3c010204u) : 1.0f;
        const float inv = 1.0f / sx;
        if (t < d) {
#pragma unroll
            for (int b = 0; b < MHC_LANES; ++b) sh.nx8[b * d + t] = quant_one(xl[b] * r, inv);
        }
        if (t == 0) sh.r_sx = sx;
    }
    __syncthreads();
    // Phi8 rows: p[k] = (sx * s_k) * idot(phi_q[k], nx8)
    {
        const float sx = sh.r_sx;
        const int per = nc / 16;
        if constexpr (MF) {
            const int h = phi_holder(wave);
            if (h >= 0) {
                const int acc = dot_row<PC>(q.r0, sh.nx8, per, lane);
                const int acc1 = dot_row<PC>(q.r1, sh.nx8, per, lane);
                if (lane == 0) {
                    sh.p[h] = (sx * q.ps0) * (float)acc;
                    sh.p[h + PHI_MF] = (sx * q.ps1) * (float)acc1;
                }
                if (h + 2 * PHI_MF < MHC_COLS) {
                    const int acc2 = dot_row<PC>(q.r2, sh.nx8, per, lane);
                    if (lane == 0) sh.p[h + 2 * PHI_MF] = (sx * q.ps2) * (float)acc2;
                }
            }
        } else if (wave >= 1) {
            const int acc = dot_row<PC>(q.r0, sh.nx8, per, lane);
            if (lane == 0) sh.p[wave - 1] = (sx * q.ps0) * (float)acc;
            if (wave - 1 + PHI_B < MHC_COLS) {
                const int acc1 = dot_row<PC>(q.r1, sh.nx8, per, lane);
                if (lane == 0) sh.p[wave - 1 + PHI_B] = (sx * q.ps1) * (float)acc1;
            }
        }
    }
    __syncthreads();
    // The pre gate hp (sigmoid) in every wavefront, then u and x1.
    float hp[MHC_LANES];
    {
        float g = 0.0f;
        if (lane < MHC_LANES) {
            const float off = lane == N.lane ? 4.0f : -4.0f;
            const float zz = ((sh.p[lane] * N.a_pre) + off) + N.b_pre[lane];
            g = 1.0f / (lexpf(-zz) + 1.0f);
        }
#pragma unroll
        for (int b = 0; b < MHC_LANES; ++b)
            hp[b] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, g), b));
    }
    float u = 0.0f, x1 = 0.0f;
    if (t < d) {
        u = xl[0] * hp[0];
#pragma unroll
        for (int b = 1; b < MHC_LANES; ++b) u = __builtin_fmaf(xl[b], hp[b], u);
        x1 = u;
        put_t(sh.tA, TP_D, t, x1);
        if (N.site >= 0) put_t(sh.tB, TP_D, t, q.kr);
    }
    __syncthreads();
    if (N.site >= 0) {
        // alpha = sigmoid(dot16(x1 / |x1|, k / |k|) / sqrt(d)); x1 += alpha * conv
        if (wave == 1) {
            const float rk = rinv(dot16_t<true>(sh.tB, sh.tB, TP_D, d, lane), d);
            if (lane == 0) sh.r_b = rk;
        }
        const float rx = block_rinv_t(sh.tA, TP_D, d, &sh.r_a);
        const float rk = sh.r_b;
        if (t < d) {
            put_t(sh.tA, TP_D, t, x1 * rx);
            put_t(sh.tB, TP_D, t, q.kr * rk);
        }
        __syncthreads();
        if (wave == 0) {
            const float dd = dot16_t<false>(sh.tA, sh.tB, TP_D, d, lane);
            if (lane == 0) sh.r_c = 1.0f / (lexpf((-dd) / __builtin_sqrtf((float)d)) + 1.0f);
        }
        __syncthreads();
        const float alpha = sh.r_c;
        if (t < d) {
            x1 = __builtin_fmaf(q.ev, alpha, x1);
            put_t(sh.tA, TP_D, t, x1);
        }
        __syncthreads();
    }
    // hloc = norm_apply16(x1, rinv(dot16(x1)), norm_in), then A8.
    {
        const float r = block_rinv_t(sh.tA, TP_D, d, &sh.r_b);
        if (t < d) {
            const float tt = x1 * r;
            sh.h[t] = __builtin_fmaf(tt, h2f_late(q.norm), tt);
            S.u[t] = u;
            S.x1[t] = x1;
        }
    }
    if (t < MHC_COLS) S.p[t] = sh.p[t];
    __syncthreads();
    const int groups = (d + GROUP - 1) / GROUP;
    for (int g = wave; g < groups; g += LT / 64) {
        const int p0 = g * GROUP + lane, p1 = p0 + 64;
        a8_group(p0 < d ? sh.h[p0] : 0.0f, p1 < d ? sh.h[p1] : 0.0f, lane, in_bits, S.xq_in + (size_t)g * GROUP,
                 S.sx_in + g);
    }
}

// The head's input (step.rs:706-728, chunk.rs:331-347): lane mean, zcn with
// the f32 final norm into `hid`, A8 into activation row `arow`.
__device__ void head_in(const Dims& D, const SessDev& S, float fnorm, int head_bits, int arow, LayerShared& sh,
                        const float (&xl)[MHC_LANES]) {
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, d = D.d;
    float mean = 0.0f;
    if (t < d) {
        mean = (((xl[0] + xl[1]) + xl[2]) + xl[3]) * 0.25f;
        put_t(sh.tA, TP_D, t, mean);
    }
    __syncthreads();
    {
        const float r = block_rinv_t(sh.tA, TP_D, d, &sh.r_a);
        if (t < d) {
            const float tt = mean * r;
            const float h = __builtin_fmaf(tt, fnorm, tt);
            sh.x2[t] = h;
            S.hid[(size_t)arow * d + t] = h;
            // NatState::last_hidden: the last row returned (the launch's last block)
            if (blockIdx.x == gridDim.x - 1) S.last_hid[t] = h;
        }
    }
    __syncthreads();
    const int groups = (d + GROUP - 1) / GROUP;
    for (int g = wave; g < groups; g += LT / 64) {
        const int p0 = g * GROUP + lane, p1 = p0 + 64;
        a8_group(p0 < d ? sh.x2[p0] : 0.0f, p1 < d ? sh.x2[p1] : 0.0f, lane, head_bits,
                 S.xq_in + ((size_t)arow * groups + g) * GROUP, S.sx_in + (size_t)arow * groups + g);
    }
}

}  // namespace

// BATCH (a feed of several rows): two rows per CU (at most 64 VGPRs), so
// the next layer's Phi8 rows are read at the start of the mHC read instead
// of beside the MLP.
//
// The operands of everything the first barrier waits for lead the arguments
// as scalars (the previous layer's staged tables and post norm, the row
// buffers, d and row0), so they are preloaded into SGPRs at wave launch.
template <bool PREV, bool NEXT, bool BATCH, int PC>
__global__ __launch_bounds__(LT) __attribute__((amdgpu_waves_per_eu(BATCH ? 8 : 1))) void k_layer(
    const uint4* stage, const float* o, const float* p, float* xs, const float* x1, const float* u, int d, int row0,
    Dims D, Globals G, SessDev S, LayerDev P, LayerDev N, int in_bits, int head_bits, int head_row0) {
    constexpr bool has_prev = PREV, has_next = NEXT;
    __shared__ LayerShared sh;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nc = MHC_LANES * d;
    const int Gd = (d + GROUP - 1) / GROUP;
    // this block's row of every row buffer
    const int row = row0 + blockIdx.x;
    SessDev R = S;
    R.xs = xs + (size_t)row * nc;
    R.u = const_cast<float*>(u) + (size_t)row * d;
    R.x1 = const_cast<float*>(x1) + (size_t)row * d;
    R.p = const_cast<float*>(p) + (size_t)row * 64;
    R.o = const_cast<float*>(o) + (size_t)row * d;
    R.ekv += (size_t)row * 2 * d;
    R.evals += (size_t)row * d;
    R.xq_in += (size_t)row * Gd * GROUP;
    R.sx_in += (size_t)row * Gd;
    // every global read first, then the LDS stores; thread t < d holds
    // element t of each lane
    const int td = min(t, d - 1);
    float xl[MHC_LANES];
#pragma unroll
    for (int k = 0; k < MHC_LANES; ++k) xl[k] = R.xs[k * d + td];
    OutRegs qo;
    if constexpr (has_prev) qo = load_out(d, stage, P.post_norm, G, R, P);
    InRegs<PC> qi;
    float fnorm = 0.0f;
    // Without a previous layer nothing else loads: the next layer's reads
    // go now.  With one they go after the first barrier: the Phi8 rows are
    // half the kernel's bytes and are not needed before the mHC read, so
    // they stay out of the way of the tables the MLP waits for.
    if constexpr (has_next && !has_prev) qi = load_in<!BATCH, PC, !BATCH>(D, R, N);
    if constexpr (!has_next) fnorm = G.final_norm[min(t, d - 1)];
    float m = 0.0f;
    if (t == 0) sh.mix_count = 0;
    // With a previous layer the lanes' transposed copy is written by its
    // mHC write (over the MLP's buffers, which store_out fills now).
    if constexpr (!has_prev) {
        if (t < d) {
#pragma unroll
            for (int k = 0; k < MHC_LANES; ++k) {
                put_t(sh.tX, TP_X, k * d + t, xl[k]);
                m = fmaxf(m, fabsf(xl[k]));
            }
        }
    }
    if constexpr (has_prev) store_out(d, qo, sh);
    __syncthreads();
    if constexpr (has_next && has_prev) qi = load_in<false, PC, !BATCH>(D, R, N);
    // The Phi8 rows (72 KB at d = 768, ~16 cycles of the CU's address unit
    // per 1 KB wavefront load): one row alone issues them where wavefront 0
    // runs cond_weights, the longest chain of the MLP, and the other
    // wavefronts wait for it anyway (issued right after the first barrier
    // they held the post norm's barrier back); batched, once the MLP's
    // registers are free.
    if constexpr (has_prev)
        m = layer_out(
            D, S, P, qo, sh, xl,
            [&]() __attribute__((always_inline)) {
                if constexpr (has_next && !BATCH) load_phi<PC, true>(D, N, qi);
            },
            [&]() __attribute__((always_inline)) {
                if constexpr (has_next && BATCH) load_phi<PC, false>(D, N, qi);
            });
    // the wavefronts' maxima of |xs| for the mHC read
    m = wave_max_nonneg(m);
    if (lane == 0) sh.red[wave] = m;
    __syncthreads();
    // (the new lanes go back to HBM last: nothing here reads them there, and
    // stores issued earlier would sit in the memory counter ahead of loads
    // that are waited for)
    if constexpr (has_next)
        layer_in<BATCH && !has_prev, PC, !BATCH>(D, R, N, qi, in_bits, sh, xl);
    else if ((int)blockIdx.x >= head_row0)  // (uniform over the block)
        head_in(D, S, fnorm, head_bits, blockIdx.x - head_row0, sh, xl);  // row i - row0 - head_row0
    if constexpr (has_prev) {
        if (t < d) {
#pragma unroll
            for (int k = 0; k < MHC_LANES; ++k) R.xs[k * d + t] = xl[k];
            // the cell of layer P: the lane mean after its mHC write
            // (step.rs:672-694, chunk.rs:310, lane_mean infer.rs:1707-1711)
            if (S.cells)
                S.cells[((size_t)row * (D.layers + 1) + P.index + 1) * d + t] =
                    (((xl[0] + xl[1]) + xl[2]) + xl[3]) * 0.25f;
        }
    }
}

template <bool BATCH, int PC>
static void launch_layer(const Dims& D, const Globals& G, const SessDev& S, const LayerDev* prev,
                         const LayerDev* next, int row0, int rows, int in_bits, int head_bits, int head_row0,
                         hipStream_t s) {
    const LayerDev none{};
    const uint4* stage = prev ? reinterpret_cast<const uint4*>(prev->stage) : nullptr;
#define NH_LAYER(HP, HN, PV, NX)                                                                                  \
    hipLaunchKernelGGL((k_layer<HP, HN, BATCH, PC>), dim3(rows), dim3(LT), 0, s, stage, S.o, S.p, S.xs, S.x1,     \
                       S.u, D.d, row0, D, G, S, PV, NX, in_bits, head_bits, head_row0)
    if (prev && next)
        NH_LAYER(true, true, *prev, *next);
    else if (next)
        NH_LAYER(false, true, none, *next);
    else if (prev)
        NH_LAYER(true, false, *prev, none);
    else
        NH_LAYER(false, false, none, none);
#undef NH_LAYER
}

hipError_t fwd_layer(const Dims& D, const Globals& G, const SessDev& S, const LayerDev* prev, const LayerDev* next,
                     int row0, int rows, int in_bits, int head_bits, hipStream_t s, int head_row0) {
    // A feed's 64-VGPR kernel sized for a Phi8 row of at most three 1 KB
    // chunks (d <= 768: no spills) or of four.  The one-row kernel has no
    // register cap and keeps the four-chunk form (measured no faster with
    // three).
    if (rows > 1) {
        if (MHC_LANES * D.d <= 3 * 1024)
            launch_layer<true, 3>(D, G, S, prev, next, row0, rows, in_bits, head_bits, head_row0, s);
        else
            launch_layer<true, PHI_CHUNKS>(D, G, S, prev, next, row0, rows, in_bits, head_bits, head_row0, s);
    } else {
        launch_layer<false, PHI_CHUNKS>(D, G, S, prev, next, row0, rows, in_bits, head_bits, head_row0, s);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ units
// sinkhorn64 (infer.rs:2501-2528) by 16 lanes, lane = 4 r + c holding
// e[r][c]: row sums ((e0 + e1) + (e2 + e3)), column sums
// ((e[c] + e[4 + c]) + (e[8 + c] + e[12 + c])), 20 rounds, in f64.
// A double moved across lanes by one DPP pattern (both halves).
template <int CTRL>
__device__ __forceinline__ double dpp64(double x) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, x);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, (unsigned long long)(unsigned)lo | ((unsigned long long)(unsigned)hi << 32));
}

__device__ __forceinline__ float sinkhorn_lane(float z, int lane) {
    const int r = (lane >> 2) & 3;
    // the row's four elements by DPP quad broadcasts (row r is a quad)
    const int zi = __builtin_bit_cast(int, z);
    const float z0 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, zi, 0x00, 0xF, 0xF, false)),
                z1 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, zi, 0x55, 0xF, 0xF, false)),
                z2 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, zi, 0xAA, 0xF, 0xF, false)),
                z3 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, zi, 0xFF, 0xF, 0xF, false));
    const double m = (double)fmaxf(fmaxf(z0, z1), fmaxf(z2, z3));
    double e = exp((double)z - m);
    // Both sums are (x0 + x1) + (x2 + x3) over the row's (column's)
    // elements in order.  A row's lanes are a quad: lane c gets element
    // c ^ j from quad permutes j = 1, 2, 3, and since IEEE addition is
    // commutative, (y0 + y1) + (y2 + y3) over them is the same sum in every
    // lane.  A column's elements sit 4 lanes apart: rotations by 4, 8, 12
    // within the 16 lanes bring rows r +- 1, r +- 2, r -+ 1, so the sum
    // pairs (w0 + w1) + (w2 + w3) when row r and the first rotation's row
    // differ in bit 0 only, else (w0 + w3) + (w1 + w2); the first
    // rotation's row comes from rotating r itself.
    const int r1 = __builtin_amdgcn_update_dpp(0, r, 0x124, 0xF, 0xF, false);
    const bool pair01 = (r ^ r1) == 1;
    for (int it = 0; it < 20; ++it) {
        {
            const double y1 = dpp64<0xB1>(e), y2 = dpp64<0x4E>(e), y3 = dpp64<0x1B>(e);
            const double inv = 1.0 / ((e + y1) + (y2 + y3));
            e *= inv;
        }
        {
            const double w1 = dpp64<0x124>(e), w2 = dpp64<0x128>(e), w3 = dpp64<0x12C>(e);
            const double sa = (e + w1) + (w2 + w3), sb = (e + w3) + (w1 + w2);
            const double inv = 1.0 / (pair01 ? sa : sb);
            e *= inv;
        }
    }
    return (float)e;
}

// The post and residual gates of the layer (step.rs:636-660), written
// after the 24 mHC projections of a row: hpost[j] = 2 sigmoid(p_post[j]
// a_post + off_j + b_post[j]) at 24, hres = sinkhorn64(fma(p_res, a_res,
// b_res)) at 28.  One wavefront, beside the attention output of the row.
__device__ __forceinline__ void post_gates(float* p, const LayerDev& L, int lane) {
    const int k = lane & 15;
    const float z = __builtin_fmaf(p[2 * MHC_LANES + k], L.a_res, L.b_res[k]);
    const float hr = sinkhorn_lane(z, lane);
    if (lane < 16) p[MHC_COLS + MHC_LANES + lane] = hr;
    if (lane < MHC_LANES) {
        const float off = lane == L.lane ? 0.0f : -4.0f;
        const float zz = ((p[MHC_LANES + lane] * L.a_post) + off) + L.b_post[lane];
        p[MHC_COLS + lane] = 2.0f / (lexpf(-zz) + 1.0f);
    }
}


// A unit's inputs for lane i of feed row `row` (position pos): the pre-tap
// value, the taps, the earlier pre-tap rows (rows of the same feed from the
// projection, older ones from the history ring), and (normed units) the
// norm scale and the row's RoPE entry.  Every load is unconditional (lanes,
// taps and rows past the ranges read a clamped in-range address; `norm` is
// read for every unit, used by the normed ones) and raw, so all of them
// issue before the first wait.
struct UnitIn {
    float cur, rc, rs;
    uint16_t nrm;
    uint16_t w[DG_MAX_TAPS];
    float h[DG_MAX_TAPS];
};

template <int TAPS, bool EXACT>
__device__ __forceinline__ UnitIn unit_load(const Dims& D, const SessDev& S, int layer, int pos, int row, int start,
                                            int cw, int cc, int len, const uint16_t* w, const uint16_t* norm, int i) {
    const float* hist = S.hist + (size_t)layer * D.hist_slots * D.W;
    const int ii = i < len ? i : 0;
    UnitIn u{};
    u.cur = S.proj[(size_t)row * D.nq + start + ii];
#pragma unroll
    for (int j = 0; j < TAPS; ++j) {
        const int jj = EXACT || j < D.taps ? j : D.taps - 1;
        u.w[j] = w[(size_t)jj * cw + cc + ii];
        if (j > 0) {
            const int pj = pos >= jj ? pos - jj : 0;
            const float* src = jj <= row ? S.proj + (size_t)(row - jj) * D.nq
                                         : hist + (size_t)(pj % D.hist_slots) * D.W;
            u.h[j] = src[start + ii];
        }
    }
    {
        const int qi = i < D.qk ? i : 0, half = D.qk / 2, f = qi < half ? qi : qi - half;
        u.nrm = norm[qi];
        u.rc = S.rope_c[row * half + f];
        u.rs = S.rope_s[row * half + f];
    }
    return u;
}

// The unit's post-tap value (zcn16 and RoPE when `normed`): the causal conv
// over the row and the earlier pre-tap rows, v = w0 cur, then
// fma(w_j, row_{pos - j}, v) (a row the history no longer holds, before
// D.hist_lo, is zero; hist_lo <= the feed's first position, so rows of the
// feed always count); the row's pre-tap value goes to the ring at pos.
template <int TAPS, bool EXACT>
__device__ __forceinline__ float unit_finish(const Dims& D, const SessDev& S, int layer, int pos, int start, int len,
                                             const UnitIn& u, bool normed, int i, bool write_hist) {
    float v = 0.0f;
    if (i < len) {
        v = h2f(u.w[0]) * u.cur;
#pragma unroll
        for (int j = 1; j < TAPS; ++j)
            if (EXACT || j < D.taps) v = __builtin_fmaf(h2f(u.w[j]), pos - j >= D.hist_lo ? u.h[j] : 0.0f, v);
        if (write_hist) S.hist[((size_t)layer * D.hist_slots + pos % D.hist_slots) * D.W + start + i] = u.cur;
    }
    if (normed) {
        const int qk = D.qk;
        const float ss = dot16_lanes(v, qk, i);
        const float r = rinv(ss, qk);
        if (i < qk) {
            const float tt = v * r;
            v = __builtin_fmaf(tt, h2f(u.nrm), tt);
        }
        const int half = qk / 2, f = i < half ? i : i - half;
        const float a = __shfl(v, f, 64), b = __shfl(v, f + half, 64);
        if (i < qk) v = i < half ? __builtin_fmaf(-u.rs, b, u.rc * a) : __builtin_fmaf(u.rs, a, u.rc * b);
    }
    return v;
}

// Block i: row i's units, one wavefront per unit (q heads, k heads,
// v heads; step.rs:481-556, chunk.rs:202-253), lane = element: the causal
// conv over the row and the pre-tap rows before it (fma from the newest
// back; a row before position 0 contributes fma(w, 0, v)), then for q and
// k the head zcn16 and RoPE, and for k and v the int8 cache append.  Rows
// of the same feed are read from the projection, earlier ones from the
// history ring; the row's pre-tap values go to the ring at a slot no row of
// the feed reads.
template <int TAPS, bool EXACT>
__global__ __launch_bounds__(MAX_UNITS * 64) void k_units(Dims D, SessDev S, LayerDev L, int layer, int p0, int t) {
    const int unit = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), i = threadIdx.x & 63;
    const int row = blockIdx.x, pos = p0 + row;
    const int nh = D.nh, nkv = D.nkv, qk = D.qk, vd = D.vd;
    const int qd = nh * qk, kd = nkv * qk, vdim = nkv * vd;
    // the unit's inputs (wave-uniform branches, each with constant argument
    // fields); waves past the units load the last v unit's and ignore them
    const int uu = min(unit, nh + 2 * nkv - 1);
    int start, len;
    UnitIn u;
    if (uu < nh) {
        start = uu * qk, len = qk;
        u = unit_load<TAPS, EXACT>(D, S, layer, pos, row, start, qd, uu * qk, qk, L.q_taps, L.q_norm, i);
    } else if (uu < nh + nkv) {
        const int kh = uu - nh;
        start = qd + kh * qk, len = qk;
        u = unit_load<TAPS, EXACT>(D, S, layer, pos, row, start, kd, kh * qk, qk, L.k_taps, L.k_norm, i);
    } else {
        const int vh = uu - nh - nkv;
        start = qd + kd + vh * vd, len = vd;
        u = unit_load<TAPS, EXACT>(D, S, layer, pos, row, start, vdim, vh * vd, vd, L.v_taps, L.k_norm, i);
    }
    if (unit >= nh + 2 * nkv) return;
    const float v = unit_finish<TAPS, EXACT>(D, S, layer, pos, start, len, u, unit < nh + nkv, i, t <= FWD_ROWS);
    if (unit < nh) {
        if (i < qk) S.qbuf[(size_t)row * qd + start + i] = v;
    } else {
        const float s = wave_quant_scale(i < len ? v : 0.0f);
        const int8_t q = quant_one(v, 1.0f / s);
        const size_t lc = (size_t)layer * D.cap;
        const int slot = slot_of(D, pos);
        // A ring shorter than the feed gives two of its rows one slot: the
        // later position keeps it (the slot map says so; the reference's
        // members would race there).
        const bool taken = D.ring > 0 && pos >= D.sink && pos + D.ring < p0 + t;
        if (taken) return;
        if (unit < nh + nkv) {
            const int kh = unit - nh;
            if (i < qk) S.k8[((lc + slot) * nkv + kh) * qk + i] = q;
            if (i == 0) S.ks[(lc + slot) * nkv + kh] = s;
        } else {
            const int vh = unit - nh - nkv;
            if (i < vd) S.v8t[(((size_t)layer * nkv + vh) * vd + i) * D.vcap + slot] = q;
            if (i == 0) S.vs[(lc + slot) * nkv + vh] = s;
        }
    }
}

hipError_t fwd_units(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int t, hipStream_t s) {
    const int units = D.nh + 2 * D.nkv;
    switch (D.taps) {
#define NH_UNITS(TP, EX) \
    hipLaunchKernelGGL((k_units<TP, EX>), dim3(t), dim3(units * 64), 0, s, D, S, L, layer, p0, t)
        case 1: NH_UNITS(1, true); break;
        case 2: NH_UNITS(2, true); break;
        case 3: NH_UNITS(3, true); break;
        case 4: NH_UNITS(4, true); break;
        default: NH_UNITS(DG_MAX_TAPS, false);
#undef NH_UNITS
    }
    return hipGetLastError();
}

// The sum of an integer over each group of four lanes (DPP quad permutes;
// integer adds are exact in any order).
__device__ __forceinline__ int quad_sum_i32(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    return v;
}

// -------------------------------------------------------------- attention
// attend_head_ref (infer.rs:1871-2007), one workgroup per (query head,
// key chunk): q as int8 (scale x INV_SQRT_QK), int8 scores
// (k-scale x dot) x qs for the 4-blocked prefix and (k-scale x qs) x dot
// for the rest, the chunk max, chunk_exp (nexp over the 4-blocked prefix
// summed in 8 lane classes, lexpf over the tail, infer.rs:2222-2279), the
// weights times v-scales as 21-bit digits (digits21, infer.rs:2171-2220)
// and their exact integer P.V with the int8 values.  The chunk's key rows,
// scales and value columns are staged in LDS with every load in flight at
// once (value dwords of the transposed cache from the dword boundary at or
// before the chunk's first slot; the digits are shifted by the same
// offset, so bytes before the first key meet zero digits), and P.V runs
// four keys per sdot4.
// The two coarse key ranges of a query at pos under an attention span
// (key_ranges, infer.rs:1781-1791): [lo, max(lo, min(sink, pos + 1))) and
// [min(max(end - ring, sink), pos + 1), pos + 1); the ring part is not cut
// by the layer's window.
__host__ __device__ inline void span_ranges(const Dims& D, const KeySpan& K, int lo, int pos, int& alo, int& ahi,
                                            int& blo, int& bhi) {
    alo = lo;
    ahi = max(lo, min(D.sink, pos + 1));
    blo = min(max(K.end - D.ring, D.sink), pos + 1);
    bhi = pos + 1;
}

__host__ __device__ inline int span_overlap(int lo, int hi, int a, int b) { return max(0, min(hi, b) - max(lo, a)); }

// The number of keys: the span's live runs cut to the two ranges.
__host__ __device__ inline int span_count(const KeySpan& K, int alo, int ahi, int blo, int bhi) {
    int n = 0;
    for (int r = 0; r < K.nrun; ++r)
        n += span_overlap(K.lo[r], K.hi[r], alo, ahi) + span_overlap(K.lo[r], K.hi[r], blo, bhi);
    return n;
}

// The position of key k (ascending: every position of the first range lies
// below the sink, every one of the second at or past it).
__device__ __forceinline__ int span_key(const KeySpan& K, int alo, int ahi, int blo, int bhi, int k) {
    for (int r = 0; r < K.nrun; ++r) {
        const int ca = span_overlap(K.lo[r], K.hi[r], alo, ahi);
        if (k < ca) return max(K.lo[r], alo) + k;
        k -= ca;
        const int cb = span_overlap(K.lo[r], K.hi[r], blo, bhi);
        if (k < cb) return max(K.lo[r], blo) + k;
        k -= cb;
    }
    return 0;
}

// The key count of a query at pos: every position from the window's start
// without a span.
__device__ __forceinline__ int key_count(const Dims& D, const KeySpan& K, bool span, int window, int pos) {
    const int lo = window_lo(window, pos);
    if (!span) return pos + 1 - lo;
    int alo, ahi, blo, bhi;
    span_ranges(D, K, lo, pos, alo, ahi, blo, bhi);
    return span_count(K, alo, ahi, blo, bhi);
}

constexpr int ATT_KPITCH = MAX_HEAD_DIM + 16;        // key row (80 bytes: 8 rows cover the 32 banks)
constexpr int ATT_PITCH = ATT_CHUNK_MAX + 8;         // value / digit row: 3 alignment bytes + 256 keys + tail
constexpr int ATT_VDW = (ATT_CHUNK_MAX + 3 + 3) / 4; // value dwords per column

//
// With an attention span (SPAN) the keys are the span's live positions (the
// reference's key runs) in their KV slots (slot_of): each key's slot is
// found first, then the key rows, scales and value bytes are gathered from
// those slots (value column j = key j, no alignment offset).
template <bool SPAN>
__global__ __launch_bounds__(ATT_THREADS) void k_attend(Dims D, SessDev S, LayerDev L, int layer, int p0, int rows,
                                                        KeySpan K) {
    const int row = blockIdx.x / D.nh, hh = blockIdx.x % D.nh, ci = blockIdx.y, t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63, pos = p0 + row;
    const int nkv = D.nkv, qk = D.qk, vd = D.vd, kvh = hh / (D.nh / nkv);
    const int lo = window_lo(L.window, pos);
    int alo = 0, ahi = 0, blo = 0, bhi = 0, n;
    if constexpr (SPAN) {
        span_ranges(D, K, lo, pos, alo, ahi, blo, bhi);
        n = span_count(K, alo, ahi, blo, bhi);
    } else {
        n = pos + 1 - lo;
    }
    int count, chunk;
    key_chunks(n, nkv, rows > 1, count, chunk);
    if (ci >= count) return;
    const int c0 = ci * chunk, len = min(chunk, n - c0), blocked = len / 4 * 4, slot0 = lo + c0;
    const int sh = SPAN ? 0 : slot0 & 3, base = slot0 - sh, cols = sh + len;
    __shared__ alignas(16) int8_t ks8[ATT_CHUNK_MAX][ATT_KPITCH];
    __shared__ alignas(16) int8_t vs8[MAX_HEAD_DIM][ATT_PITCH];
    __shared__ float kss[ATT_CHUNK_MAX], vss[ATT_CHUNK_MAX];
    __shared__ alignas(16) int8_t q8[MAX_HEAD_DIM];
    __shared__ float sc[ATT_CHUNK_MAX];
    __shared__ alignas(16) int8_t dig[3][ATT_PITCH];
    __shared__ float red[ATT_THREADS / 64];
    __shared__ float s_qs, s_sum;
    __shared__ int kslot[SPAN ? ATT_CHUNK_MAX : 1];
    const size_t lc = (size_t)layer * D.cap;
    // every load first (unconditional, at clamped in-range addresses)
    const float qv = S.qbuf[((size_t)row * D.nh + hh) * qk + min(lane, qk - 1)];
    constexpr int KR = ATT_CHUNK_MAX * 4 / ATT_THREADS, VR = (MAX_HEAD_DIM * ATT_VDW + ATT_THREADS - 1) / ATT_THREADS;
    const int rq = qk / 16, vdw = (cols + 3) / 4;
    if constexpr (SPAN) {
        if (t < len) kslot[t] = slot_of(D, span_key(K, alo, ahi, blo, bhi, c0 + t));
        __syncthreads();
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            const int e = t + r * ATT_THREADS, i = e >> 2, c = e & 3;
            if (i < len && c < rq)
                reinterpret_cast<uint4*>(ks8[i])[c] =
                    reinterpret_cast<const uint4*>(S.k8 + ((lc + kslot[i]) * nkv + kvh) * qk)[c];
        }
        if (t < len) {
            kss[t] = S.ks[(lc + kslot[t]) * nkv + kvh];
            vss[t] = S.vs[(lc + kslot[t]) * nkv + kvh];
        }
        const int8_t* vcol = S.v8t + ((size_t)layer * nkv + kvh) * vd * D.vcap;
        for (int e = t; e < vd * len; e += ATT_THREADS) {
            const int dm = e / len, i = e % len;
            vs8[dm][i] = vcol[(size_t)dm * D.vcap + kslot[i]];
        }
        if (wave == 0) {
            const float s = wave_quant_scale(lane < qk ? qv : 0.0f);
            if (lane < qk) q8[lane] = quant_one(qv, 1.0f / s);
            if (lane == 0) s_qs = s * bits_f32(0x3e13cd3au);
        }
    } else {
        uint4 kr[KR];
        uint32_t vw[VR];
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            const int e = t + r * ATT_THREADS, i = min(e >> 2, len - 1), c = min(e & 3, rq - 1);
            kr[r] = reinterpret_cast<const uint4*>(S.k8 + ((lc + slot0 + i) * nkv + kvh) * qk)[c];
        }
        float ksr, vsr;
        {
            const int i = min(t, len - 1);
            ksr = S.ks[(lc + slot0 + i) * nkv + kvh];
            vsr = S.vs[(lc + slot0 + i) * nkv + kvh];
        }
        const int8_t* vcol = S.v8t + ((size_t)layer * nkv + kvh) * vd * D.vcap + base;
#pragma unroll
        for (int r = 0; r < VR; ++r) {
            const int e = t + r * ATT_THREADS, dm = min(e / ATT_VDW, vd - 1), k = min(e % ATT_VDW, vdw - 1);
            vw[r] = reinterpret_cast<const uint32_t*>(vcol + (size_t)dm * D.vcap)[k];
        }
        if (wave == 0) {
            const float s = wave_quant_scale(lane < qk ? qv : 0.0f);
            if (lane < qk) q8[lane] = quant_one(qv, 1.0f / s);
            if (lane == 0) s_qs = s * bits_f32(0x3e13cd3au);
        }
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            const int e = t + r * ATT_THREADS, i = e >> 2, c = e & 3;
            if (i < len && c < rq) reinterpret_cast<uint4*>(ks8[i])[c] = kr[r];
        }
        if (t < len) {
            kss[t] = ksr;
            vss[t] = vsr;
        }
#pragma unroll
        for (int r = 0; r < VR; ++r) {
            const int e = t + r * ATT_THREADS, dm = e / ATT_VDW, k = e % ATT_VDW;
            if (dm < vd && k < vdw) {
                if (4 * k + 3 < cols) {
                    reinterpret_cast<uint32_t*>(vs8[dm])[k] = vw[r];
                } else {
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        if (4 * k + b < cols) vs8[dm][4 * k + b] = (int8_t)(vw[r] >> (8 * b));
                }
            }
        }
    }
    __syncthreads();
    const float qs = s_qs;
    float mx = -__builtin_inff();
    {
        uint4 qw[MAX_HEAD_DIM / 16];
#pragma unroll
        for (int c = 0; c < MAX_HEAD_DIM / 16; ++c)
            qw[c] = c < rq ? reinterpret_cast<const uint4*>(q8)[c] : make_uint4(0, 0, 0, 0);
        for (int i = t; i < len; i += ATT_THREADS) {
            int dot = 0;
            // every 16-byte chunk of the key row, the query's past qk zero
            // (the integer dot is the same; no branch between the reads)
#pragma unroll
            for (int c = 0; c < MAX_HEAD_DIM / 16; ++c) {
                const uint4 kv = reinterpret_cast<const uint4*>(ks8[i])[c];
                dot = __builtin_amdgcn_sdot4((int)kv.x, (int)qw[c].x, dot, false);
                dot = __builtin_amdgcn_sdot4((int)kv.y, (int)qw[c].y, dot, false);
                dot = __builtin_amdgcn_sdot4((int)kv.z, (int)qw[c].z, dot, false);
                dot = __builtin_amdgcn_sdot4((int)kv.w, (int)qw[c].w, dot, false);
            }
            const float ksc = kss[i];
            const float sv = i < blocked ? (ksc * (float)dot) * qs : (ksc * qs) * (float)dot;
            sc[i] = sv;
            mx = fmaxf(mx, sv);
        }
    }
    mx = wave_max_ordered(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int i = t; i < len; i += ATT_THREADS) sc[i] = i < blocked ? nexp(sc[i] - mx) : lexpf(sc[i] - mx);
    __syncthreads();
    if (wave == 0) {
        // a[k] over the 8-blocks' first halves plus a trailing 4-block,
        // b[k] over their second halves (lane 4 hi + k sums sc[8 b + 4 hi + k]
        // over b in order, batches of 8 loads ahead of their adds)
        float acc = 0.0f;
        const int nb8 = len / 8;
        if (lane < 8) {
            const int k = lane & 3, hi = lane >> 2;
            const float* col = &sc[hi * 4 + k];
            int b = 0;
            for (; b + 8 <= nb8; b += 8) {
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = col[(b + j) * 8];
#pragma unroll
                for (int j = 0; j < 8; ++j) acc += v[j];
            }
            for (; b < nb8; ++b) acc += col[b * 8];
            if (hi == 0 && len - nb8 * 8 >= 4) acc += sc[nb8 * 8 + k];
        }
        // t = a + b; (t0 + t1) + (t2 + t3) (DPP; exact in lane 0)
        const float tk = acc + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc),
                                                                                       0x104, 0xF, 0xF, false));
        const int ti = __builtin_bit_cast(int, tk);
        const float t0 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x00, 0xF, 0xF, false));
        const float t1 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x55, 0xF, 0xF, false));
        const float t2 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xAA, 0xF, 0xF, false));
        const float t3 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xFF, 0xF, 0xF, false));
        float sum = (t0 + t1) + (t2 + t3);
        int i = blocked;
        if (len - i >= 2) {
            sum = (sc[i] + sum) + sc[i + 1];
            i += 2;
        }
        if (len - i == 1) sum += sc[i];
        if (lane == 0) s_sum = sum;
    }
    __syncthreads();
    float wmax = 0.0f;
    for (int i = t; i < len; i += ATT_THREADS) {
        const float w = sc[i] * vss[i];
        sc[i] = w;
        wmax = fmaxf(wmax, w);
    }
    wmax = wave_max_nonneg(wmax);
    if (lane == 0) red[wave] = wmax;
    __syncthreads();
    wmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float qw = bits_f32(0x49fffff8u) / wmax;
    for (int i = t; i < len; i += ATT_THREADS) {
        const int32_t wq = (int32_t)roundf(sc[i] * qw);
        dig[0][sh + i] = (int8_t)(wq >> 14);
        dig[1][sh + i] = (int8_t)((wq >> 7) & 127);
        dig[2][sh + i] = (int8_t)(wq & 127);
    }
    // zero digits in the first dword before the keys and the last one past them
    if (t < 4) {
        const int j0 = t, j1 = cols + t;
        if (j0 < sh) dig[0][j0] = dig[1][j0] = dig[2][j0] = 0;
        if (j1 < (cols + 3) / 4 * 4) dig[0][j1] = dig[1][j1] = dig[2][j1] = 0;
    }
    __syncthreads();
    const float cw = wmax * bits_f32(0x35000004u);
    const int dm = t >> 2, part = t & 3;
    int a = 0, b = 0, c = 0;
    if (dm < vd) {
        // exact integer P.V: four keys per sdot4, 16 per thread step
        const int* vrow = reinterpret_cast<const int*>(vs8[dm]);
        const int* d0 = reinterpret_cast<const int*>(dig[0]);
        const int* d1 = reinterpret_cast<const int*>(dig[1]);
        const int* d2 = reinterpret_cast<const int*>(dig[2]);
        int i = part;
        for (; 4 * (i + 12) < cols; i += 16) {
            int v[4], x0[4], x1[4], x2[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[q] = vrow[i + 4 * q];
                x0[q] = d0[i + 4 * q];
                x1[q] = d1[i + 4 * q];
                x2[q] = d2[i + 4 * q];
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                a = __builtin_amdgcn_sdot4(x0[q], v[q], a, false);
                b = __builtin_amdgcn_sdot4(x1[q], v[q], b, false);
                c = __builtin_amdgcn_sdot4(x2[q], v[q], c, false);
            }
        }
        for (; 4 * i < cols; i += 4) {
            const int v = vrow[i];
            a = __builtin_amdgcn_sdot4(d0[i], v, a, false);
            b = __builtin_amdgcn_sdot4(d1[i], v, b, false);
            c = __builtin_amdgcn_sdot4(d2[i], v, c, false);
        }
    }
    a = quad_sum_i32(a);
    b = quad_sum_i32(b);
    c = quad_sum_i32(c);
    const size_t pi = ((size_t)row * D.nh + hh) * D.max_chunks + ci;
    if (dm < vd && part == 0)
        S.po[pi * vd + dm] = __builtin_fmaf(16384.0f, (float)a, __builtin_fmaf(128.0f, (float)b, (float)c)) * cw;
    if (t == 0) {
        S.pm[pi] = mx;
        S.psum[pi] = s_sum;
    }
}

// LDS writes of a wavefront visible to its other lanes (its LDS operations
// complete in order; the fence waits for them and keeps the compiler from
// moving accesses across).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// attend_head_ref for all the query heads that share a kv head: one
// workgroup per (row or pair of rows, kv head, key chunk) stages the
// chunk's key rows, scales and value columns once (as k_attend does).  The two integer dot
// products run on the matrix cores, since an int32 sum is the same in any
// order: the scores of every head against 16 keys are one
// v_mfma_i32_16x16x64_i8 (A = the heads' int8 queries, B = the key rows),
// and P.V is a product of the three 7-bit digit planes of every head (A,
// rows plane * 8 + head) with the value columns (B), 64 keys per step.
// Between them wavefront h runs query head h's float steps as the reference
// orders them: the chunk max, chunk_exp with its sum order (lanes 0-7 run
// the eight lane-class chains), the weights and the 21-bit digits.
constexpr int AG_WAVES = 8;   // query heads per kv head this kernel takes
constexpr int AG_T = AG_WAVES * 64;
constexpr int AG_COLS = 320;  // value / digit columns: 15 alignment + 256 keys, in whole 64-column steps
constexpr int AG_KPL = ATT_CHUNK_MAX / 64;  // keys per lane in the head steps
constexpr int AG_TP = ATT_CHUNK_MAX / 8 + 4;  // a lane class's exps (16-byte rows, room for the trailing 4-block)

// RP rows per workgroup (RP = 2: two consecutive rows whose window start
// and chunk ranges agree, which the launch checks for the whole feed): the
// chunk is staged once by all RP * 512 threads, then row rr's 8 wavefronts
// (threads rr * 512 ...) run its scores, head steps and P.V over its own
// keys, a prefix of the staged ones; a feed with an odd count of rows
// leaves the last workgroup's second row empty.
template <int RP>
__global__ __launch_bounds__(AG_T * RP) __attribute__((amdgpu_waves_per_eu(RP == 2 ? 8 : 1))) void k_attend_group(
    const float* qbuf, const int8_t* k8l, const float* ksl, const float* vsl, const int8_t* v8l, int p0, int rows,
    int wv, int geom, Dims D, SessDev S, LayerDev L, int layer) {
    // (the staging's operands lead the arguments as scalars, preloaded at
    // wave launch: the queries, the layer's key rows, scales and value
    // columns, the window | value stride << 16 and the geometry
    // nh | nkv | qk | vd; the parameters and the loads need no read of the
    // argument segment)
    const int g_nh = geom & 255, g_nkv = (geom >> 8) & 255, g_qk = (geom >> 16) & 255,
              g_vd = (int)((unsigned)geom >> 24), window = wv & 0xffff, vcap = (int)((unsigned)wv >> 16);
    constexpr int NTT = AG_T * RP;
    // (the row half and the wavefront are wave-uniform: in scalar registers,
    // so the lengths and bounds derived from them are too)
    const int tb = threadIdx.x, rr = __builtin_amdgcn_readfirstlane(tb / AG_T), t = tb % AG_T;
    // The block's parameters (three divisions by runtime values) are worked
    // out once, by wavefront 0, and handed over through LDS: ~200 scalar
    // instructions per wavefront would otherwise queue on the CU's scalar
    // unit for every resident wavefront before any load is issued.  The
    // longest rows first; the staged range is row A's (the block's rows
    // share lo and the chunking).
    __shared__ int prm[6];
    if (tb < 64) {
        const int pr = (int)blockIdx.x / g_nkv, rA = rows - 1 - RP * pr, pA = p0 + rA;
        const int l0 = window_lo(window, pA);
        int cnt, chk;
        key_chunks(pA + 1 - l0, g_nkv, rows > 1, cnt, chk);
        if (tb == 0) {
            prm[0] = rA;
            prm[1] = (int)blockIdx.x - pr * g_nkv;
            prm[2] = l0;
            prm[3] = cnt;
            prm[4] = chk;
            prm[5] = g_nh / g_nkv;
        }
    }
    __syncthreads();
    const int rowA = __builtin_amdgcn_readfirstlane(prm[0]), kvh = __builtin_amdgcn_readfirstlane(prm[1]);
    const int lo = __builtin_amdgcn_readfirstlane(prm[2]), count = __builtin_amdgcn_readfirstlane(prm[3]);
    const int chunk = __builtin_amdgcn_readfirstlane(prm[4]), hpg = __builtin_amdgcn_readfirstlane(prm[5]);
    const int ci = blockIdx.y;
    if (ci >= count) return;
    const int row = rowA - rr;
    const bool live = RP == 1 || row >= 0;  // (wave-uniform)
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63, posA = p0 + rowA,
              pos = p0 + (live ? row : 0);
    const int nkv = g_nkv, qk = g_qk, vd = g_vd;
    const int nA = posA + 1 - lo, n = pos + 1 - lo;
    const int c0 = ci * chunk, lenA = min(chunk, nA - c0), slot0 = lo + c0;
    const int len = live ? min(chunk, n - c0) : 0, blocked = len / 4 * 4;
    // value columns and digits from slot base = slot0 rounded down to 16
    // bytes (column j = key + sh)
    const int sh = slot0 & 15, base = slot0 - sh, colsA = sh + lenA, cols = sh + len;
    __shared__ alignas(16) int8_t vs8[MAX_HEAD_DIM][AG_COLS];
    __shared__ float kss[ATT_CHUNK_MAX], vss[ATT_CHUNK_MAX];
    __shared__ alignas(16) int8_t q8s[RP][AG_WAVES][MAX_HEAD_DIM];
    __shared__ float qscs[RP][AG_WAVES];
    // The key rows are read by the score products only; the scores, digits
    // and P.V sums then take their space (three one-row blocks or two
    // two-row blocks fit on a CU).
    __shared__ union {
        alignas(16) int8_t ks8[ATT_CHUNK_MAX][ATT_KPITCH];
        struct {
            alignas(16) float sc[RP][AG_WAVES][8 * AG_TP];
            alignas(16) int8_t dig[RP][AG_WAVES][3][AG_COLS];
            int32_t pv[RP][3][AG_WAVES][MAX_HEAD_DIM];
        };
    } lds;
    auto& ks8 = lds.ks8;
    auto& sc = lds.sc[rr];
    auto& dig = lds.dig[rr];
    auto& pv = lds.pv[rr];
    auto& q8 = q8s[rr];
    auto& qsc = qscs[rr];
    const int hw = min(wave, hpg - 1), hh = kvh * hpg + hw;
    // every load first (unconditional, at clamped in-range addresses)
    const float qv = qbuf[((size_t)(live ? row : 0) * g_nh + hh) * qk + min(lane, qk - 1)];
    constexpr int VQ = AG_COLS / 16;  // 16-byte value chunks per column
    constexpr int KR = ATT_CHUNK_MAX * 4 / NTT, VR = (MAX_HEAD_DIM * VQ + NTT - 1) / NTT;
    const int rq = qk / 16, vq = (colsA + 15) / 16;
    // buffer resources over the chunk's key rows (this kv head's, from
    // slot0), their scales and the value columns (from base)
    const int kstride = nkv * qk;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(k8l + (size_t)slot0 * kstride + kvh * qk, (size_t)lenA * kstride);
    const __amdgpu_buffer_rsrc_t rks = make_rsrc(ksl + (size_t)slot0 * nkv + kvh, (size_t)lenA * nkv * 4);
    const __amdgpu_buffer_rsrc_t rvs = make_rsrc(vsl + (size_t)slot0 * nkv + kvh, (size_t)lenA * nkv * 4);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(v8l + (size_t)kvh * vd * vcap + base, (size_t)vd * vcap);
    u32x4 kr[KR], vw[VR];
#pragma unroll
    for (int r = 0; r < KR; ++r) {
        const int e = tb + r * NTT, i = min(e >> 2, lenA - 1), c = min(e & 3, rq - 1);
        kr[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, __mul24(i, kstride) + c * 16, 0, 0));
    }
    float ksr, vsr;
    {
        const int i = min(tb, lenA - 1);
        ksr = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rks, __mul24(i, nkv) * 4, 0, 0));
        vsr = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvs, __mul24(i, nkv) * 4, 0, 0));
    }
#pragma unroll
    for (int r = 0; r < VR; ++r) {
        const int e = tb + r * NTT, dm = min(e / VQ, vd - 1), k = min(e % VQ, vq - 1);
        vw[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, __mul24(dm, vcap) + k * 16, 0, 0));
    }
    // the int8 query of this wavefront's head, zero past qk (the key rows'
    // bytes there are not staged)
    const float s = wave_quant_scale(lane < qk ? qv : 0.0f);
    q8[wave][lane] = lane < qk ? quant_one(qv, 1.0f / s) : (int8_t)0;
    if (lane == 0) qsc[wave] = s * bits_f32(0x3e13cd3au);
#pragma unroll
    for (int r = 0; r < KR; ++r) {
        const int e = tb + r * NTT, i = e >> 2, c = e & 3;
        if (i < lenA && c < rq) reinterpret_cast<u32x4*>(ks8[i])[c] = kr[r];
    }
    if (tb < lenA) {
        kss[tb] = ksr;
        vss[tb] = vsr;
    }
    // whole chunks: the bytes before column sh and past the keys meet zero
    // digits in P.V
#pragma unroll
    for (int r = 0; r < VR; ++r) {
        const int e = tb + r * NTT, dm = e / VQ, k = e % VQ;
        if (dm < vd && k < vq) reinterpret_cast<u32x4*>(vs8[dm])[k] = vw[r];
    }
    __syncthreads();
    const int mr = lane & 15, mq = lane >> 4;  // MFMA lane: row / column mr, 16-byte k-block mq
    // scores: key tile kt (16 keys) per MFMA, tiles split over the wavefronts
    // (at most KT per wavefront); lane (mq, mr) gets heads 4 mq + v against
    // key 16 kt + mr, kept in registers until every key row has been read
    constexpr int KT = ATT_CHUNK_MAX / 16 / AG_WAVES;
    v4i dk[KT];
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        const int kt = wave + j * AG_WAVES;
        if (kt * 16 < len) {
            const v4i a = mr < AG_WAVES ? *reinterpret_cast<const v4i*>(&q8[mr][16 * mq]) : v4i{0, 0, 0, 0};
            const v4i b = *reinterpret_cast<const v4i*>(&ks8[kt * 16 + mr][16 * mq]);
            dk[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, v4i{0, 0, 0, 0}, 0, 0, 0);
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        const int i = (wave + j * AG_WAVES) * 16 + mr;
        if (i < len) {
            const float ksc = kss[i];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int h = 4 * mq + v;
                if (h < hpg) {
                    const float qs = qsc[h];
                    sc[h][i] = i < blocked ? (ksc * (float)dk[j][v]) * qs : (ksc * qs) * (float)dk[j][v];
                }
            }
        }
    }
    __syncthreads();
    float mx = -__builtin_inff(), sum = 0.0f, cw = 0.0f;
    if (live && wave < hpg) {
        // key i = lane + 64 j of the head in register e[j]: score, exp, weight
        float* scw = sc[wave];
        float e[AG_KPL];
#pragma unroll
        for (int j = 0; j < AG_KPL; ++j) {
            const int i = lane + 64 * j;
            e[j] = i < len ? scw[i] : -__builtin_inff();
            mx = fmaxf(mx, e[j]);
        }
        mx = wave_max_ordered(mx);
#pragma unroll
        for (int j = 0; j < AG_KPL; ++j) {
            const int i = lane + 64 * j;
            if (i < len) e[j] = i < blocked ? nexp(e[j] - mx) : lexpf(e[j] - mx);
        }
        // the exps by lane class, key i at (i % 8) * AG_TP + i / 8 (over the
        // scores, which this wavefront has read)
#pragma unroll
        for (int j = 0; j < AG_KPL; ++j) {
            const int i = lane + 64 * j;
            if (i < len) scw[(i & 7) * AG_TP + (i >> 3)] = e[j];
        }
        wave_lds_sync();
        {
            // chunk_exp's order (infer.rs:2222-2279): a[k] over the 8-blocks'
            // first halves plus a trailing 4-block, b[k] over their second
            // halves (lane 4 hi + k), then t = a + b, (t0 + t1) + (t2 + t3)
            float acc = 0.0f;
            const int nb8 = len / 8;
            if (lane < 8) {
                // the class's first nb8 exps in order, four per 16-byte read
                // (nb8 is wave-uniform: scalar loop bounds, no selects)
                const float4* tr = reinterpret_cast<const float4*>(scw + lane * AG_TP);
                int b = 0;
                for (; b + 4 <= nb8; b += 4) {
                    const float4 x = tr[b >> 2];
                    acc += x.x;
                    acc += x.y;
                    acc += x.z;
                    acc += x.w;
                }
                if (b < nb8) {
                    const float4 x = tr[b >> 2];
                    acc += x.x;
                    if (b + 1 < nb8) acc += x.y;
                    if (b + 2 < nb8) acc += x.z;
                }
                if (lane < 4 && len - nb8 * 8 >= 4) acc += scw[lane * AG_TP + nb8];
            }
            const float tk = acc + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                                 0, __builtin_bit_cast(int, acc), 0x104, 0xF, 0xF, false));
            const int ti = __builtin_bit_cast(int, tk);
            const float t0 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x00, 0xF, 0xF, false));
            const float t1 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x55, 0xF, 0xF, false));
            const float t2 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xAA, 0xF, 0xF, false));
            const float t3 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xFF, 0xF, 0xF, false));
            sum = (t0 + t1) + (t2 + t3);
            int i = blocked;
            if (len - i >= 2) {
                sum = (scw[(i & 7) * AG_TP + (i >> 3)] + sum) + scw[((i + 1) & 7) * AG_TP + ((i + 1) >> 3)];
                i += 2;
            }
            if (len - i == 1) sum += scw[(i & 7) * AG_TP + (i >> 3)];
        }
        float wmax = 0.0f;
#pragma unroll
        for (int j = 0; j < AG_KPL; ++j) {
            const int i = lane + 64 * j;
            if (i < len) {
                e[j] = e[j] * vss[i];
                wmax = fmaxf(wmax, e[j]);
            }
        }
        wmax = wave_max_nonneg(wmax);
        const float qwt = bits_f32(0x49fffff8u) / wmax;
        int8_t(*dg)[AG_COLS] = dig[wave];
#pragma unroll
        for (int j = 0; j < AG_KPL; ++j) {
            const int i = lane + 64 * j;
            if (i < len) {
                const int32_t wq = (int32_t)roundf(e[j] * qwt);
                dg[0][sh + i] = (int8_t)(wq >> 14);
                dg[1][sh + i] = (int8_t)((wq >> 7) & 127);
                dg[2][sh + i] = (int8_t)(wq & 127);
            }
        }
        // zero digits before the keys and from their end to the last step's
        if (lane < sh) dg[0][lane] = dg[1][lane] = dg[2][lane] = 0;
        const int j1 = cols + lane;
        if (j1 < (cols + 63) / 64 * 64) dg[0][j1] = dg[1][j1] = dg[2][j1] = 0;
        cw = wmax * bits_f32(0x35000004u);
    }
    __syncthreads();
    // P.V: row tile rt (rows plane * 8 + head) x value-dimension tile dt per
    // job, 64 columns per step
    if (live) {
        const int ndt = (vd + 15) / 16, nsteps = (cols + 63) / 64;
        for (int job = wave; job < 2 * ndt; job += AG_WAVES) {
            const int rt = job / ndt, dt = job % ndt;
            const int R = rt * 16 + mr, j = R >> 3, h = R & 7, dm = min(dt * 16 + mr, MAX_HEAD_DIM - 1);
            v4i acc = {0, 0, 0, 0};
            for (int st = 0; st < nsteps; ++st) {
                const int c = st * 64 + 16 * mq;
                const v4i a = j < 3 ? *reinterpret_cast<const v4i*>(&dig[h][j][c]) : v4i{0, 0, 0, 0};
                const v4i b = *reinterpret_cast<const v4i*>(&vs8[dm][c]);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int R2 = rt * 16 + 4 * mq + v, j2 = R2 >> 3;
                if (j2 < 3) pv[j2][R2 & 7][dt * 16 + mr] = acc[v];
            }
        }
    }
    __syncthreads();
    if (live && wave < hpg) {
        const size_t pi = ((size_t)row * D.nh + hh) * D.max_chunks + ci;
        if (lane < vd) {
            const int a = pv[0][wave][lane], b = pv[1][wave][lane], c = pv[2][wave][lane];
            S.po[pi * vd + lane] = __builtin_fmaf(16384.0f, (float)a, __builtin_fmaf(128.0f, (float)b, (float)c)) * cw;
        }
        if (lane == 0) {
            S.pm[pi] = mx;
            S.psum[pi] = sum;
        }
    }
}

hipError_t fwd_attend(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int t,
                      const KeySpan* span, hipStream_t s) {
    if (span)
        hipLaunchKernelGGL(k_attend<true>, dim3(t * D.nh, D.max_chunks), dim3(ATT_THREADS), 0, s, D, S, L, layer, p0,
                           t, *span);
    else if (D.nh / D.nkv <= AG_WAVES && D.nh < 256 && D.nkv < 256 && D.qk < 256 && D.vd < 256 &&
             L.window >= 0 && L.window < 65536 && D.vcap < 65536) {
        // the most chunks a row of the feed needs
        int most = 1;
        for (int i = 0; i < t; ++i) {
            const int pos = p0 + i, n = pos + 1 - window_lo(L.window, pos);
            int count, chunk;
            key_chunks(n, D.nkv, t > 1, count, chunk);
            most = count > most ? count : most;
        }
        // consecutive rows whose window start and chunking agree share a
        // workgroup (every pair of the feed, else none); rows of one chunk
        // each agree whatever its length (the chunk is all their keys)
        bool pairs = t > 1;
        for (int i = t - 1; i > 0 && pairs; i -= 2) {
            const int pa = p0 + i, pb = pa - 1, la = window_lo(L.window, pa), lb = window_lo(L.window, pb);
            int ca, sa, cb, sb;
            key_chunks(pa + 1 - la, D.nkv, true, ca, sa);
            key_chunks(pb + 1 - lb, D.nkv, true, cb, sb);
            pairs = la == lb && ca == cb && (ca == 1 || sa == sb);
        }
        const size_t lc = (size_t)layer * D.cap;
        const int8_t* k8l = S.k8 + lc * D.nkv * D.qk;
        const float* ksl = S.ks + lc * D.nkv;
        const float* vsl = S.vs + lc * D.nkv;
        const int8_t* v8l = S.v8t + (size_t)layer * D.nkv * D.vd * D.vcap;
        const int geom = D.nh | D.nkv << 8 | D.qk << 16 | D.vd << 24, wv = L.window | D.vcap << 16;
        if (pairs)
            hipLaunchKernelGGL(k_attend_group<2>, dim3((t + 1) / 2 * D.nkv, most), dim3(2 * AG_T), 0, s, S.qbuf, k8l,
                               ksl, vsl, v8l, p0, t, wv, geom, D, S, L, layer);
        else
            hipLaunchKernelGGL(k_attend_group<1>, dim3(t * D.nkv, most), dim3(AG_T), 0, s, S.qbuf, k8l, ksl, vsl,
                               v8l, p0, t, wv, geom, D, S, L, layer);
    }
    else
        hipLaunchKernelGGL(k_attend<false>, dim3(t * D.nh, D.max_chunks), dim3(ATT_THREADS), 0, s, D, S, L, layer,
                           p0, t, KeySpan{});
    return hipGetLastError();
}

// The chunk merge (infer.rs:1990-2006), the head gate
// (att / (nexp(-gate) + 1), step.rs:558-572) and A8 of the heads: wavefront
// g merges the two halves of A8 group g (elements 128 g + lane and
// 128 g + 64 + lane) and quantizes them, so no wavefront waits for another;
// the last wavefront computes the row's post gates meanwhile.
__global__ __launch_bounds__(LT) void k_attn_out(Dims D, SessDev S, LayerDev L, int layer, int p0, int rows,
                                                 int out_bits, KeySpan KS, int span) {
    static_assert((FWD_MAX_D + GROUP - 1) / GROUP < LT / 64, "the A8 groups leave the last wavefront free");
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, vd = D.vd, K = D.nh * vd;
    const int row = blockIdx.x, pos = p0 + row, Ga = (K + GROUP - 1) / GROUP;
    // A feed of several chunks: the tap history of its last rows (the units
    // have read every earlier row by now; only the rows the ring keeps are
    // written, so no two rows share a slot)
    if (rows > FWD_ROWS && row >= rows - D.hist_slots) {
        float* h = S.hist + ((size_t)layer * D.hist_slots + pos % D.hist_slots) * D.W;
        const float* src = S.proj + (size_t)row * D.nq;
        for (int k = t; k < D.W; k += LT) h[k] = src[k];
    }
    if (wave == LT / 64 - 1) {
        post_gates(S.p + (size_t)row * 64, L, lane);
        return;
    }
    if (wave >= Ga) return;
    const int n = key_count(D, KS, span != 0, L.window, pos);
    int count, chunk;
    key_chunks(n, D.nkv, rows > 1, count, chunk);
    auto merged = [&](int q) -> float {
        if (q >= K) return 0.0f;
        const int hh = q / vd, i = q % vd;
        const size_t base = ((size_t)row * D.nh + hh) * D.max_chunks;
        float out;
        if (count == 1) {
            const float inv = 1.0f / S.psum[base];
            out = S.po[base * vd + i] * inv;
        } else {
            float big = -1e30f;
            for (int p = 0; p < count; ++p) big = fmaxf(big, S.pm[base + p]);
            float acc = 0.0f, total = 0.0f;
            for (int p = 0; p < count; ++p) {
                const float w = lexpf(S.pm[base + p] - big);
                acc = __builtin_fmaf(S.po[(base + p) * vd + i], w, acc);
                total = __builtin_fmaf(w, S.psum[base + p], total);
            }
            const float inv = 1.0f / total;
            out = acc * inv;
        }
        return out / (nexp(-S.proj[(size_t)row * D.nq + D.W + q]) + 1.0f);
    };
    const float v0 = merged(wave * GROUP + lane), v1 = merged(wave * GROUP + 64 + lane);
    a8_group(v0, v1, lane, out_bits, S.xq_att + ((size_t)row * Ga + wave) * GROUP, S.sx_att + (size_t)row * Ga + wave);
}

hipError_t fwd_attn_out(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int t, int out_bits,
                        const KeySpan* span, hipStream_t s) {
    hipLaunchKernelGGL(k_attn_out, dim3(t), dim3(LT), 0, s, D, S, L, layer, p0, t, out_bits,
                       span ? *span : KeySpan{}, span ? 1 : 0);
    return hipGetLastError();
}

// ------------------------------------------------------- decode attention
// One decode token's units, attention, gate and A8 in one launch while the
// position's keys form a single chunk (key_chunks gives one chunk below
// 64 k keys; the arithmetic of k_units, k_attend and k_attn_out for one
// row).  Block g owns the heads of A8 group g (GROUP / vd heads sharing one
// kv head): 16 wavefronts, the attention on 256 threads per head.  The
// waves of the heads' query units and of the kv head's new key and value
// compute them first (the same values in every block of the kv group; its
// first block appends them to the cache and the history ring) while the
// other waves stage the keys' int8 rows, scales and values in LDS.  With no
// cross-block data the group's A8 runs in the block.  One more block
// computes the row's post gates.
constexpr int DG_HEAD_T = 256;
constexpr int DG_THREADS = 1024;  // 16 wavefronts: the attention's HP * 256 threads, the rest stage keys

constexpr int DG_PITCH = ATT_CHUNK_MAX + 8;      // value / digit row: 3 alignment bytes + 256 slots + dword tail
constexpr int DG_KPITCH = MAX_HEAD_DIM + 16;     // key row (80 bytes: 8 rows cover the 32 banks)
constexpr int DG_VDW = (ATT_CHUNK_MAX + 3 + 3) / 4;  // value dwords per column (alignment offset + slots)

template <int HP, int TAPS, bool EXACT>
__global__ __launch_bounds__(DG_THREADS) void k_dec_group(const int8_t* k8l, const float* ksl, const float* vsl,
                                                          int8_t* v8l, int p0, int lo, int geom, int vcap, Dims D,
                                                          SessDev S, LayerDev L, int layer, int out_bits) {
    constexpr int NT = HP * DG_HEAD_T;  // the attention's threads (the rest only stage keys)
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int nh = geom & 255, nkv = (geom >> 8) & 255, qk = (geom >> 16) & 255, vd = (int)((unsigned)geom >> 24),
              group = nh / nkv;
    const int qd = nh * qk, kd = nkv * qk, vdim = nkv * vd;
    if ((int)blockIdx.x * HP >= nh) {
        if (wave == 0) post_gates(S.p, L, lane);
        return;
    }
    const int hh0 = blockIdx.x * HP, kvh = hh0 / group;
    const bool owner = hh0 % group == 0;
    const int n = p0 + 1 - lo, blocked = n / 4 * 4;
    // value columns and digits are kept from slot lo - sh (a dword
    // boundary of the cache row): column index j = i + sh for key i
    const int sh = lo & 3, base = lo - sh;
    const int h = t / DG_HEAD_T, u = t % DG_HEAD_T, hw = u >> 6;  // head, thread and wavefront in it
    const bool attends = t < NT;  // (wave-uniform)
    __shared__ alignas(16) int8_t ks8[ATT_CHUNK_MAX][DG_KPITCH];  // key rows by slot - lo
    __shared__ alignas(16) int8_t vs8[MAX_HEAD_DIM][DG_PITCH];    // value columns by slot - base
    __shared__ float kss[ATT_CHUNK_MAX], vss[ATT_CHUNK_MAX];
    __shared__ alignas(16) int8_t q8[HP][MAX_HEAD_DIM];
    __shared__ float sc[HP][ATT_CHUNK_MAX];
    __shared__ alignas(16) int8_t dig[HP][3][DG_PITCH];
    __shared__ float red[HP][DG_HEAD_T / 64], wred[HP][DG_HEAD_T / 64];
    __shared__ float s_qs[HP], s_sum[HP];
    __shared__ float att[HP * MAX_HEAD_DIM];
    __shared__ float gden[HP * MAX_HEAD_DIM];  // exp(-gate) + 1 of output hh0 * vd + j
    // Waves 0 .. HP-1 load the query units' inputs, the next two those of
    // the new key and value, and the rest (the staging waves) the keys
    // before the position: int8 rows (16-byte chunks), scales and value
    // dwords.  A wavefront's loads land at about a kilobyte per thousand
    // cycles, so the units' few loads are kept apart from the keys' and
    // the keys' are spread over many wavefronts.  The role is wave-uniform
    // (scalar branches, each with constant argument fields: selecting the
    // fields by role would copy the argument struct to scratch); within a
    // role the loads are unconditional, at clamped in-range addresses (a
    // load under a lane condition gets waited for at the branch's end), and
    // what lies past the keys is never stored.
    const int role = __builtin_amdgcn_readfirstlane(wave < HP ? 0 : min(wave - HP + 1, 3));  // 0 q, 1 k, 2 v, 3 keys
    constexpr int NS = DG_THREADS - (HP + 2) * 64;  // staging threads
    constexpr int KR = (ATT_CHUNK_MAX * 4 + NS - 1) / NS, VR = (MAX_HEAD_DIM * DG_VDW + NS - 1) / NS,
                  SR = (ATT_CHUNK_MAX + NS - 1) / NS;
    const int nold = n - 1, rq = qk / 16, vdw = (sh + nold + 3) / 4, ts = t - (HP + 2) * 64;
    UnitIn ui;
    u32x4 kr[KR];  // (a native vector: an array of HIP's uint4 is kept on the stack)
    uint32_t vw[VR];
    float ksr[SR], vsr[SR];
    if (role == 0) {
        ui = unit_load<TAPS, EXACT>(D, S, layer, p0, 0, (hh0 + wave) * qk, qd, (hh0 + wave) * qk, qk, L.q_taps,
                                    L.q_norm, lane);
    } else if (role == 1) {
        ui = unit_load<TAPS, EXACT>(D, S, layer, p0, 0, qd + kvh * qk, kd, kvh * qk, qk, L.k_taps, L.k_norm, lane);
    } else if (role == 2) {
        ui = unit_load<TAPS, EXACT>(D, S, layer, p0, 0, qd + kd + kvh * vd, vdim, kvh * vd, vd, L.v_taps, L.k_norm,
                                    lane);
    } else {
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            const int e = ts + r * NS, i = min(e >> 2, n - 1), c = min(e & 3, rq - 1);
            kr[r] = reinterpret_cast<const u32x4*>(k8l + ((size_t)(lo + i) * nkv + kvh) * qk)[c];
        }
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int i = min(ts + r * NS, n - 1);
            ksr[r] = ksl[(size_t)(lo + i) * nkv + kvh];
            vsr[r] = vsl[(size_t)(lo + i) * nkv + kvh];
        }
        const int8_t* vcol = v8l + (size_t)kvh * vd * vcap + base;
#pragma unroll
        for (int r = 0; r < VR; ++r) {
            const int e = ts + r * NS, dm = min(e / DG_VDW, vd - 1), k = min(e % DG_VDW, max(vdw - 1, 0));
            vw[r] = reinterpret_cast<const uint32_t*>(vcol + (size_t)dm * vcap)[k];
        }
    }
    // the head gates of the group's HP * vd = GROUP outputs, one per thread
    // of the query waves, whose units finish well before the staging
    const float gate = S.proj[D.W + hh0 * vd + min(t, HP * vd - 1)];
    // the units
    if (wave < HP) {
        const float v = unit_finish<TAPS, EXACT>(D, S, layer, p0, (hh0 + wave) * qk, qk, ui, true, lane, true);
        const float s = wave_quant_scale(lane < qk ? v : 0.0f);
        if (lane < qk) q8[wave][lane] = quant_one(v, 1.0f / s);
        if (lane == 0) s_qs[wave] = s * bits_f32(0x3e13cd3au);
        if (t < HP * vd) gden[t] = nexp(-gate) + 1.0f;
    } else if (wave == HP) {
        const float v = unit_finish<TAPS, EXACT>(D, S, layer, p0, qd + kvh * qk, qk, ui, true, lane, owner);
        const float s = wave_quant_scale(lane < qk ? v : 0.0f);
        const int8_t q = quant_one(v, 1.0f / s);
        if (lane < qk) {
            ks8[n - 1][lane] = q;
            if (owner) S.k8[(((size_t)layer * D.cap + p0) * nkv + kvh) * qk + lane] = q;
        }
        if (lane == 0) {
            kss[n - 1] = s;
            if (owner) S.ks[((size_t)layer * D.cap + p0) * nkv + kvh] = s;
        }
    } else if (wave == HP + 1) {
        const float v = unit_finish<TAPS, EXACT>(D, S, layer, p0, qd + kd + kvh * vd, vd, ui, false, lane, owner);
        const float s = wave_quant_scale(lane < vd ? v : 0.0f);
        const int8_t q = quant_one(v, 1.0f / s);
        if (lane < vd) {
            vs8[lane][sh + n - 1] = q;
            if (owner) v8l[((size_t)kvh * vd + lane) * vcap + p0] = q;
        }
        if (lane == 0) {
            vss[n - 1] = s;
            if (owner) S.vs[((size_t)layer * D.cap + p0) * nkv + kvh] = s;
        }
    } else {
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            const int e = ts + r * NS, i = e >> 2, c = e & 3;
            if (i < nold && c < rq) reinterpret_cast<u32x4*>(ks8[i])[c] = kr[r];
        }
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int i = ts + r * NS;
            if (i < nold) {
                kss[i] = ksr[r];
                vss[i] = vsr[r];
            }
        }
        // value bytes of keys 0 .. nold - 1 (columns sh .. sh + nold - 1);
        // the bytes before sh and past the keys meet zero digits
#pragma unroll
        for (int r = 0; r < VR; ++r) {
            const int e = ts + r * NS, dm = e / DG_VDW, k = e % DG_VDW;
            if (dm < vd && k < vdw) {
                if (4 * k + 3 < sh + nold) {
                    reinterpret_cast<uint32_t*>(vs8[dm])[k] = vw[r];
                } else {
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        if (4 * k + b < sh + nold) vs8[dm][4 * k + b] = (int8_t)(vw[r] >> (8 * b));
                }
            }
        }
    }
    __syncthreads();
    // attend_head_ref over the one chunk, one head per 256 threads (the
    // staging waves only meet the barriers)
    float mx = -__builtin_inff(), wmax = 0.0f;
    if (attends) {
        const float qs = s_qs[h];
        uint4 qv[MAX_HEAD_DIM / 16];
#pragma unroll
        for (int c = 0; c < MAX_HEAD_DIM / 16; ++c)
            qv[c] = c < rq ? reinterpret_cast<const uint4*>(q8[h])[c] : make_uint4(0, 0, 0, 0);
        for (int i = u; i < n; i += DG_HEAD_T) {
            // (four partial integer sums: exact in any order; every 16-byte
            // chunk of the key row, the query's past qk zero, so no branch
            // sits between the reads)
            int dp[4] = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < MAX_HEAD_DIM / 16; ++c) {
                const uint4 kv = reinterpret_cast<const uint4*>(ks8[i])[c];
                dp[0] = __builtin_amdgcn_sdot4((int)kv.x, (int)qv[c].x, dp[0], false);
                dp[1] = __builtin_amdgcn_sdot4((int)kv.y, (int)qv[c].y, dp[1], false);
                dp[2] = __builtin_amdgcn_sdot4((int)kv.z, (int)qv[c].z, dp[2], false);
                dp[3] = __builtin_amdgcn_sdot4((int)kv.w, (int)qv[c].w, dp[3], false);
            }
            const int dot = (dp[0] + dp[1]) + (dp[2] + dp[3]);
            const float ksc = kss[i];
            const float sv = i < blocked ? (ksc * (float)dot) * qs : (ksc * qs) * (float)dot;
            sc[h][i] = sv;
            mx = fmaxf(mx, sv);
        }
        mx = wave_max_ordered(mx);
        if (lane == 0) red[h][hw] = mx;
    }
    __syncthreads();
    if (attends) {
        // the exps (kept in sc for the sum) and the max of the value
        // weights w = p * vscale, which the digits need and the sum does not
        mx = fmaxf(fmaxf(red[h][0], red[h][1]), fmaxf(red[h][2], red[h][3]));
        for (int i = u; i < n; i += DG_HEAD_T) {
            const float e = i < blocked ? nexp(sc[h][i] - mx) : lexpf(sc[h][i] - mx);
            sc[h][i] = e;
            wmax = fmaxf(wmax, e * vss[i]);
        }
        wmax = wave_max_nonneg(wmax);
        if (lane == 0) wred[h][hw] = wmax;
    }
    __syncthreads();
    if (attends) {
        if (hw == 0) {
            // lane 4 hi + k sums sc[8 b + 4 hi + k] over b in order, the
            // loads of a batch of 8 issued ahead of its adds
            float acc = 0.0f;
            const int nb8 = n / 8;
            if (lane < 8) {
                const int k = lane & 3, hi = lane >> 2;
                const float* col = &sc[h][hi * 4 + k];
                int b = 0;
                for (; b + 8 <= nb8; b += 8) {
                    float v[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = col[(b + j) * 8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc += v[j];
                }
                for (; b < nb8; ++b) acc += col[b * 8];
                if (hi == 0 && n - nb8 * 8 >= 4) acc += sc[h][nb8 * 8 + k];
            }
            // t[k] = a[k] + b[k] (lane 4 + k brought to lane k by a DPP row
            // shift), then (t0 + t1) + (t2 + t3) by quad broadcasts: exact in
            // lane 0, which alone uses it
            const float tk = acc + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                                 0, __builtin_bit_cast(int, acc), 0x104, 0xF, 0xF, false));
            const int ti = __builtin_bit_cast(int, tk);
            const float t0 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x00, 0xF, 0xF, false));
            const float t1 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x55, 0xF, 0xF, false));
            const float t2 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xAA, 0xF, 0xF, false));
            const float t3 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xFF, 0xF, 0xF, false));
            float sum = (t0 + t1) + (t2 + t3);
            int i = blocked;
            if (n - i >= 2) {
                sum = (sc[h][i] + sum) + sc[h][i + 1];
                i += 2;
            }
            if (n - i == 1) sum += sc[h][i];
            if (lane == 0) s_sum[h] = sum;
        }
        // the 21-bit digits of the weights, beside the sum (wave 0 joins
        // once its sum is done); w is recomputed from the same two factors
        wmax = fmaxf(fmaxf(wred[h][0], wred[h][1]), fmaxf(wred[h][2], wred[h][3]));
        const float qw = bits_f32(0x49fffff8u) / wmax;
        for (int i = u; i < n; i += DG_HEAD_T) {
            const float w = sc[h][i] * vss[i];
            const int32_t wq = (int32_t)roundf(w * qw);
            dig[h][0][sh + i] = (int8_t)(wq >> 14);
            dig[h][1][sh + i] = (int8_t)((wq >> 7) & 127);
            dig[h][2][sh + i] = (int8_t)(wq & 127);
        }
        // zero digits in the first dword before the keys and the last one past them
        if (u < 4) {
            const int j0 = u, j1 = sh + n + u;
            if (j0 < sh) dig[h][0][j0] = dig[h][1][j0] = dig[h][2][j0] = 0;
            if (j1 < (sh + n + 3) / 4 * 4) dig[h][0][j1] = dig[h][1][j1] = dig[h][2][j1] = 0;
        }
    }
    __syncthreads();
    if (attends) {
        // exact integer P.V: four columns per sdot4, 16 per thread step
        const float inv_sum = 1.0f / s_sum[h];
        const float cw = wmax * bits_f32(0x35000004u);
        const int dm = u >> 2, part = u & 3, cols = sh + n;
        int a = 0, b = 0, c = 0;
        if (dm < vd) {
            const int* vrow = reinterpret_cast<const int*>(vs8[dm]);
            const int* d0 = reinterpret_cast<const int*>(dig[h][0]);
            const int* d1 = reinterpret_cast<const int*>(dig[h][1]);
            const int* d2 = reinterpret_cast<const int*>(dig[h][2]);
            int i = part;
            for (; 4 * (i + 12) < cols; i += 16) {
                int v[4], x0[4], x1[4], x2[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v[q] = vrow[i + 4 * q];
                    x0[q] = d0[i + 4 * q];
                    x1[q] = d1[i + 4 * q];
                    x2[q] = d2[i + 4 * q];
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    a = __builtin_amdgcn_sdot4(x0[q], v[q], a, false);
                    b = __builtin_amdgcn_sdot4(x1[q], v[q], b, false);
                    c = __builtin_amdgcn_sdot4(x2[q], v[q], c, false);
                }
            }
            for (; 4 * i < cols; i += 4) {
                const int v = vrow[i];
                a = __builtin_amdgcn_sdot4(d0[i], v, a, false);
                b = __builtin_amdgcn_sdot4(d1[i], v, b, false);
                c = __builtin_amdgcn_sdot4(d2[i], v, c, false);
            }
        }
        a = quad_sum_i32(a);
        b = quad_sum_i32(b);
        c = quad_sum_i32(c);
        if (dm < vd && part == 0) {
            const float po = __builtin_fmaf(16384.0f, (float)a, __builtin_fmaf(128.0f, (float)b, (float)c)) * cw;
            const float out = po * inv_sum;
            att[h * vd + dm] = out / gden[h * vd + dm];
        }
    }
    __syncthreads();
    if (wave == 0) {
        const int K = HP * vd;
        a8_group(lane < K ? att[lane] : 0.0f, lane + 64 < K ? att[lane + 64] : 0.0f, lane, out_bits,
                 S.xq_att + (size_t)blockIdx.x * GROUP, S.sx_att + blockIdx.x);
    }
}

bool dec_group_fits(const Dims& D, int p0, int window) {
    const int lo = (window > 0 && p0 + 1 > window) ? p0 + 1 - window : 0, n = p0 + 1 - lo;
    int k = 2 * NATIVE_TEAM / D.nkv;
    if (k < 1) k = 1;
    int c = (n + 255) / 256;
    if (k * 64 <= n && c < k) c = k;
    if (c > 1 || n > ATT_CHUNK_MAX || D.ring > 0) return false;
    if (GROUP % D.vd != 0 || D.taps > DG_MAX_TAPS) return false;
    const int hp = GROUP / D.vd;
    return (hp == 2 || hp == 4) && D.nh % hp == 0 && (D.nh / D.nkv) % hp == 0 && D.qk % 16 == 0 && D.nh < 256 &&
           D.nkv < 256 && D.qk < 256 && D.vd < 256;
}

hipError_t fwd_dec_attn(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int out_bits,
                        hipStream_t s) {
    const int hp = GROUP / D.vd, blocks = D.nh / hp + 1;
    // The staging loads' operands lead the arguments (scalars, preloaded
    // into SGPRs at wave launch): the layer's key rows, scales and value
    // columns, the window start and the geometry (nh, nkv, qk, vd < 256).
    const size_t lc = (size_t)layer * D.cap;
    const int8_t* k8l = S.k8 + lc * D.nkv * D.qk;
    const float* ksl = S.ks + lc * D.nkv;
    const float* vsl = S.vs + lc * D.nkv;
    int8_t* v8l = S.v8t + (size_t)layer * D.nkv * D.vd * D.vcap;
    const int lo = window_lo(L.window, p0), geom = D.nh | D.nkv << 8 | D.qk << 16 | D.vd << 24;
    // exact tap counts 1..4, clamped loads up to DG_MAX_TAPS otherwise
#define NH_DG(HP, TP, EX)                                                                                        \
    hipLaunchKernelGGL((k_dec_group<HP, TP, EX>), dim3(blocks), dim3(DG_THREADS), 0, s, k8l, ksl, vsl, v8l, p0, \
                       lo, geom, D.vcap, D, S, L, layer, out_bits)
#define NH_DG_TAPS(HP)                          \
    switch (D.taps) {                           \
        case 1: NH_DG(HP, 1, true); break;      \
        case 2: NH_DG(HP, 2, true); break;      \
        case 3: NH_DG(HP, 3, true); break;      \
        case 4: NH_DG(HP, 4, true); break;      \
        default: NH_DG(HP, DG_MAX_TAPS, false); \
    }
    if (hp == 2) {
        NH_DG_TAPS(2)
    } else {
        NH_DG_TAPS(4)
    }
#undef NH_DG_TAPS
#undef NH_DG
    return hipGetLastError();
}

// Chunk parts the merge of k_dec_chunks loads at once.
constexpr int MERGE_AHEAD = 8;

// One decode token's units, attention, gate and A8 in one launch for any
// key count and with an attention span: attend_head_ref's chunks
// (key_chunks, infer.rs:1888-1893,2093-2101) run in blocks of their own.
// Block (g, c) owns A8 group g's heads (as k_dec_group) and key chunk c:
// its query waves compute the heads' query units (every block of the group
// the same values), the last chunk's blocks also the kv head's new key and
// value (the first of them appends them to the cache and the history
// ring), and the staging waves load the chunk's cached keys, scales and
// values (by position; with a span, through the chunk's KV slots: from the
// chunk's slot runs, or found first into LDS when the runs do not fit).  Each chunk's attention gives the reference's part (max, sum,
// P.V, infer.rs:1918-1987); one chunk finishes in its block.  With several,
// each block stores its heads' parts and counts itself in (agent-scope
// release); the group's block that counts last merges the parts in chunk
// order (infer.rs:1990-2006), divides by the head gate and runs the
// group's A8, then clears the count.  No block waits for another.  One
// more block computes the row's post gates.
// Under a span, the KV slots of each key chunk as runs of consecutive keys
// in consecutive slots (a span's live positions are a few position runs;
// past the sink a run's slots only break where the ring wraps), worked out
// on the host per launch: chunk c's run r holds its keys key0 ..
// key0 + len - 1 (chunk-local) at slots slot0 .. slot0 + len - 1; unused
// runs have key0 = RUN_NONE and len 0 (so the last run starting at or
// before a key is the key's run).
constexpr int DC_RUNS = 4;         // runs per chunk
constexpr int DC_RUN_CHUNKS = 8;   // chunks
constexpr int RUN_NONE = 1 << 30;
constexpr int RUN_CHUNK = 128;     // the most keys a chunk has on the run path
struct ChunkRuns {
    int nrun[DC_RUN_CHUNKS];
    int key0[DC_RUN_CHUNKS][DC_RUNS], slot0[DC_RUN_CHUNKS][DC_RUNS], len[DC_RUN_CHUNKS][DC_RUNS];
};

// One chunk's runs, read once into registers.
struct Runs {
    int k0[DC_RUNS], s0[DC_RUNS];
};

// The slot of chunk-local key j (j within the chunk's runs): the last run
// starting at or before j (selects, no branches).
__device__ __forceinline__ int run_slot(const Runs& q, int j) {
    int slot = q.s0[0] + (j - q.k0[0]);
#pragma unroll
    for (int r = 1; r < DC_RUNS; ++r) slot = j >= q.k0[r] ? q.s0[r] + (j - q.k0[r]) : slot;
    return slot;
}

// RUNS (with SPAN, chunks of at most RUN_CHUNK keys): the staging reads
// keys, scales and value bytes at slots taken from the chunk's slot runs
// (R) in registers, with no slot list in LDS and no barrier for it, and
// gathers RUN_CHUNK value bytes per column instead of ATT_CHUNK_MAX.
template <int HP, int TAPS, bool EXACT, bool SPAN, bool RUNS>
__global__ __launch_bounds__(DG_THREADS) void k_dec_chunks(Dims D, SessDev S, LayerDev L, int layer, int p0,
                                                           int out_bits, KeySpan K, int n, int nchunks, int chunk,
                                                           ChunkRuns R) {
    constexpr int NT = HP * DG_HEAD_T;  // the attention's threads
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int nh = D.nh, nkv = D.nkv, qk = D.qk, vd = D.vd, group = nh / nkv;
    const int qd = nh * qk, kd = nkv * qk, vdim = nkv * vd;
    const int ngroups = nh / HP;
    if ((int)blockIdx.x >= ngroups * nchunks) {
        if (wave == 0) post_gates(S.p, L, lane);
        return;
    }
    const int g = blockIdx.x / nchunks, ci = blockIdx.x % nchunks;
    const int hh0 = g * HP, kvh = hh0 / group;
    const bool last = ci == nchunks - 1;              // the chunk holding the new key (key n - 1 = p0)
    const bool owner = last && hh0 % group == 0;      // appends the new key and value
    const int c0 = ci * chunk, len = min(chunk, n - c0), blocked = len / 4 * 4;
    const int nold = last ? len - 1 : len;            // keys read from the cache
    const int lo = window_lo(L.window, p0);
    // without a span the chunk's keys are positions (= slots) slot0 ..;
    // value columns and digits are kept from the dword boundary at or
    // before slot0 (column j = i + sh for key i); with one, column j = key j
    const int slot0 = lo + c0, sh = SPAN ? 0 : slot0 & 3, base = slot0 - sh;
    const int h = t / DG_HEAD_T, u = t % DG_HEAD_T, hw = u >> 6;
    const bool attends = t < NT;  // (wave-uniform)
    __shared__ alignas(16) int8_t ks8[ATT_CHUNK_MAX][DG_KPITCH];
    __shared__ alignas(16) int8_t vs8[MAX_HEAD_DIM][DG_PITCH];
    __shared__ float kss[ATT_CHUNK_MAX], vss[ATT_CHUNK_MAX];
    __shared__ int kslot[SPAN && !RUNS ? ATT_CHUNK_MAX : 1];
    __shared__ alignas(16) int8_t q8[HP][MAX_HEAD_DIM];
    __shared__ float sc[HP][ATT_CHUNK_MAX];
    __shared__ alignas(16) int8_t dig[HP][3][DG_PITCH];
    __shared__ float red[HP][DG_HEAD_T / 64], wred[HP][DG_HEAD_T / 64];
    __shared__ float s_qs[HP], s_sum[HP];
    __shared__ float att[HP * MAX_HEAD_DIM];
    __shared__ float gden[HP * MAX_HEAD_DIM];
    __shared__ int s_merge;
    const size_t lc = (size_t)layer * D.cap;
    const int role = __builtin_amdgcn_readfirstlane(wave < HP ? 0 : min(wave - HP + 1, 3));  // 0 q, 1 k, 2 v, 3 keys
    constexpr int NS = DG_THREADS - (HP + 2) * 64;  // staging threads
    constexpr int KR = (ATT_CHUNK_MAX * 4 + NS - 1) / NS, SR = (ATT_CHUNK_MAX + NS - 1) / NS;
    // values: dwords of the columns without a span, bytes gathered by slot
    // with one (RUNS: chunks of at most RUN_CHUNK keys, so RUN_CHUNK
    // elements per column)
    constexpr int VR = RUNS ? (MAX_HEAD_DIM * RUN_CHUNK + NS - 1) / NS
                     : SPAN ? (MAX_HEAD_DIM * ATT_CHUNK_MAX + NS - 1) / NS
                            : (MAX_HEAD_DIM * DG_VDW + NS - 1) / NS;
    // the chunk's runs, read once, unconditionally
    Runs q{};
    if constexpr (RUNS) {
#pragma unroll
        for (int r = 0; r < DC_RUNS; ++r) {
            q.k0[r] = R.key0[ci][r];
            q.s0[r] = R.slot0[ci][r];
        }
    }
    const int rq = qk / 16, vdw = (sh + nold + 3) / 4, ts = t - (HP + 2) * 64;
    const int8_t* vcol = S.v8t + ((size_t)layer * nkv + kvh) * vd * D.vcap;
    UnitIn ui;
    u32x4 kr[KR];
    uint32_t vw[VR];
    float ksr[SR], vsr[SR];
    if (role == 0) {
        ui = unit_load<TAPS, EXACT>(D, S, layer, p0, 0, (hh0 + wave) * qk, qd, (hh0 + wave) * qk, qk, L.q_taps,
                                    L.q_norm, lane);
    } else if (role == 1) {
        if (last)
            ui = unit_load<TAPS, EXACT>(D, S, layer, p0, 0, qd + kvh * qk, kd, kvh * qk, qk, L.k_taps, L.k_norm, lane);
    } else if (role == 2) {
        if (last)
            ui = unit_load<TAPS, EXACT>(D, S, layer, p0, 0, qd + kd + kvh * vd, vdim, kvh * vd, vd, L.v_taps,
                                        L.k_norm, lane);
    } else if constexpr (RUNS) {
        // keys and scales at their runs' slots; values as the runs' dwords
        // (clamped in-range: past nold, or past the runs' dwords, nothing is
        // stored)
        const int im = max(nold - 1, 0);
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            const int e = ts + r * NS, i = min(e >> 2, im), c = min(e & 3, rq - 1);
            kr[r] = reinterpret_cast<const u32x4*>(S.k8 + ((lc + run_slot(q, i)) * nkv + kvh) * qk)[c];
        }
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int sl = run_slot(q, min(ts + r * NS, im));
            ksr[r] = S.ks[(lc + sl) * nkv + kvh];
            vsr[r] = S.vs[(lc + sl) * nkv + kvh];
        }
        // element e: column dm = e / RUN_CHUNK, key i = e % RUN_CHUNK
#pragma unroll
        for (int r = 0; r < VR; ++r) {
            const int e = ts + r * NS, dm = min(e / RUN_CHUNK, vd - 1), i = min(e % RUN_CHUNK, im);
            vw[r] = (uint8_t)vcol[(size_t)dm * D.vcap + run_slot(q, i)];
        }
    } else if constexpr (!SPAN) {
        // (clamped in-range addresses: past nold nothing is stored; with no
        // cached key the clamp reads the new position's own slot)
        const int im = max(nold - 1, 0);
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            const int e = ts + r * NS, i = min(e >> 2, im), c = min(e & 3, rq - 1);
            kr[r] = reinterpret_cast<const u32x4*>(S.k8 + ((lc + slot0 + i) * nkv + kvh) * qk)[c];
        }
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int i = min(ts + r * NS, im);
            ksr[r] = S.ks[(lc + slot0 + i) * nkv + kvh];
            vsr[r] = S.vs[(lc + slot0 + i) * nkv + kvh];
        }
#pragma unroll
        for (int r = 0; r < VR; ++r) {
            const int e = ts + r * NS, dm = min(e / DG_VDW, vd - 1), k = min(e % DG_VDW, max(vdw - 1, 0));
            vw[r] = reinterpret_cast<const uint32_t*>(vcol + base + (size_t)dm * D.vcap)[k];
        }
    } else {
        // the chunk's KV slots: key c0 + i at its position in the span's runs
        if (ts < len) {
            int alo, ahi, blo, bhi;
            span_ranges(D, K, lo, p0, alo, ahi, blo, bhi);
            kslot[ts] = slot_of(D, span_key(K, alo, ahi, blo, bhi, c0 + ts));
        }
    }
    if constexpr (SPAN && !RUNS) {
        __syncthreads();  // the slots
        if (role == 3) {
            const int im = max(nold - 1, 0);
#pragma unroll
            for (int r = 0; r < KR; ++r) {
                const int e = ts + r * NS, i = min(e >> 2, im), c = min(e & 3, rq - 1);
                kr[r] = reinterpret_cast<const u32x4*>(S.k8 + ((lc + kslot[i]) * nkv + kvh) * qk)[c];
            }
#pragma unroll
            for (int r = 0; r < SR; ++r) {
                const int sl = kslot[min(ts + r * NS, im)];
                ksr[r] = S.ks[(lc + sl) * nkv + kvh];
                vsr[r] = S.vs[(lc + sl) * nkv + kvh];
            }
#pragma unroll
            for (int r = 0; r < VR; ++r) {
                const int e = ts + r * NS, dm = min(e / ATT_CHUNK_MAX, vd - 1), i = min(e % ATT_CHUNK_MAX, im);
                vw[r] = (uint8_t)vcol[(size_t)dm * D.vcap + kslot[i]];
            }
        }
    }
    const float gate = S.proj[D.W + hh0 * vd + min(t, HP * vd - 1)];
    if (wave < HP) {
        // the query history row is written once (by the last chunk's block)
        const float v = unit_finish<TAPS, EXACT>(D, S, layer, p0, (hh0 + wave) * qk, qk, ui, true, lane, last);
        const float s = wave_quant_scale(lane < qk ? v : 0.0f);
        if (lane < qk) q8[wave][lane] = quant_one(v, 1.0f / s);
        if (lane == 0) s_qs[wave] = s * bits_f32(0x3e13cd3au);
        if (t < HP * vd) gden[t] = nexp(-gate) + 1.0f;
    } else if (wave == HP) {
        if (last) {
            const float v = unit_finish<TAPS, EXACT>(D, S, layer, p0, qd + kvh * qk, qk, ui, true, lane, owner);
            const float s = wave_quant_scale(lane < qk ? v : 0.0f);
            const int8_t q = quant_one(v, 1.0f / s);
            const int slot = slot_of(D, p0);
            if (lane < qk) {
                ks8[len - 1][lane] = q;
                if (owner) S.k8[((lc + slot) * nkv + kvh) * qk + lane] = q;
            }
            if (lane == 0) {
                kss[len - 1] = s;
                if (owner) S.ks[(lc + slot) * nkv + kvh] = s;
            }
        }
    } else if (wave == HP + 1) {
        if (last) {
            const float v = unit_finish<TAPS, EXACT>(D, S, layer, p0, qd + kd + kvh * vd, vd, ui, false, lane, owner);
            const float s = wave_quant_scale(lane < vd ? v : 0.0f);
            const int8_t q = quant_one(v, 1.0f / s);
            const int slot = slot_of(D, p0);
            if (lane < vd) {
                vs8[lane][sh + len - 1] = q;
                if (owner) S.v8t[(((size_t)layer * nkv + kvh) * vd + lane) * D.vcap + slot] = q;
            }
            if (lane == 0) {
                vss[len - 1] = s;
                if (owner) S.vs[(lc + slot) * nkv + kvh] = s;
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            const int e = ts + r * NS, i = e >> 2, c = e & 3;
            if (i < nold && c < rq) reinterpret_cast<u32x4*>(ks8[i])[c] = kr[r];
        }
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int i = ts + r * NS;
            if (i < nold) {
                kss[i] = ksr[r];
                vss[i] = vsr[r];
            }
        }
        if constexpr (RUNS) {
#pragma unroll
            for (int r = 0; r < VR; ++r) {
                const int e = ts + r * NS, dm = e / RUN_CHUNK, i = e % RUN_CHUNK;
                if (dm < vd && i < nold) vs8[dm][i] = (int8_t)vw[r];
            }
        } else if constexpr (SPAN) {
#pragma unroll
            for (int r = 0; r < VR; ++r) {
                const int e = ts + r * NS, dm = e / ATT_CHUNK_MAX, i = e % ATT_CHUNK_MAX;
                if (dm < vd && i < nold) vs8[dm][i] = (int8_t)vw[r];
            }
        } else {
#pragma unroll
            for (int r = 0; r < VR; ++r) {
                const int e = ts + r * NS, dm = e / DG_VDW, k = e % DG_VDW;
                if (dm < vd && k < vdw) {
                    if (4 * k + 3 < sh + nold) {
                        reinterpret_cast<uint32_t*>(vs8[dm])[k] = vw[r];
                    } else {
#pragma unroll
                        for (int b = 0; b < 4; ++b)
                            if (4 * k + b < sh + nold) vs8[dm][4 * k + b] = (int8_t)(vw[r] >> (8 * b));
                    }
                }
            }
        }
    }
    __syncthreads();
    // the chunk's attend_head_ref steps, one head per 256 threads
    float mx = -__builtin_inff(), wmax = 0.0f;
    if (attends) {
        const float qs = s_qs[h];
        uint4 qv[MAX_HEAD_DIM / 16];
#pragma unroll
        for (int c = 0; c < MAX_HEAD_DIM / 16; ++c)
            qv[c] = c < rq ? reinterpret_cast<const uint4*>(q8[h])[c] : make_uint4(0, 0, 0, 0);
        for (int i = u; i < len; i += DG_HEAD_T) {
            int dp[4] = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < MAX_HEAD_DIM / 16; ++c) {
                const uint4 kv = reinterpret_cast<const uint4*>(ks8[i])[c];
                dp[0] = __builtin_amdgcn_sdot4((int)kv.x, (int)qv[c].x, dp[0], false);
                dp[1] = __builtin_amdgcn_sdot4((int)kv.y, (int)qv[c].y, dp[1], false);
                dp[2] = __builtin_amdgcn_sdot4((int)kv.z, (int)qv[c].z, dp[2], false);
                dp[3] = __builtin_amdgcn_sdot4((int)kv.w, (int)qv[c].w, dp[3], false);
            }
            const int dot = (dp[0] + dp[1]) + (dp[2] + dp[3]);
            const float ksc = kss[i];
            const float sv = i < blocked ? (ksc * (float)dot) * qs : (ksc * qs) * (float)dot;
            sc[h][i] = sv;
            mx = fmaxf(mx, sv);
        }
        mx = wave_max_ordered(mx);
        if (lane == 0) red[h][hw] = mx;
    }
    __syncthreads();
    if (attends) {
        mx = fmaxf(fmaxf(red[h][0], red[h][1]), fmaxf(red[h][2], red[h][3]));
        for (int i = u; i < len; i += DG_HEAD_T) {
            const float e = i < blocked ? nexp(sc[h][i] - mx) : lexpf(sc[h][i] - mx);
            sc[h][i] = e;
            wmax = fmaxf(wmax, e * vss[i]);
        }
        wmax = wave_max_nonneg(wmax);
        if (lane == 0) wred[h][hw] = wmax;
    }
    __syncthreads();
    if (attends) {
        if (hw == 0) {
            // chunk_exp's sum order (as k_dec_group)
            float acc = 0.0f;
            const int nb8 = len / 8;
            if (lane < 8) {
                const int k = lane & 3, hi = lane >> 2;
                const float* col = &sc[h][hi * 4 + k];
                int b = 0;
                for (; b + 8 <= nb8; b += 8) {
                    float v[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = col[(b + j) * 8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc += v[j];
                }
                for (; b < nb8; ++b) acc += col[b * 8];
                if (hi == 0 && len - nb8 * 8 >= 4) acc += sc[h][nb8 * 8 + k];
            }
            const float tk = acc + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                                 0, __builtin_bit_cast(int, acc), 0x104, 0xF, 0xF, false));
            const int ti = __builtin_bit_cast(int, tk);
            const float t0 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x00, 0xF, 0xF, false));
            const float t1 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0x55, 0xF, 0xF, false));
            const float t2 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xAA, 0xF, 0xF, false));
            const float t3 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ti, 0xFF, 0xF, 0xF, false));
            float sum = (t0 + t1) + (t2 + t3);
            int i = blocked;
            if (len - i >= 2) {
                sum = (sc[h][i] + sum) + sc[h][i + 1];
                i += 2;
            }
            if (len - i == 1) sum += sc[h][i];
            if (lane == 0) s_sum[h] = sum;
        }
        wmax = fmaxf(fmaxf(wred[h][0], wred[h][1]), fmaxf(wred[h][2], wred[h][3]));
        const float qw = bits_f32(0x49fffff8u) / wmax;
        for (int i = u; i < len; i += DG_HEAD_T) {
            const float w = sc[h][i] * vss[i];
            const int32_t wq = (int32_t)roundf(w * qw);
            dig[h][0][sh + i] = (int8_t)(wq >> 14);
            dig[h][1][sh + i] = (int8_t)((wq >> 7) & 127);
            dig[h][2][sh + i] = (int8_t)(wq & 127);
        }
        if (u < 4) {
            const int j0 = u, j1 = sh + len + u;
            if (j0 < sh) dig[h][0][j0] = dig[h][1][j0] = dig[h][2][j0] = 0;
            if (j1 < (sh + len + 3) / 4 * 4) dig[h][0][j1] = dig[h][1][j1] = dig[h][2][j1] = 0;
        }
    }
    __syncthreads();
    if (attends) {
        const float cw = wmax * bits_f32(0x35000004u);
        const int dm = u >> 2, part = u & 3, cols = sh + len;
        int a = 0, b = 0, c = 0;
        if (dm < vd) {
            const int* vrow = reinterpret_cast<const int*>(vs8[dm]);
            const int* d0 = reinterpret_cast<const int*>(dig[h][0]);
            const int* d1 = reinterpret_cast<const int*>(dig[h][1]);
            const int* d2 = reinterpret_cast<const int*>(dig[h][2]);
            int i = part;
            for (; 4 * (i + 12) < cols; i += 16) {
                int v[4], x0[4], x1[4], x2[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v[q] = vrow[i + 4 * q];
                    x0[q] = d0[i + 4 * q];
                    x1[q] = d1[i + 4 * q];
                    x2[q] = d2[i + 4 * q];
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    a = __builtin_amdgcn_sdot4(x0[q], v[q], a, false);
                    b = __builtin_amdgcn_sdot4(x1[q], v[q], b, false);
                    c = __builtin_amdgcn_sdot4(x2[q], v[q], c, false);
                }
            }
            for (; 4 * i < cols; i += 4) {
                const int v = vrow[i];
                a = __builtin_amdgcn_sdot4(d0[i], v, a, false);
                b = __builtin_amdgcn_sdot4(d1[i], v, b, false);
                c = __builtin_amdgcn_sdot4(d2[i], v, c, false);
            }
        }
        a = quad_sum_i32(a);
        b = quad_sum_i32(b);
        c = quad_sum_i32(c);
        if (dm < vd && part == 0) {
            const float po = __builtin_fmaf(16384.0f, (float)a, __builtin_fmaf(128.0f, (float)b, (float)c)) * cw;
            if (nchunks == 1) {
                att[h * vd + dm] = (po * (1.0f / s_sum[h])) / gden[h * vd + dm];
            } else {
                const size_t pi = (size_t)(hh0 + h) * D.max_chunks + ci;
                S.po[pi * vd + dm] = po;
                if (dm == 0) {
                    S.pm[pi] = mx;
                    S.psum[pi] = s_sum[h];
                }
            }
        }
    }
    if (nchunks > 1) {
        // count this block in; the group's last block merges
        __syncthreads();
        if (t == 0) {
            const int before = __hip_atomic_fetch_add(S.dcount + g, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            s_merge = before == nchunks - 1;
        }
        __syncthreads();
        if (!s_merge) return;
        if (t < HP * vd) {
            // merge_parts (infer.rs:2143-2166) in chunk order.  The first
            // MERGE_AHEAD parts' loads are all issued before any is used (the
            // parts come from other CUs, a memory round trip each), and their
            // exponentials are independent of one another; only the two fma
            // chains run in chunk order.  Parts past those (over 2,048 keys)
            // are read one by one.
            constexpr int MA = MERGE_AHEAD;
            const int hh = hh0 + t / vd, i = t % vd;
            const size_t pb = (size_t)hh * D.max_chunks;
            float mv[MA], ov[MA], sv[MA];
#pragma unroll
            for (int p = 0; p < MA; ++p) {
                const size_t pp = pb + min(p, nchunks - 1);
                mv[p] = __hip_atomic_load(S.pm + pp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ov[p] = __hip_atomic_load(S.po + pp * vd + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                sv[p] = __hip_atomic_load(S.psum + pp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            float big = -1e30f;
#pragma unroll
            for (int p = 0; p < MA; ++p) big = fmaxf(big, mv[p]);  // (clamped repeats change no maximum)
            for (int p = MA; p < nchunks; ++p)
                big = fmaxf(big, __hip_atomic_load(S.pm + pb + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            float w[MA];
#pragma unroll
            for (int p = 0; p < MA; ++p) w[p] = lexpf(mv[p] - big);
            float acc = 0.0f, total = 0.0f;
#pragma unroll
            for (int p = 0; p < MA; ++p) {
                if (p < nchunks) {
                    acc = __builtin_fmaf(ov[p], w[p], acc);
                    total = __builtin_fmaf(w[p], sv[p], total);
                }
            }
            for (int p = MA; p < nchunks; ++p) {
                const float m = __hip_atomic_load(S.pm + pb + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float o = __hip_atomic_load(S.po + (pb + p) * vd + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float sm = __hip_atomic_load(S.psum + pb + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float wp = lexpf(m - big);
                acc = __builtin_fmaf(o, wp, acc);
                total = __builtin_fmaf(wp, sm, total);
            }
            const float inv = 1.0f / total;
            att[t] = (acc * inv) / gden[t];
        }
        if (t == 0) __hip_atomic_store(S.dcount + g, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (wave == 0) {
        const int Kg = HP * vd;
        a8_group(lane < Kg ? att[lane] : 0.0f, lane + 64 < Kg ? att[lane + 64] : 0.0f, lane, out_bits,
                 S.xq_att + (size_t)g * GROUP, S.sx_att + g);
    }
}

bool dec_chunks_fits(const Dims& D) {
    if (GROUP % D.vd != 0 || D.taps > DG_MAX_TAPS) return false;
    const int hp = GROUP / D.vd;
    return (hp == 2 || hp == 4) && D.nh % hp == 0 && (D.nh / D.nkv) % hp == 0 && D.qk % 16 == 0 &&
           D.nh / hp <= DCOUNT_SLOTS;
}

// The slot runs of every key chunk of position p0 under span K (keys in
// span_key's order: per live run, its part below the sink, then its part in
// the ring's range; a ring part's slots break where the ring wraps); false
// when a chunk needs more than DC_RUNS runs or there are more than
// DC_RUN_CHUNKS chunks.
static bool chunk_runs(const Dims& D, const KeySpan& K, int lo, int p0, int n, int count, int chunk, ChunkRuns& R) {
    if (count > DC_RUN_CHUNKS || chunk > RUN_CHUNK || D.ring <= 0) return false;
    int alo, ahi, blo, bhi;
    span_ranges(D, K, lo, p0, alo, ahi, blo, bhi);
    R = ChunkRuns{};
    for (int c = 0; c < DC_RUN_CHUNKS; ++c)
        for (int r = 0; r < DC_RUNS; ++r) R.key0[c][r] = RUN_NONE;
    int k = 0;  // keys so far
    auto add = [&](int pa, int pb) -> bool {
        // positions pa .. pb - 1 (all below the sink or all in the ring's range)
        while (pa < pb) {
            int m = pb - pa, slot = pa;
            if (pa >= D.sink) {
                slot = (pa - D.sink) % D.ring + D.sink;
                m = std::min(m, D.sink + D.ring - slot);  // to the ring's wrap
            }
            // the keys k .. k + m - 1 at slots slot .., cut into chunks
            for (int j = 0; j < m;) {
                const int c = (k + j) / chunk, cend = std::min(n, (c + 1) * chunk);
                const int take = std::min(m - j, cend - (k + j));
                if (c >= count || R.nrun[c] >= DC_RUNS) return false;
                const int r = R.nrun[c]++;
                R.key0[c][r] = k + j - c * chunk;
                R.slot0[c][r] = slot + j;
                R.len[c][r] = take;
                j += take;
            }
            k += m;
            pa += m;
        }
        return true;
    };
    for (int r = 0; r < K.nrun; ++r) {
        if (!add(std::max(K.lo[r], alo), std::min(K.hi[r], ahi))) return false;
        if (!add(std::max(K.lo[r], blo), std::min(K.hi[r], bhi))) return false;
    }
    return k == n;
}

hipError_t fwd_dec_chunks(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int out_bits,
                          const KeySpan* span, hipStream_t s) {
    const int hp = GROUP / D.vd, lo = window_lo(L.window, p0);
    int n = p0 + 1 - lo;
    if (span) {
        int alo, ahi, blo, bhi;
        span_ranges(D, *span, lo, p0, alo, ahi, blo, bhi);
        n = span_count(*span, alo, ahi, blo, bhi);
    }
    int count, chunk;
    key_chunks(n, D.nkv, false, count, chunk);
    if (n < 1 || count < 1 || count > D.max_chunks || chunk > ATT_CHUNK_MAX) return hipErrorInvalidValue;
    const int blocks = D.nh / hp * count + 1;
    const KeySpan K = span ? *span : KeySpan{};
    ChunkRuns R{};
    const bool runs = span && chunk_runs(D, K, lo, p0, n, count, chunk, R);
#define NH_DC(HP, TP, EX, SP, RN)                                                                                      \
    hipLaunchKernelGGL((k_dec_chunks<HP, TP, EX, SP, RN>), dim3(blocks), dim3(DG_THREADS), 0, s, D, S, L, layer, p0, \
                       out_bits, K, n, count, chunk, R)
#define NH_DC_TAPS(HP, SP, RN)                          \
    switch (D.taps) {                                   \
        case 1: NH_DC(HP, 1, true, SP, RN); break;      \
        case 2: NH_DC(HP, 2, true, SP, RN); break;      \
        case 3: NH_DC(HP, 3, true, SP, RN); break;      \
        case 4: NH_DC(HP, 4, true, SP, RN); break;      \
        default: NH_DC(HP, DG_MAX_TAPS, false, SP, RN); \
    }
    if (hp == 2) {
        if (runs) {
            NH_DC_TAPS(2, true, true)
        } else if (span) {
            NH_DC_TAPS(2, true, false)
        } else {
            NH_DC_TAPS(2, false, false)
        }
    } else {
        if (runs) {
            NH_DC_TAPS(4, true, true)
        } else if (span) {
            NH_DC_TAPS(4, true, false)
        } else {
            NH_DC_TAPS(4, false, false)
        }
    }
#undef NH_DC_TAPS
#undef NH_DC
    return hipGetLastError();
}

// ----------------------------------------------------------------- argmax
// k_argmax: block_argmax (above) by one workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int n, uint32_t* __restrict__ dst) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const uint32_t r = block_argmax<1024>(x, n, sv, si);
    if (threadIdx.x == 0) dst[0] = r;
}

hipError_t fwd_argmax(const float* logits, int n, uint32_t* dst, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, logits, n, dst);
    return hipGetLastError();
}

// ------------------------------------------------------------------- Phi8
// Phi8::new (infer.rs:850-867): each row requantized to int8 with its own
// quant_i8 scale.  One workgroup per row.
__global__ __launch_bounds__(256) void k_phi8(const float* __restrict__ rows, int width, int8_t* __restrict__ q,
                                              float* __restrict__ scale) {
    const int r = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const float* x = rows + (size_t)r * width;
    float m = 0.0f;
    for (int i = t; i < width; i += 256) m = fmaxf(m, fabsf(x[i]));
    m = wave_max_nonneg(m);
    __shared__ float red[4];
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = m > 0.0f ? m * bits_f32(0x3c010204u) : 1.0f;
    const float inv = 1.0f / s;
    for (int i = t; i < width; i += 256) q[(size_t)r * width + i] = quant_one(x[i], inv);
    if (t == 0) scale[r] = s;
}

hipError_t fwd_phi8(const float* rows, int nrows, int width, int8_t* q, float* scale, hipStream_t s) {
    if (nrows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_phi8, dim3(nrows), dim3(256), 0, s, rows, width, q, scale);
    return hipGetLastError();
}

}  // namespace nh
