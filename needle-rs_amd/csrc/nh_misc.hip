// Smaller kernels on the CQ path: sparse single-row logits, dequantized
// rows (embedding lookups) and the CQ-W4 weight quantizer.
#include "nh_device.h"
#include "nh_internal.h"

namespace nh {

// ---------------------------------------------------------------- single rows
// QMat::single_row (crates/needle-engine/src/qlinear.rs:454-456): the
// prefill block combine for token 0, acc = fma(S_g, (norm * cbs) * sx_g, acc).
// One wavefront per id: lane = 4 * gs + l covers groups gs, gs + 16, ...;
// the quad sum of its four decode lanes is the group total (exact), and the
// fma chain runs over groups in order with the totals fetched by shuffle.
constexpr int SR_WAVES = 4;
constexpr int SR_MAX_GROUPS = 32;

template <int BITS>
__global__ __launch_bounds__(SR_WAVES * 64) void k_single_rows(const void* __restrict__ codes,
                                                               const uint16_t* __restrict__ norms,
                                                               const uint4* __restrict__ xq,
                                                               const float* __restrict__ sx,
                                                               const uint32_t* __restrict__ ids, int n, int out,
                                                               int G, float cbs, Lut lut, float* __restrict__ vals,
                                                               float* __restrict__ logits, int logits_n) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i = blockIdx.x * SR_WAVES + wave;
    if (i >= n) return;
    const uint32_t row = ids[i];
    const bool ok = row < (uint32_t)out;
    const uint32_t rr = ok ? row : 0u;
    const int l = lane & 3, gs = lane >> 2;
    const int tile = rr / TILE_ROWS, rt = rr % TILE_ROWS;
    int tot[SR_MAX_GROUPS / 16];
#pragma unroll
    for (int j = 0; j < SR_MAX_GROUPS / 16; ++j) {
        const int g = gs + 16 * j;
        int s = 0;
        if (g < G) {
            const size_t ci = ((size_t)tile * G + g) * 64 + rt * 4 + l;
            const uint4* xp = xq + (g * 4 + l) * 2;
            if constexpr (BITS == 4)
                s = dot_chunk(reinterpret_cast<const uint4*>(codes)[ci], xp[0], xp[1], lut);
            else
                s = dot_chunk2(reinterpret_cast<const uint2*>(codes)[ci], xp[0], xp[1], lut.a_lo);
        }
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        tot[j] = s;
    }
    float acc = 0.0f;
    for (int g = 0; g < G; ++g) {
        int s = __shfl(tot[g / 16], 4 * (g % 16), 64);
        float norm = f16_bits_to_f32(norms[(size_t)rr * G + g]);
        float sc = (norm * cbs) * sx[g];
        acc = __builtin_fmaf((float)s, sc, acc);
    }
    if (lane == 0) {
        float v = ok ? acc : __builtin_nanf("");
        if (vals) vals[i] = v;
        if (logits && row < (uint32_t)logits_n) logits[row] = v;
    }
}

hipError_t launch_single_rows(const nh_qmat* w, const nh_qact* a, const uint32_t* ids, int n, float* out,
                              float* scatter_logits, int scatter_n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (w->m.groups > SR_MAX_GROUPS) return hipErrorInvalidValue;
    const Lut lut{w->m.lut.a_hi, w->m.lut.a_lo, w->m.lut.b_hi, w->m.lut.b_lo};
    auto kern = w->m.bits == 2 ? k_single_rows<2> : k_single_rows<4>;
    hipLaunchKernelGGL(kern, dim3((n + SR_WAVES - 1) / SR_WAVES), dim3(SR_WAVES * 64), 0, s, w->d_codes, w->d_norms,
                       (const uint4*)a->d_xq, a->d_sx, ids, n, w->m.out, w->m.groups, w->m.cbs, lut, out,
                       scatter_logits, scatter_n);
    return hipGetLastError();
}

__global__ void k_fill(float* __restrict__ p, float v, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

hipError_t launch_fill(float* p, float v, int n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill, dim3((n + 255) / 256), dim3(256), 0, s, p, v, n);
    return hipGetLastError();
}

// ----------------------------------------------------------------- row lookup
// QMat::row (crates/needle-engine/src/qlinear.rs:309-323): per group
// cb[code] * norm, then the normalised rotation.  One wavefront per
// (id, group), two positions per lane.
template <int BITS>
__global__ __launch_bounds__(256) void k_rows(const void* __restrict__ codes, const uint16_t* __restrict__ norms,
                                              const float* __restrict__ fsel, const uint32_t* __restrict__ ids,
                                              int n, int out, int G, int in_dim, float* __restrict__ dst) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int unit = blockIdx.x * 4 + wave;
    if (unit >= n * G) return;
    const int i = unit / G, g = unit % G;
    const uint32_t row = ids[i];
    const bool ok = row < (uint32_t)out;
    float v0, v1;
    row_group<BITS>(codes, norms, fsel, G, ok ? row : 0u, g, lane, v0, v1);
    if (!ok) v0 = v1 = __builtin_nanf("");
    const int p0 = g * GROUP + lane, p1 = p0 + 64;
    float* o = dst + (size_t)i * in_dim;
    if (p0 < in_dim) o[p0] = v0;
    if (p1 < in_dim) o[p1] = v1;
}

hipError_t launch_rows(const nh_qmat* w, const uint32_t* ids, int n, float* out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int units = n * w->m.groups;
    auto kern = w->m.bits == 2 ? k_rows<2> : k_rows<4>;
    hipLaunchKernelGGL(kern, dim3((units + 3) / 4), dim3(256), 0, s, w->d_codes, w->d_norms, w->d_fsel, ids, n,
                       w->m.out, w->m.groups, w->m.in_dim, out);
    return hipGetLastError();
}

// ------------------------------------------------------------------- cq_pack
// cq_pack (crates/needle-core/src/quant.rs:233-256) for 4-bit group-128:
// per (row, group) the zero-padded group is rotated, its L2 norm is the
// sequential f32 sum of squares in position order then sqrtf
// (quant.rs:127-135), every element snaps to nearest(v / max(norm, 1e-12))
// (quant.rs:119-124, ties low), the norm is stored f16 (round to nearest
// even) and the indices are packed LSB-first (quant.rs:185-198).  Output is
// the archive layout: packed[rows][groups * 64], norms[rows][groups].
__global__ __launch_bounds__(256) void k_cq_pack(const float* __restrict__ w, int rows, int d, int G,
                                                 const float* __restrict__ cb, uint8_t* __restrict__ packed,
                                                 uint16_t* __restrict__ norms) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int unit = blockIdx.x * 4 + wave;
    const bool active = unit < rows * G;
    __shared__ float sq[4][GROUP];
    __shared__ float scb[16];
    if (threadIdx.x < 16) scb[threadIdx.x] = cb[threadIdx.x];
    const int row = active ? unit / G : 0, g = active ? unit % G : 0;
    const int p0 = g * GROUP + lane, p1 = p0 + 64;
    const float* src = w + (size_t)row * d;
    float v0 = (active && p0 < d) ? src[p0] : 0.0f;
    float v1 = (active && p1 < d) ? src[p1] : 0.0f;
    fwht128(v0, v1, lane);
    const float hs = bits_f32(0x3db504f3u);
    v0 *= hs;
    v1 *= hs;
    sq[wave][lane] = v0 * v0;
    sq[wave][lane + 64] = v1 * v1;
    __syncthreads();
    if (!active) return;
    float norm = 0.0f;
    for (int i = 0; i < GROUP; ++i) norm = norm + sq[wave][i];
    norm = __builtin_sqrtf(norm);
    const float denom = norm > 1e-12f ? norm : 1e-12f;
    auto nearest = [&](float x) -> uint32_t {
        int pos = 0;
        while (pos < 16 && scb[pos] < x) ++pos;
        pos = pos < 1 ? 1 : (pos > 15 ? 15 : pos);
        const float lo = scb[pos - 1], hi = scb[pos];
        return fabsf(x - lo) <= fabsf(x - hi) ? (uint32_t)(pos - 1) : (uint32_t)pos;
    };
    const uint32_t i0 = nearest(v0 / denom);
    const uint32_t i1 = nearest(v1 / denom);
    const uint32_t n0 = __shfl_down(i0, 1, 64);
    const uint32_t n1 = __shfl_down(i1, 1, 64);
    uint8_t* prow = packed + (size_t)row * G * 64 + (size_t)g * 64;
    if ((lane & 1) == 0) {
        prow[lane >> 1] = (uint8_t)(i0 | (n0 << 4));
        prow[32 + (lane >> 1)] = (uint8_t)(i1 | (n1 << 4));
    }
    if (lane == 0) norms[(size_t)row * G + g] = __builtin_bit_cast(uint16_t, (_Float16)norm);
}

hipError_t launch_cq_pack(const float* w, int rows, int d, int groups, const float* cb, uint8_t* packed,
                          uint16_t* norms, hipStream_t s) {
    const int units = rows * groups;
    if (units <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_cq_pack, dim3((units + 3) / 4), dim3(256), 0, s, w, rows, d, groups, cb, packed, norms);
    return hipGetLastError();
}

}  // namespace nh
