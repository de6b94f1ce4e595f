// Decode GEMV: one token against a CQ-W4 matrix with the reference's decode
// combine (crates/needle-engine/src/qlinear.rs:340-350): four float lanes
// per row, lane l fed by positions p with (p % 32) / 8 == l, scale
// (sx * cbs) * norm, lane_l = fma(sum_l, scale, lane_l) over groups in
// order, y = (l0 + l1) + (l2 + l3).
//
// HBM-bound.  A workgroup owns one 16-row tile.  Its S wavefronts split the
// tile's groups (GPS each); in a wavefront, lane = 4 * row + l, so each
// load instruction reads the tile-group block (16 rows x 4 lanes x 16 B)
// as 1 KiB of contiguous HBM.  A lane's 16 bytes are exactly its decode
// lane's 32 codes of the group, so its integer sum is the reference's
// lane sum L[n][g][l] (qlinear.rs:327-337) with no cross-lane reduction.
// Every load (codes, activations, norms, scales) is issued before any
// arithmetic, so a launch costs one memory round trip; each wavefront
// turns its groups into (float(L), scale) pairs and wave 0 runs the
// group-ordered fma chain from LDS.
#include "nh_device.h"
#include "nh_internal.h"

namespace nh {

template <int GPS, int S, bool DBG>
__global__ __launch_bounds__(S * 64) void k_gemv(const uint4* __restrict__ codes, const uint16_t* __restrict__ norms,
                                                 const uint4* __restrict__ xq, const float* __restrict__ sx,
                                                 float* __restrict__ y, int32_t* __restrict__ dbg, int out,
                                                 float cbs, Lut lut) {
    constexpr int G = GPS * S;
    static_assert(S * 64 >= G * 8, "one thread per activation uint4");
    const int tile = blockIdx.x;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane >> 2, l = lane & 3;
    const int n = tile * TILE_ROWS + r;
    const int g0 = wave * GPS;

    // The token's activations (G * 128 bytes) go to LDS once per workgroup;
    // their load is issued first so waiting for it does not wait for the
    // code stream behind it.
    __shared__ uint4 xs[G * 8];
    uint4 xv = make_uint4(0, 0, 0, 0);
    if (threadIdx.x < G * 8) xv = xq[threadIdx.x];
    uint4 c[GPS];
    uint16_t nb[GPS];
    float sxv[GPS];
#pragma unroll
    for (int j = 0; j < GPS; ++j) c[j] = load_stream(codes + ((size_t)(tile * G + g0 + j) * 64 + lane));
#pragma unroll
    for (int j = 0; j < GPS; ++j) {
        nb[j] = norms[(size_t)n * G + g0 + j];
        sxv[j] = sx[g0 + j];
    }
    if (threadIdx.x < G * 8) xs[threadIdx.x] = xv;
    __syncthreads();
    float lf[GPS], sc[GPS];
#pragma unroll
    for (int j = 0; j < GPS; ++j) {
        const uint4* xp = xs + ((g0 + j) * 4 + l) * 2;
        const int isum = dot_chunk(c[j], xp[0], xp[1], lut);
        if (DBG && n < out) dbg[((size_t)n * G + g0 + j) * 4 + l] = isum;
        lf[j] = (float)isum;
        sc[j] = (sxv[j] * cbs) * f16_bits_to_f32(nb[j]);
    }

    float acc = 0.0f;
    if constexpr (S == 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) acc = __builtin_fmaf(lf[g], sc[g], acc);
    } else {
        __shared__ float2 part[G][64];
#pragma unroll
        for (int j = 0; j < GPS; ++j) part[g0 + j][lane] = make_float2(lf[j], sc[j]);
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float2 p = part[g][lane];
            acc = __builtin_fmaf(p.x, p.y, acc);
        }
    }
    // (l0 + l1) + (l2 + l3) across the row's four lanes.
    float t = acc + __shfl_xor(acc, 1, 64);
    float u = t + __shfl_xor(t, 2, 64);
    if (y && l == 0 && n < out) y[n] = u;
}

template <int GPS, int S>
static hipError_t run(const nh_qmat* w, const nh_qact* a, float* y, int32_t* dbg, hipStream_t s) {
    const QMatMeta& m = w->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    dim3 grid(m.out_pad / TILE_ROWS), block(S * 64);
    if (dbg)
        hipLaunchKernelGGL((k_gemv<GPS, S, true>), grid, block, 0, s, w->d_codes, w->d_norms,
                           (const uint4*)a->d_xq, a->d_sx, y, dbg, m.out, m.cbs, lut);
    else
        hipLaunchKernelGGL((k_gemv<GPS, S, false>), grid, block, 0, s, w->d_codes, w->d_norms,
                           (const uint4*)a->d_xq, a->d_sx, y, dbg, m.out, m.cbs, lut);
    return hipGetLastError();
}

// Groups per wavefront and wavefronts per tile for each supported group
// count: two to four groups per lane keeps 2-4 KiB of loads in flight per
// wavefront while giving the big shapes several wavefronts per CU.
hipError_t launch_gemv(const nh_qmat* w, const nh_qact* a, float* y, int col0, int32_t* dbg, hipStream_t s) {
    float* yc = y ? y + col0 : nullptr;
    switch (w->m.groups) {
    case 1: return run<1, 1>(w, a, yc, dbg, s);
    case 2: return run<2, 1>(w, a, yc, dbg, s);
    case 3: return run<3, 1>(w, a, yc, dbg, s);
    case 4: return run<2, 2>(w, a, yc, dbg, s);
    case 5: return run<5, 1>(w, a, yc, dbg, s);
    case 6: return run<3, 2>(w, a, yc, dbg, s);
    case 8: return run<2, 4>(w, a, yc, dbg, s);
    case 12: return run<3, 4>(w, a, yc, dbg, s);
    case 16: return run<4, 4>(w, a, yc, dbg, s);
    case 24: return run<4, 6>(w, a, yc, dbg, s);
    case 32: return run<4, 8>(w, a, yc, dbg, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace nh
