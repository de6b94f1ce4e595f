// The decode GEMV's tile (one 16-row tile of a CQ matrix against one
// token, the reference's decode combine) and the launch shapes by group
// count, shared by the library's two GEMV translation units: nh_gemv.hip
// (streamed matrices, the debug partials, the tall-matrix grid and the read
// floors) and nh_gemv_res.hip (resident matrices, built with the kernel
// arguments preloaded into scalar registers).
#pragma once

#include <type_traits>

#include "nh_device.h"
#include "nh_internal.h"

namespace nh {

// NT: the code loads carry the non-temporal hint (a matrix read once per
// sweep of more than the caches hold); without it (a resident matrix, read
// again at every token) their lines stay cached.
template <int GPS, int S, int BITS, bool DBG, bool NT>
__device__ __forceinline__ void gemv_tile(const void* __restrict__ codes, const uint16_t* __restrict__ norms,
                                          const uint4* __restrict__ xq, const float* __restrict__ sx,
                                          float* __restrict__ y, int32_t* __restrict__ dbg, int out, int G, float cbs,
                                          Lut lut, int tile) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane >> 2, l = lane & 3;
    const int n = tile * TILE_ROWS + r;
    const int g0 = wave * GPS;

    // The token's activations, issued ahead of the code stream.  With one
    // group per wavefront a lane reads its decode lane's 32 bytes itself (the
    // 16 rows' lanes with the same l share them: one 128-byte span per
    // wavefront, an L2 hit after the first workgroup) and no barrier waits
    // for the slowest wavefront; with more, the G * 128 bytes go to LDS once
    // per workgroup (two direct reads per group measured slower there).
    constexpr bool DIRECT = GPS == 1;
    static_assert(DIRECT || S * 64 >= GPS * S * 8, "one thread per activation uint4");
    __shared__ uint4 xs[DIRECT ? 1 : GPS * S * 8];
    uint4 xa[GPS], xb[GPS], xv = make_uint4(0, 0, 0, 0);
    if constexpr (DIRECT) {
        const int g = g0 < G ? g0 : 0;
        xa[0] = xq[(g * 4 + l) * 2];
        xb[0] = xq[(g * 4 + l) * 2 + 1];
    } else if (threadIdx.x < G * 8) {
        xv = xq[threadIdx.x];
    }
    // A lane's chunk: 16 bytes (4-bit: 32 codes) or 8 (2-bit: 32 codes).
    using Chunk = typename std::conditional<BITS == 4, uint4, uint2>::type;
    Chunk c[GPS];
    uint16_t nb[GPS];
    float sxv[GPS];
#pragma unroll
    for (int j = 0; j < GPS; ++j) {
        // Groups past G (when S * GPS > G) reload group 0; never used.
        const int g = g0 + j < G ? g0 + j : 0;
        if constexpr (BITS == 4) {
            const uint4* p = reinterpret_cast<const uint4*>(codes) + ((size_t)(tile * G + g) * 64 + lane);
            c[j] = NT ? load_stream(p) : *p;
        } else
            c[j] = reinterpret_cast<const uint2*>(codes)[(size_t)(tile * G + g) * 64 + lane];
        nb[j] = norms[(size_t)n * G + g];
        sxv[j] = sx[g];
    }
    if constexpr (!DIRECT) {
        if (threadIdx.x < G * 8) xs[threadIdx.x] = xv;
        __syncthreads();
    }
    float lf[GPS], sc[GPS];
#pragma unroll
    for (int j = 0; j < GPS; ++j) {
        uint4 x0, x1;
        if constexpr (DIRECT) {
            x0 = xa[j];
            x1 = xb[j];
        } else {
            const int g = g0 + j < G ? g0 + j : 0;
            const uint4* xp = xs + (g * 4 + l) * 2;
            x0 = xp[0];
            x1 = xp[1];
        }
        int isum;
        if constexpr (BITS == 4)
            isum = dot_chunk(c[j], x0, x1, lut);
        else
            isum = dot_chunk2(c[j], x0, x1, lut.a_lo);
        if (DBG && n < out && g0 + j < G) dbg[((size_t)n * G + g0 + j) * 4 + l] = isum;
        lf[j] = (float)isum;
        sc[j] = (sxv[j] * cbs) * f16_bits_to_f32(nb[j]);
    }

    float acc = 0.0f;
    if constexpr (S == 1) {
#pragma unroll
        for (int j = 0; j < GPS; ++j)
            if (j < G) acc = __builtin_fmaf(lf[j], sc[j], acc);
    } else {
        __shared__ float2 part[GPS * S][64];
#pragma unroll
        for (int j = 0; j < GPS; ++j) part[g0 + j][lane] = make_float2(lf[j], sc[j]);
        __syncthreads();
        if (wave != 0) return;
        for (int g = 0; g < G; ++g) {
            const float2 p = part[g][lane];
            acc = __builtin_fmaf(p.x, p.y, acc);
        }
    }
    // (l0 + l1) + (l2 + l3) across the row's four lanes.
    const float t = acc + quad_xor1(acc);
    const float u = t + quad_xor2(t);
    if (y && l == 0 && n < out) y[n] = u;
}

// A launch shape: GPS groups per wavefront, S wavefronts per tile.
template <int GPS_, int S_>
struct GemvShape {
    static constexpr int GPS = GPS_, S = S_;
};

// Groups per wavefront (GPS) and wavefronts per tile (S) by group count:
// two to four groups per lane keeps 2-4 KiB of loads in flight per
// wavefront while giving the big shapes several wavefronts per CU (at
// K = 2048, 8 wavefronts x 2 groups measured 2.4 % faster than 4 x 4; at
// K = 768, 6 x 1 5 % faster than 2 x 3).  Any G up to 32 maps to the
// smallest listed G' >= G (wavefronts skip the groups past G).  f is called
// with the shape (a GemvShape) and returns its launch status.
template <typename F>
__host__ hipError_t gemv_shape(int G, F&& f) {
    if (G <= 1) return f(GemvShape<1, 1>{});
    if (G <= 2) return f(GemvShape<2, 1>{});
    if (G <= 3) return f(GemvShape<3, 1>{});
    if (G <= 4) return f(GemvShape<2, 2>{});
    if (G <= 6) return f(GemvShape<1, 6>{});
    if (G <= 8) return f(GemvShape<2, 4>{});
    if (G <= 12) return f(GemvShape<3, 4>{});
    if (G <= 16) return f(GemvShape<2, 8>{});
    if (G <= 24) return f(GemvShape<4, 6>{});
    if (G <= 32) return f(GemvShape<4, 8>{});
    return hipErrorInvalidValue;
}

// The same for several same-shaped products in one launch.
template <typename F>
__host__ hipError_t gemv_batch_shape(int G, F&& f) {
    if (G <= 1) return f(GemvShape<1, 1>{});
    if (G <= 2) return f(GemvShape<2, 1>{});
    if (G <= 3) return f(GemvShape<3, 1>{});
    if (G <= 4) return f(GemvShape<2, 2>{});
    if (G <= 6) return f(GemvShape<3, 2>{});
    if (G <= 8) return f(GemvShape<2, 4>{});
    if (G <= 12) return f(GemvShape<3, 4>{});
    if (G <= 16) return f(GemvShape<4, 4>{});
    if (G <= 24) return f(GemvShape<4, 6>{});
    if (G <= 32) return f(GemvShape<4, 8>{});
    return hipErrorInvalidValue;
}

// The resident matrices' products (nh_gemv_res.hip): one token, and several
// same-shaped products in one launch.
hipError_t launch_gemv_resident(const nh_qmat* w, const nh_qact* a, float* y, hipStream_t s);
hipError_t launch_gemv_batch_resident(const nh_qmat* w, const GemvBatch& b, int n, hipStream_t s);

}  // namespace nh
