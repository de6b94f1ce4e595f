// Decode GEMV: one token against a CQ matrix with the reference's decode
// combine (crates/needle-engine/src/qlinear.rs:340-350): four float lanes
// per row, lane l fed by positions p with (p % 32) / 8 == l (4-bit) or
// (p % 64) / 16 == l (2-bit, qlinear.rs:333), scale
// (sx * cbs) * norm, lane_l = fma(sum_l, scale, lane_l) over groups in
// order, y = (l0 + l1) + (l2 + l3).
//
// HBM-bound.  A workgroup owns one 16-row tile.  Its S wavefronts split the
// tile's groups (GPS each); in a wavefront, lane = 4 * row + l, so each
// load instruction reads the tile-group block (16 rows x 4 lanes x 16 B)
// as 1 KiB (4-bit; 512 B for 2-bit) of contiguous HBM.  A lane's 16 (8)
// bytes are exactly its decode lane's 32 codes of the group, so its integer sum is the reference's
// lane sum L[n][g][l] (qlinear.rs:327-337) with no cross-lane reduction.
// Every load (codes, activations, norms, scales) is issued before any
// arithmetic, so a launch costs one memory round trip; each wavefront
// turns its groups into (float(L), scale) pairs and wave 0 runs the
// group-ordered fma chain from LDS.
#include <string.h>

#include "nh_gemv_tile.h"

namespace nh {

// Workgroups per CU of the streaming variant, and the tile count from which
// it replaces one workgroup per tile (8 tiles per workgroup).
constexpr int STREAM_WG_PER_CU = 4;

template <int GPS, int S, int BITS, bool DBG, bool NT>
__global__ __launch_bounds__(S * 64) void k_gemv(const void* __restrict__ codes, const uint16_t* __restrict__ norms,
                                                 const uint4* __restrict__ xq, const float* __restrict__ sx,
                                                 float* __restrict__ y, int32_t* __restrict__ dbg, int out, int G,
                                                 float cbs, Lut lut) {
    gemv_tile<GPS, S, BITS, DBG, NT>(codes, norms, xq, sx, y, dbg, out, G, cbs, lut, blockIdx.x);
}

// Several same-shaped products in one launch (blockIdx.y picks the member),
// e.g. the engram key | value products of every site.
template <int GPS, int S, int BITS, bool NT>
__global__ __launch_bounds__(S * 64) void k_gemv_batch(GemvBatch b, int out, int G, float cbs, Lut lut) {
    const int e = blockIdx.y;
    gemv_tile<GPS, S, BITS, false, NT>(b.codes[e], b.norms[e], b.xq[e], b.sx[e], b.y[e], nullptr, out, G, cbs, lut,
                                       blockIdx.x);
}

// The same product for very tall matrices (4-bit): a persistent grid of a
// few workgroups per CU, each staging the token's activations once and
// walking tiles blockIdx.x, + gridDim.x, ...; a tile's codes and norms are
// loaded while the previous tile combines (two tiles per loop turn, so the
// register buffers alternate statically; the combine slots alternate too,
// so one barrier per tile suffices).
template <int GPS, int S>
__global__ __launch_bounds__(S * 64) void k_gemv_stream(const uint4* __restrict__ codes,
                                                        const uint16_t* __restrict__ norms,
                                                        const uint4* __restrict__ xq, const float* __restrict__ sx,
                                                        float* __restrict__ y, int out, int G, float cbs, Lut lut,
                                                        int tiles) {
    static_assert(S * 64 >= GPS * S * 8, "one thread per activation uint4");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane >> 2, l = lane & 3;
    const int g0 = wave * GPS;
    __shared__ uint4 xs[GPS * S * 8];
    __shared__ float2 part[2][GPS * S][64];
    if ((int)threadIdx.x < G * 8) xs[threadIdx.x] = xq[threadIdx.x];
    float sxc[GPS];
#pragma unroll
    for (int j = 0; j < GPS; ++j) sxc[j] = sx[g0 + j < G ? g0 + j : 0] * cbs;
    struct Tile {
        uint4 c[GPS];
        uint16_t nb[GPS];
    };
    auto load = [&](Tile& b, int tile) __attribute__((always_inline)) {
        const int tl = tile < tiles ? tile : tiles - 1;  // past the end: reload the last tile, never stored
#pragma unroll
        for (int j = 0; j < GPS; ++j) {
            const int g = g0 + j < G ? g0 + j : 0;
            b.c[j] = load_stream(codes + ((size_t)(tl * G + g) * 64 + lane));
            b.nb[j] = norms[(size_t)(tl * TILE_ROWS + r) * G + g];
        }
    };
    auto combine = [&](const Tile& b, int tile, int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < GPS; ++j) {
            const int g = g0 + j < G ? g0 + j : 0;
            const uint4* xp = xs + (g * 4 + l) * 2;
            const float lf = (float)dot_chunk(b.c[j], xp[0], xp[1], lut);
            part[slot][g0 + j][lane] = make_float2(lf, sxc[j] * f16_bits_to_f32(b.nb[j]));
        }
        __syncthreads();
        if (wave == 0 && tile < tiles) {
            float acc = 0.0f;
            for (int g = 0; g < G; ++g) {
                const float2 p = part[slot][g][lane];
                acc = __builtin_fmaf(p.x, p.y, acc);
            }
            // (l0 + l1) + (l2 + l3) across the row's four lanes.
            const float t = acc + quad_xor1(acc);
            const float u = t + quad_xor2(t);
            const int n = tile * TILE_ROWS + r;
            if (l == 0 && n < out) y[n] = u;
        }
    };
    Tile ta, tb;
    load(ta, blockIdx.x);
    __syncthreads();  // the activations
    const int step = gridDim.x;
    for (int tile = blockIdx.x; tile < tiles; tile += 2 * step) {
        load(tb, tile + step);
        combine(ta, tile, 0);
        load(ta, tile + 2 * step);
        combine(tb, tile + step, 1);
    }
}

// A 4-bit matrix tall enough for the persistent streaming grid.
static bool gemv_tall(const nh_qmat* w) {
    return w->m.bits == 4 && w->m.out_pad / TILE_ROWS >= 8 * device_cus() * STREAM_WG_PER_CU;
}

// Streamed matrices (codes read with the non-temporal hint) and the debug
// partials; a resident matrix's product is launched by nh_gemv_res.hip.
template <int GPS, int S, int BITS>
static hipError_t run(const nh_qmat* w, const nh_qact* a, float* y, int32_t* dbg, hipStream_t s) {
    const QMatMeta& m = w->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    dim3 grid(m.out_pad / TILE_ROWS), block(S * 64);
    if (BITS == 4 && !dbg && gemv_tall(w)) {
        const int tiles = m.out_pad / TILE_ROWS, slots = device_cus() * STREAM_WG_PER_CU;
        hipLaunchKernelGGL((k_gemv_stream<GPS, S>), dim3(slots), block, 0, s, (const uint4*)w->d_codes, w->d_norms,
                           (const uint4*)a->d_xq, a->d_sx, y, m.out, m.groups, m.cbs, lut, tiles);
        return hipGetLastError();
    }
    auto kern = dbg ? k_gemv<GPS, S, BITS, true, true> : k_gemv<GPS, S, BITS, false, true>;
    hipLaunchKernelGGL(kern, grid, block, 0, s, w->d_codes, w->d_norms, (const uint4*)a->d_xq, a->d_sx, y, dbg, m.out,
                       m.groups, m.cbs, lut);
    return hipGetLastError();
}

template <int BITS>
static hipError_t dispatch(const nh_qmat* w, const nh_qact* a, float* y, int32_t* dbg, hipStream_t s) {
    return gemv_shape(w->m.groups, [&](auto sh) {
        return run<decltype(sh)::GPS, decltype(sh)::S, BITS>(w, a, y, dbg, s);
    });
}

template <int BITS>
static hipError_t dispatch_batch(const nh_qmat* w, const GemvBatch& b, int n, hipStream_t s) {
    const QMatMeta& m = w->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    return gemv_batch_shape(m.groups, [&](auto sh) {
        constexpr int GPS = decltype(sh)::GPS, S = decltype(sh)::S;
        hipLaunchKernelGGL((k_gemv_batch<GPS, S, BITS, true>), dim3(m.out_pad / TILE_ROWS, n), dim3(S * 64), 0, s, b,
                           m.out, m.groups, m.cbs, lut);
        return hipGetLastError();
    });
}

bool gemv_batchable(const nh_qmat* const* w, int n) {
    if (n < 1 || n > GEMV_BATCH_MAX) return false;
    for (int i = 1; i < n; ++i)
        if (w[i]->m.out != w[0]->m.out || w[i]->m.groups != w[0]->m.groups || w[i]->m.bits != w[0]->m.bits ||
            w[i]->m.cbs != w[0]->m.cbs || memcmp(&w[i]->m.lut, &w[0]->m.lut, sizeof(LutTables)) != 0)
            return false;
    return true;
}

hipError_t launch_gemv_batch(const nh_qmat* const* w, const nh_qact* const* a, float* const* y, int n, hipStream_t s) {
    GemvBatch b{};
    for (int i = 0; i < n; ++i) {
        b.codes[i] = w[i]->d_codes;
        b.norms[i] = w[i]->d_norms;
        b.xq[i] = (const uint4*)a[i]->d_xq;
        b.sx[i] = a[i]->d_sx;
        b.y[i] = y[i];
    }
    if (w[0]->resident) return launch_gemv_batch_resident(w[0], b, n, s);
    return w[0]->m.bits == 2 ? dispatch_batch<2>(w[0], b, n, s) : dispatch_batch<4>(w[0], b, n, s);
}

// Read floors of the decode product, for measurement only.  The tile form
// issues exactly the loads k_gemv<GPS, S, 4> issues (codes with the
// streaming hint, norms, activations, scales) in its grid, and no
// arithmetic or LDS; the stream form reads the codes and the norms as a
// plain grid-stride stream of 16-byte loads, four in flight per lane.  An
// empty asm statement consumes the loaded values, so the loads stay.  With
// STORE the tile form then ends as the product does: a workgroup barrier
// (every wavefront's loads have arrived) and wavefront 0's store of one
// float per row; without it, nothing is stored.
template <int GPS, int S, bool STORE>
__global__ __launch_bounds__(S * 64) void k_read_floor_tile(const uint4* __restrict__ codes,
                                                            const uint16_t* __restrict__ norms,
                                                            const uint4* __restrict__ xq,
                                                            const float* __restrict__ sx, int G,
                                                            float* __restrict__ y, int out) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane >> 2, l = lane & 3;
    const int n = blockIdx.x * TILE_ROWS + r, g0 = wave * GPS;
    uint32_t x = 0;
    if (GPS == 1) {
        const int g = g0 < G ? g0 : 0;
        const uint4 a = xq[(g * 4 + l) * 2], b = xq[(g * 4 + l) * 2 + 1];
        x ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
    } else if ((int)threadIdx.x < G * 8) {
        const uint4 a = xq[threadIdx.x];
        x ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    uint4 c[GPS];
    uint32_t nb[GPS], sv[GPS];
#pragma unroll
    for (int j = 0; j < GPS; ++j) {
        const int g = g0 + j < G ? g0 + j : 0;
        c[j] = load_stream(codes + ((size_t)(blockIdx.x * G + g) * 64 + lane));
        nb[j] = norms[(size_t)n * G + g];
        sv[j] = __float_as_uint(sx[g]);
    }
#pragma unroll
    for (int j = 0; j < GPS; ++j) x ^= c[j].x ^ c[j].y ^ c[j].z ^ c[j].w ^ nb[j] ^ sv[j];
    asm volatile("" ::"v"(x));
    if constexpr (STORE) {
        __syncthreads();
        if (wave == 0 && l == 0 && n < out) y[n] = __uint_as_float(x & 0x3fffffffu);
    }
}

__global__ __launch_bounds__(256) void k_read_floor_stream(const uint4* __restrict__ a, size_t na,
                                                          const uint4* __restrict__ b, size_t nb) {
    constexpr int U = 4;
    const size_t stride = (size_t)gridDim.x * 256 * U;
    uint32_t x = 0;
    for (size_t i = (size_t)blockIdx.x * 256 * U + threadIdx.x; i < na + nb; i += stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t k = i + (size_t)u * 256;
            const size_t kk = k < na + nb ? k : 0;
            v[u] = load_stream(kk < na ? a + kk : b + (kk - na));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    asm volatile("" ::"v"(x));
}

template <int GPS, int S>
static hipError_t run_floor(const nh_qmat* w, const nh_qact* a, float* y, hipStream_t s) {
    auto kern = y ? k_read_floor_tile<GPS, S, true> : k_read_floor_tile<GPS, S, false>;
    hipLaunchKernelGGL(kern, dim3(w->m.out_pad / TILE_ROWS), dim3(S * 64), 0, s, (const uint4*)w->d_codes,
                       w->d_norms, (const uint4*)a->d_xq, a->d_sx, w->m.groups, y, w->m.out);
    return hipGetLastError();
}

hipError_t launch_read_floor(const nh_qmat* w, const nh_qact* a, int mode, float* y, hipStream_t s) {
    if (mode == 1) {
        // 16-byte units: codes out_pad x G x 64 bytes, norms out_pad x G x 2 bytes (out_pad: a multiple of 16)
        const size_t na = (size_t)w->m.out_pad * w->m.groups * 64 / 16, nb = (size_t)w->m.out_pad * w->m.groups * 2 / 16;
        const int grid = (int)((na + nb + 256 * 4 - 1) / (256 * 4));
        hipLaunchKernelGGL(k_read_floor_stream, dim3(grid), dim3(256), 0, s, (const uint4*)w->d_codes, na,
                           (const uint4*)w->d_norms, nb);
        return hipGetLastError();
    }
    if (mode != 2) y = nullptr;
    const int G = w->m.groups;  // the shapes dispatch<4> picks
    if (G <= 1) return run_floor<1, 1>(w, a, y, s);
    if (G <= 2) return run_floor<2, 1>(w, a, y, s);
    if (G <= 3) return run_floor<3, 1>(w, a, y, s);
    if (G <= 4) return run_floor<2, 2>(w, a, y, s);
    if (G <= 6) return run_floor<1, 6>(w, a, y, s);
    if (G <= 8) return run_floor<2, 4>(w, a, y, s);
    if (G <= 12) return run_floor<3, 4>(w, a, y, s);
    if (G <= 16) return run_floor<2, 8>(w, a, y, s);
    if (G <= 24) return run_floor<4, 6>(w, a, y, s);
    if (G <= 32) return run_floor<4, 8>(w, a, y, s);
    return hipErrorInvalidValue;
}

hipError_t launch_gemv(const nh_qmat* w, const nh_qact* a, float* y, int col0, int32_t* dbg, hipStream_t s) {
    float* yc = y ? y + col0 : nullptr;
    if (w->resident && !dbg && !gemv_tall(w)) return launch_gemv_resident(w, a, yc, s);
    return w->m.bits == 2 ? dispatch<2>(w, a, yc, dbg, s) : dispatch<4>(w, a, yc, dbg, s);
}

}  // namespace nh
