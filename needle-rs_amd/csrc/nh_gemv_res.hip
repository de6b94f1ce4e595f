// The decode GEMV of resident matrices (a loaded model's weights, read
// again at every token, so their code loads keep their cache lines): the
// same tile as nh_gemv.hip's (nh_gemv_tile.h), in a translation unit built
// with the kernel arguments preloaded into scalar registers, since these
// launches (one per product of every decode step) start from a few dozen
// to a few hundred workgroups that wait on their arguments first.
#include "nh_gemv_tile.h"

namespace nh {

template <int GPS, int S, int BITS>
__global__ __launch_bounds__(S * 64) void k_gemv_res(const void* __restrict__ codes, const uint16_t* __restrict__ norms,
                                                     const uint4* __restrict__ xq, const float* __restrict__ sx,
                                                     float* __restrict__ y, int out, int G, float cbs, Lut lut) {
    gemv_tile<GPS, S, BITS, false, false>(codes, norms, xq, sx, y, nullptr, out, G, cbs, lut, blockIdx.x);
}

// Several same-shaped products in one launch (blockIdx.y picks the member).
template <int GPS, int S, int BITS>
__global__ __launch_bounds__(S * 64) void k_gemv_batch_res(GemvBatch b, int out, int G, float cbs, Lut lut) {
    const int e = blockIdx.y;
    gemv_tile<GPS, S, BITS, false, false>(b.codes[e], b.norms[e], b.xq[e], b.sx[e], b.y[e], nullptr, out, G, cbs,
                                          lut, blockIdx.x);
}

template <int BITS>
static hipError_t res_one(const nh_qmat* w, const nh_qact* a, float* y, hipStream_t s) {
    const QMatMeta& m = w->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    return gemv_shape(m.groups, [&](auto sh) {
        constexpr int GPS = decltype(sh)::GPS, S = decltype(sh)::S;
        hipLaunchKernelGGL((k_gemv_res<GPS, S, BITS>), dim3(m.out_pad / TILE_ROWS), dim3(S * 64), 0, s, w->d_codes,
                           w->d_norms, (const uint4*)a->d_xq, a->d_sx, y, m.out, m.groups, m.cbs, lut);
        return hipGetLastError();
    });
}

template <int BITS>
static hipError_t res_batch(const nh_qmat* w, const GemvBatch& b, int n, hipStream_t s) {
    const QMatMeta& m = w->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    return gemv_batch_shape(m.groups, [&](auto sh) {
        constexpr int GPS = decltype(sh)::GPS, S = decltype(sh)::S;
        hipLaunchKernelGGL((k_gemv_batch_res<GPS, S, BITS>), dim3(m.out_pad / TILE_ROWS, n), dim3(S * 64), 0, s, b,
                           m.out, m.groups, m.cbs, lut);
        return hipGetLastError();
    });
}

hipError_t launch_gemv_resident(const nh_qmat* w, const nh_qact* a, float* y, hipStream_t s) {
    return w->m.bits == 2 ? res_one<2>(w, a, y, s) : res_one<4>(w, a, y, s);
}

hipError_t launch_gemv_batch_resident(const nh_qmat* w, const GemvBatch& b, int n, hipStream_t s) {
    return w->m.bits == 2 ? res_batch<2>(w, b, n, s) : res_batch<4>(w, b, n, s);
}

}  // namespace nh
