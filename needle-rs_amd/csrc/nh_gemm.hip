// Prefill / batched W4A8 product on int8 MFMA with the reference's prefill
// combine (crates/needle-engine/src/qlinear.rs:353-363): per token t and
// row n, S = the exact int32 group sum, sc = (norm * cbs) * sx for block
// tokens and norm * (cbs * sx) for the rest, acc = fma(S, sc, acc) over
// groups in order.  Block tokens are t < rows / 4 * 4 (qlinear.rs:397) or
// an explicit per-token flag.
//
// v_mfma_i32_16x16x64_i8: MFMA row i = weight row, column j = token.  A
// group (128 inputs) is two MFMAs (k = 64 each) into a fresh int32
// accumulator, which the epilogue turns into the float fma chain, so every
// group sum is exact and separately scaled.  Lane L holds A/B bytes of the
// same k-slice (L / 16), and both operands draw that slice from the same
// 16-byte block of the group's activation order, so the dot product runs
// over exactly the group's 128 products whatever order the instruction
// visits k in.  The 4-bit codes are expanded to int8 in registers with two
// v_perm lookups per four codes.
#include "nh_device.h"
#include "nh_internal.h"

namespace nh {

constexpr int GEMM_WAVES = 4;

// One workgroup: GEMM_WAVES row tiles (16 rows each) x BMT token tiles (16
// tokens each).  Wave w computes rows of tile blockIdx.x * 4 + w.
template <int BMT, bool DBG>
__global__ __launch_bounds__(GEMM_WAVES * 64) void k_gemm(
    const uint2* __restrict__ codes, const uint16_t* __restrict__ norms, const uint4* __restrict__ xq,
    const float* __restrict__ sx, const uint8_t* __restrict__ block, int blocked, float* __restrict__ y, int ldy,
    int col0, int32_t* __restrict__ dbg, int out, int tiles, int M, int G, float cbs, Lut lut) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int tile = blockIdx.x * GEMM_WAVES + wave;
    if (tile >= tiles) return;
    const int m0 = blockIdx.y * (16 * BMT);
    const int r = lane & 15, q = lane >> 4;
    const int lA0 = q >> 1, lA1 = 2 + (q >> 1);

    // Per token tile: this lane's token, its block flag.
    int mt[BMT];
    bool blk[BMT];
#pragma unroll
    for (int t = 0; t < BMT; ++t) {
        mt[t] = m0 + 16 * t + r;
        const int m = mt[t];
        blk[t] = m < M ? (block ? block[m] != 0 : m < blocked) : true;
    }

    float acc[BMT][4];
#pragma unroll
    for (int t = 0; t < BMT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][v] = 0.0f;

    for (int g = 0; g < G; ++g) {
        const size_t base = ((size_t)tile * G + g) * 64;
        const uint2 c0 = codes[(base + r * 4 + lA0) * 2 + (q & 1)];
        const uint2 c1 = codes[(base + r * 4 + lA1) * 2 + (q & 1)];
        uint32_t e0, e1, e2, e3, f0, f1, f2, f3;
        expand8(c0.x, lut, e0, e1);
        expand8(c0.y, lut, e2, e3);
        expand8(c1.x, lut, f0, f1);
        expand8(c1.y, lut, f2, f3);
        const v4i a0 = {(int)e0, (int)e1, (int)e2, (int)e3};
        const v4i a1 = {(int)f0, (int)f1, (int)f2, (int)f3};
        float nf[4], nc[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            nf[v] = f16_bits_to_f32(norms[(size_t)(tile * TILE_ROWS + 4 * q + v) * G + g]);
            nc[v] = nf[v] * cbs;
        }
#pragma unroll
        for (int t = 0; t < BMT; ++t) {
            const int m = mt[t];
            const uint4* xp = xq + ((size_t)m * G + g) * 8;
            const uint4 b0 = xp[q], b1 = xp[4 + q];
            const v4i bb0 = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w};
            const v4i bb1 = {(int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
            v4i d = {0, 0, 0, 0};
            d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bb0, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bb1, d, 0, 0, 0);
            const float sxm = sx[(size_t)m * G + g];
            if (DBG && m < M) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int n = tile * TILE_ROWS + 4 * q + v;
                    if (n < out) dbg[((size_t)m * out + n) * G + g] = d[v];
                }
            }
            if (blk[t]) {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf((float)d[v], nc[v] * sxm, acc[t][v]);
            } else {
                const float cs = cbs * sxm;
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf((float)d[v], nf[v] * cs, acc[t][v]);
            }
        }
    }
    if (!y) return;
#pragma unroll
    for (int t = 0; t < BMT; ++t) {
        const int m = mt[t];
        if (m >= M) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = tile * TILE_ROWS + 4 * q + v;
            if (n < out) y[(size_t)m * ldy + col0 + n] = acc[t][v];
        }
    }
}

template <int BMT>
static hipError_t run(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                      int32_t* dbg, hipStream_t s) {
    const QMatMeta& m = w->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    const int tiles = m.out_pad / TILE_ROWS;
    const int M = a->rows;
    dim3 grid((tiles + GEMM_WAVES - 1) / GEMM_WAVES, (M + 16 * BMT - 1) / (16 * BMT)), blockdim(GEMM_WAVES * 64);
    const int blocked = M / 4 * 4;
    if (dbg)
        hipLaunchKernelGGL((k_gemm<BMT, true>), grid, blockdim, 0, s, (const uint2*)w->d_codes, w->d_norms,
                           (const uint4*)a->d_xq, a->d_sx, block, blocked, y, ldy, col0, dbg, m.out, tiles, M,
                           m.groups, m.cbs, lut);
    else
        hipLaunchKernelGGL((k_gemm<BMT, false>), grid, blockdim, 0, s, (const uint2*)w->d_codes, w->d_norms,
                           (const uint4*)a->d_xq, a->d_sx, block, blocked, y, ldy, col0, dbg, m.out, tiles, M,
                           m.groups, m.cbs, lut);
    return hipGetLastError();
}

hipError_t launch_gemm(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                       int32_t* dbg, hipStream_t s) {
    const int M = a->rows;
    if (M <= 16) return run<1>(w, a, block, y, ldy, col0, dbg, s);
    if (M <= 32) return run<2>(w, a, block, y, ldy, col0, dbg, s);
    return run<4>(w, a, block, y, ldy, col0, dbg, s);
}

}  // namespace nh
