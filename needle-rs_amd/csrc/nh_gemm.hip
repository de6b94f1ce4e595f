// Prefill / batched W4A8 product on int8 MFMA with the reference's prefill
// combine (crates/needle-engine/src/qlinear.rs:353-363): per token t and
// row n, S = the exact int32 group sum, sc = (norm * cbs) * sx for block
// tokens and norm * (cbs * sx) for the rest, acc = fma(S, sc, acc) over
// groups in order.  Block tokens are t < rows / 4 * 4 (qlinear.rs:397) or
// an explicit per-token flag.
//
// Workgroup tile: 64 weight rows x BM tokens; wavefront w owns rows
// 16w..16w+15 (one MFMA row tile) against all BM tokens.  The K dimension
// is walked in chunks of up to GC groups: a chunk's activations (int8),
// scales and norms are staged in LDS by the whole workgroup (double
// buffered, the next chunk's global loads in flight during this chunk's
// math), and each wavefront keeps its own rows' 4-bit codes for the chunk
// in registers, expanding them to int8 (two v_perm lookups per four codes)
// right before use.  Inside a chunk the groups run back to back with no
// barrier: per group two v_mfma_i32_16x16x64_i8 per token tile into a fresh
// int32 accumulator, then the float epilogue.
//
// MFMA operand note: lane L supplies A and B bytes of the same k-slice
// (L / 16), both cut from the same 16-byte block of the group's activation
// order, so each MFMA sums exactly its 64 products whatever order the
// instruction visits k in.
#include <type_traits>

#include "nh_device.h"
#include "nh_internal.h"

namespace nh {

constexpr int GEMM_ROWS = 64;  // weight rows per workgroup (4 wavefronts x 16)
constexpr int GC = 8;          // groups per LDS chunk

__device__ __forceinline__ int swz(int tok, int b) { return b ^ (tok & 7); }

template <int BM>
__host__ __device__ constexpr size_t gemm_lds_bytes(int nbuf) {
    return (size_t)nbuf * ((size_t)BM * GC * 128 + (size_t)BM * GC * 8 + (size_t)GEMM_ROWS * GC * 8);
}

template <int BM, bool GENERAL, bool DBG>
__global__ __launch_bounds__(256) void k_gemm(const uint2* __restrict__ codes, const uint16_t* __restrict__ norms,
                                              const uint4* __restrict__ xq, const float* __restrict__ sx,
                                              const uint8_t* __restrict__ block, int blocked, float* __restrict__ y,
                                              int ldy, int col0, int32_t* __restrict__ dbg, int out, int out_pad,
                                              int M, int G, float cbs, Lut lut) {
    constexpr int TT = BM / 16;  // token tiles per wavefront
    // LDS chunk buffer: activations [tok][gi][blk] (128 B per token-group),
    // scales [gi][tok] float2, norms [gi][row] float2.
    constexpr int XB = BM * GC * 128;
    constexpr int SB = BM * GC * 8;
    constexpr int BUF_BYTES = XB + SB + GEMM_ROWS * GC * 8;
    extern __shared__ uint4 lds[];
    char* const lbase = reinterpret_cast<char*>(lds);
    const int nchunks = (G + GC - 1) / GC;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
    const int r = lane & 15, q = lane >> 4;
    const int row0 = blockIdx.x * GEMM_ROWS;
    const int m0 = blockIdx.y * BM;
    const int tile = (row0 >> 4) + wave;  // this wavefront's 16-row code tile
    const bool tile_ok = tile * 16 < out_pad;
    const int ctile = tile_ok ? tile : 0;  // clamped: loads stay in bounds

    // Per-lane LDS byte offsets inside a chunk buffer; everything that
    // varies with the tile t, the group gi or the row v is a compile-time
    // constant folded into the ds_read offset field.
    const uint32_t xo0 = (uint32_t)(r * GC * 128 + swz(r, q) * 16);      // B fragment, k-half 0
    const uint32_t xo1 = (uint32_t)(r * GC * 128 + swz(r, 4 + q) * 16);  // k-half 1
    const uint32_t so = XB + r * 8;                                       // + gi * BM * 8 + t * 128
    const uint32_t no = XB + SB + (wave * 16 + 4 * q) * 8;                // + gi * 512 + v * 8

    // Global sources.  Codes: the two 8-byte pieces per group of this lane's
    // A fragments (chunks l = q/2 and 2 + q/2, dword pair q & 1).
    const uint2* cb0 = codes + (((size_t)ctile * G * 64 + r * 4 + (q >> 1)) * 2 + (q & 1));
    const uint2* cb1 = cb0 + 4;  // chunk l + 2
    // Activations: lane j fills slot j of a token's 1 KiB row: group j / 8,
    // physical block j % 8 = logical block ^ (tok & 7).
    const int xg = lane >> 3, xpb = lane & 7;
    // Scales / norms staged through registers: thread tid covers entries
    // tid and tid + 256 of the [gi][tok] / [gi][row] tables.
    float s_reg[2], n_reg[2];
    uint2 cwa[GC][2], cwb[GC][2];

    // Reads past the last group of a row land in the next row or in the
    // allocation's tail padding (one chunk's worth, see nh_api.hip); those
    // slots are staged but never used.
    const size_t xrow = (size_t)G * 8;  // uint4 per token row
    auto stage_load = [&](int c, int b, uint2 (&cdst)[GC][2]) __attribute__((always_inline)) {
        const int gb = c * GC;
        char* xdst = lbase + b * BUF_BYTES;
        const uint4* xs = xq + (size_t)(m0 + wave) * xrow + (gb + xg) * 8 + (xpb ^ wave);
#pragma unroll
        for (int i = 0; i < BM / 4; ++i) {
            const int tok = i * 4 + wave;
            // physical block xpb holds logical block xpb ^ (tok & 7); tok & 7
            // alternates between wave and wave + 4 with i.
            const uint4* src = xs + (size_t)i * 4 * xrow + ((i & 1) ? ((xpb ^ wave ^ 4) - (xpb ^ wave)) : 0);
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(xdst + tok * (GC * 128)), 16,
                                             0, 0);
        }
        s_reg[0] = sx[(size_t)(m0 + (tid % BM)) * G + gb + tid / BM];
        if constexpr (BM * GC > 256) s_reg[1] = sx[(size_t)(m0 + (tid % BM)) * G + gb + (256 + tid) / BM];
        const int nrow = row0 + (tid & 63) < out_pad ? row0 + (tid & 63) : 0;
        n_reg[0] = f16_bits_to_f32(norms[(size_t)nrow * G + gb + (tid >> 6)]);
        n_reg[1] = f16_bits_to_f32(norms[(size_t)nrow * G + gb + 4 + (tid >> 6)]);
        const uint2* c0 = cb0 + (size_t)gb * 128;
        const uint2* c1 = cb1 + (size_t)gb * 128;
#pragma unroll
        for (int k = 0; k < GC; ++k) {
            cdst[k][0] = c0[k * 128];
            cdst[k][1] = c1[k * 128];
        }
    };
    // After the staged loads landed: the register-staged tables.
    auto stage_store = [&](int b) __attribute__((always_inline)) {
        float2* sdst = reinterpret_cast<float2*>(lbase + b * BUF_BYTES + XB);
        float2* ndst = reinterpret_cast<float2*>(lbase + b * BUF_BYTES + XB + SB);
        sdst[tid] = make_float2(s_reg[0], cbs * s_reg[0]);
        if constexpr (BM * GC > 256) sdst[256 + tid] = make_float2(s_reg[1], cbs * s_reg[1]);
        ndst[tid] = make_float2(n_reg[0], n_reg[0] * cbs);
        ndst[256 + tid] = make_float2(n_reg[1], n_reg[1] * cbs);
    };

    // ---- per-lane output bookkeeping: token column r of each tile
    bool blk[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int m = m0 + t * 16 + r;
        blk[t] = !GENERAL || (m < M ? (block ? block[m] != 0 : m < blocked) : true);
    }
    float acc[TT][4];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][v] = 0.0f;

    // One group: all B fragments, every tile's two MFMAs into its own
    // accumulator (independent, so they pipeline), then the epilogues.
    auto do_group = [&](const uint2 (&cg)[2], const char* bb, int gi, int g) __attribute__((always_inline)) {
        uint32_t e0, e1, e2, e3, f0, f1, f2, f3;
        expand8(cg[0].x, lut, e0, e1);
        expand8(cg[0].y, lut, e2, e3);
        expand8(cg[1].x, lut, f0, f1);
        expand8(cg[1].y, lut, f2, f3);
        const v4i a0 = {(int)e0, (int)e1, (int)e2, (int)e3};
        const v4i a1 = {(int)f0, (int)f1, (int)f2, (int)f3};
        v4i b0[TT], b1[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            b0[t] = *reinterpret_cast<const v4i*>(bb + xo0 + t * 16 * GC * 128 + gi * 128);
            b1[t] = *reinterpret_cast<const v4i*>(bb + xo1 + t * 16 * GC * 128 + gi * 128);
        }
        float2 nr[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) nr[v] = *reinterpret_cast<const float2*>(bb + no + gi * GEMM_ROWS * 8 + v * 8);
        float2 sc[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) sc[t] = *reinterpret_cast<const float2*>(bb + so + gi * BM * 8 + t * 128);
        v4i d[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) d[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0[t], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < TT; ++t) d[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1[t], d[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            if (DBG) {
                const int m = m0 + t * 16 + r;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int n = row0 + wave * 16 + 4 * q + v;
                    if (m < M && n < out) dbg[((size_t)m * out + n) * G + g] = d[t][v];
                }
            }
            if (!GENERAL) {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf((float)d[t][v], nr[v].y * sc[t].x, acc[t][v]);
            } else {
                const float tf = blk[t] ? sc[t].x : sc[t].y;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float rf = blk[t] ? nr[v].y : nr[v].x;
                    acc[t][v] = __builtin_fmaf((float)d[t][v], rf * tf, acc[t][v]);
                }
            }
        }
    };
    // One chunk from LDS buffer B with codes cg, prefetching chunk c + 1
    // (into the other buffer and code registers cn) first.
    auto do_chunk = [&](auto Bc, int c, const uint2 (&cg)[GC][2], uint2 (&cn)[GC][2]) __attribute__((always_inline)) {
        constexpr int B = decltype(Bc)::value;
        const bool more = c + 1 < nchunks;
        if (more) stage_load(c + 1, B ^ 1, cn);
        const int gb = c * GC;
        const int gcc = min(GC, G - gb);
        const char* bb = lbase + B * BUF_BYTES;
#pragma unroll
        for (int gi = 0; gi < GC; ++gi) {
            if (gi >= gcc) break;
            do_group(cg[gi], bb, gi, gb + gi);
        }
        if (more) {
            // Buffer B ^ 1 was last read in the previous chunk, which every
            // wavefront left through the barrier below.
            __builtin_amdgcn_s_waitcnt(0);
            stage_store(B ^ 1);
            __syncthreads();
        }
    };

    stage_load(0, 0, cwa);
    __builtin_amdgcn_s_waitcnt(0);
    stage_store(0);
    __syncthreads();
    // Chunks in pairs so buffers and code registers alternate statically.
    for (int c = 0; c < nchunks; c += 2) {
        do_chunk(std::integral_constant<int, 0>{}, c, cwa, cwb);
        if (c + 1 < nchunks) do_chunk(std::integral_constant<int, 1>{}, c + 1, cwb, cwa);
    }
    if (!y || !tile_ok) return;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const int m = m0 + t * 16 + r;
        if (m >= M) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = row0 + wave * 16 + 4 * q + v;
            if (n < out) y[(size_t)m * ldy + col0 + n] = acc[t][v];
        }
    }
}

template <int BM, bool GENERAL>
static hipError_t run(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                      int32_t* dbg, hipStream_t s) {
    const QMatMeta& m = w->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    const int M = a->rows;
    const int nchunks = (m.groups + GC - 1) / GC;
    const size_t lds = gemm_lds_bytes<BM>(nchunks > 1 ? 2 : 1);
    dim3 grid((m.out_pad + GEMM_ROWS - 1) / GEMM_ROWS, (M + BM - 1) / BM), blockdim(256);
    const int blocked = M / 4 * 4;
    if (dbg)
        hipLaunchKernelGGL((k_gemm<BM, GENERAL, true>), grid, blockdim, lds, s, (const uint2*)w->d_codes, w->d_norms,
                           (const uint4*)a->d_xq, a->d_sx, block, blocked, y, ldy, col0, dbg, m.out, m.out_pad, M,
                           m.groups, m.cbs, lut);
    else
        hipLaunchKernelGGL((k_gemm<BM, GENERAL, false>), grid, blockdim, lds, s, (const uint2*)w->d_codes,
                           w->d_norms, (const uint4*)a->d_xq, a->d_sx, block, blocked, y, ldy, col0, dbg, m.out,
                           m.out_pad, M, m.groups, m.cbs, lut);
    return hipGetLastError();
}

template <int BM>
static void set_lds_limits() {
    hipFuncSetAttribute((const void*)k_gemm<BM, false, false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)gemm_lds_bytes<BM>(2));
    hipFuncSetAttribute((const void*)k_gemm<BM, true, false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)gemm_lds_bytes<BM>(2));
    hipFuncSetAttribute((const void*)k_gemm<BM, false, true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)gemm_lds_bytes<BM>(2));
    hipFuncSetAttribute((const void*)k_gemm<BM, true, true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)gemm_lds_bytes<BM>(2));
}

hipError_t launch_gemm(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                       int32_t* dbg, hipStream_t s) {
    static bool limits = false;
    if (!limits) {
        set_lds_limits<32>();
        set_lds_limits<64>();
        limits = true;
    }
    // Tokens past rows / 4 * 4 (or flagged) take the remainder combine.
    const bool general = block != nullptr || a->rows % 4 != 0;
    // Activation buffers hold whole multiples of 64 token rows, so both tile
    // heights read inside the allocation.
    if (a->rows <= 32)
        return general ? run<32, true>(w, a, block, y, ldy, col0, dbg, s) : run<32, false>(w, a, block, y, ldy, col0, dbg, s);
    return general ? run<64, true>(w, a, block, y, ldy, col0, dbg, s) : run<64, false>(w, a, block, y, ldy, col0, dbg, s);
}

}  // namespace nh
