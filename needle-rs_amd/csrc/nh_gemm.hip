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

__device__ __forceinline__ int swz(int tok, int b) { return b ^ (tok & 7); }

// LDS bytes of one chunk buffer: activations [tok][gi][blk] (128 B per
// token-group), scales [gi][tok] float2, norms [gi][row] float2.
template <int BM, int NW, int GC>
__host__ __device__ constexpr int gemm_buf_bytes() {
    return BM * GC * 128 + BM * GC * 8 + 16 * NW * GC * 8;
}

// NW wavefronts, each owning 16 weight rows (one MFMA row tile) against all
// BM tokens of the workgroup; K walked in chunks of GC groups.
template <int BM, int NW, int GC, bool GENERAL, bool DBG>
__global__ __launch_bounds__(64 * NW, 2) void k_gemm(
    const uint2* __restrict__ codes, const uint16_t* __restrict__ norms, const uint4* __restrict__ xq,
    const float* __restrict__ sx, const uint8_t* __restrict__ block, int blocked, float* __restrict__ y, int ldy,
    int col0, int32_t* __restrict__ dbg, int out, int out_pad, int M, int G, float cbs, Lut lut) {
    constexpr int T = 64 * NW;
    constexpr int ROWS = 16 * NW;
    constexpr int TT = BM / 16;  // token tiles per wavefront
    constexpr int XB = BM * GC * 128;
    constexpr int SB = BM * GC * 8;
    constexpr int BUF_BYTES = gemm_buf_bytes<BM, NW, GC>();
    constexpr int XINST = BM * GC * 8 / 64;  // 1 KiB global->LDS instructions per chunk
    static_assert(XINST % NW == 0, "activation staging splits evenly over wavefronts");
    static_assert((ROWS * GC) % T == 0 && (BM * GC) <= 2 * T, "table staging fits the thread count");
    extern __shared__ uint4 lds[];
    char* const lbase = reinterpret_cast<char*>(lds);
    const int nchunks = (G + GC - 1) / GC;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
    const int r = lane & 15, q = lane >> 4;
    const int row0 = blockIdx.x * ROWS;
    const int m0 = blockIdx.y * BM;
    const int tile = (row0 >> 4) + wave;  // this wavefront's 16-row code tile
    const bool tile_ok = tile * 16 < out_pad;
    const int ctile = tile_ok ? tile : 0;  // clamped: loads stay in bounds

    // Per-lane LDS byte offsets inside a chunk buffer; tile, group and row
    // terms are compile-time constants folded into the ds_read offsets.
    const uint32_t xo0 = (uint32_t)(r * GC * 128 + swz(r, q) * 16);
    const uint32_t xo1 = (uint32_t)(r * GC * 128 + swz(r, 4 + q) * 16);
    const uint32_t so = XB + r * 8;                         // + gi * BM * 8 + t * 128
    const uint32_t no = XB + SB + (wave * 16 + 4 * q) * 8;  // + gi * ROWS * 8 + v * 8

    // Codes: the two 8-byte pieces per group of this lane's A fragments
    // (chunks l = q/2 and 2 + q/2, dword pair q & 1).
    const uint2* cb0 = codes + (((size_t)ctile * G * 64 + r * 4 + (q >> 1)) * 2 + (q & 1));
    const uint2* cb1 = cb0 + 4;
    constexpr int SPT = (BM * GC + T - 1) / T;  // scale entries per thread
    constexpr int NPT = ROWS * GC / T;         // norm entries per thread
    float s_reg[SPT], n_reg[NPT];
    uint2 cwa[GC][2], cwb[GC][2];

    // Reads past the last group of a row land in the next row or in the
    // allocation's tail padding (8 groups' worth, see nh_internal.h); those
    // slots are staged but never used.
    const size_t xrow = (size_t)G * 8;  // uint4 per token row
    auto stage_load = [&](int c, int b, uint2 (&cdst)[GC][2]) __attribute__((always_inline)) {
        const int gb = c * GC;
        char* xdst = lbase + b * BUF_BYTES;
#pragma unroll
        for (int i = 0; i < XINST / NW; ++i) {
            const int k = i * NW + wave;  // this instruction's 1 KiB of the chunk buffer
            const int u = k * 64 + lane;  // uint4 slot
            const int tok = u / (GC * 8), rem = u % (GC * 8);
            const int gi = rem >> 3, blk = (rem & 7) ^ (tok & 7);
            const uint4* src = xq + (size_t)(m0 + tok) * xrow + (gb + gi) * 8 + blk;
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(xdst + k * 1024), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int L = i * T + tid;  // [gi][tok]
            const int Lc = L < BM * GC ? L : 0;
            s_reg[i] = sx[(size_t)(m0 + Lc % BM) * G + gb + Lc / BM];
        }
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
            const int L = i * T + tid;  // [gi][row]
            const int row = L % ROWS;
            const int nrow = row0 + row < out_pad ? row0 + row : 0;
            n_reg[i] = f16_bits_to_f32(norms[(size_t)nrow * G + gb + L / ROWS]);
        }
        const uint2* c0 = cb0 + (size_t)gb * 128;
        const uint2* c1 = cb1 + (size_t)gb * 128;
#pragma unroll
        for (int kk = 0; kk < GC; ++kk) {
            cdst[kk][0] = c0[kk * 128];
            cdst[kk][1] = c1[kk * 128];
        }
    };
    // After the staged loads landed: the register-staged tables.
    auto stage_store = [&](int b) __attribute__((always_inline)) {
        float2* sdst = reinterpret_cast<float2*>(lbase + b * BUF_BYTES + XB);
        float2* ndst = reinterpret_cast<float2*>(lbase + b * BUF_BYTES + XB + SB);
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int L = i * T + tid;
            if (L < BM * GC) sdst[L] = make_float2(s_reg[i], cbs * s_reg[i]);
        }
#pragma unroll
        for (int i = 0; i < NPT; ++i) ndst[i * T + tid] = make_float2(n_reg[i], n_reg[i] * cbs);
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
        for (int v = 0; v < 4; ++v) nr[v] = *reinterpret_cast<const float2*>(bb + no + gi * ROWS * 8 + v * 8);
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

template <int BM, int NW, int GC, bool GENERAL>
static hipError_t run(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                      int32_t* dbg, hipStream_t s) {
    const QMatMeta& m = w->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    const int M = a->rows;
    const int nchunks = (m.groups + GC - 1) / GC;
    const size_t lds = (size_t)(nchunks > 1 ? 2 : 1) * gemm_buf_bytes<BM, NW, GC>();
    dim3 grid((m.out_pad + 16 * NW - 1) / (16 * NW), (M + BM - 1) / BM), blockdim(64 * NW);
    const int blocked = M / 4 * 4;
    auto kern = dbg ? k_gemm<BM, NW, GC, GENERAL, true> : k_gemm<BM, NW, GC, GENERAL, false>;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemm<BM, NW, GC, GENERAL, true>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 2 * gemm_buf_bytes<BM, NW, GC>());
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)k_gemm<BM, NW, GC, GENERAL, false>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 2 * gemm_buf_bytes<BM, NW, GC>());
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL(kern, grid, blockdim, lds, s, (const uint2*)w->d_codes, w->d_norms, (const uint4*)a->d_xq,
                       a->d_sx, block, blocked, y, ldy, col0, dbg, m.out, m.out_pad, M, m.groups, m.cbs, lut);
    return hipGetLastError();
}

template <int BM, int NW, int GC>
static hipError_t pick(bool general, const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy,
                       int col0, int32_t* dbg, hipStream_t s) {
    return general ? run<BM, NW, GC, true>(w, a, block, y, ldy, col0, dbg, s)
                   : run<BM, NW, GC, false>(w, a, block, y, ldy, col0, dbg, s);
}

hipError_t launch_gemm(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                       int32_t* dbg, hipStream_t s) {
    // Tokens past rows / 4 * 4 (or flagged) take the remainder combine.
    const bool general = block != nullptr || a->rows % 4 != 0;
    // Four wavefronts (64 rows) per workgroup and 8-group chunks measured
    // fastest on the prefill shapes (eight wavefronts sharing one staging
    // were slower at M = 64 and no faster at M = 1024).  Activation buffers
    // hold whole multiples of 64 token rows, so both tile heights read
    // inside them.
    if (a->rows <= 32) return pick<32, 4, 8>(general, w, a, block, y, ldy, col0, dbg, s);
    return pick<64, 4, 8>(general, w, a, block, y, ldy, col0, dbg, s);
}

}  // namespace nh
