// Prefill / batched W4A8 product on int8 MFMA with the reference's prefill
// combine (crates/needle-engine/src/qlinear.rs:353-363): per token t and
// row n, S = the exact int32 group sum, sc = (norm * cbs) * sx for block
// tokens and norm * (cbs * sx) for the rest, acc = fma(S, sc, acc) over
// groups in order.  Block tokens are t < rows / 4 * 4 (qlinear.rs:397) or
// an explicit per-token flag.
//
// Weights: the GEMM reads the matrix's int8 copy (made once at upload by
// k_expand_w8 from the 4-bit codes), stored as the MFMA A fragments
// themselves: per 16-row tile and group, [half h][lane][16 bytes], 2 KiB.
// Keeping the int4 -> int8 expansion out of the product removes half of
// its vector-ALU work; the copy costs in_dim bytes per row of HBM.
//
// Work item: a panel of ROWS = 16 * NW weight rows x BM tokens; wavefront
// w owns the 16-row MFMA tile w of the panel against all BM tokens.  The
// grid is persistent: each workgroup walks its items (blockIdx.x,
// + gridDim.x, ...) and every item's K dimension in chunks of GC groups (GC
// divides G), as one flat sequence of steps.  A step's activations (int8),
// scales and norms are staged in LDS by the whole workgroup, double
// buffered; each wavefront's A fragments go straight to registers.  The
// next step's global loads (possibly the next item's first chunk) are in
// flight while this step computes; the activations are then written to the
// other LDS buffer.  Per group: two v_mfma_i32_16x16x64_i8 per token tile
// into a fresh int32 accumulator, then the float epilogue.
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

// The per-product operands of one launch; blockIdx.y picks the product
// (the products of a launch share shape, code tables and token rows).
constexpr int GEMM_BATCH_MAX = 8;
struct GemmSrcs {
    const uint4* w8[GEMM_BATCH_MAX];
    const uint2* codes[GEMM_BATCH_MAX];
    const uint16_t* norms[GEMM_BATCH_MAX];
    const uint4* xq[GEMM_BATCH_MAX];
    const float* sx[GEMM_BATCH_MAX];
    float* y[GEMM_BATCH_MAX];
};

// The int8 A-fragment copy of a tiled code matrix: one wavefront per
// (16-row tile, group).  Lane L = 16 q + r holds row r's k-block q of each
// 64-wide half: the 8-byte code pieces of chunks l = q / 2 (half 0) and
// 2 + q / 2 (half 1), dword pair q & 1, expanded to int8.
//
// 2-bit: the B operand's k-block q of half h is activation bytes
// h * 64 + q * 16 .. + 16, i.e. decode lane l = 2 h + q / 2's chunk, dword
// d' = q % 2 of it (packed dword 4 d' + l), fields k = 0..3 as 4-byte
// blocks; the A fragment expands the same packed dword field by field.
template <int BITS>
__global__ __launch_bounds__(64) void k_expand_w8(const void* __restrict__ codes, uint4* __restrict__ w8, Lut lut) {
    const int tg = blockIdx.x;  // tile * G + g
    const int lane = threadIdx.x;
    const int r = lane & 15, q = lane >> 4;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t e0, e1, e2, e3;
        if constexpr (BITS == 4) {
            const uint2 cw = reinterpret_cast<const uint2*>(codes)[((size_t)tg * 64 + r * 4 + (q >> 1)) * 2 + (q & 1) + h * 4];
            expand8(cw.x, lut, e0, e1);
            expand8(cw.y, lut, e2, e3);
        } else {
            const uint2 cw = reinterpret_cast<const uint2*>(codes)[(size_t)tg * 64 + r * 4 + 2 * h + (q >> 1)];
            const uint32_t w = (q & 1) ? cw.y : cw.x;
            e0 = expand2(w, 0, lut.a_lo);
            e1 = expand2(w, 1, lut.a_lo);
            e2 = expand2(w, 2, lut.a_lo);
            e3 = expand2(w, 3, lut.a_lo);
        }
        w8[((size_t)tg * 2 + h) * 64 + lane] = make_uint4(e0, e1, e2, e3);
    }
}

hipError_t launch_expand_w8(const nh_qmat* w, hipStream_t s) {
    const QMatMeta& m = w->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    const int blocks = (m.out + PANEL_ROWS - 1) / PANEL_ROWS * (PANEL_ROWS / 16) * m.groups;
    auto kern = m.bits == 2 ? k_expand_w8<2> : k_expand_w8<4>;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64), 0, s, (const void*)w->d_codes, w->d_w8, lut);
    return hipGetLastError();
}

// Dynamic LDS bytes of one step buffer: activations [tok][gi][blk] (128 B
// per token-group, 16-byte blocks swizzled by token).  The scale
// ([gi][tok]) and norm ([gi][row]) float2 tables are a static LDS array.
template <int BM, int GC>
__host__ __device__ constexpr int gemm_act_bytes() {
    return BM * GC * 128;
}

// One group's A fragments as held in registers: the int8 fragments
// themselves (halves 0 and 1), or (W4) the 4-bit code pieces they expand
// from, expanded right before use.
template <bool W4>
struct AFrag {
    v4i h[2];
};
template <>
struct AFrag<true> {
    uint32_t c[4];
};

template <int BM, int NW, int GC, bool GENERAL, bool DBG, bool W4>
__global__ __launch_bounds__(64 * NW, DBG ? 1 : 2) void k_gemm(
    GemmSrcs src, Lut lut, const uint8_t* __restrict__ block, int blocked, int ldy, int col0, int vec_store,
    int32_t* __restrict__ dbg, int out, int out_alloc, int cap_rows, int M, int G, float cbs, int panels, int items) {
    const int mb = blockIdx.y;
    const uint4* __restrict__ w8 = src.w8[mb];
    const uint2* __restrict__ codes = src.codes[mb];
    const uint16_t* __restrict__ norms = src.norms[mb];
    const uint4* __restrict__ xq = src.xq[mb];
    const float* __restrict__ sx = src.sx[mb];
    float* __restrict__ y = src.y[mb];
    constexpr int T = 64 * NW;
    constexpr int ROWS = 16 * NW;
    constexpr int TT = BM / 16;  // token tiles per wavefront
    constexpr int XB = BM * GC * 128;
    constexpr int SB = BM * GC * 8;
    constexpr int TAB = BM * GC + ROWS * GC;  // float2 entries per table buffer
    static_assert(XB % (1024 * NW) == 0, "activation staging splits evenly over wavefronts");
    constexpr int XPT = XB / 1024 / NW;           // 16-byte activation loads per thread per step
    constexpr int SPT = (BM * GC + T - 1) / T;    // scale entries per thread
    constexpr int NPT = (ROWS * GC + T - 1) / T;  // norm entries per thread
    extern __shared__ uint4 lds[];
    __shared__ float2 tabs[2][TAB];
    char* const lbase = reinterpret_cast<char*>(lds);
    const int nchunks = G / GC;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
    const int r = lane & 15, q = lane >> 4;
    const int my_items = (items - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int nsteps = my_items * nchunks;
    if (nsteps <= 0) return;

    // Per-lane constants.  Activation slot u = (i * NW + wave) * 64 + lane
    // of a step buffer holds token u / (8 GC), group (u / 8) % GC and
    // 16-byte block (u % 8) ^ (token & 7) of that token's group.
    uint32_t xoff[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        const int u = (i * NW + wave) * 64 + lane;
        const int tok = u / (GC * 8), rem = u % (GC * 8);
        xoff[i] = (uint32_t)(tok * G * 128 + (rem >> 3) * 128 + ((rem & 7) ^ (tok & 7)) * 16);
    }
    const uint32_t xo0 = (uint32_t)(r * GC * 128 + swz(r, q) * 16);
    const uint32_t xo1 = (uint32_t)(r * GC * 128 + swz(r, 4 + q) * 16);
    const uint32_t so = r * 8;                          // + gi * BM * 8 + t * 128
    const uint32_t no = SB + (wave * 16 + 4 * q) * 8;  // + gi * ROWS * 8 + v * 8

    // Table entries this thread stages: scales [gi][tok], norms [gi][row]
    // (threads past a table's end reload entry 0, never stored).
    uint32_t soff[SPT], noff[NPT];
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
        const int L = i * T + tid < BM * GC ? i * T + tid : 0;
        soff[i] = (uint32_t)((L % BM) * G + L / BM);
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int L = i * T + tid < ROWS * GC ? i * T + tid : 0;
        noff[i] = (uint32_t)((L % ROWS) * G + L / ROWS);
    }
    // 4-bit A pieces: chunks l = q / 2 and 2 + q / 2 of row r, dword pair
    // q & 1 (uint2 units within a tile-group block).
    const uint32_t coff = (uint32_t)((r * 4 + (q >> 1)) * 2 + (q & 1));

    // Step bookkeeping: item k of this workgroup, chunk c.  The division
    // runs once per item.
    struct Pos {
        int k, c, row0, m0;
    };
    auto set_item = [&](Pos& p) __attribute__((always_inline)) {
        const int item = (int)blockIdx.x + p.k * (int)gridDim.x;
        const int tt = item / panels;
        p.row0 = (item - tt * panels) * ROWS;
        p.m0 = tt * BM;
    };
    auto advance = [&](Pos& p) __attribute__((always_inline)) {
        if (++p.c == nchunks) {
            p.c = 0;
            if (p.k + 1 < my_items) {
                ++p.k;
                set_item(p);
            } else {
                p.c = nchunks - 1;  // past the last step: reload the last step
            }
        }
    };

    u32x4 xr[XPT];
    float s_reg[SPT];
    uint16_t n_reg[NPT];
    AFrag<W4> aa[GC], ab[GC];

    // The global loads of step p: activations, tables and this wavefront's
    // A fragments into registers.  Tables stay raw until stage_store (a
    // conversion here would wait on every load in flight).
    // Buffer resources over the inputs: every staging load is a buffer load
    // with a loop-invariant per-lane offset and the step's uniform offset in
    // a scalar register, so a step computes no vector addresses (and no
    // address temporary reuses a register a load is still filling).  Device
    // matrix copies hold whole 64-row panels: no row clamps.
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xq, (size_t)cap_rows * G * 128);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(sx, (size_t)cap_rows * G * 4);
    const __amdgpu_buffer_rsrc_t rn = make_rsrc(norms, (size_t)out_alloc * G * 2);
    const __amdgpu_buffer_rsrc_t ra =
        W4 ? make_rsrc(codes, (size_t)out_alloc * G * 64) : make_rsrc(w8, (size_t)out_alloc * G * 128);
    auto stage_load = [&](const Pos& p, AFrag<W4> (&adst)[GC]) __attribute__((always_inline)) {
        const int gb = p.c * GC;
        const int xs = (p.m0 * G + gb) * 128;
#pragma unroll
        for (int i = 0; i < XPT; ++i)
            xr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)xoff[i], xs, 0));
#pragma unroll
        for (int i = 0; i < SPT; ++i)
            s_reg[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)soff[i] * 4,
                                                                                     (p.m0 * G + gb) * 4, 0));
#pragma unroll
        for (int i = 0; i < NPT; ++i)
            n_reg[i] = __builtin_amdgcn_raw_buffer_load_b16(rn, (int)noff[i] * 2, (p.row0 * G + gb) * 2, 0);
        const int tg = ((p.row0 >> 4) + wave) * G + gb;  // this wavefront's tile, first group
        if constexpr (W4) {
#pragma unroll
            for (int gi = 0; gi < GC; ++gi) {
                const auto c0 = __builtin_amdgcn_raw_buffer_load_b64(ra, (int)coff * 8 + gi * 1024, tg * 1024, 0);
                const auto c1 = __builtin_amdgcn_raw_buffer_load_b64(ra, (int)coff * 8 + gi * 1024 + 32, tg * 1024, 0);
                adst[gi].c[0] = (uint32_t)c0[0];
                adst[gi].c[1] = (uint32_t)c0[1];
                adst[gi].c[2] = (uint32_t)c1[0];
                adst[gi].c[3] = (uint32_t)c1[1];
            }
        } else {
#pragma unroll
            for (int gi = 0; gi < GC; ++gi) {
                adst[gi].h[0] = __builtin_amdgcn_raw_buffer_load_b128(ra, lane * 16 + gi * 2048, tg * 2048, 0);
                adst[gi].h[1] = __builtin_amdgcn_raw_buffer_load_b128(ra, lane * 16 + gi * 2048 + 1024, tg * 2048, 0);
            }
        }
    };
    // After the loads landed: activations and tables into LDS buffer b.
    auto stage_store = [&](int b) __attribute__((always_inline)) {
        char* xdst = lbase + b * XB;
#pragma unroll
        for (int i = 0; i < XPT; ++i) *reinterpret_cast<u32x4*>(xdst + (i * NW + wave) * 1024 + lane * 16) = xr[i];
#pragma unroll
        for (int i = 0; i < SPT; ++i) {
            const int L = i * T + tid;
            if ((BM * GC) % T == 0 || L < BM * GC) tabs[b][L] = make_float2(s_reg[i], cbs * s_reg[i]);
        }
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
            const int L = i * T + tid;
            const float nv = f16_bits_to_f32(n_reg[i]);
            if ((ROWS * GC) % T == 0 || L < ROWS * GC) tabs[b][BM * GC + L] = make_float2(nv, nv * cbs);
        }
    };

    float acc[TT][4];
    bool blk[TT];
    Pos cur{0, 0, 0, 0}, nxt, done{0, 0, 0, 0};
    set_item(cur);
    auto begin_item = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const int m = cur.m0 + t * 16 + r;
            blk[t] = !GENERAL || (m < M ? (block ? block[m] != 0 : m < blocked) : true);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[t][v] = 0.0f;
        }
    };
    auto end_item = [&](const Pos& p) __attribute__((always_inline)) {
        if (!y) return;
        const int n0 = p.row0 + wave * 16 + 4 * q;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const int m = p.m0 + t * 16 + r;
            if (m >= M) continue;
            float* dst = y + (size_t)m * ldy + col0 + n0;
            if (vec_store && n0 + 3 < out) {
                *reinterpret_cast<float4*>(dst) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (n0 + v < out) dst[v] = acc[t][v];
            }
        }
    };

    // One group: B fragments from LDS, every token tile's two MFMAs into its
    // own accumulator (independent, so they pipeline), then the epilogues.
    auto do_group = [&](const AFrag<W4> (&ag)[GC], const char* bb, const char* tb, int gi) __attribute__((always_inline)) {
        v4i a0, a1;
        if constexpr (W4) {
            uint32_t e0, e1, e2, e3, f0, f1, f2, f3;
            expand8(ag[gi].c[0], lut, e0, e1);
            expand8(ag[gi].c[1], lut, e2, e3);
            expand8(ag[gi].c[2], lut, f0, f1);
            expand8(ag[gi].c[3], lut, f2, f3);
            a0 = v4i{(int)e0, (int)e1, (int)e2, (int)e3};
            a1 = v4i{(int)f0, (int)f1, (int)f2, (int)f3};
        } else {
            a0 = ag[gi].h[0];
            a1 = ag[gi].h[1];
        }
        v4i b0[TT], b1[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            b0[t] = *reinterpret_cast<const v4i*>(bb + xo0 + t * 16 * GC * 128 + gi * 128);
            b1[t] = *reinterpret_cast<const v4i*>(bb + xo1 + t * 16 * GC * 128 + gi * 128);
        }
        float2 nr[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) nr[v] = *reinterpret_cast<const float2*>(tb + no + gi * ROWS * 8 + v * 8);
        float2 sc[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) sc[t] = *reinterpret_cast<const float2*>(tb + so + gi * BM * 8 + t * 128);
        v4i d[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) d[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0[t], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < TT; ++t) d[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1[t], d[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            if (DBG) {
                const int m = cur.m0 + t * 16 + r;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int n = cur.row0 + wave * 16 + 4 * q + v;
                    if (m < M && n < out) dbg[((size_t)m * out + n) * G + cur.c * GC + gi] = d[t][v];
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
    // Step `cur` from LDS buffer B with A fragments ag, prefetching step
    // `nxt` (into the other buffer and fragment registers an) first.
    //
    // The prefetch, its LDS stores and the barrier run on every step (the
    // last step reloads its own, cached, data): with no path that skips
    // them, the compiler's wait before this step's first use of its A
    // registers counts the prefetch loads as issued after them and does not
    // wait for the prefetch.
    auto do_step = [&](auto Bc, const AFrag<W4> (&ag)[GC], AFrag<W4> (&an)[GC]) __attribute__((always_inline)) {
        constexpr int B = decltype(Bc)::value;
        nxt = cur;
        advance(nxt);
        stage_load(nxt, an);
        if (cur.c == 0) {
            // The previous item's outputs are stored here, behind this
            // step's prefetch: the wait at the start of the next step's
            // prefetch (for registers it reuses) then finds them long done.
            if (cur.k > 0) end_item(done);
            begin_item();
        }
        const char* bb = lbase + B * XB;
        const char* tb = reinterpret_cast<const char*>(&tabs[B][0]);
        // Scheduling fences keep the prefetch loads ahead of the compute and
        // its LDS stores behind it (hoisted stores would wait for the
        // prefetch in the middle of the compute).
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int gi = 0; gi < GC; ++gi) do_group(ag, bb, tb, gi);
        __builtin_amdgcn_sched_barrier(0);
        // Buffer B ^ 1 was last read in the previous step, which every
        // wavefront left through the barrier below.
        stage_store(B ^ 1);
        __syncthreads();
        if (cur.c == nchunks - 1) done = cur;
        cur = nxt;
    };

    stage_load(cur, aa);
    stage_store(0);
    __syncthreads();
    // Steps in pairs so buffers and fragment registers alternate statically.
    for (int s = 0; s < nsteps; s += 2) {
        do_step(std::integral_constant<int, 0>{}, aa, ab);
        if (s + 1 < nsteps) do_step(std::integral_constant<int, 1>{}, ab, aa);
    }
    end_item(done);
}

// Workgroups of one kernel that fit on a CU at once.
template <typename K>
static int occupancy(K kern, int threads, size_t lds) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds) != hipSuccess || n < 1) n = 1;
    return n;
}

// n same-shaped products (w[i] x a[i] into y[i]) in one launch.
struct GemmSet {
    const nh_qmat* const* w;
    const nh_qact* const* a;
    float* const* y;
    int n;
};

template <int BM, int NW, int GC, bool GENERAL, bool W4>
static hipError_t run(const GemmSet& g, const uint8_t* block, int ldy, int col0, int32_t* dbg, hipStream_t s) {
    constexpr int ROWS = 16 * NW;
    const QMatMeta& m = g.w[0]->m;
    const Lut lut{m.lut.a_hi, m.lut.a_lo, m.lut.b_hi, m.lut.b_lo};
    const int M = g.a[0]->rows;
    const int panels = (m.out_pad + ROWS - 1) / ROWS;
    const int ttiles = (M + BM - 1) / BM;
    const int items = panels * ttiles;
    const size_t lds = 2 * (size_t)gemm_act_bytes<BM, GC>();
    auto kern = dbg ? k_gemm<BM, NW, GC, GENERAL, true, W4> : k_gemm<BM, NW, GC, GENERAL, false, W4>;
    static int per_cu = 0;
    if (!per_cu) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemm<BM, NW, GC, GENERAL, true, W4>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)k_gemm<BM, NW, GC, GENERAL, false, W4>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        per_cu = occupancy(k_gemm<BM, NW, GC, GENERAL, false, W4>, 64 * NW, lds);
    }
    // Persistent grid: at most one resident wave of workgroups over all the
    // launch's products, each taking the same number of items.
    const int slots = device_cus() * per_cu;
    const int rounds = (g.n * items + slots - 1) / slots;
    const int grid = (items + rounds - 1) / rounds;
    GemmSrcs src{};
    int vec = ldy % 4 == 0 && col0 % 4 == 0;
    for (int i = 0; i < g.n; ++i) {
        src.w8[i] = (const uint4*)g.w[i]->d_w8;
        src.codes[i] = (const uint2*)g.w[i]->d_codes;
        src.norms[i] = g.w[i]->d_norms;
        src.xq[i] = (const uint4*)g.a[i]->d_xq;
        src.sx[i] = g.a[i]->d_sx;
        src.y[i] = g.y[i];
        vec &= (uintptr_t)g.y[i] % 16 == 0;
    }
    hipLaunchKernelGGL(kern, dim3(grid, g.n), dim3(64 * NW), lds, s, src, lut, block, M / 4 * 4, ldy, col0, vec, dbg,
                       m.out, (m.out + PANEL_ROWS - 1) / PANEL_ROWS * PANEL_ROWS, g.a[0]->cap_rows, M, m.groups,
                       m.cbs, panels, items);
    return hipGetLastError();
}

// BM-token tiles on NW wavefronts with the largest chunk (3, 4, 2 or 1
// groups) that divides G.
template <int BM, int NW, bool W4>
static hipError_t run_gc(bool general, const GemmSet& g, const uint8_t* block, int ldy, int col0, int32_t* dbg,
                         hipStream_t s) {
    const int G = g.w[0]->m.groups;
#define NH_GEMM_GC(GCV)                                                               \
    if (G % GCV == 0)                                                                 \
        return general ? run<BM, NW, GCV, true, W4>(g, block, ldy, col0, dbg, s) \
                       : run<BM, NW, GCV, false, W4>(g, block, ldy, col0, dbg, s);
    NH_GEMM_GC(3)
    NH_GEMM_GC(4)
    NH_GEMM_GC(2)
#undef NH_GEMM_GC
    return general ? run<BM, NW, 1, true, W4>(g, block, ldy, col0, dbg, s)
                   : run<BM, NW, 1, false, W4>(g, block, ldy, col0, dbg, s);
}

static hipError_t gemm_dispatch(const GemmSet& g, const uint8_t* block, int ldy, int col0, int32_t* dbg,
                                hipStream_t s) {
    const nh_qmat* w = g.w[0];
    const nh_qact* a = g.a[0];
    // Tokens past rows / 4 * 4 (or flagged) take the remainder combine.
    const bool general = block != nullptr || a->rows % 4 != 0;
    // Activation buffers hold whole multiples of ACT_PAD token rows, so
    // every token tile reads inside them.
    static_assert(ACT_PAD % 64 == 0, "token tiles stay inside the activation buffer");
    // The steps wait on load latency more than on arithmetic, so what pays
    // is parallel work: take the largest tile that still gives every CU an
    // item (and is no taller than the tokens), else the smallest.  Measured
    // on the prefill and LM-head shapes: 64 x 64 tiles with one-group steps
    // (four workgroups per CU) for the largest products, 64-row x 32-token
    // tiles with 3-group steps in the middle, 32-row x 16-token tiles for
    // prompt chunks and small batches.  Up to 16 tokens the product is
    // bound by the weight stream, so it reads the 4-bit codes (half the
    // bytes of the int8 copy) and expands them in the kernel.
    const int M = a->rows, cus = device_cus(), out_pad = w->m.out_pad;
    // (items over all the launch's products)
    auto items = [&](int rows, int bm) { return (long)g.n * ((out_pad + rows - 1) / rows) * ((M + bm - 1) / bm); };
    if (M > 48 && items(64, 64) >= cus)
        return general ? run<64, 4, 1, true, false>(g, block, ldy, col0, dbg, s)
                       : run<64, 4, 1, false, false>(g, block, ldy, col0, dbg, s);
    if (M > 16 && items(64, 32) >= cus) return run_gc<32, 4, false>(general, g, block, ldy, col0, dbg, s);
    if (M <= 16 && w->m.bits == 4) return run_gc<16, 2, true>(general, g, block, ldy, col0, dbg, s);
    return run_gc<16, 2, false>(general, g, block, ldy, col0, dbg, s);
}

hipError_t launch_gemm(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                       int32_t* dbg, hipStream_t s) {
    const GemmSet g{&w, &a, &y, 1};
    return gemm_dispatch(g, block, ldy, col0, dbg, s);
}

bool gemm_batchable(const nh_qmat* const* w, const nh_qact* const* a, int n) {
    if (n < 1 || n > GEMM_BATCH_MAX || !gemv_batchable(w, n)) return false;
    for (int i = 1; i < n; ++i)
        if (w[i]->m.in_dim != w[0]->m.in_dim || a[i]->rows != a[0]->rows || a[i]->cap_rows != a[0]->cap_rows ||
            a[i]->bits != a[0]->bits)
            return false;
    return true;
}

hipError_t launch_gemm_batch(const nh_qmat* const* w, const nh_qact* const* a, float* const* y, int n,
                             const uint8_t* block, int ldy, hipStream_t s) {
    const GemmSet g{w, a, y, n};
    return gemm_dispatch(g, block, ldy, 0, nullptr, s);
}

}  // namespace nh
