// Device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nh_internal.h"


namespace nh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// The value of lane (lane ^ 1) / (lane ^ 2) within each group of four
// lanes, by DPP quad permutes (no LDS round trip, unlike a shuffle).
__device__ __forceinline__ float quad_xor1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_xor2(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}

// The value of lane (lane ^ H), H = 4 or 8, within each row of 16 lanes:
// two DPP row shifts (lane i reads i + H, resp. i - H) and a select.
template <int H>
__device__ __forceinline__ float row_xor(float v, int lane) {
    const int up = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + H, 0xF, 0xF, false);
    const int dn = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x110 + H, 0xF, 0xF, false);
    return __builtin_bit_cast(float, (lane & H) ? dn : up);
}

// The value of lane (lane ^ 16), by a swizzle in xor mode (no address
// computation, unlike a shuffle).
__device__ __forceinline__ float lane_xor16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1F | (16 << 10)));
}

// The value of lane (lane ^ h) for h = 1, 2, 4, 8, 16, 32.
__device__ __forceinline__ float lane_xor(float v, int h, int lane) {
    switch (h) {
        case 1: return quad_xor1(v);
        case 2: return quad_xor2(v);
        case 4: return row_xor<4>(v, lane);
        case 8: return row_xor<8>(v, lane);
        case 16: return lane_xor16(v);
        default: return __shfl_xor(v, h, 64);
    }
}

// A raw buffer resource over `bytes` bytes at p (gfx9 descriptor word 3):
// loads through it take a scalar base and 32-bit lane offsets (no 64-bit
// address arithmetic per lane), and read zero past the range.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)(bytes < 0xffffffffu ? bytes : 0xffffffffu),
                                             0x00020000);
}

// A streamed 16-byte load (read once, non-temporal hint).
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// The v_perm code tables, passed by value (scalar registers).
struct Lut {
    uint32_t a_hi, a_lo, b_hi, b_lo;
};

// Four selector bytes (each 0..15) -> four int8 codebook values:
// perm(A, s) ^ perm(B, s ^ 8).  v_perm_b32 returns table bytes for
// selector values 0..7 and 0x00 / 0xFF constants for 8..15; the tables are
// solved on the host so the XOR of the two lookups is the codebook byte.
__device__ __forceinline__ uint32_t expand4(uint32_t s, const Lut& t) {
    return __builtin_amdgcn_perm(t.a_hi, t.a_lo, s) ^ __builtin_amdgcn_perm(t.b_hi, t.b_lo, s ^ 0x08080808u);
}

// One packed code dword (8 codes, LSB-first nibbles) -> int8 weights of its
// even positions (lo) and odd positions (hi).
__device__ __forceinline__ void expand8(uint32_t w, const Lut& t, uint32_t& lo, uint32_t& hi) {
    lo = expand4(w & 0x0F0F0F0Fu, t);
    hi = expand4((w >> 4) & 0x0F0F0F0Fu, t);
}

// Exact integer sum of one 16-byte code chunk (32 weights: dwords k = 0..3
// of one decode lane) against its 32 activation bytes (x0 = k 0,1; x1 = k
// 2,3, each dword pair [even positions, odd positions]).
__device__ __forceinline__ int dot_chunk(uint4 c, uint4 x0, uint4 x1, const Lut& t) {
    uint32_t lo, hi;
    int acc = 0;
    expand8(c.x, t, lo, hi);
    acc = __builtin_amdgcn_sdot4((int)lo, (int)x0.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)hi, (int)x0.y, acc, false);
    expand8(c.y, t, lo, hi);
    acc = __builtin_amdgcn_sdot4((int)lo, (int)x0.z, acc, false);
    acc = __builtin_amdgcn_sdot4((int)hi, (int)x0.w, acc, false);
    expand8(c.z, t, lo, hi);
    acc = __builtin_amdgcn_sdot4((int)lo, (int)x1.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)hi, (int)x1.y, acc, false);
    expand8(c.w, t, lo, hi);
    acc = __builtin_amdgcn_sdot4((int)lo, (int)x1.z, acc, false);
    acc = __builtin_amdgcn_sdot4((int)hi, (int)x1.w, acc, false);
    return acc;
}

// Four 2-bit code fields k of a packed dword (one per byte) -> four int8
// codebook values: one v_perm lookup in the 4-byte table t (byte c = value
// of code c; selector bytes 0..3 pick bytes of the second operand).
__device__ __forceinline__ uint32_t expand2(uint32_t w, int k, uint32_t t) {
    return __builtin_amdgcn_perm(0u, t, (w >> (2 * k)) & 0x03030303u);
}

// Exact integer sum of one 2-bit chunk (packed dwords l and 4 + l of a
// group: 32 codes of decode lane l) against its 32 activation bytes: x0
// holds dword l's fields k = 0..3 as four 4-byte blocks, x1 dword 4 + l's.
__device__ __forceinline__ int dot_chunk2(uint2 c, uint4 x0, uint4 x1, uint32_t t) {
    int acc = 0;
    acc = __builtin_amdgcn_sdot4((int)expand2(c.x, 0, t), (int)x0.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)expand2(c.x, 1, t), (int)x0.y, acc, false);
    acc = __builtin_amdgcn_sdot4((int)expand2(c.x, 2, t), (int)x0.z, acc, false);
    acc = __builtin_amdgcn_sdot4((int)expand2(c.x, 3, t), (int)x0.w, acc, false);
    acc = __builtin_amdgcn_sdot4((int)expand2(c.y, 0, t), (int)x1.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)expand2(c.y, 1, t), (int)x1.y, acc, false);
    acc = __builtin_amdgcn_sdot4((int)expand2(c.y, 2, t), (int)x1.z, acc, false);
    acc = __builtin_amdgcn_sdot4((int)expand2(c.y, 3, t), (int)x1.w, acc, false);
    return acc;
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// The 128-point unnormalised Sylvester FWHT of a group held two elements
// per lane (position p = lane in v0, p = lane + 64 in v1), stages
// h = 1, 2, ..., 64 as crates/needle-core/src/quant.rs:91-105 orders them:
// x[j] = a + b, x[j + h] = a - b.  Each output is one add of the same two
// operands as on the CPU, so the result is bit-identical.
__device__ __forceinline__ void fwht128(float& v0, float& v1, int lane) {
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
        float p0 = lane_xor(v0, h, lane);
        float p1 = lane_xor(v1, h, lane);
        bool upper = (lane & h) != 0;
        v0 = upper ? (p0 - v0) : (v0 + p0);
        v1 = upper ? (p1 - v1) : (v1 + p1);
    }
    float a = v0, b = v1;
    v0 = a + b;
    v1 = a - b;
}

// Wavefront reductions.  The maximum over the 64 lanes of values >= +0
// (absolute values, exps and their weights): their bit patterns order as
// unsigned integers as the values do, so four DPP integer max steps
// (within quads, then rows of 16 by rotations of 4 and 8) and the four
// rows' maxima read into scalar registers give the exact maximum, in ~a
// third of the instructions of a float reduction (which also quiets each
// operand).  All 64 lanes must be active.
__device__ __forceinline__ unsigned umax_dpp_step(unsigned x, unsigned y) { return x > y ? x : y; }
__device__ __forceinline__ float wave_max_nonneg(float v) {
    unsigned x = __builtin_bit_cast(unsigned, v);
    x = umax_dpp_step(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false));
    x = umax_dpp_step(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false));
    x = umax_dpp_step(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x124, 0xF, 0xF, false));
    x = umax_dpp_step(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false));
    const unsigned r0 = (unsigned)__builtin_amdgcn_readlane((int)x, 0), r1 = (unsigned)__builtin_amdgcn_readlane((int)x, 16),
                   r2 = (unsigned)__builtin_amdgcn_readlane((int)x, 32), r3 = (unsigned)__builtin_amdgcn_readlane((int)x, 48);
    return __builtin_bit_cast(float, umax_dpp_step(umax_dpp_step(r0, r1), umax_dpp_step(r2, r3)));
}

// The same for any non-NaN values (scores): the key b ^ ((b >> 31) &
// 0x7fffffff) of bit pattern b orders as a signed integer as the values do
// (negative values get their magnitude bits flipped) and is its own
// inverse.  (-0 keys below +0: no score here is -0.)  All 64 lanes must be
// active.
__device__ __forceinline__ int imax_dpp_step(int x, int y) { return x > y ? x : y; }
__device__ __forceinline__ float wave_max_ordered(float v) {
    const int b = __builtin_bit_cast(int, v);
    int x = b ^ ((b >> 31) & 0x7fffffff);
    x = imax_dpp_step(x, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
    x = imax_dpp_step(x, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
    x = imax_dpp_step(x, __builtin_amdgcn_update_dpp(0, x, 0x124, 0xF, 0xF, false));
    x = imax_dpp_step(x, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
    const int r0 = __builtin_amdgcn_readlane(x, 0), r1 = __builtin_amdgcn_readlane(x, 16),
              r2 = __builtin_amdgcn_readlane(x, 32), r3 = __builtin_amdgcn_readlane(x, 48);
    const int k = imax_dpp_step(imax_dpp_step(r0, r1), imax_dpp_step(r2, r3));
    return __builtin_bit_cast(float, k ^ ((k >> 31) & 0x7fffffff));
}

// The minimum of an integer over the 64 lanes by the same four DPP steps
// and four lane reads.  All 64 lanes must be active.
__device__ __forceinline__ int imin_dpp_step(int x, int y) { return x < y ? x : y; }
__device__ __forceinline__ int wave_min_i32(int x) {
    x = imin_dpp_step(x, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
    x = imin_dpp_step(x, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
    x = imin_dpp_step(x, __builtin_amdgcn_update_dpp(0, x, 0x124, 0xF, 0xF, false));
    x = imin_dpp_step(x, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
    return imin_dpp_step(imin_dpp_step(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
                         imin_dpp_step(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// `(v * inv).round().clamp(-128, 127) as i8` (crates/needle-engine/src/qlinear.rs:137-139).
__device__ __forceinline__ int8_t quant_one(float v, float inv) {
    float r = roundf(v * inv);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    return (int8_t)(int)r;
}

__device__ __forceinline__ float bits_f32(uint32_t b) { return __builtin_bit_cast(float, b); }

// The stored selector of natural position p: 4-bit dword d = p / 8 is
// dword d / 4 of lane d % 4's 16-byte chunk; 2-bit dword d = p / 16 is
// dword d / 4 of lane d % 4's 8-byte chunk, field p % 4 of byte (p / 4) % 4.
template <int BITS>
__device__ __forceinline__ uint32_t code_sel_at(const void* codes, int tile, int G, int g, int rt, int p) {
    const size_t ci = ((size_t)tile * G + g) * 64 + rt * 4;
    if constexpr (BITS == 4) {
        const int d = p >> 3;
        const uint32_t* chunk = (const uint32_t*)(reinterpret_cast<const uint4*>(codes) + ci + (d & 3));
        return (chunk[d >> 2] >> (4 * (p & 7))) & 15u;
    } else {
        const int d = p >> 4;
        const uint32_t* chunk = (const uint32_t*)(reinterpret_cast<const uint2*>(codes) + ci + (d & 3));
        return (chunk[d >> 2] >> (8 * ((p >> 2) & 3) + 2 * (p & 3))) & 3u;
    }
}

// The dequantized values of positions lane and lane + 64 of (row, group g)
// of a tiled matrix: QMat::row (crates/needle-engine/src/qlinear.rs:309-323),
// cb[code] * norm, then the normalised rotation (quant.rs:109-115).
template <int BITS>
__device__ __forceinline__ void row_group(const void* codes, const uint16_t* norms, const float* fsel, int G,
                                          uint32_t row, int g, int lane, float& v0, float& v1) {
    const int tile = row / TILE_ROWS, rt = row % TILE_ROWS;
    const float norm = f16_bits_to_f32(norms[(size_t)row * G + g]);
    v0 = fsel[code_sel_at<BITS>(codes, tile, G, g, rt, lane)] * norm;
    v1 = fsel[code_sel_at<BITS>(codes, tile, G, g, rt, lane + 64)] * norm;
    fwht128(v0, v1, lane);
    const float hs = bits_f32(0x3db504f3u);
    v0 *= hs;
    v1 *= hs;
}

// prep_group (crates/needle-engine/src/qlinear.rs:149-164) for one group
// held by one wavefront (positions lane, lane + 64): rotate, scale
// (quant.rs:109-115), quantize with the group's amax scale (qlinear.rs:77-88)
// and store the int8 codes at act_offset(p, bits) of the group's 128-byte
// block `q`, the scale at `s_out`.
__device__ __forceinline__ void a8_group(float v0, float v1, int lane, int bits, int8_t* q, float* s_out) {
    fwht128(v0, v1, lane);
    const float hs = bits_f32(0x3db504f3u);
    v0 *= hs;
    v1 *= hs;
    const float m = wave_max_nonneg(fmaxf(fabsf(v0), fabsf(v1)));
    const float s = m > 0.0f ? m * bits_f32(0x3c010204u) : 1.0f;
    const float inv = 1.0f / s;
    q[act_offset(lane, bits)] = quant_one(v0, inv);
    q[act_offset(lane + 64, bits)] = quant_one(v1, inv);
    if (lane == 0) *s_out = s;
}

}  // namespace nh
