// Fused RMSNorm -> 128-point FWHT -> int8 activation quantizer (A8).
//
// One workgroup per token row.  With a norm scale, the row's zero-centred
// RMSNorm comes first: ss = dot16(x, x) in the reference's accumulator
// order (crates/needle-engine/src/infer.rs:369-419, portable branch
// 401-418), r = 1 / sqrtf(ss / n + 1e-6) (infer.rs:422-424) and
// h = fma(x * r, s, x * r) (norm_apply16, infer.rs:614-635).  Then every
// 128-group is rotated (crates/needle-core/src/quant.rs:109-115) and
// quantized (crates/needle-engine/src/qlinear.rs:77-88, 152-164).  The
// int8 codes are written in the GEMV/GEMM activation order (act_offset),
// not the reference's act_pos order: the integer sums they feed are
// order-free, and nh_qact_download restores act_pos for checks.
#include "nh_device.h"
#include "nh_internal.h"

namespace nh {

constexpr int ACT_THREADS = 256;
constexpr int ACT_MAX_DIM = 32 * GROUP;  // 4096 inputs (16 KiB of LDS)

__global__ __launch_bounds__(ACT_THREADS) void k_act_prep(const float* __restrict__ x, int in_dim, int groups,
                                                          int bits, const uint16_t* __restrict__ norm_scale,
                                                          int8_t* __restrict__ xq, float* __restrict__ sx) {
    const int row = blockIdx.x;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    __shared__ float xr[ACT_MAX_DIM];
    __shared__ float s_r;
    // The row once from HBM, coalesced; every later read is LDS.
    const float* xg = x + (size_t)row * in_dim;
    for (int i = threadIdx.x; i < in_dim; i += ACT_THREADS) xr[i] = xg[i];
    __syncthreads();

    float r = 1.0f;
    if (norm_scale) {
        if (wave == 0) {
            // dot16: lane i16 = j * 4 + l carries accumulator a[j][l] over
            // chunks c ascending: a = fma(x[16c + i16], x[16c + i16], a).
            float a = 0.0f;
            if (lane < 16) {
                for (int c = 0; c < in_dim / 16; ++c) {
                    float v = xr[c * 16 + lane];
                    a = __builtin_fmaf(v, v, a);
                }
            }
            // t[l] = ((a[2][l] + a[3][l]) + a[1][l]) + a[0][l]; lane l < 4
            // reads a[j][l] from lane 4j + l.
            float a0 = __shfl(a, lane & 3, 64);
            float a1 = __shfl(a, 4 + (lane & 3), 64);
            float a2 = __shfl(a, 8 + (lane & 3), 64);
            float a3 = __shfl(a, 12 + (lane & 3), 64);
            float t = ((a2 + a3) + a1) + a0;
            float t0 = __shfl(t, 0, 64), t1 = __shfl(t, 1, 64), t2 = __shfl(t, 2, 64), t3 = __shfl(t, 3, 64);
            float ss = (t0 + t1) + (t2 + t3);
            float v = ss / (float)in_dim + 1e-6f;
            float rr = 1.0f / __builtin_sqrtf(v);
            if (lane == 0) s_r = rr;
        }
        __syncthreads();
        r = s_r;
    }

    for (int g = wave; g < groups; g += ACT_THREADS / 64) {
        int p0 = g * GROUP + lane, p1 = p0 + 64;
        float v0 = p0 < in_dim ? xr[p0] : 0.0f;
        float v1 = p1 < in_dim ? xr[p1] : 0.0f;
        if (norm_scale) {
            if (p0 < in_dim) {
                float t = v0 * r;
                v0 = __builtin_fmaf(t, f16_bits_to_f32(norm_scale[p0]), t);
            }
            if (p1 < in_dim) {
                float t = v1 * r;
                v1 = __builtin_fmaf(t, f16_bits_to_f32(norm_scale[p1]), t);
            }
        }
        a8_group(v0, v1, lane, bits, xq + ((size_t)row * groups + g) * GROUP, sx + (size_t)row * groups + g);
    }
}

hipError_t launch_act_prep(const float* x, int rows, int in_dim, int groups, int bits, const uint16_t* norm_scale,
                           int8_t* xq, float* sx, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_act_prep, dim3(rows), dim3(ACT_THREADS), 0, s, x, in_dim, groups, bits, norm_scale, xq, sx);
    return hipGetLastError();
}

}  // namespace nh
