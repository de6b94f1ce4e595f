// The C ABI (include/needle_hip.h): handles, upload and re-layout of CQ
// matrices into HBM, dispatch to the gfx950 kernels, errors.
//
// HBM code layout ("tiled"): the 64 code bytes of (row n, group g) are
// split by decode lane l = (p % 32) / 8 (crates/needle-engine/src/qlinear.rs:333):
// lane l owns packed dwords d = l, l + 4, l + 8, l + 12 of the group, 16
// bytes called the chunk (n, g, l).  Chunks are stored
//   chunk (n, g, l) at uint4 index ((n / 16 * groups + g) * 16 + n % 16) * 4 + l
// so one wavefront load (lane = 4 * (n % 16) + l) reads the 1 KiB block of
// a 16-row tile and one group.  Each nibble holds the code's v_perm
// selector (LutTables::sel_of_code), not the code.  Norms stay
// [rows][groups] f16.
#include <string.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <thread>

#include "../../include/needle_hip.h"
#include "nh_internal.h"

namespace nh {

static thread_local std::string g_err;
static int g_device = -1;
static int g_cus = 0;
static bool g_lut_ok = false;
static LutTables g_lut4;
static int8_t g_cb8[16];
static float g_cb4[16];
static float g_cbs4;
static std::mutex g_init_mu;

// The staging of nh_qlinear_apply_static: one A8 activation of up to
// STATIC_ROWS rows and 32 groups (int8 codes, then the f32 scales).  Each
// GPU holds its own copy from the library's load to the end of the process.
// In host code `scratch` is only a handle for hipGetSymbolAddress; its
// device address, one per device, is g_scratch[device], set by nh_init.
constexpr int STATIC_ROWS = ACT_PAD;
constexpr int STATIC_GROUPS = 32;
constexpr size_t SCRATCH_XQ = (size_t)STATIC_ROWS * STATIC_GROUPS * GROUP;
constexpr size_t SCRATCH_BYTES = SCRATCH_XQ + (size_t)STATIC_ROWS * STATIC_GROUPS * 4;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
static void* g_scratch[MAX_DEVICES];

void set_error(const std::string& msg) { g_err = msg; }

int device_cus() { return g_cus > 0 ? g_cus : 1; }

bool ready() { return g_device >= 0 && g_lut_ok; }

static int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

static int hip_fail(hipError_t e, const char* what) {
    return fail(NH_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

#define NH_HIP(call, what)                          \
    do {                                            \
        hipError_t e_ = (call);                     \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

static inline float bits_to_f32(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}

// ---------------------------------------------------------------- codebook
// quant.rs:30-47 (LM4) / 65-68: 4-bit Lloyd-Max centroids over sqrt(128),
// f64 then rounded once to f32.
static const uint64_t LM4_BITS[16] = {0xc005ae0f408928fbull, 0xc0005b0b8a516d54ull, 0xbff9841ff0758fc8ull,
                                      0xbff3bbbebadac679ull, 0xbfed82c6dd21f59eull, 0xbfe47717151708b5ull,
                                      0xbfd7d9b9e4b565faull, 0xbfbd4ca474b8559bull, 0x3fc2683e9154fce2ull,
                                      0x3fd9daf49368793aull, 0x3fe586b43e57d29dull, 0x3feec3d50cbc3b33ull,
                                      0x3ff4688db93b85f1ull, 0x3ffa3164906b428full, 0x4000ace7bbde2442ull,
                                      0x4005ed98d06f2a4aull};

static void codebook4(float* cb) {
    const double s = std::sqrt(128.0);
    for (int i = 0; i < 16; ++i) {
        double c;
        memcpy(&c, &LM4_BITS[i], 8);
        cb[i] = (float)(c / s);
    }
}

// quant.rs:19 (LM2), 15 (TERNARY_C), 55-68: the 2-bit centroids and the
// ternary record's three levels over sqrt(128).  Returns the count.
static const uint64_t LM2_BITS[4] = {0xbff81b52e4028034ull, 0xbfdce467275b97c2ull, 0x3fdcfd177c54d348ull,
                                     0x3ff828af1c856640ull};
static int codebook2(bool ternary, float* cb) {
    const double s = std::sqrt(128.0);
    if (ternary) {
        const double t = 1.2240064;
        cb[0] = (float)(-t / s);
        cb[1] = (float)(0.0 / s);
        cb[2] = (float)(t / s);
        return 3;
    }
    for (int i = 0; i < 4; ++i) {
        double c;
        memcpy(&c, &LM2_BITS[i], 8);
        cb[i] = (float)(c / s);
    }
    return 4;
}

// quant.rs:20-29 (LM3): the 3-bit centroids, only written into archive
// codebook blocks (no 3-bit matmul records are read).
static const uint64_t LM3_BITS[8] = {0xc00121468f3c6b81ull, 0xbff556e7125deacaull, 0xbfe7f2e0f9d592abull,
                                     0xbfce6e4509e1aa2cull, 0x3fd000bb25e4dfa5ull, 0x3fe82dc469b936a5ull,
                                     0x3ff568607ac227c5ull, 0x40012e5beccc8fdaull};

// int8_codebook (qlinear.rs:211-216): scale = amax * K127, values
// round-half-away(v * (1 / scale)) saturated.
static void int8_codebook(const float* cb, int n, int8_t* cb8, float* scale) {
    float m = 0.0f;
    for (int i = 0; i < n; ++i) m = std::max(m, std::fabs(cb[i]));
    const float k127 = bits_to_f32(0x3c010204u);
    const float s = m > 0.0f ? m * k127 : 1.0f;
    const float inv = 1.0f / s;
    for (int i = 0; i < n; ++i) {
        float v = std::round(cb[i] * inv);
        v = std::min(std::max(v, -128.0f), 127.0f);
        cb8[i] = (int8_t)(int)v;
    }
    *scale = s;
}

// v_perm_b32 byte select over the 8-byte table t (low dword = src1):
// 0..7 a table byte, 8..11 the sign of byte 1/3/5/7 replicated, 12 zero,
// 13..15 0xFF.
static uint8_t perm_byte(uint64_t t, uint32_t sel) {
    if (sel >= 13) return 0xff;
    if (sel == 12) return 0x00;
    if (sel >= 8) return ((t >> (8 * (2 * (sel - 8) + 1))) & 0x80) ? 0xff : 0x00;
    return (uint8_t)(t >> (8 * sel));
}

// Find tables A, B and a code -> selector map with
// perm(A, s) ^ perm(B, s ^ 8) == cb8[code] for all 16 codes.  The constant
// bytes depend on the signs of A and B's odd bytes, so every sign pattern
// is tried and kept only if self-consistent.
static bool solve_lut(const int8_t* vals, LutTables* out) {
    uint8_t sel_of_code[16];
    for (int i = 0; i < 16; ++i) sel_of_code[i] = (uint8_t)i;
    uint32_t rng = 12345u;
    for (int attempt = 0; attempt < 4096; ++attempt) {
        if (attempt > 0) {
            for (int i = 15; i > 0; --i) {
                rng = rng * 1664525u + 1013904223u;
                int j = (int)((rng >> 8) % (uint32_t)(i + 1));
                std::swap(sel_of_code[i], sel_of_code[j]);
            }
        }
        uint8_t code_of_sel[16];
        for (int c = 0; c < 16; ++c) code_of_sel[sel_of_code[c]] = (uint8_t)c;
        for (int signs = 0; signs < 256; ++signs) {
            auto cA = [&](uint32_t v) -> uint8_t {  // perm(A, v) for v >= 8 under the assumed signs
                if (v >= 13) return 0xff;
                if (v == 12) return 0;
                return ((signs >> (v - 8)) & 1) ? 0xff : 0;
            };
            auto cB = [&](uint32_t v) -> uint8_t {
                if (v >= 13) return 0xff;
                if (v == 12) return 0;
                return ((signs >> (4 + v - 8)) & 1) ? 0xff : 0;
            };
            uint64_t A = 0, B = 0;
            for (uint32_t s = 0; s < 8; ++s) A |= (uint64_t)((uint8_t)vals[code_of_sel[s]] ^ cB(s ^ 8)) << (8 * s);
            for (uint32_t s = 8; s < 16; ++s)
                B |= (uint64_t)((uint8_t)vals[code_of_sel[s]] ^ cA(s)) << (8 * (s - 8));
            bool ok = true;
            for (uint32_t s = 0; s < 16 && ok; ++s)
                ok = (uint8_t)(perm_byte(A, s) ^ perm_byte(B, s ^ 8)) == (uint8_t)vals[code_of_sel[s]];
            if (!ok) continue;
            out->a_hi = (uint32_t)(A >> 32);
            out->a_lo = (uint32_t)A;
            out->b_hi = (uint32_t)(B >> 32);
            out->b_lo = (uint32_t)B;
            memcpy(out->sel_of_code, sel_of_code, 16);
            memcpy(out->code_of_sel, code_of_sel, 16);
            return true;
        }
    }
    return false;
}

static bool ensure_tables() {
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (g_lut_ok) return true;
    codebook4(g_cb4);
    int8_codebook(g_cb4, 16, g_cb8, &g_cbs4);
    if (!solve_lut(g_cb8, &g_lut4)) return false;
    g_lut_ok = true;
    return true;
}

// ---------------------------------------------------------------- upload
// Archive-layout codes (rows x groups*64) -> tiled selector layout.
static void relayout(const uint8_t* packed, int out, int out_pad, int groups, const LutTables& lut,
                     std::vector<uint32_t>& tiled) {
    tiled.assign((size_t)out_pad * groups * 16, 0u);
    // nibble-pair byte -> selector-pair byte
    uint8_t map[256];
    for (int b = 0; b < 256; ++b) map[b] = (uint8_t)(lut.sel_of_code[b & 15] | (lut.sel_of_code[b >> 4] << 4));
    auto work = [&](int r0, int r1) {
        for (int n = r0; n < r1; ++n)
            for (int g = 0; g < groups; ++g) {
                const uint8_t* src = packed + ((size_t)n * groups + g) * 64;
                for (int l = 0; l < 4; ++l)
                    for (int k = 0; k < 4; ++k) {
                        const uint8_t* s = src + 4 * (4 * k + l);
                        uint32_t v = (uint32_t)map[s[0]] | ((uint32_t)map[s[1]] << 8) | ((uint32_t)map[s[2]] << 16) |
                                     ((uint32_t)map[s[3]] << 24);
                        size_t idx = ((((size_t)(n / TILE_ROWS) * groups + g) * TILE_ROWS + n % TILE_ROWS) * 4 + l) * 4 + k;
                        tiled[idx] = v;
                    }
            }
    };
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if ((size_t)out * groups < 4096) nt = 1;
    std::vector<std::thread> th;
    int per = (out + (int)nt - 1) / (int)nt;
    for (unsigned t = 0; t < nt; ++t) {
        int a = std::min(out, (int)t * per), b = std::min(out, (int)(t + 1) * per);
        if (a < b) th.emplace_back(work, a, b);
    }
    for (auto& t : th) t.join();
}

// 2-bit archive codes (rows x groups*32, four codes per byte, LSB first) ->
// tiled: decode lane l = (p % 64) / 16 owns packed dwords l and 4 + l of a
// group, stored as the pair at uint2 index
// ((n / 16 * groups + g) * 16 + n % 16) * 4 + l.
static void relayout2(const uint8_t* packed, int out, int out_pad, int groups, std::vector<uint32_t>& tiled) {
    tiled.assign((size_t)out_pad * groups * 8, 0u);
    for (int n = 0; n < out; ++n)
        for (int g = 0; g < groups; ++g) {
            const uint8_t* src = packed + ((size_t)n * groups + g) * 32;
            for (int l = 0; l < 4; ++l)
                for (int h = 0; h < 2; ++h) {
                    uint32_t v;
                    memcpy(&v, src + 4 * (4 * h + l), 4);
                    tiled[(((size_t)(n / TILE_ROWS) * groups + g) * TILE_ROWS + n % TILE_ROWS) * 8 + l * 2 + h] = v;
                }
        }
}

// QMat::build (qlinear.rs:244-265) for the code width `bits` (2 or 4), with
// from_cq's ternary remap (qlinear.rs:222-227): code 3 is the first level,
// codes 0..2 the rest; codes without a level are 0.
static int upload(std::vector<uint8_t>&& packed, std::vector<uint16_t>&& norms, int out, int in_dim, int bits,
                  bool ternary, nh_qmat** h) {
    const int groups = (in_dim + GROUP - 1) / GROUP;
    const int out_pad = (out + TILE_ROWS - 1) / TILE_ROWS * TILE_ROWS;
    nh_qmat* q = new nh_qmat();
    QMatMeta& m = q->m;
    m.out = out;
    m.out_pad = out_pad;
    m.in_dim = in_dim;
    m.groups = groups;
    m.bits = bits;
    m.ternary = ternary;
    std::vector<uint32_t> tiled;
    const int out_alloc = (out + PANEL_ROWS - 1) / PANEL_ROWS * PANEL_ROWS;
    float fsel[16] = {0};
    if (bits == 4) {
        m.cbs = g_cbs4;
        memcpy(m.vals, g_cb8, 16);
        memcpy(m.fvals, g_cb4, sizeof g_cb4);
        m.lut = g_lut4;
        relayout(packed.data(), out, out_alloc, groups, m.lut, tiled);
        for (int s = 0; s < 16; ++s) fsel[s] = m.fvals[m.lut.code_of_sel[s]];
    } else {
        float cb[4];
        int8_t cb8[4];
        const int ncb = codebook2(ternary, cb);
        int8_codebook(cb, ncb, cb8, &m.cbs);
        memset(m.vals, 0, sizeof m.vals);
        memset(m.fvals, 0, sizeof m.fvals);
        memset(&m.lut, 0, sizeof m.lut);
        for (int c = 0; c < 4; ++c) {
            const int k = ternary ? (c == 3 ? 0 : c + 1) : c;
            m.vals[c] = k < ncb ? cb8[k] : 0;
            m.fvals[c] = k < ncb ? cb[k] : 0.0f;
            m.lut.a_lo |= (uint32_t)(uint8_t)m.vals[c] << (8 * c);
            m.lut.sel_of_code[c] = m.lut.code_of_sel[c] = (uint8_t)c;
            fsel[c] = m.fvals[c];
        }
        relayout2(packed.data(), out, out_alloc, groups, tiled);
    }
    std::vector<uint16_t> np((size_t)out_alloc * groups, 0);
    memcpy(np.data(), norms.data(), (size_t)out * groups * 2);
    hipError_t e;
    if ((e = hipMalloc(&q->d_codes, tiled.size() * 4)) != hipSuccess ||
        (e = hipMalloc(&q->d_w8, (size_t)out_alloc * groups * 128)) != hipSuccess ||
        (e = hipMalloc(&q->d_norms, np.size() * 2)) != hipSuccess || (e = hipMalloc(&q->d_fsel, 64)) != hipSuccess) {
        nh_qmat_free(q);
        return fail(NH_ENOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    }
    if ((e = hipMemcpy(q->d_codes, tiled.data(), tiled.size() * 4, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(q->d_norms, np.data(), np.size() * 2, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(q->d_fsel, fsel, 64, hipMemcpyHostToDevice)) != hipSuccess ||
        (e = launch_expand_w8(q, nullptr)) != hipSuccess || (e = hipDeviceSynchronize()) != hipSuccess) {
        nh_qmat_free(q);
        return hip_fail(e, "upload");
    }
    q->h_packed = std::move(packed);
    q->h_norms = std::move(norms);
    *h = q;
    return NH_OK;
}

static int check_ready() {
    if (g_device < 0 || !g_lut_ok) return fail(NH_ESTATE, "nh_init has not been called");
    return NH_OK;
}

// ------------------------------------------------------------ seeded inputs
// threefry2x32 (crates/needle-train/src/rand.rs:139-153).
static void threefry(uint32_t k0, uint32_t k1, uint32_t x0, uint32_t x1, uint32_t* o) {
    static const uint32_t R[2][4] = {{13, 15, 26, 6}, {17, 29, 16, 24}};
    const uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
    x0 += ks[0];
    x1 += ks[1];
    for (uint32_t round = 0; round < 5; ++round) {
        for (int i = 0; i < 4; ++i) {
            x0 += x1;
            uint32_t r = R[round % 2][i];
            x1 = ((x1 << r) | (x1 >> (32 - r))) ^ x0;
        }
        x0 += ks[(round + 1) % 3];
        x1 += ks[(round + 2) % 3] + round + 1;
    }
    o[0] = x0;
    o[1] = x1;
}

// XLA's f32 ErfInv (rand.rs:166-202).
static float erfinv_f32(float x) {
    float w = -logf((1.0f - x) * (1.0f + x));
    float p;
    if (w < 5.0f) {
        static const float c[8] = {3.4327394e-7f,  -3.5233877e-06f, -4.3915065e-6f, 0.00021858087f,
                                   -0.001253725f, -0.0041776816f,  0.24664073f,    1.5014094f};
        w = w - 2.5f;
        p = 2.8102264e-8f;
        for (int i = 0; i < 8; ++i) p = c[i] + p * w;
    } else {
        static const float c[8] = {0.00010095056f, 0.0013493432f, -0.0036734284f, 0.0057395077f,
                                   -0.0076224613f, 0.0094388705f, 1.001674f,      2.8329768f};
        w = sqrtf(w) - 3.0f;
        p = -0.00020021426f;
        for (int i = 0; i < 8; ++i) p = c[i] + p * w;
    }
    if (std::fabs(x) == 1.0f) return x * INFINITY;
    return p * x;
}

}  // namespace nh

using namespace nh;

extern "C" {

int nh_version(void) { return 101; }

int nh_codebook(int bits, float* out) {
    if (!out) return fail(NH_EINVAL, "null output");
    switch (bits) {
        case 2: return codebook2(false, out);
        case 3: {
            const double s = std::sqrt(128.0);
            for (int i = 0; i < 8; ++i) {
                double c;
                memcpy(&c, &LM3_BITS[i], 8);
                out[i] = (float)(c / s);
            }
            return 8;
        }
        case 4: codebook4(out); return 16;
        case 5: return codebook2(true, out);
        default: return fail(NH_EINVAL, "no CQ codebook for this width");
    }
}

const char* nh_last_error(void) { return g_err.c_str(); }

int nh_init(int device) {
    int count = 0;
    NH_HIP(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count) return fail(NH_EDEVICE, "no such HIP device");
    hipDeviceProp_t prop;
    NH_HIP(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(NH_EDEVICE, std::string("device is ") + prop.gcnArchName + ", this library is built for gfx950");
    NH_HIP(hipSetDevice(device), "hipSetDevice");
    NH_HIP(hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, device), "hipDeviceGetAttribute");
    if (!ensure_tables()) return fail(NH_EDEVICE, "no v_perm table pair reproduces the int8 codebook");
    if (device < MAX_DEVICES) {
        // this device's copy of the static staging, with the device current
        std::lock_guard<std::mutex> lk(g_init_mu);
        if (!g_scratch[device]) {
            void* p = nullptr;
            NH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
            g_scratch[device] = p;
        }
    }
    g_device = device;
    return NH_OK;
}

int nh_qmat_from_cq(const uint8_t* packed, uint64_t packed_bytes, const uint16_t* norms, uint64_t norms_count,
                    int out, int in_dim, int bits, int group, nh_qmat** h) {
    if (int rc = check_ready()) return rc;
    if (!h || !packed || !norms) return fail(NH_EINVAL, "null argument");
    if (group != GROUP) return fail(NH_EINVAL, "CQ group size " + std::to_string(group) + " is not supported");
    // Widths of quant.rs:12,51-60: 2 and 4 bits, and ternary records (5),
    // which pack at 2 bits (quant.rs:286).
    if (bits != 2 && bits != 4 && bits != 5)
        return fail(NH_EINVAL, "CQ records of " + std::to_string(bits) + " bits are not supported");
    const bool ternary = bits == 5;
    const int cbits = ternary ? 2 : bits;
    if (out <= 0 || in_dim <= 0) return fail(NH_EINVAL, "empty matrix");
    const int groups = (in_dim + GROUP - 1) / GROUP;
    if (groups > 32) return fail(NH_EINVAL, "in_dim above 4096 is not supported");
    const uint64_t row_bytes = (uint64_t)groups * GROUP * cbits / 8;
    if (packed_bytes < row_bytes * (uint64_t)out) return fail(NH_ESMALL, "packed blob shorter than out x row_bytes");
    if (norms_count < (uint64_t)groups * out) return fail(NH_ESMALL, "norms shorter than out x groups");
    std::vector<uint8_t> p(packed, packed + row_bytes * out);
    std::vector<uint16_t> nn(norms, norms + (size_t)groups * out);
    return upload(std::move(p), std::move(nn), out, in_dim, cbits, ternary, h);
}

int nh_qmat_from_f32(const float* w, int out, int in_dim, nh_qmat** h) {
    if (int rc = check_ready()) return rc;
    if (!h || !w) return fail(NH_EINVAL, "null argument");
    if (out <= 0 || in_dim <= 0) return fail(NH_EINVAL, "empty matrix");
    const int groups = (in_dim + GROUP - 1) / GROUP;
    if (groups > 32) return fail(NH_EINVAL, "in_dim above 4096 is not supported");
    float* dw = nullptr;
    float* dcb = nullptr;
    uint8_t* dp = nullptr;
    uint16_t* dn = nullptr;
    const size_t nw = (size_t)out * in_dim, np = (size_t)out * groups * 64, nn = (size_t)out * groups;
    hipError_t e = hipMalloc(&dw, nw * 4);
    if (e == hipSuccess) e = hipMalloc(&dcb, 64);
    if (e == hipSuccess) e = hipMalloc(&dp, np);
    if (e == hipSuccess) e = hipMalloc(&dn, nn * 2);
    std::vector<uint8_t> packed(np);
    std::vector<uint16_t> norms(nn);
    if (e == hipSuccess) e = hipMemcpy(dw, w, nw * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dcb, g_cb4, 64, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_cq_pack(dw, out, in_dim, groups, dcb, dp, dn, nullptr);
    if (e == hipSuccess) e = hipMemcpy(packed.data(), dp, np, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(norms.data(), dn, nn * 2, hipMemcpyDeviceToHost);
    hipFree(dw);
    hipFree(dcb);
    hipFree(dp);
    hipFree(dn);
    if (e != hipSuccess) return hip_fail(e, "cq_pack");
    return upload(std::move(packed), std::move(norms), out, in_dim, 4, false, h);
}

int nh_qlinear_new(nh_qmat* const* parts, int n, nh_qmat** h) {
    if (int rc = check_ready()) return rc;
    if (!parts || n <= 0 || !h) return fail(NH_EINVAL, "no parts");
    for (int i = 0; i < n; ++i)
        if (!parts[i]) return fail(NH_EINVAL, "null part");
    const QMatMeta& m0 = parts[0]->m;
    int out = 0;
    for (int i = 0; i < n; ++i) {
        const QMatMeta& m = parts[i]->m;
        if (m.in_dim != m0.in_dim) return fail(NH_EINVAL, "fused parts must share in_dim");
        if (m.bits != m0.bits || m.cbs != m0.cbs || memcmp(m.vals, m0.vals, 16) != 0)
            return fail(NH_EINVAL, "fused parts must share a code width");
        out += m.out;
    }
    std::vector<uint8_t> packed;
    std::vector<uint16_t> norms;
    for (int i = 0; i < n; ++i) {
        packed.insert(packed.end(), parts[i]->h_packed.begin(), parts[i]->h_packed.end());
        norms.insert(norms.end(), parts[i]->h_norms.begin(), parts[i]->h_norms.end());
    }
    return upload(std::move(packed), std::move(norms), out, m0.in_dim, m0.bits, m0.ternary, h);
}

int nh_qmat_slice_rows(const nh_qmat* h, int r0, int r1, nh_qmat** out) {
    if (int rc = check_ready()) return rc;
    if (!h || !out) return fail(NH_EINVAL, "null argument");
    if (r0 < 0 || r1 <= r0 || r1 > h->m.out) return fail(NH_EINVAL, "row range outside the matrix");
    const size_t rb = h->h_packed.size() / h->m.out, G = h->m.groups;
    std::vector<uint8_t> packed(h->h_packed.begin() + r0 * rb, h->h_packed.begin() + r1 * rb);
    std::vector<uint16_t> norms(h->h_norms.begin() + r0 * G, h->h_norms.begin() + r1 * G);
    return upload(std::move(packed), std::move(norms), r1 - r0, h->m.in_dim, h->m.bits, h->m.ternary, out);
}

int nh_qmat_free(nh_qmat* h) {
    if (!h) return NH_OK;
    if (h->d_codes) hipFree(h->d_codes);
    if (h->d_w8) hipFree(h->d_w8);
    if (h->d_norms) hipFree(h->d_norms);
    if (h->d_fsel) hipFree(h->d_fsel);
    delete h;
    return NH_OK;
}

int nh_qmat_shape(const nh_qmat* h, int* out, int* in_dim, int* bits) {
    if (!h) return fail(NH_EINVAL, "null matrix");
    if (out) *out = h->m.out;
    if (in_dim) *in_dim = h->m.in_dim;
    if (bits) *bits = h->m.bits;
    return NH_OK;
}

int64_t nh_qmat_bytes(const nh_qmat* h) {
    if (!h) return fail(NH_EINVAL, "null matrix");
    return (int64_t)h->m.out * h->m.groups * (GROUP * h->m.bits / 8) + (int64_t)h->m.out * h->m.groups * 2;
}

int nh_qmat_download(const nh_qmat* h, uint8_t* packed, uint64_t packed_bytes, uint16_t* norms, uint64_t norms_count) {
    if (!h) return fail(NH_EINVAL, "null matrix");
    if (packed) {
        if (packed_bytes < h->h_packed.size()) return fail(NH_ESMALL, "packed buffer too small");
        memcpy(packed, h->h_packed.data(), h->h_packed.size());
    }
    if (norms) {
        if (norms_count < h->h_norms.size()) return fail(NH_ESMALL, "norms buffer too small");
        memcpy(norms, h->h_norms.data(), h->h_norms.size() * 2);
    }
    return NH_OK;
}

int nh_qmat_rows(const nh_qmat* h, const uint32_t* ids, int n, float* out, void* stream) {
    if (int rc = check_ready()) return rc;
    if (!h || (n > 0 && (!ids || !out)) || n < 0) return fail(NH_EINVAL, "bad arguments");
    NH_HIP(launch_rows(h, ids, n, out, (hipStream_t)stream), "rows");
    return NH_OK;
}

int nh_qact_new(int rows, int in_dim, int bits, nh_qact** a) {
    if (int rc = check_ready()) return rc;
    if (!a || rows <= 0 || in_dim <= 0) return fail(NH_EINVAL, "bad activation shape");
    if (bits != 2 && bits != 4) return fail(NH_EINVAL, "activation layouts exist for 2- and 4-bit codes");
    const int groups = (in_dim + GROUP - 1) / GROUP;
    if (groups > 32) return fail(NH_EINVAL, "in_dim above 4096 is not supported");
    nh_qact* q = new nh_qact();
    q->cap_rows = (rows + ACT_PAD - 1) / ACT_PAD * ACT_PAD;
    q->rows = 0;
    q->in_dim = in_dim;
    q->groups = groups;
    q->bits = bits;
    const size_t nx = (size_t)q->cap_rows * groups * GROUP, ns = (size_t)q->cap_rows * groups;
    hipError_t e = hipMalloc(&q->d_xq, nx);
    if (e == hipSuccess) e = hipMalloc(&q->d_sx, ns * 4);
    if (e == hipSuccess) e = hipMemset(q->d_xq, 0, nx);
    if (e == hipSuccess) e = hipMemset(q->d_sx, 0, ns * 4);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        nh_qact_free(q);
        return fail(NH_ENOMEM, std::string("activation allocation: ") + hipGetErrorString(e));
    }
    *a = q;
    return NH_OK;
}

int nh_qact_free(nh_qact* a) {
    if (!a) return NH_OK;
    if (a->d_xq) hipFree(a->d_xq);
    if (a->d_sx) hipFree(a->d_sx);
    delete a;
    return NH_OK;
}

int nh_qact_rows(const nh_qact* a) {
    if (!a) return fail(NH_EINVAL, "null activation");
    return a->rows;
}

int nh_act_prep(nh_qact* a, const float* x, int rows, int in_dim, const uint16_t* norm_scale, void* stream) {
    if (int rc = check_ready()) return rc;
    if (!a || !x) return fail(NH_EINVAL, "null argument");
    if (rows <= 0 || rows > a->cap_rows) return fail(NH_EINVAL, "rows outside the activation's capacity");
    if (in_dim != a->in_dim) return fail(NH_EINVAL, "in_dim does not match the activation");
    if (norm_scale && in_dim % 16 != 0) return fail(NH_EINVAL, "the fused norm needs in_dim a multiple of 16");
    NH_HIP(launch_act_prep(x, rows, in_dim, a->groups, a->bits, norm_scale, a->d_xq, a->d_sx, (hipStream_t)stream),
           "act_prep");
    a->rows = rows;
    return NH_OK;
}

int nh_qact_download(const nh_qact* a, int8_t* xq, uint64_t xq_bytes, float* sx, uint64_t sx_count) {
    if (!a) return fail(NH_EINVAL, "null activation");
    const size_t nx = (size_t)a->rows * a->groups * GROUP, ns = (size_t)a->rows * a->groups;
    if ((xq && xq_bytes < nx) || (sx && sx_count < ns)) return fail(NH_ESMALL, "buffer too small");
    NH_HIP(hipDeviceSynchronize(), "sync");
    if (xq) {
        std::vector<int8_t> t(nx);
        NH_HIP(hipMemcpy(t.data(), a->d_xq, nx, hipMemcpyDeviceToHost), "download xq");
        // act_pos (qlinear.rs:145-147): 2-bit (p % 4) * 32 + p / 4, 4-bit
        // (p % 2) * 64 + p / 2.
        for (size_t u = 0; u < (size_t)a->rows * a->groups; ++u)
            for (int p = 0; p < GROUP; ++p) {
                const int ap = a->bits == 2 ? (p % 4) * 32 + p / 4 : (p % 2) * 64 + p / 2;
                xq[u * GROUP + ap] = t[u * GROUP + act_offset(p, a->bits)];
            }
    }
    if (sx) NH_HIP(hipMemcpy(sx, a->d_sx, ns * 4, hipMemcpyDeviceToHost), "download sx");
    return NH_OK;
}

static int check_pair(const nh_qmat* w, const nh_qact* a) {
    if (int rc = check_ready()) return rc;
    if (!w || !a) return fail(NH_EINVAL, "null argument");
    if (a->rows <= 0) return fail(NH_EINVAL, "activation holds no rows (nh_act_prep first)");
    if (w->m.groups != a->groups || w->m.bits != a->bits)
        return fail(NH_EINVAL, "matrix and activation differ in groups or code width");
    return NH_OK;
}

// QLinear::apply's two steps over a staging activation (xq, sx) of
// `cap_rows` rows: A8 of x, then the product (decode combine for one row,
// prefill combine for more) into y[rows][out].
static int apply_into(const nh_qmat* w, const float* x, int rows, float* y, int8_t* xq, float* sx, int cap_rows,
                      hipStream_t st) {
    nh_qact a{};
    a.cap_rows = cap_rows;
    a.rows = rows;
    a.in_dim = w->m.in_dim;
    a.groups = w->m.groups;
    a.bits = w->m.bits;
    a.d_xq = xq;
    a.d_sx = sx;
    NH_HIP(launch_act_prep(x, rows, a.in_dim, a.groups, a.bits, nullptr, xq, sx, st), "apply: act_prep");
    hipError_t e = rows == 1 ? launch_gemv(w, &a, y, 0, nullptr, st)
                             : launch_gemm(w, &a, nullptr, y, w->m.out, 0, nullptr, st);
    NH_HIP(e, "apply: product");
    return NH_OK;
}

static int check_apply(const nh_qmat* w, const float* x, int rows, const float* y) {
    if (int rc = check_ready()) return rc;
    if (!w || !x || !y) return fail(NH_EINVAL, "null argument");
    if (rows <= 0) return fail(NH_EINVAL, "no rows");
    if (w->m.groups > 32) return fail(NH_EINVAL, "in_dim above 4096 is not supported");
    return NH_OK;
}

int nh_qlinear_apply(const nh_qmat* w, const float* x, int rows, float* y, void* stream) {
    if (int rc = check_apply(w, x, rows, y)) return rc;
    hipStream_t st = (hipStream_t)stream;
    const int cap = (rows + ACT_PAD - 1) / ACT_PAD * ACT_PAD;
    const size_t nx = (size_t)cap * w->m.groups * GROUP, ns = (size_t)cap * w->m.groups;
    void* buf = nullptr;
    NH_HIP(hipMallocAsync(&buf, nx + ns * 4, st), "apply: staging allocation");
    const int rc = apply_into(w, x, rows, y, (int8_t*)buf, (float*)((uint8_t*)buf + nx), cap, st);
    const hipError_t e = hipFreeAsync(buf, st);
    if (rc != NH_OK) return rc;
    NH_HIP(e, "apply: staging release");
    return NH_OK;
}

int nh_qlinear_apply_static(const nh_qmat* w, const float* x, int rows, float* y, void* stream) {
    if (int rc = check_apply(w, x, rows, y)) return rc;
    if (rows > STATIC_ROWS) return fail(NH_EINVAL, "nh_qlinear_apply_static takes at most 64 rows");
    int dev = -1;
    NH_HIP(hipGetDevice(&dev), "hipGetDevice");
    void* p = dev >= 0 && dev < MAX_DEVICES ? g_scratch[dev] : nullptr;
    if (!p) return fail(NH_ESTATE, "nh_init has not been called for the current device");
    // Nothing in the staging needs to start at zero: act_prep writes the
    // rows' codes and scales, and the products store no padding row.
    return apply_into(w, x, rows, y, (int8_t*)p, (float*)((uint8_t*)p + SCRATCH_XQ), STATIC_ROWS,
                      (hipStream_t)stream);
}

int nh_matmul(const nh_qmat* w, const nh_qact* a, float* y, int ldy, int col0, void* stream) {
    if (int rc = check_pair(w, a)) return rc;
    if (!y) return fail(NH_EINVAL, "null output");
    if (col0 < 0 || (a->rows > 1 && ldy < col0 + w->m.out)) return fail(NH_EINVAL, "ldy/col0 do not fit the rows");
    hipError_t e = a->rows == 1 ? launch_gemv(w, a, y, col0, nullptr, (hipStream_t)stream)
                                : launch_gemm(w, a, nullptr, y, ldy, col0, nullptr, (hipStream_t)stream);
    NH_HIP(e, "matmul");
    return NH_OK;
}

int nh_matmul_flags(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                    void* stream) {
    if (int rc = check_pair(w, a)) return rc;
    if (!y || !block) return fail(NH_EINVAL, "null argument");
    if (col0 < 0 || ldy < col0 + w->m.out) return fail(NH_EINVAL, "ldy/col0 do not fit the rows");
    NH_HIP(launch_gemm(w, a, block, y, ldy, col0, nullptr, (hipStream_t)stream), "matmul_flags");
    return NH_OK;
}

int nh_single_rows(const nh_qmat* w, const nh_qact* a, const uint32_t* ids, int n, float* out, void* stream) {
    if (int rc = check_pair(w, a)) return rc;
    if (n < 0 || (n > 0 && (!ids || !out))) return fail(NH_EINVAL, "bad arguments");
    NH_HIP(launch_single_rows(w, a, ids, n, out, nullptr, 0, (hipStream_t)stream), "single_rows");
    return NH_OK;
}

int nh_head_logits_sparse(const nh_qmat* w, const nh_qact* a, const uint32_t* ids, int n, int out_rows, float* logits,
                          void* stream) {
    if (int rc = check_pair(w, a)) return rc;
    if (n < 0 || (n > 0 && !ids) || !logits || out_rows <= 0 || out_rows > w->m.out)
        return fail(NH_EINVAL, "bad arguments");
    const float neg = bits_to_f32(0xf149f2cau);  // NEG, crates/needle-engine/src/infer.rs:36
    NH_HIP(launch_fill(logits, neg, out_rows, (hipStream_t)stream), "fill");
    NH_HIP(launch_single_rows(w, a, ids, n, nullptr, logits, out_rows, (hipStream_t)stream), "sparse logits");
    return NH_OK;
}

int nh_debug_partials(const nh_qmat* w, const nh_qact* a, int32_t* out, void* stream) {
    if (int rc = check_pair(w, a)) return rc;
    if (!out) return fail(NH_EINVAL, "null output");
    hipError_t e = a->rows == 1 ? launch_gemv(w, a, nullptr, 0, out, (hipStream_t)stream)
                                : launch_gemm(w, a, nullptr, nullptr, 0, 0, out, (hipStream_t)stream);
    NH_HIP(e, "partials");
    return NH_OK;
}

int nh_debug_read_floor(const nh_qmat* w, const nh_qact* a, int mode, float* y, void* stream) {
    if (int rc = check_pair(w, a)) return rc;
    if (w->m.bits != 4 || a->rows != 1 || mode < 0 || mode > 2)
        return fail(NH_EINVAL, "a 4-bit one-token product, mode 0, 1 or 2");
    if (mode == 2 && !y) return fail(NH_EINVAL, "mode 2 stores to y");
    NH_HIP(launch_read_floor(w, a, mode, y, (hipStream_t)stream), "read floor");
    return NH_OK;
}

int nh_normal(uint32_t key0, uint32_t key1, uint64_t n, float* out) {
    if (!out && n) return fail(NH_EINVAL, "null output");
    const float lo = bits_to_f32(0xbf7fffffu);  // nextafter(-1, 0)
    const float hi = 1.0f;
    const float sqrt2 = bits_to_f32(0x3fb504f3u);
    auto work = [&](uint64_t a, uint64_t b) {
        for (uint64_t i = a; i < b; ++i) {
            uint32_t o[2];
            threefry(key0, key1, (uint32_t)(i >> 32), (uint32_t)i, o);
            uint32_t bits = o[0] ^ o[1];
            float f = bits_to_f32((bits >> 9) | 0x3f800000u) - 1.0f;
            float u = f * (hi - lo);
            u = u + lo;
            u = std::isnan(u) ? lo : std::max(lo, u);
            out[i] = sqrt2 * erfinv_f32(u);
        }
    };
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < (1u << 16)) nt = 1;
    std::vector<std::thread> th;
    uint64_t per = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        uint64_t a = std::min<uint64_t>(n, t * per), b = std::min<uint64_t>(n, (t + 1) * per);
        if (a < b) th.emplace_back(work, a, b);
    }
    for (auto& t : th) t.join();
    return NH_OK;
}

int nh_split(uint32_t key0, uint32_t key1, uint32_t* out4) {
    if (!out4) return fail(NH_EINVAL, "null output");
    threefry(key0, key1, 0, 0, out4);
    threefry(key0, key1, 0, 1, out4 + 2);
    return NH_OK;
}

}  // extern "C"
