// Internal declarations shared by the runtime (nh_api.hip) and the kernel
// translation units.  gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

namespace nh {

constexpr int GROUP = 128;
// Rows per tile of the HBM code layout: one tile-group block is 16 rows x
// 4 lanes x 16 bytes = 1 KiB, read by one wavefront load.
constexpr int TILE_ROWS = 16;
// Rows the device copies of a matrix (codes, int8 fragments, norms) are
// padded to: the GEMM reads whole panels of up to 64 rows without clamping
// row indices; padding rows hold zeros and are never stored.
constexpr int PANEL_ROWS = 64;
// Token rows an activation buffer is padded to (the GEMM reads whole
// 64-token tiles; padding rows hold zeros and are never stored).
constexpr int ACT_PAD = 64;

// The int8 codebook as v_perm tables: value(s) = perm(A, s) ^ perm(B, s ^ 8)
// for the 4-bit selector s a code is stored as.
struct LutTables {
    uint32_t a_hi, a_lo, b_hi, b_lo;
    uint8_t sel_of_code[16];   // code -> stored selector nibble
    uint8_t code_of_sel[16];   // inverse
};

struct QMatMeta {
    int out;       // logical rows
    int out_pad;   // rows padded to TILE_ROWS
    int in_dim;
    int groups;
    int bits;                // 2 or 4 bits per code
    bool ternary;            // a ternary record (2-bit codes, remapped)
    float cbs;               // int8 codebook scale
    int8_t vals[16];         // code -> int8 codebook value
    float fvals[16];         // code -> f32 codebook value
    // 4-bit: the v_perm table pair and selector map.  2-bit: codes are
    // stored as they are and lut.a_lo holds vals[0..3] as bytes (one v_perm
    // lookup with the 2-bit code as selector).
    LutTables lut;
};

}  // namespace nh

struct nh_qmat {
    nh::QMatMeta m;
    // HBM: codes in the tiled layout (see nh_api.hip), norms [out_pad][groups]
    // f16 bits, and the per-selector f32 codebook for row dequantization.
    uint4* d_codes = nullptr;
    uint16_t* d_norms = nullptr;
    // The same codes as int8 MFMA A fragments for the GEMM: per 16-row tile
    // and group, [half][lane][16 bytes] (k_expand_w8).
    uint4* d_w8 = nullptr;
    float* d_fsel = nullptr;
    // Read again at every token (a loaded model's weights): the decode
    // product's code loads then keep their lines cached instead of streaming
    // them past (the default, for matrices swept once).
    bool resident = false;
    // Host copy of the archive-layout codes and norms (fusion, download).
    std::vector<uint8_t> h_packed;   // out x groups*64
    std::vector<uint16_t> h_norms;   // out x groups
};

struct nh_weights;

struct nh_qact {
    int cap_rows;   // allocated rows (multiple of ACT_PAD)
    int rows;       // rows of the last prep
    int in_dim;
    int groups;
    int bits;
    int8_t* d_xq = nullptr;   // [cap_rows][groups][128], tiled act order
    float* d_sx = nullptr;    // [cap_rows][groups]
};

namespace nh {

// Error plumbing: kernels' host launchers return hipError_t.
void set_error(const std::string& msg);
// Compute units of the device selected by nh_init.
int device_cus();
// nh_init has selected a device and built the code tables.
bool ready();

// Byte offset (0..127) inside a group's activation block of natural
// position p, for the code width `bits` of the matrices it feeds.  Each
// decode lane l (qlinear.rs:333) owns 32 contiguous bytes at l * 32.
//  4-bit: dword d = p / 8 of the packed codes belongs to lane l = d % 4 and
//    is the k = d / 4 -th dword of its chunk; its even positions meet bytes
//    0..3 of an 8-byte block, its odd ones bytes 4..7.
//  2-bit: dword d = p / 16 belongs to lane l = d % 4 (positions with
//    (p % 64) / 16 == l) as its d / 4 -th dword; the 2-bit field k = p % 4
//    of its byte b = (p / 4) % 4 meets byte b of 4-byte block k.
__host__ __device__ inline int act_offset(int p, int bits) {
    if (bits == 2) {
        const int d = p >> 4, l = d & 3;
        return l * 32 + ((d >> 2) * 4 + (p & 3)) * 4 + ((p >> 2) & 3);
    }
    const int d = p >> 3, j = p & 7;
    const int l = d & 3, k = d >> 2;
    return ((l * 4 + k) << 3) + ((j & 1) ? 4 + (j >> 1) : (j >> 1));
}

// The small per-layer tensors of a .cact layer in their canonical walk
// order (crates/needle-engine/src/weights.rs:322-371).
enum SmallKind {
    S_NORM_IN = 0, S_Q_TAPS, S_K_TAPS, S_V_TAPS, S_Q_NORM, S_K_NORM, S_POST_NORM, S_ATTN_GATE, S_PRE_HADA,
    S_D1, S_D2, S_B2, S_D3, S_D4, S_KRON0, S_KRON1, S_KRON2, S_KRON3, S_KRON4, S_KRON5, S_COND_V, S_COND_U,
    SMALL_KINDS
};

// The non-matmul tensors of an archive widened to f32 (f16 records exactly),
// as Cursor::next yields them (weights.rs:106-110).
struct ArchiveSmall {
    std::vector<std::vector<std::vector<float>>> layer;  // [layer][SmallKind] (empty: absent)
    std::vector<std::vector<float>> mhc;                  // a_pre, a_post, a_res, b_pre, b_post, b_res
    std::vector<float> perm1, perm2, final_norm;
    std::vector<std::vector<float>> etaps;                // per engram site
};

// nh_weights_load, and with `small` set the small tensors too (an error if
// one of them is a CQ record).
int load_archive(const uint8_t* bytes, uint64_t n, nh_weights** w, ArchiveSmall* small);

// Same-shaped decode products launched together (k_gemv_batch).
constexpr int GEMV_BATCH_MAX = 16;
struct GemvBatch {
    const void* codes[GEMV_BATCH_MAX];
    const uint16_t* norms[GEMV_BATCH_MAX];
    const uint4* xq[GEMV_BATCH_MAX];
    const float* sx[GEMV_BATCH_MAX];
    float* y[GEMV_BATCH_MAX];
};
// Whether n matrices share out, groups, code width and tables.
bool gemv_batchable(const nh_qmat* const* w, int n);
hipError_t launch_gemv_batch(const nh_qmat* const* w, const nh_qact* const* a, float* const* y, int n, hipStream_t s);

// Launchers (one per kernel translation unit).
hipError_t launch_act_prep(const float* x, int rows, int in_dim, int groups, int bits, const uint16_t* norm_scale,
                           int8_t* xq, float* sx, hipStream_t s);
hipError_t launch_gemv(const nh_qmat* w, const nh_qact* a, float* y, int col0, int32_t* dbg_lanes, hipStream_t s);
// The decode product's read floors (0: its loads in its grid, 1: a plain stream of its bytes).
hipError_t launch_read_floor(const nh_qmat* w, const nh_qact* a, int mode, float* y, hipStream_t s);
hipError_t launch_expand_w8(const nh_qmat* w, hipStream_t s);
hipError_t launch_gemm(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                       int32_t* dbg_totals, hipStream_t s);
// Same-shaped prefill products in one launch (blockIdx.y picks the product):
// gemv_batchable matrices, activations of equal rows, width and capacity.
bool gemm_batchable(const nh_qmat* const* w, const nh_qact* const* a, int n);
hipError_t launch_gemm_batch(const nh_qmat* const* w, const nh_qact* const* a, float* const* y, int n,
                             const uint8_t* block, int ldy, hipStream_t s);
hipError_t launch_single_rows(const nh_qmat* w, const nh_qact* a, const uint32_t* ids, int n, float* out,
                              float* scatter_logits, int scatter_n, hipStream_t s);
hipError_t launch_fill(float* p, float v, int n, hipStream_t s);
hipError_t launch_rows(const nh_qmat* w, const uint32_t* ids, int n, float* out, hipStream_t s);
hipError_t launch_cq_pack(const float* w, int rows, int d, int groups, const float* cb, uint8_t* packed,
                          uint16_t* norms, hipStream_t s);

}  // namespace nh
