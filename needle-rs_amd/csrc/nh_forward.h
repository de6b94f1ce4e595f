// The Needle-3 decode step on the GPU: the geometry, per-layer weights and
// per-session state the forward kernels (nh_forward.hip) take by value,
// shared with the host side that builds them (nh_model.cpp).
//
// Every pointer is device memory.  Small per-layer weights are f16 bits as
// the reference's LayerF16 keeps them (crates/needle-engine/src/infer.rs:
// 887-938); Phi8 is the int8 requantization of the dequantized mHC rows
// (infer.rs:850-867).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nh {

constexpr int FWD_MAX_D = 1024;     // d_model (the Hadamard MLP pads to 1024)
constexpr int HADA_NB = 32;         // Kronecker factor side (hada_n = 1024)
constexpr int HADA_N = HADA_NB * HADA_NB;
constexpr int COND_RANK = 8;        // HADA_COND_RANK (crates/needle-core/src/config.rs:13)
constexpr int MHC_LANES = 4;        // the step is written for 4 residual lanes
constexpr int MHC_COLS = 2 * MHC_LANES + MHC_LANES * MHC_LANES;  // pre | post | res = 24
constexpr int MAX_UNITS = 16;       // q heads + k heads + v heads (one wavefront each)
constexpr int MAX_HEAD_DIM = 64;
constexpr int MAX_SITES = 16;
constexpr int MAX_TABLES = 16;
constexpr int ENGRAM_TAPS = 4;      // ENGRAM_CONV_TAPS (config.rs:10)
constexpr int ATT_CHUNK_MAX = 256;  // key_chunks never makes a chunk longer
constexpr int ATT_THREADS = 256;
constexpr int FWD_ROWS = 32;        // token rows of one prompt chunk (infer.rs:1105-1132)
constexpr int BATCH_ROWS = 512;     // token rows of one feed: whole chunks of a prompt fed together
constexpr int ACT_ROWS = BATCH_ROWS;  // rows of an A8 buffer (a multiple of the GEMM's 64-token tiles)
constexpr int ROLLBACK = 32;        // ROLLBACK (crates/needle-engine/src/model.rs:181-183)
constexpr int ROPE_RING = 128;      // RoPE rows kept by position (the reference's list holds at most 66)
constexpr int DG_MAX_TAPS = 8;      // conv taps the unit kernels are written for
constexpr int SPAN_RUNS = 24;       // runs of live positions an attention span passes to a feed
constexpr int STATUS_SPIN = 1;      // a bounded in-kernel wait gave up (SessDev::status)
constexpr int SPIN_LIMIT = 1 << 20; // polls of a bounded wait (~64 cycles each, ~30 ms)
constexpr int DCOUNT_SLOTS = 16;    // arrival counters of the decode attention's chunk blocks

struct Dims {
    int d, nh, nkv, qk, vd, lanes, taps, layers;
    int W;      // (nh + nkv) * qk + nkv * vd: the pre-tap q | k | v width
    int nq;     // W + nh * vd: the fused q | k | v | gate rows
    int hist_slots;  // the history ring, position p at p % hist_slots: room for every row the
                     // reference's history can hold, 2 (taps - 1 + ROLLBACK) + FWD_ROWS
    int vocab, out_rows;
    int sites, ntab, eheads, seed_stride, slots, sub, dilation;
    int orders[4];
    int cap;    // session positions
    int vcap;   // row stride of the transposed int8 values: cap + 4 rounded up to 16
    int max_chunks;  // attention chunks a position can need
    int spin_limit;  // polls of an in-kernel wait before it gives up (SPIN_LIMIT)
    // per-feed state, set by the host before each feed
    int hist_lo;     // the first position the conv history still holds (LayerState::hist,
                     // crates/needle-engine/src/infer.rs:968-980): older rows read as zero
    int rope_prev;   // 1: a single token right after the newest RoPE row (the recurrence)
    int sink, ring;  // Session::attend (model.rs:62-66); ring 0: no span
};

// The keys an attention span leaves a feed (key_ranges,
// crates/needle-engine/src/infer.rs:1781-1826): the runs of positions in
// [0, sink) and [max(end - ring, sink), end) whose KV slot still holds them
// (the slot map), ascending.  A query at pos sees these runs cut to
// [lo, min(sink, pos + 1)) and [min(max(end - ring, sink), pos + 1), pos + 1).
struct KeySpan {
    int end;
    int nrun;
    int lo[SPAN_RUNS], hi[SPAN_RUNS];
};

struct LayerDev {
    const uint16_t* stage;  // the six Kronecker factors [32][32], cond_v [d][8], cond_u [8][1024]
    const uint16_t *d1, *d2, *b2, *d3, *d4;
    const uint16_t *norm_in, *post_norm, *pre_hada, *q_taps, *k_taps, *v_taps, *q_norm, *k_norm;
    const int8_t* phi_q;  // [24][lanes * d]
    const float* phi_s;   // [24]
    float a_pre, a_post, a_res;
    float ga;             // sigmoid(attn_gate), f32 expf on the host
    float b_pre[4], b_post[4], b_res[16];
    int site;             // engram site gating this layer, or -1
    int index;            // the layer's index (its post block writes cell depth index + 1)
    int lane;             // l % lanes
    int window;           // sliding window (0: attends to every position)
};

struct Globals {
    const float* final_norm;  // [d] f32
    const int32_t *perm1, *perm2;
    const float *freq;        // RoPE: powf(theta, i * (-2 / qk))
    const float *sd, *cd;     // RoPE: sincosf(freq)
    const float* etaps;       // [sites][4][d] f32
};

// One session's state, all device memory.  Row buffers hold the rows of
// the current feed (BATCH_ROWS at most); activations feed the products.
struct SessDev {
    float* xs;        // [rows][4][d] residual lanes
    float* u;         // [rows][d] mHC read of the layer
    float* x1;        // [rows][d] after the engram gate
    float* p;         // [rows][64]: the 24 mHC gate projections, then hpost
                      // [4] at 24 and the Sinkhorn mixing hres [16] at 28
    float* proj;      // [rows][nq] q | k | v | gate
    float* qbuf;      // [rows][nh][qk] rotated queries
    float* o;         // [rows][d] attention output projection
    float* ekv;       // [sites][rows][2d] engram key | value
    float* evals;     // [sites][rows][d] engram conv
    float* logits;    // [out_rows]
    float* rope_c;    // [rows][qk/2] the feed's RoPE rows
    float* rope_s;
    float* rope_rc;   // [ROPE_RING][qk/2] the RoPE rows of recent positions, position p at p % ROPE_RING
    float* rope_rs;
    float* hid;       // [rows][d] final normed hidden states of the rows a feed outputs
    float* last_hid;  // [d] NatState::last_hidden
    uint32_t* tokens; // [cap]
    float* po;        // [rows][nh][max_chunks][vd] attention chunk partials
    float* pm;        // [rows][nh][max_chunks]
    float* psum;      // [rows][nh][max_chunks]
    float* hist;      // [layers][hist_slots][W] ring of pre-tap rows
    int8_t* k8;       // [layers][cap][nkv][qk]
    float* ks;        // [layers][cap][nkv]
    int8_t* v8t;      // [layers][nkv][vd][vcap]
    float* vs;        // [layers][cap][nkv]
    int8_t* ev8;      // [sites][cap][d]
    float* evs;       // [sites][cap][d / 32]
    int8_t* xq_in;    // [ACT_ROWS][G(d)][128] the layer inputs (K = d)
    float* sx_in;     // [ACT_ROWS][G(d)]
    int8_t* xq_att;   // [ACT_ROWS][G(nh vd)][128] the gated heads
    float* sx_att;
    int8_t* xq_eng;   // [sites][ACT_ROWS][G(d)][128] the engram rows
    float* sx_eng;
    int32_t* argmax;  // scratch of the greedy pick
    int32_t* status;  // STATUS_* bits set by a kernel that gave up a wait; the host reads and clears it
    uint8_t* flags;   // [rows] the prefill combine's block flag of each row of the feed
    int32_t* dcount;  // [DCOUNT_SLOTS] chunk blocks of an A8 head group counted in; zero between launches
    float* cells;     // [rows][layers + 1][d] the feed's cells (lane means after the embedding
                      // and after each layer's mHC write), or null when not wanted; set per feed
};

// A CQ matrix read by rows (the embedding, the engram tables).
struct RowSrc {
    const void* codes;
    const uint16_t* norms;
    const float* fsel;
    int out, groups, bits;
};

struct BeginArgs {
    RowSrc emb;
    RowSrc tab[MAX_SITES];
    int eng_bits[MAX_SITES];  // code width of each site's key | value matrix
};

// Launchers (nh_forward.hip).  A feed is rows p0 .. p0 + t - 1: one token
// (a decode step), one prompt chunk (t <= 32), or several whole chunks of
// at least two tokens each fed together (t <= BATCH_ROWS, chunk c = rows
// 32c .. 32c + 31): every row keeps its chunk's semantics (the block flag of
// its products, nested key chunking, sincosf RoPE rows).
// The start of a feed: the embedding rows into the lanes, the RoPE rows, and
// per engram site the hashed table rows as A8 rows.  pick (t = 1): the
// row's token is first taken as the argmax of S.logits and stored at
// S.tokens[p0].
hipError_t fwd_begin(const Dims& D, const Globals& G, const SessDev& S, const BeginArgs& B, int p0, int t,
                     hipStream_t s, bool pick = false);
hipError_t fwd_engram_hist(const Dims& D, const Globals& G, const SessDev& S, int p0, int t, hipStream_t s);
// The per-layer boundary for rows row0 .. row0 + rows - 1: the Hadamard MLP
// and mHC write of layer `prev` (null: none, the lanes hold the embedding
// rows; with S.cells its lane means go to cell depth prev->index + 1), then
// the mHC read, engram gate, input norm and A8 of layer `next` (null: for
// rows i >= row0 + head_row0, the head's lane mean and final norm into hid
// row i - row0 - head_row0 and its A8 into that activation row).
hipError_t fwd_layer(const Dims& D, const Globals& G, const SessDev& S, const LayerDev* prev, const LayerDev* next,
                     int row0, int rows, int in_bits, int head_bits, hipStream_t s, int head_row0 = 0);
hipError_t fwd_units(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int t, hipStream_t s);
// `span`: the keys of a session with an attention span (null: none).
hipError_t fwd_attend(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int t,
                      const KeySpan* span, hipStream_t s);
// Also writes the tap history of a feed of several chunks (there the units
// leave it: a row could overwrite a ring slot another row still reads).
hipError_t fwd_attn_out(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int t, int out_bits,
                        const KeySpan* span, hipStream_t s);
// One decode token's units, attention, gate and A8 in one launch (the three
// launches above for a single row), for positions whose keys form one chunk
// and geometries with 2 or 4 heads per A8 group (dec_group_fits).
bool dec_group_fits(const Dims& D, int p0, int window);
hipError_t fwd_dec_attn(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int out_bits,
                        hipStream_t s);
// The same for any key count and with an attention span (`span`, or null):
// the position's key chunks in blocks of their own, merged by the last.
bool dec_chunks_fits(const Dims& D);
hipError_t fwd_dec_chunks(const Dims& D, const SessDev& S, const LayerDev& L, int layer, int p0, int out_bits,
                          const KeySpan* span, hipStream_t s);
hipError_t fwd_argmax(const float* logits, int n, uint32_t* dst, hipStream_t s);
hipError_t fwd_phi8(const float* rows, int nrows, int width, int8_t* q, float* scale, hipStream_t s);

}  // namespace nh
