/*
 * needle_hip.h -- C ABI of the MI355X (gfx950) packed CQ-W4 x A8 runtime.
 *
 * Drop-in for the operator level of needle-rs's packed CQ runtime
 * (crates/needle-engine/src/qlinear.rs): a Rust `needle-hip` crate binds
 * these with `extern "C"` declarations and the
 * QMat/QAct/QLinear methods forward to them.  Conventions follow the
 * reference's C API (crates/needle-ffi/src/lib.rs:30-33,180-183): every
 * entry point returns an int, 0 (or a count) on success and a negative
 * NH_E* code on failure, with the reason in nh_last_error().  Nothing
 * aborts across the ABI; the reference's assert!/panic sites
 * (qlinear.rs:221,469) become NH_EINVAL.
 *
 * Memory: matrices and activations are opaque handles that own device
 * memory (HBM).  Activation inputs, outputs and id lists are DEVICE
 * pointers; archive bytes (nh_qmat_from_cq) and f32 weights
 * (nh_qmat_from_f32) are HOST pointers borrowed for the call only, like
 * needle_load (lib.rs:57-77).  `stream` is a hipStream_t (NULL: the null
 * stream).  Calls on one handle are serialized by the caller, as the
 * reference's engine mutex does (lib.rs:18-28).
 */
#ifndef NEEDLE_HIP_H
#define NEEDLE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NH_OK 0
#define NH_EINVAL (-1)   /* bad argument or shape (the reference asserts) */
#define NH_ESMALL (-2)   /* caller buffer too small (needle_complete's -2) */
#define NH_EDEVICE (-3)  /* HIP runtime error / no gfx950 device */
#define NH_ENOMEM (-4)   /* device allocation failed */
#define NH_ESTATE (-5)   /* nh_init not called */

typedef struct nh_qmat nh_qmat; /* a CQ matrix resident in HBM (QMat / fused QLinear) */
typedef struct nh_qact nh_qact; /* rotated int8 activations resident in HBM (QAct) */
typedef struct nh_weights nh_weights; /* every matmul weight of a .cact archive in HBM (QWeights) */
typedef struct nh_model nh_model;     /* a loaded model for the decode step (Model) */
typedef struct nh_session nh_session; /* one sequence's decoding state in HBM (Session) */

/* ---- runtime ----------------------------------------------------------- */
/* Select the device and prepare the code tables.  No reference counterpart
 * (the CPU engine needs no device); idempotent per device. */
int nh_init(int device);
/* Text of the last failure on this thread (needle_last_error, lib.rs:180-183). */
const char* nh_last_error(void);
/* Library ABI version (major*100 + minor). */
int nh_version(void);
/* quant::codebook(bits, 128) (crates/needle-core/src/quant.rs:52-68): the
 * f32 centroids of a code width (2, 3, 4; 5 = ternary) into out[16];
 * returns their count. */
int nh_codebook(int bits, float* out);

/* ---- matrices (QMat, qlinear.rs:43-61) --------------------------------- */
/* QMat::from_cq (qlinear.rs:220-236) over a .cact CQ blob as CqView holds
 * it (crates/needle-core/src/cact.rs:497-525): `packed` is out x row_bytes
 * (row_bytes = in_pad * bits / 8; ternary records pack at 2 bits),
 * `norms` is out x groups f16 bit patterns.  group must be 128 (the
 * reference asserts); bits is 2, 4 or 5 (ternary, quant.rs:12, with the
 * code remap of qlinear.rs:226-227).  The blob is re-laid out into the
 * tiled HBM layout (plus an int8 copy for the batched products) during
 * the call. */
int nh_qmat_from_cq(const uint8_t* packed, uint64_t packed_bytes, const uint16_t* norms, uint64_t norms_count,
                    int out, int in_dim, int bits, int group, nh_qmat** h);
/* QMat::from_f32 (qlinear.rs:239-242): cq_pack (crates/needle-core/src/quant.rs:233-256)
 * of host f32 w[out][in_dim] run on the GPU, then uploaded as from_cq. */
int nh_qmat_from_f32(const float* w, int out, int in_dim, nh_qmat** h);
/* QLinear::new (qlinear.rs:501-519): parts fused by row concatenation
 * (q|k|v|gate, crates/needle-engine/src/weights.rs:484-490).  The parts
 * stay valid and owned by the caller. */
int nh_qlinear_new(nh_qmat* const* parts, int n, nh_qmat** h);
/* QMat::slice_rows (qlinear.rs:268-276): rows r0..r1 of h as their own
 * matrix (per-layer slices of stacked records, weights.rs:383-388). */
int nh_qmat_slice_rows(const nh_qmat* h, int r0, int r1, nh_qmat** out);
int nh_qmat_free(nh_qmat* h);
/* out, in_dim, bits of a matrix. */
int nh_qmat_shape(const nh_qmat* h, int* out, int* in_dim, int* bits);
/* QMat::bytes (qlinear.rs:287-289): packed codes + f16 norms. */
int64_t nh_qmat_bytes(const nh_qmat* h);
/* The archive-layout codes and norms back on the host (for .cact export and
 * checks): out x in_pad*bits/8 bytes and out x groups f16. */
int nh_qmat_download(const nh_qmat* h, uint8_t* packed, uint64_t packed_bytes, uint16_t* norms, uint64_t norms_count);
/* QMat::row (qlinear.rs:309-323) for each id: out[i][in_dim] = dequantized
 * row ids[i] (embedding / engram lookups). */
int nh_qmat_rows(const nh_qmat* h, const uint32_t* ids, int n, float* out, void* stream);

/* ---- activations (QAct, qlinear.rs:63-72) ------------------------------ */
/* QAct::empty_rows (qlinear.rs:175-178): room for up to `rows` token rows,
 * in the layout of `bits`-bit matrices (2 or 4; a ternary matrix reads
 * the 2-bit layout, nh_qmat_shape reports its bits as 2). */
int nh_qact_new(int rows, int in_dim, int bits, nh_qact** a);
int nh_qact_free(nh_qact* a);
/* QAct::new (qlinear.rs:191-207): x[rows][in_dim] f32 -> per (row, 128-group)
 * FWHT, int8 (amax * K127, round half away), scale.  With a non-NULL f16
 * `norm_scale[in_dim]` the zero-centred RMSNorm is fused in front:
 * zcn16 / norm_apply16 (crates/needle-engine/src/infer.rs:455-473,614-635)
 * as the decode and prefill drivers apply it
 * (crates/needle-engine/src/infer/step.rs:470-479, infer/chunk.rs:187-193). */
int nh_act_prep(nh_qact* a, const float* x, int rows, int in_dim, const uint16_t* norm_scale, void* stream);
/* Current token count of an activation. */
int nh_qact_rows(const nh_qact* a);
/* The int8 codes in the reference's act_pos layout (qlinear.rs:145-147)
 * and the scales, on the host: xq[rows][groups][128], sx[rows][groups]. */
int nh_qact_download(const nh_qact* a, int8_t* xq, uint64_t xq_bytes, float* sx, uint64_t sx_count);

/* ---- products ---------------------------------------------------------- */
/* QMat::matmul_into (qlinear.rs:468-487): y[t*ldy + col0 + r] for every
 * token t and row r.  One token: the decode combine (qlinear.rs:340-350),
 * else the prefill combine (qlinear.rs:353-363) with block = t < rows/4*4
 * (qlinear.rs:397). */
int nh_matmul(const nh_qmat* w, const nh_qact* a, float* y, int ldy, int col0, void* stream);
/* QLinear::apply (qlinear.rs:555-557): y[rows][out] = the products of w
 * with QAct::new(x, rows, in_dim, act_bits) (DEVICE x[rows][in_dim] f32,
 * DEVICE y), the decode combine for one row, the prefill combine for more.
 * The activation staging is allocated and released on `stream` by the call. */
int nh_qlinear_apply(const nh_qmat* w, const float* x, int rows, float* y, void* stream);
/* No counterpart in the reference: nh_qlinear_apply for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  It allocates nothing: the activation staging is a
 * static device array of 270,336 bytes that each GPU the library runs on
 * holds until the process ends.  At most 64 rows and in_dim <= 4096 (32
 * groups); larger inputs return NH_EINVAL.  Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU (other streams,
 * threads or processes) race and must be serialized by the caller.
 * nh_init must have been called for the current device. */
int nh_qlinear_apply_static(const nh_qmat* w, const float* x, int rows, float* y, void* stream);
/* The prefill combine with one block flag per token (1: (norm*cbs)*sx,
 * 0: norm*(cbs*sx)): a batched feed of several <=32-token chunks gives
 * each token its in-chunk flag (crates/needle-engine/src/infer.rs:1105-1132). */
int nh_matmul_flags(const nh_qmat* w, const nh_qact* a, const uint8_t* block, float* y, int ldy, int col0,
                    void* stream);
/* QMat::single_row (qlinear.rs:454-456) for each id: out[i] = row ids[i]
 * against token 0 with the block combine. */
int nh_single_rows(const nh_qmat* w, const nh_qact* a, const uint32_t* ids, int n, float* out, void* stream);
/* Model::head_logits_sparse (crates/needle-engine/src/infer.rs:1145-1166):
 * logits[out_rows] = NEG except the ids, scored with single_row. */
int nh_head_logits_sparse(const nh_qmat* w, const nh_qact* a, const uint32_t* ids, int n, int out_rows,
                          float* logits, void* stream);
/* The exact integer partial sums (qlinear.rs:325-337,356), for the
 * bit-exact check: one token -> int32 lanes[out][groups][4]; more ->
 * int32 totals[rows][out][groups]. */
int nh_debug_partials(const nh_qmat* w, const nh_qact* a, int32_t* out, void* stream);

/* No reference counterpart (measurement): the read floors of the decode
 * product of a 4-bit w with a one-token a.  mode 0 issues exactly the loads
 * the decode GEMV issues (codes, norms, activations, scales), in its grid,
 * with no arithmetic; mode 1 reads the codes and norms as a plain
 * grid-stride stream; mode 2 is mode 0 ending as the product does (a
 * workgroup barrier, then one float per row stored to y[0 .. w's out), a
 * value with no meaning).  Modes 0 and 1 write nothing and ignore y. */
int nh_debug_read_floor(const nh_qmat* w, const nh_qact* a, int mode, float* y, void* stream);

/* ---- archives (QWeights, crates/needle-engine/src/weights.rs:136-148) --- */
/* Weights::from_archive_mode with fast = true (weights.rs:314-467) over the
 * bytes of a .cact archive (Archive::from_raw, crates/needle-core/src/cact.rs:577-583),
 * borrowed for the call only as needle_load borrows them
 * (crates/needle-ffi/src/lib.rs:57-77).  The header, codebook and directory
 * are parsed with the reference's checks (cact.rs:120-131,213-230,593-614),
 * the canonical record order is walked and checked (weights.rs:318-464),
 * and only then is anything uploaded, so a malformed archive returns
 * NH_EINVAL (with the reference's message) even without nh_init.  CQ records
 * upload as nh_qmat_from_cq, f16/f32 matmul records as nh_qmat_from_f32
 * (Cursor::big, weights.rs:113-128).  The matrices are fused as QWeights
 * holds them: q|k|v|gate and out per layer, the mHC pre|post|res rows of
 * each layer, engram key|value per site; engram tables and the embedding
 * stay whole. */
int nh_weights_load(const uint8_t* bytes, uint64_t n, nh_weights** w);
int nh_weights_free(nh_weights* w);
/* The 49 header words in archive order (cact.rs:80-118); copies up to n of
 * them and returns 49. */
int nh_weights_header(const nh_weights* w, uint32_t* words, int n);
#define NH_W_EMBEDDING 0    /* QWeights::embedding (index 0) */
#define NH_W_QKVG 1         /* QWeights::qkvg[layer] */
#define NH_W_OUT 2          /* QWeights::out[layer] */
#define NH_W_PHI 3          /* QWeights::phi[layer] */
#define NH_W_ENGRAM_TABLE 4 /* QWeights::engram_tables[site] */
#define NH_W_ENGRAM_KV 5    /* QWeights::engram_kv[site] */
/* Number of matrices of a kind. */
int nh_weights_count(const nh_weights* w, int kind);
/* A matrix of a kind, owned by w (valid until nh_weights_free). */
int nh_weights_get(const nh_weights* w, int kind, int index, const nh_qmat** m);
/* QWeights::bytes (weights.rs:151-155): packed codes + f16 norms of every matrix. */
int64_t nh_weights_bytes(const nh_weights* w);

/* ---- the model and its sessions (crates/needle-engine/src/model.rs) ---- */
/* Model::quantized over Weights::from_archive_mode(fast = true)
 * (model.rs:248-262) with the native tables (Tables::new,
 * crates/needle-engine/src/infer.rs:869-960): the archive as nh_weights_load
 * reads it, plus its small per-layer weights narrowed to f16
 * (LayerF16::new, infer.rs:905-938), the mHC rows requantized per row
 * (Phi8, infer.rs:850-867), the RoPE tables and gate constants, all in HBM.
 * Bytes are borrowed for the call only (needle_load, crates/needle-ffi/src/
 * lib.rs:57-77).  The decode step covers the Needle-3 geometry family
 * (4 mHC lanes, d_model in (512, 1024], head dims <= 64, engram sub-tables
 * of 128); anything else is NH_EINVAL naming the property. */
int nh_model_load(const uint8_t* bytes, uint64_t n, nh_model** m);
int nh_model_free(nh_model* m);
/* The model's matmul weights (owned by m). */
int nh_model_weights(const nh_model* m, const nh_weights** w);
/* Config::out_rows (crates/needle-core/src/config.rs:299-301): logits per step. */
int nh_model_out_rows(const nh_model* m);
/* Model::session (model.rs:264-280) with room for `cap` positions: the KV
 * caches, tap and engram histories and every activation in one HBM
 * allocation. */
int nh_session_new(const nh_model* m, int cap, nh_session** s);
int nh_session_free(nh_session* s);
/* Session::len (model.rs:72-74). */
int nh_session_len(const nh_session* s);
/* Back to an empty session (Model::session again, without reallocating):
 * no attention span, no cell tracking. */
int nh_session_reset(nh_session* s);
/* Outputs (crates/needle-engine/src/model.rs:150-160): what a feed returns. */
#define NH_OUT_NONE 0        /* nothing: the head is not run */
#define NH_OUT_LAST_LOGITS 1 /* logits of the last position [1][out_rows] */
#define NH_OUT_ALL_LOGITS 2  /* logits of every new position [n][out_rows] (head_logits per row) */
#define NH_OUT_HIDDEN 3      /* final normed hidden state of every new position [n][d_model] */
#define NH_OUT_LAST_HIDDEN 4 /* final normed hidden state of the last position [1][d_model] */
/* Model::forward (model.rs:304-306) on the native path (forward_native,
 * crates/needle-engine/src/infer.rs:1105-1132) with any Outputs: chunks of 32
 * tokens, LastLogits / LastHidden from the last chunk only (infer.rs:
 * 1111-1116), the rows a chunk returns as chunk_job picks them
 * (infer/chunk.rs:331-353).  `out` is DEVICE memory for out_cap floats (or
 * NULL); returns the rows written (ForwardOut::rows), NH_ESMALL when they do
 * not fit.  The session keeps the last returned row's hidden state
 * (NatState::last_hidden) and, for the logits modes, its logits.  Argument
 * errors (bad ids, capacity, a small buffer) leave the session untouched;
 * any failure once feeding has begun (a span the slot map cannot express, a
 * launch error) resets it to empty, keeping its attention span. */
int nh_forward_outputs(nh_session* s, const uint32_t* toks, int n, int outputs, float* out, int64_t out_cap,
                       void* stream);
/* Model::forward_cells (model.rs:330-345): nh_forward_outputs that also
 * returns ForwardOut::cells, the feed's per-depth cells [n][L+1][d_model]
 * (L layers): the lane mean (((x0 + x1) + x2) + x3) * 0.25 of the residual
 * lanes after the embedding (depth 0) and after each layer's mHC write, as
 * the native drivers record them (infer/step.rs:240-243,672-714,
 * infer/chunk.rs:69-70,310, lane_mean infer.rs:1707-1711).  `cells` is
 * DEVICE memory for cells_cap floats (NULL: the cells go only to a tracking
 * session's store); NH_ESMALL when they do not fit.  Returns the rows of
 * `out` as nh_forward_outputs does. */
int nh_forward_cells(nh_session* s, const uint32_t* toks, int n, int outputs, float* out, int64_t out_cap,
                     float* cells, int64_t cells_cap, void* stream);
/* Session::cells = Some(vec![]) (on) or None (off) (model.rs:60-62): a
 * tracking session appends the cells of every nh_forward, nh_forward_outputs,
 * nh_forward_cells and nh_generate_greedy feed to its store (step.rs:730-732,
 * chunk.rs:353-355), which rollback, rewind_zeroed and a prefill re-feed
 * truncate to the session's length (model.rs:108-110,118-121,
 * infer.rs:1096-1099).  nh_prefill appends none: prefill_native runs its
 * feeds with want_cells = false (infer.rs:1089,1100).  Tracking starts at an
 * empty session (NH_EINVAL otherwise); the first call allocates the store,
 * cap x (L+1) x d_model floats in HBM.  nh_session_reset turns it off. */
int nh_session_track_cells(nh_session* s, int on);
/* The number of cell rows a tracking session holds (Session::cells.len() /
 * ((L+1) d_model)); NH_EINVAL when it does not track them. */
int nh_session_cell_rows(const nh_session* s);
/* Rows row0 .. row0 + n - 1 of a tracking session's cells into DEVICE
 * dst[n][L+1][d_model]; returns n. */
int nh_session_cells(const nh_session* s, int row0, int n, float* dst, void* stream);
/* Model::prefill on the native path (prefill_native, infer.rs:1078-1101):
 * with an attention span, a position in max(end - ring, sink) .. len whose KV
 * slot another position holds now starts a re-feed from there with the
 * conv history zeroed; else as nh_forward_outputs. */
int nh_prefill(nh_session* s, const uint32_t* toks, int n, int outputs, float* out, int64_t out_cap, void* stream);
/* Session::clone (model.rs:53-55): a new session with a copy of every cache
 * (one device-to-device copy on `stream`, then a synchronization).  A source
 * whose bounded wait gave up and has not been reported yet is refused
 * (NH_EDEVICE; the source's next feed reports it). */
int nh_session_clone(const nh_session* s, void* stream, nh_session** out);
/* Session::attend = Some((sink, ring)) (model.rs:62-66; ring 0: None): every
 * query sees the first `sink` positions and the last `ring`; positions past
 * the sink share `ring` KV slots (slot_of, infer.rs:1749-1756) and a slot map
 * (mark_slots / key_ranges, infer.rs:1770-1826) skips a position whose slot
 * another has taken since.  Any ring is taken; with a ring shorter than 32 a
 * feed longer than the ring is refused (NH_EINVAL, the session untouched):
 * two rows of its chunk would share a KV slot, where the reference's team
 * members race, and a row could see no key at all. */
int nh_session_set_attend(nh_session* s, int sink, int ring);
/* Session::rollback (model.rs:81-113, NatState::rollback infer.rs:1053-1071):
 * drop the last n <= 32 positions without recomputing; the KV slots and the
 * slot map keep what they hold. */
int nh_session_rollback(nh_session* s, int n);
/* Session::rewind_zeroed (model.rs:115-121, infer.rs:1039-1051): forget
 * positions len.. as the engine's context-overflow re-feed does: the KV cache
 * keeps what it holds, the conv history and the RoPE state start over. */
int nh_session_rewind_zeroed(nh_session* s, int len);
/* No reference counterpart (a test hook): the polls a bounded in-kernel
 * wait makes before it gives up (default 1 << 20, about 30 ms).  A wait
 * that gives up lets its kernel end and marks the session.  Each feed ends
 * by queueing a copy of that mark to pinned host memory; the first
 * nh_forward*, nh_prefill or nh_generate_greedy call made after the stream
 * has passed the copy (any call after a synchronization, and
 * nh_generate_greedy itself, which waits for its own) returns NH_EDEVICE
 * and resets the session.  No call waits for earlier work to check it.
 * 0 makes every such wait give up at once, for tests of that path. */
int nh_session_debug_spin_limit(nh_session* s, int limit);
/* No reference counterpart (the reference's calls are synchronous and a
 * failure surfaces in the call that caused it): waits for everything queued
 * on `stream` and reports a bounded wait that gave up in the session's feeds
 * so far (NH_EDEVICE, the session reset, as above), so a caller that wants
 * the failure attributed to the feed that caused it calls this after the
 * feed.  NH_OK when none did. */
int nh_session_sync(nh_session* s, void* stream);
/* No reference counterpart (a test hook for the failure path): the
 * `after`-th feed from now (each nh_forward* / nh_prefill chunk group or
 * greedy step counts one) fails with NH_EDEVICE before it launches anything,
 * as a feed does whose attention span the slot map cannot express; 0 turns
 * it off. */
int nh_session_debug_fail_feed(nh_session* s, int after);
/* NatState::last_hidden (infer.rs:1014-1016) into DEVICE h[d_model]. */
int nh_session_last_hidden(const nh_session* s, float* h, void* stream);
/* Model::head_logits (infer.rs:1135-1141) of the session's last hidden state
 * into DEVICE logits[out_rows]. */
int nh_session_head_logits(nh_session* s, float* logits, void* stream);
/* Model::head_logits_sparse (infer.rs:1145-1166) of the session's last hidden
 * state: DEVICE ids[n], DEVICE logits[out_rows] (NEG off the ids), as the
 * agent's sparse decode scores its candidates (agent.rs:398-409). */
int nh_session_head_logits_sparse(nh_session* s, const uint32_t* ids, int n, float* logits, void* stream);
/* Model::forward (model.rs:304-306) with Outputs::LastLogits for HOST token
 * ids, fed as forward_native feeds them (crates/needle-engine/src/infer.rs:
 * 1105-1132): chunks of 32 tokens through chunk_job
 * (crates/needle-engine/src/infer/chunk.rs:32-358, the products over the
 * chunk's rows with the prefill combine), a single-token chunk through
 * step_native (crates/needle-engine/src/infer/step.rs:171-760).  `logits`
 * (DEVICE, out_rows floats, or NULL) receives the last token's; with n = 0
 * they are the logits the session already holds (NH_EINVAL without any). */
int nh_forward(nh_session* s, const uint32_t* toks, int n, float* logits, void* stream);
/* generate::argmax (crates/needle-engine/src/generate.rs:42-50) on the
 * device: the first index of the maximum of DEVICE x[n] into DEVICE dst[0];
 * NaNs never win, and a NaN x[0] gives 0, as the reference's loop does. */
int nh_argmax(const float* x, int n, uint32_t* dst, void* stream);
/* The greedy loop of generate (crates/needle-engine/src/generate.rs:87-139)
 * at temperature 0, on the device: `steps` times argmax of the current
 * logits (generate.rs:42-50, the first maximum), then a step on that token.
 * The picked ids land in HOST `out` at the end (one synchronization); the
 * last step's logits in `logits` (DEVICE, or NULL).  No stop token: the
 * caller cuts at EOS.  A step that fails resets the session to empty
 * (keeping its attention span), as a failed nh_forward_outputs does. */
int nh_generate_greedy(nh_session* s, int steps, uint32_t* out, float* logits, void* stream);

/* ---- seeded inputs (host) ---------------------------------------------- */
/* jax.random.normal for float32 from a threefry key, as
 * crates/needle-train/src/rand.rs:205-217 computes it, into host memory. */
int nh_normal(uint32_t key0, uint32_t key1, uint64_t n, float* out);
/* jax.random.split (rand.rs:161-163): out = {key0, key1, sub0, sub1}. */
int nh_split(uint32_t key0, uint32_t key1, uint32_t* out4);

#ifdef __cplusplus
}
#endif
#endif
