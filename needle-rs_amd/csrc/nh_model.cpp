// The Needle-3 model and its decoding sessions on the GPU: Model::quantized
// plus the native tables (crates/needle-engine/src/model.rs:248-262,
// crates/needle-engine/src/infer.rs:869-960), Model::session
// (model.rs:264-280) with the native state in HBM (NatState,
// infer.rs:966-1071), and Model::forward over single-token steps
// (step_native, crates/needle-engine/src/infer/step.rs:171-760).
//
// nh_model_load reads the archive with the matmul loader, then uploads the
// small per-layer weights narrowed to f16 as LayerF16::new does
// (infer.rs:905-938), the mHC rows requantized per row (Phi8,
// infer.rs:850-867, dequantized on the device with QMat::row), the RoPE
// tables powf / sincosf (Tables::new, infer.rs:942-947) and the gate
// constants.  A session is one HBM arena: residual lanes, KV caches, tap
// and engram histories, activation buffers and logits.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/needle_hip.h"
#include "nh_forward.h"
#include "nh_internal.h"

namespace {

constexpr size_t ALIGN = 256;

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int fail(int code, const std::string& msg) {
    nh::set_error(msg);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(NH_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

#define NH_TRY(call, what)                                   \
    do {                                                     \
        hipError_t e_ = (call);                              \
        if (e_ != hipSuccess) return hip_fail(e_, what);     \
    } while (0)

// f16::from_f32 of the `half` crate: round to nearest even, overflow to
// infinity, subnormals kept, NaN stays NaN.
uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
    const int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const int shift = 14 - e;
        const uint32_t half = 1u << (shift - 1);
        uint32_t r = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1);
        if (rem > half || (rem == half && (r & 1))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) ++r;
    return (uint16_t)(sign | r);
}

// Host staging of one device buffer: 256-byte aligned sections.
struct Arena {
    std::vector<uint8_t> host;
    size_t put(const void* p, size_t bytes) {
        const size_t off = round_up(host.size(), ALIGN);
        host.resize(off + bytes, 0);
        if (bytes && p) memcpy(host.data() + off, p, bytes);
        return off;
    }
    size_t reserve(size_t bytes) { return put(nullptr, bytes); }
};

// A device arena of zeroed sections, laid out before allocation.
struct Layout {
    size_t size = 0;
    size_t take(size_t bytes) {
        const size_t off = round_up(size, ALIGN);
        size = off + std::max<size_t>(bytes, 1);
        return off;
    }
};

int key_chunk_count(int n, int nkv) {
    // key_chunks (infer.rs:2093-2101)
    int k = std::max(1, 2 * 4 / nkv);
    int c = (n + 255) / 256;
    if (k * 64 <= n && c < k) c = k;
    c = std::max(c, 1);
    const int chunk = ((n + c - 1) / c + 15) / 16 * 16;
    return chunk ? (n + chunk - 1) / chunk : 0;
}

}  // namespace

struct nh_model {
    nh_weights* w = nullptr;
    uint32_t header[49];
    nh::Dims dims{};
    nh::Globals glob{};
    nh::BeginArgs begin{};
    std::vector<nh::LayerDev> layers;
    std::vector<const nh_qmat*> qkvg, out, ekv;
    nh_qmat* head = nullptr;  // the embedding's first out_rows rows (shares its memory)
    int head_bits = 4;
    void* d_small = nullptr;

    ~nh_model() {
        if (d_small) (void)hipFree(d_small);
        delete head;
        nh_weights_free(w);
    }
};

struct nh_session {
    const nh_model* m = nullptr;
    nh::Dims dims{};
    nh::SessDev S{};
    void* d_buf = nullptr;
    size_t bytes = 0;
    int len = 0;
    bool have_logits = false;  // S.logits holds the logits of position len - 1
    bool have_hidden = false;  // S.last_hid holds NatState::last_hidden
    // Host mirrors of the reference's session state: the rows LayerState::
    // hist holds (the same in every layer, infer.rs:968-980), the length of
    // NatState::rope (infer.rs:1716-1747), Session::attend and the slot map
    // (model.rs:62-66, infer.rs:1000-1006), and the token ids.
    int hrows = 0;
    int rope_n = 0;
    int sink = 0, ring = 0;
    std::vector<int64_t> slot_pos;
    std::vector<uint32_t> toks;
    nh_qact a_in{}, a_att{};
    std::vector<nh_qact> a_eng;
    // The status word as the stream last copied it (pinned), behind
    // ev_status; pending while that copy has not been read.
    int32_t* h_status = nullptr;
    hipEvent_t ev_status = nullptr;
    bool status_pending = false;
    // Session::cells (model.rs:60-62): when tracked, the cell rows the feeds
    // appended, [ncells][layers + 1][d] in a buffer of cap rows.
    bool track_cells = false;
    float* d_cells = nullptr;
    int ncells = 0;
    int fail_in = 0;  // test hook: the feed that fails on purpose (0: none)

    size_t cell_floats() const { return (size_t)(dims.layers + 1) * dims.d; }
    ~nh_session() {
        if (ev_status) (void)hipEventDestroy(ev_status);
        if (h_status) (void)hipHostFree(h_status);
        if (d_cells) (void)hipFree(d_cells);
        if (d_buf) (void)hipFree(d_buf);
    }
};

namespace {

// The geometry the decode step is written for, from the header and the
// loaded matrices; an error names the first unsupported property.
int check_geometry(nh_model* m, const nh::ArchiveSmall& sm) {
    const uint32_t* h = m->header;
    nh::Dims& D = m->dims;
    D.vocab = (int)h[5];
    D.out_rows = h[6] > 0 ? (int)h[6] : (int)h[5];  // Config::out_rows (config.rs:299-301)
    D.d = (int)h[7];
    D.nh = (int)h[8];
    D.nkv = (int)h[9];
    D.layers = (int)h[10];
    D.qk = (int)h[11];
    D.vd = (int)h[12];
    D.lanes = (int)h[15];
    D.taps = (int)h[19];
    const int window = (int)h[16];
    const uint64_t gmask = (uint64_t)h[17] | ((uint64_t)h[18] << 32);
    const int norders = (int)h[26];
    const int tables = (int)h[22];
    D.sites = (int)h[31];
    if (D.lanes != nh::MHC_LANES) return fail(NH_EINVAL, "the decode step is written for 4 mHC lanes");
    if (D.d <= nh::FWD_MAX_D / 2 || D.d > nh::FWD_MAX_D || D.d % 32 != 0)
        return fail(NH_EINVAL, "the decode step needs d_model in (512, 1024], a multiple of 32 (hada_n 1024)");
    if (D.nh <= 0 || D.nkv <= 0 || D.nh % D.nkv != 0 || D.nh + 2 * D.nkv > nh::MAX_UNITS)
        return fail(NH_EINVAL, "the decode step needs heads + 2 kv heads <= 16, heads a multiple of kv heads");
    if (D.qk <= 0 || D.qk % 16 != 0 || D.qk > nh::MAX_HEAD_DIM || D.vd <= 0 || D.vd % 4 != 0 ||
        D.vd > nh::MAX_HEAD_DIM)
        return fail(NH_EINVAL, "the decode step needs qk a multiple of 16 and vd a multiple of 4, both <= 64");
    if (D.nh * D.vd > nh::FWD_MAX_D) return fail(NH_EINVAL, "heads x vd above 1024");
    if (D.layers > 64) return fail(NH_EINVAL, "more than 64 layers");
    if (D.out_rows <= 0 || D.out_rows > D.vocab) return fail(NH_EINVAL, "out_vocab above the vocabulary");
    const int qd = D.nh * D.qk, kd = D.nkv * D.qk, vdim = D.nkv * D.vd;
    D.W = qd + kd + vdim;
    D.nq = D.W + D.nh * D.vd;
    if (D.taps <= 0) return fail(NH_EINVAL, "the decode step needs qkv conv taps");
    if (D.taps > nh::DG_MAX_TAPS)
        return fail(NH_EINVAL, "the decode step takes at most " + std::to_string(nh::DG_MAX_TAPS) + " qkv conv taps");
    // every row the reference's history can hold (rows <= 2 keep at rest,
    // keep = taps - 1 + ROLLBACK, step.rs:706-712), plus a feed's rows
    D.hist_slots = 2 * (D.taps - 1 + nh::ROLLBACK) + nh::FWD_ROWS;
    // engram geometry (config.rs:273-288 with heads = tables / orders, cact.rs:191)
    if (D.sites > nh::MAX_SITES || norders > 4) return fail(NH_EINVAL, "corrupt engram geometry");
    if (D.sites > 0) {
        if (norders <= 0 || tables <= 0 || tables % norders != 0 || tables > nh::MAX_TABLES)
            return fail(NH_EINVAL, "engram tables do not split over the orders");
        D.eheads = tables / norders;
        D.ntab = tables;
        D.sub = D.d / (norders * D.eheads);
        if (D.sub != nh::GROUP || D.ntab * D.sub > D.d)
            return fail(NH_EINVAL, "the decode step needs engram sub-tables of 128");
        D.seed_stride = h[25] > 0 ? (int)h[25] : D.eheads;
        D.slots = (int)h[20];
        if (D.slots <= 0) return fail(NH_EINVAL, "engram_slots is zero");
        int dil = 1;
        for (int i = 0; i < norders; ++i) {
            D.orders[i] = (int)h[27 + i];
            if (D.orders[i] <= 0 || D.orders[i] > 64) return fail(NH_EINVAL, "engram order out of range");
            dil = std::max(dil, D.orders[i]);
        }
        D.dilation = dil;  // Config::engram_dilation (config.rs:286-288)
    }
    // matrices
    const nh_qmat* emb = nullptr;
    nh_weights_get(m->w, NH_W_EMBEDDING, 0, &emb);
    if (emb->m.in_dim != D.d || emb->m.out != D.vocab) return fail(NH_EINVAL, "embedding shape");
    for (int l = 0; l < D.layers; ++l) {
        const nh_qmat *q = nullptr, *o = nullptr, *p = nullptr;
        nh_weights_get(m->w, NH_W_QKVG, l, &q);
        nh_weights_get(m->w, NH_W_OUT, l, &o);
        nh_weights_get(m->w, NH_W_PHI, l, &p);
        if (q->m.out != D.nq || q->m.in_dim != D.d) return fail(NH_EINVAL, "q|k|v|gate shape");
        if (o->m.out != D.d || o->m.in_dim != D.nh * D.vd) return fail(NH_EINVAL, "out projection shape");
        if (p->m.out != nh::MHC_COLS || p->m.in_dim != nh::MHC_LANES * D.d) return fail(NH_EINVAL, "mHC phi shape");
        m->qkvg.push_back(q);
        m->out.push_back(o);
    }
    for (int s = 0; s < D.sites; ++s) {
        const nh_qmat *t = nullptr, *kv = nullptr;
        nh_weights_get(m->w, NH_W_ENGRAM_TABLE, s, &t);
        nh_weights_get(m->w, NH_W_ENGRAM_KV, s, &kv);
        if (t->m.in_dim != D.sub || t->m.out != D.ntab * D.slots) return fail(NH_EINVAL, "engram table shape");
        if (kv->m.in_dim != D.d || kv->m.out != 2 * D.d) return fail(NH_EINVAL, "engram key|value shape");
        const int site = (int)h[32 + s];
        if (site < 0 || site >= D.layers) return fail(NH_EINVAL, "engram site past the last layer");
        m->ekv.push_back(kv);
    }
    // small tensors: the lengths the step reads
    const size_t d = D.d;
    auto need = [&](const std::vector<float>& v, size_t n, const char* what) -> int {
        if (v.size() < n) return fail(NH_EINVAL, std::string(what) + " is shorter than the step reads");
        return NH_OK;
    };
    for (int l = 0; l < D.layers; ++l) {
        const auto& L = sm.layer[l];
        int rc = NH_OK;
        if (!rc) rc = need(L[nh::S_NORM_IN], d, "norm_in");
        if (!rc && D.taps > 0) rc = need(L[nh::S_Q_TAPS], (size_t)D.taps * qd, "q taps");
        if (!rc && D.taps > 0) rc = need(L[nh::S_K_TAPS], (size_t)D.taps * kd, "k taps");
        if (!rc && D.taps > 0) rc = need(L[nh::S_V_TAPS], (size_t)D.taps * vdim, "v taps");
        if (!rc) rc = need(L[nh::S_Q_NORM], D.qk, "q_norm");
        if (!rc) rc = need(L[nh::S_K_NORM], D.qk, "k_norm");
        if (!rc) rc = need(L[nh::S_POST_NORM], d, "post_attn_norm");
        if (!rc) rc = need(L[nh::S_PRE_HADA], d, "pre_hada_norm");
        if (!rc) rc = need(L[nh::S_D1], d, "d1");
        if (!rc) rc = need(L[nh::S_D2], nh::HADA_N, "d2");
        if (!rc) rc = need(L[nh::S_B2], nh::HADA_N, "b2");
        if (!rc) rc = need(L[nh::S_D3], nh::HADA_N, "d3");
        if (!rc) rc = need(L[nh::S_D4], d, "d4");
        if (!rc) rc = need(L[nh::S_COND_V], d * nh::COND_RANK, "cond_v");
        if (!rc) rc = need(L[nh::S_COND_U], (size_t)nh::COND_RANK * nh::HADA_N, "cond_u");
        for (int k = 0; k < 6 && !rc; ++k) rc = need(L[nh::S_KRON0 + k], nh::HADA_N, "Kronecker factor");
        if (rc) return rc;
    }
    const size_t L = D.layers;
    if (need(sm.mhc[0], L, "mhc a_pre") || need(sm.mhc[1], L, "mhc a_post") || need(sm.mhc[2], L, "mhc a_res") ||
        need(sm.mhc[3], L * 4, "mhc b_pre") || need(sm.mhc[4], L * 4, "mhc b_post") ||
        need(sm.mhc[5], L * 16, "mhc b_res") || need(sm.final_norm, d, "final_norm"))
        return NH_EINVAL;
    for (const auto* perm : {&sm.perm1, &sm.perm2})
        for (float v : *perm)
            if (!(v >= 0.0f && v < (float)nh::HADA_N) || v != floorf(v))
                return fail(NH_EINVAL, "Hadamard permutation entry out of range");
    for (int s = 0; s < D.sites; ++s)
        if (need(sm.etaps[s], (size_t)nh::ENGRAM_TAPS * d, "engram taps")) return NH_EINVAL;
    (void)window;
    (void)gmask;
    return NH_OK;
}

int build_model(nh_model* m, const nh::ArchiveSmall& sm) {
    nh::Dims& D = m->dims;
    const uint32_t* h = m->header;
    const int window = (int)h[16];
    const uint64_t gmask = (uint64_t)h[17] | ((uint64_t)h[18] << 32);
    const int nc = nh::MHC_LANES * D.d;
    Arena A;
    struct LayerOff {
        size_t t[nh::SMALL_KINDS];
        size_t phi_q, phi_s;
    };
    std::vector<LayerOff> off(D.layers);
    auto put16 = [&](const std::vector<float>& v) {
        std::vector<uint16_t> b(v.size());
        for (size_t i = 0; i < v.size(); ++i) b[i] = f32_to_f16(v[i]);
        return A.put(b.data(), b.size() * 2);
    };
    // The tables of the layer kernel, as one block per layer: the six
    // Kronecker factors and cond_v [d][8] (staged into LDS), then cond_u
    // by column, [hada_n][8] (f16; thread t reads its column's 16 bytes).
    std::vector<size_t> stage(D.layers);
    for (int l = 0; l < D.layers; ++l) {
        for (int k = 0; k < nh::SMALL_KINDS; ++k) off[l].t[k] = put16(sm.layer[l][k]);
        std::vector<float> blk;
        for (int k = 0; k < 6; ++k) {
            const auto& f = sm.layer[l][nh::S_KRON0 + k];
            blk.insert(blk.end(), f.begin(), f.begin() + nh::HADA_N);
        }
        const auto& cv = sm.layer[l][nh::S_COND_V];
        blk.insert(blk.end(), cv.begin(), cv.begin() + (size_t)D.d * nh::COND_RANK);
        const auto& cu = sm.layer[l][nh::S_COND_U];
        for (int t = 0; t < nh::HADA_N; ++t)
            for (int k = 0; k < nh::COND_RANK; ++k) blk.push_back(cu[(size_t)k * nh::HADA_N + t]);
        stage[l] = put16(blk);
        off[l].phi_q = A.reserve((size_t)nh::MHC_COLS * nc);
        off[l].phi_s = A.reserve(nh::MHC_COLS * 4);
    }
    const size_t o_final = A.put(sm.final_norm.data(), (size_t)D.d * 4);
    std::vector<int32_t> p1(nh::HADA_N), p2(nh::HADA_N);
    for (int i = 0; i < nh::HADA_N; ++i) p1[i] = (int32_t)sm.perm1[i], p2[i] = (int32_t)sm.perm2[i];
    const size_t o_p1 = A.put(p1.data(), p1.size() * 4), o_p2 = A.put(p2.data(), p2.size() * 4);
    // Tables::new (infer.rs:942-947): freq = lpowf(theta, i * (-2 / qk)),
    // (sd, cd) = sincosf(freq), both f64 libm results rounded once as the
    // reference computes them off Apple targets (infer.rs:84-101).
    float theta;
    memcpy(&theta, &h[48], 4);
    const int half = D.qk / 2;
    std::vector<float> freq(half), sd(half), cd(half);
    const float coef = -2.0f / (float)D.qk;
    for (int i = 0; i < half; ++i) {
        const float f = (float)pow((double)theta, (double)((float)i * coef));
        double sv, cv;
        sincos((double)f, &sv, &cv);
        freq[i] = f;
        sd[i] = (float)sv;
        cd[i] = (float)cv;
    }
    const size_t o_fr = A.put(freq.data(), half * 4);
    const size_t o_sd = A.put(sd.data(), half * 4), o_cd = A.put(cd.data(), half * 4);
    std::vector<float> etaps;
    for (int s = 0; s < D.sites; ++s)
        etaps.insert(etaps.end(), sm.etaps[s].begin(), sm.etaps[s].begin() + (size_t)nh::ENGRAM_TAPS * D.d);
    const size_t o_et = A.put(etaps.data(), etaps.size() * 4);
    const size_t o_ids = A.reserve(nh::MHC_COLS * 4);

    NH_TRY(hipMalloc(&m->d_small, A.host.size()), "model tables allocation");
    NH_TRY(hipMemcpy(m->d_small, A.host.data(), A.host.size(), hipMemcpyHostToDevice), "model tables upload");
    uint8_t* base = (uint8_t*)m->d_small;

    // Phi8 per layer: QMat::row of the fused pre|post|res rows, then quant_i8.
    {
        std::vector<uint32_t> ids(nh::MHC_COLS);
        for (int i = 0; i < nh::MHC_COLS; ++i) ids[i] = i;
        NH_TRY(hipMemcpy(base + o_ids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice), "phi ids");
        float* rows = nullptr;
        NH_TRY(hipMalloc(&rows, (size_t)nh::MHC_COLS * nc * 4), "phi rows");
        hipError_t e = hipSuccess;
        for (int l = 0; l < D.layers && e == hipSuccess; ++l) {
            const nh_qmat* phi = nullptr;
            nh_weights_get(m->w, NH_W_PHI, l, &phi);
            e = nh::launch_rows(phi, (const uint32_t*)(base + o_ids), nh::MHC_COLS, rows, nullptr);
            if (e == hipSuccess)
                e = nh::fwd_phi8(rows, nh::MHC_COLS, nc, (int8_t*)(base + off[l].phi_q), (float*)(base + off[l].phi_s),
                                 nullptr);
        }
        if (e == hipSuccess) e = hipDeviceSynchronize();
        (void)hipFree(rows);
        NH_TRY(e, "Phi8");
    }

    m->glob.final_norm = (const float*)(base + o_final);
    m->glob.perm1 = (const int32_t*)(base + o_p1);
    m->glob.perm2 = (const int32_t*)(base + o_p2);
    m->glob.freq = (const float*)(base + o_fr);
    m->glob.sd = (const float*)(base + o_sd);
    m->glob.cd = (const float*)(base + o_cd);
    m->glob.etaps = (const float*)(base + o_et);

    std::vector<int> site_of(D.layers, -1);
    for (int s = 0; s < D.sites; ++s) site_of[h[32 + s]] = s;
    for (int l = 0; l < D.layers; ++l) {
        nh::LayerDev L{};
        auto p16 = [&](int k) { return (const uint16_t*)(base + off[l].t[k]); };
        L.stage = (const uint16_t*)(base + stage[l]);
        L.d1 = p16(nh::S_D1), L.d2 = p16(nh::S_D2), L.b2 = p16(nh::S_B2), L.d3 = p16(nh::S_D3), L.d4 = p16(nh::S_D4);
        L.norm_in = p16(nh::S_NORM_IN), L.post_norm = p16(nh::S_POST_NORM), L.pre_hada = p16(nh::S_PRE_HADA);
        L.q_taps = p16(nh::S_Q_TAPS), L.k_taps = p16(nh::S_K_TAPS), L.v_taps = p16(nh::S_V_TAPS);
        L.q_norm = p16(nh::S_Q_NORM), L.k_norm = p16(nh::S_K_NORM);
        L.phi_q = (const int8_t*)(base + off[l].phi_q);
        L.phi_s = (const float*)(base + off[l].phi_s);
        L.a_pre = sm.mhc[0][l], L.a_post = sm.mhc[1][l], L.a_res = sm.mhc[2][l];
        // The attention output gate 1 / (lexpf(-attn_gate) + 1) (step.rs:582).
        const float g = sm.layer[l][nh::S_ATTN_GATE][0];
        L.ga = 1.0f / ((float)exp((double)-g) + 1.0f);
        for (int j = 0; j < 4; ++j) L.b_pre[j] = sm.mhc[3][l * 4 + j], L.b_post[j] = sm.mhc[4][l * 4 + j];
        for (int j = 0; j < 16; ++j) L.b_res[j] = sm.mhc[5][l * 16 + j];
        L.site = site_of[l];
        L.index = l;
        L.lane = l % D.lanes;
        L.window = (window > 0 && !((gmask >> l) & 1)) ? window : 0;
        m->layers.push_back(L);
    }

    const nh_qmat* emb = nullptr;
    nh_weights_get(m->w, NH_W_EMBEDDING, 0, &emb);
    m->begin.emb = {emb->d_codes, emb->d_norms, emb->d_fsel, emb->m.out, emb->m.groups, emb->m.bits};
    for (int s = 0; s < D.sites; ++s) {
        const nh_qmat* t = nullptr;
        nh_weights_get(m->w, NH_W_ENGRAM_TABLE, s, &t);
        m->begin.tab[s] = {t->d_codes, t->d_norms, t->d_fsel, t->m.out, t->m.groups, t->m.bits};
        m->begin.eng_bits[s] = m->ekv[s]->m.bits;
    }
    m->head = new nh_qmat();
    m->head->m = emb->m;
    m->head->resident = true;
    m->head->m.out = D.out_rows;
    m->head->m.out_pad = (int)round_up(D.out_rows, nh::TILE_ROWS);
    m->head->d_codes = emb->d_codes;
    m->head->d_norms = emb->d_norms;
    m->head->d_fsel = emb->d_fsel;
    m->head_bits = emb->m.bits;
    return NH_OK;
}

// One product over the feed's rows: the decode combine for one row, the
// prefill combine (block = i < t / 4 * 4) for more (QMat::matmul_into,
// qlinear.rs:468-487).
// `flags`: the block flag of each row when they come from several chunks
// (null: one chunk, block = i < t / 4 * 4).
hipError_t product(const nh_qmat* w, nh_qact* a, int rows, float* y, int ldy, const uint8_t* flags, hipStream_t st) {
    a->rows = rows;
    return rows == 1 ? nh::launch_gemv(w, a, y, 0, nullptr, st) : nh::launch_gemm(w, a, flags, y, ldy, 0, nullptr, st);
}

// slot_of (crates/needle-engine/src/infer.rs:1749-1756).
int slot_of(const nh_session* s, int p) { return (s->ring > 0 && p >= s->sink) ? (p - s->sink) % s->ring + s->sink : p; }

// mark_slots (infer.rs:1770-1779).
void mark_slots(nh_session* s, int p0, int end) {
    for (int p = p0; p < end; ++p) {
        const int sl = slot_of(s, p);
        if ((int)s->slot_pos.size() <= sl) s->slot_pos.resize(sl + 1, -1);
        s->slot_pos[sl] = p;
    }
}

bool live(const nh_session* s, int p) {
    const int sl = slot_of(s, p);
    return sl < (int)s->slot_pos.size() && s->slot_pos[sl] == p;
}

// The span's keys for a feed ending at `end` (key_ranges, infer.rs:1781-1826):
// the live runs of [0, sink) and [max(end - ring, sink), end), and per row
// the reference's own run count, which it asserts stays within KEY_RUNS
// (16, infer.rs:1760,1806-1808).
int span_keys(const nh_session* s, const nh::Dims& D, const std::vector<nh::LayerDev>& layers, int p0, int end,
              nh::KeySpan* K) {
    *K = nh::KeySpan{};
    K->end = end;
    const int b0 = std::max(end - s->ring, s->sink);
    auto scan = [&](int lo, int hi) -> int {
        int a = -1;
        for (int p = lo; p <= hi; ++p) {
            const bool ok = p < hi && live(s, p);
            if (ok && a < 0) a = p;
            if (!ok && a >= 0) {
                if (K->nrun == nh::SPAN_RUNS) return fail(NH_EINVAL, "attention span: too many runs of live keys");
                K->lo[K->nrun] = a, K->hi[K->nrun] = p, ++K->nrun, a = -1;
            }
        }
        return NH_OK;
    };
    if (int rc = scan(0, std::min(s->sink, end))) return rc;
    if (int rc = scan(std::max(b0, std::min(s->sink, end)), end)) return rc;
    // the reference's runs per query row: its coarse ranges cut by liveness
    std::vector<int> windows;
    for (const auto& L : layers)
        if (std::find(windows.begin(), windows.end(), L.window) == windows.end()) windows.push_back(L.window);
    for (int pos = p0; pos < end; ++pos)
        for (int w : windows) {
            const int lo = (w > 0 && pos + 1 > w) ? pos + 1 - w : 0;
            const int ranges[2][2] = {{lo, std::max(lo, std::min(s->sink, pos + 1))},
                                      {std::min(b0, pos + 1), pos + 1}};
            int runs = 0;
            for (const auto& r : ranges) {
                bool open = false;
                for (int p = r[0]; p < r[1]; ++p) {
                    const bool ok = live(s, p);
                    if (ok && !open) ++runs;
                    open = ok;
                }
            }
            if (runs > 16) return fail(NH_EINVAL, "attention span: a query sees more than 16 key runs");
        }
    (void)D;
    return NH_OK;
}

// Rows an output mode returns for a feed of t tokens (chunk.rs:331-335).
int out_rows_of(int outputs, int t) {
    return outputs == NH_OUT_NONE ? 0 : (outputs == NH_OUT_ALL_LOGITS || outputs == NH_OUT_HIDDEN) ? t : 1;
}

int out_width(const nh_session* s, int outputs) {
    return (outputs == NH_OUT_HIDDEN || outputs == NH_OUT_LAST_HIDDEN) ? s->dims.d : s->dims.out_rows;
}

// One feed at positions s->len ..: step_native for one token, chunk_job for
// a chunk of up to 32 (forward_native, infer.rs:1105-1132), or several whole
// chunks of at least two tokens each (t <= BATCH_ROWS) as one pass through
// the layers with each row keeping its chunk's arithmetic (chunk c = rows
// 32c ..: its rows' block flags, nested key chunks and sincosf RoPE rows;
// the causal keys of a row do not depend on how the prompt was cut).
// `outputs` picks what the rows give (chunk.rs:331-353, step.rs:715-729),
// written to `out` (device, rows x width, or null to keep only the
// session's copies); for several chunks the Last* modes mean the last
// chunk's last row, All* every row.  `cells` (device, or null): the rows'
// cells [t][layers + 1][d] (step.rs:240-243,672-714, chunk.rs:69-70,310).
// pick: the greedy loop's step, whose token is the argmax of the previous
// step's logits, taken by the feed's first kernel.
int feed(nh_session* s, int t, int outputs, float* out, float* cells, hipStream_t st, bool pick = false) {
    const nh_model* m = s->m;
    nh::SessDev S = s->S;
    S.cells = cells;
    const int p0 = s->len;
    const uint8_t* flags = t > nh::FWD_ROWS ? S.flags : nullptr;
    nh::Dims D = s->dims;
    D.hist_lo = p0 - s->hrows;
    D.rope_prev = t == 1 && s->rope_n > 0;
    D.sink = s->sink;
    D.ring = s->ring;
    mark_slots(s, p0, p0 + t);
    if (s->fail_in > 0 && --s->fail_in == 0)
        return fail(NH_EDEVICE, "a feed failed on purpose (nh_session_debug_fail_feed)");
    nh::KeySpan span{};
    const nh::KeySpan* sp = nullptr;
    if (s->ring > 0) {
        if (int rc = span_keys(s, D, m->layers, p0, p0 + t, &span)) return rc;
        sp = &span;
    }
    NH_TRY(nh::fwd_begin(D, m->glob, S, m->begin, p0, t, st, pick), "feed begin");
    if (t == 1 && D.sites > 1 && nh::gemv_batchable(m->ekv.data(), D.sites)) {
        // every site's key | value product in one launch
        const nh_qact* acts[nh::GEMV_BATCH_MAX];
        float* ys[nh::GEMV_BATCH_MAX];
        for (int e = 0; e < D.sites; ++e) {
            s->a_eng[e].rows = 1;
            acts[e] = &s->a_eng[e];
            ys[e] = S.ekv + (size_t)e * nh::BATCH_ROWS * 2 * D.d;
        }
        NH_TRY(nh::launch_gemv_batch(m->ekv.data(), acts, ys, D.sites, st), "engram kv");
    } else {
        // several rows: every site's product in one GEMM launch when they
        // share shape and tables, else one launch each
        const nh_qact* acts[nh::MAX_SITES];
        float* ys[nh::MAX_SITES];
        for (int e = 0; e < D.sites; ++e) {
            s->a_eng[e].rows = t;
            acts[e] = &s->a_eng[e];
            ys[e] = S.ekv + (size_t)e * nh::BATCH_ROWS * 2 * D.d;
        }
        if (t > 1 && D.sites > 1 && nh::gemm_batchable(m->ekv.data(), acts, D.sites)) {
            NH_TRY(nh::launch_gemm_batch(m->ekv.data(), acts, ys, D.sites, flags, 2 * D.d, st), "engram kv");
        } else {
            for (int e = 0; e < D.sites; ++e)
                NH_TRY(product(m->ekv[e], &s->a_eng[e], t, ys[e], 2 * D.d, flags, st), "engram kv");
        }
    }
    NH_TRY(nh::fwd_engram_hist(D, m->glob, S, p0, t, st), "engram history");
    for (int l = 0; l < D.layers; ++l) {
        const nh::LayerDev* prev = l > 0 ? &m->layers[l - 1] : nullptr;
        NH_TRY(nh::fwd_layer(D, m->glob, S, prev, &m->layers[l], 0, t, m->qkvg[l]->m.bits, 0, st), "layer");
        NH_TRY(product(m->qkvg[l], &s->a_in, t, S.proj, D.nq, flags, st), "q|k|v|gate");
        if (t == 1 && nh::dec_group_fits(D, p0, m->layers[l].window)) {
            NH_TRY(nh::fwd_dec_attn(D, S, m->layers[l], l, p0, m->out[l]->m.bits, st), "decode attention");
        } else if (t == 1 && nh::dec_chunks_fits(D)) {
            NH_TRY(nh::fwd_dec_chunks(D, S, m->layers[l], l, p0, m->out[l]->m.bits, sp, st), "decode attention");
        } else {
            NH_TRY(nh::fwd_units(D, S, m->layers[l], l, p0, t, st), "units");
            NH_TRY(nh::fwd_attend(D, S, m->layers[l], l, p0, t, sp, st), "attend");
            NH_TRY(nh::fwd_attn_out(D, S, m->layers[l], l, p0, t, m->out[l]->m.bits, sp, st), "attention out");
        }
        NH_TRY(product(m->out[l], &s->a_att, t, S.o, D.d, flags, st), "out");
    }
    // the last layer's post block, the lane mean and final norm of the rows
    // the outputs want, then the head (head_logits per row, decode combine)
    const int rows = out_rows_of(outputs, t), row0 = t - rows;
    const int d = D.d, Gd = (d + nh::GROUP - 1) / nh::GROUP;
    const nh::LayerDev* last = D.layers > 0 ? &m->layers[D.layers - 1] : nullptr;
    if (cells && last) {
        // the last layer's post block over every row (its cells), the head's
        // input for the rows the outputs want (hid and A8 rows 0 .. rows - 1)
        NH_TRY(nh::fwd_layer(D, m->glob, S, last, nullptr, 0, t, 0, m->head_bits, st, row0), "last layer");
    }
    if (rows > 0) {
        if (!cells || !last)
            NH_TRY(nh::fwd_layer(D, m->glob, S, last, nullptr, row0, rows, 0, m->head_bits, st), "head input");
        const bool logits = outputs == NH_OUT_LAST_LOGITS || outputs == NH_OUT_ALL_LOGITS;
        for (int i = 0; i < rows && logits; ++i) {
            nh_qact a = s->a_in;
            a.d_xq += (size_t)i * Gd * nh::GROUP;
            a.d_sx += (size_t)i * Gd;
            float* y = (outputs == NH_OUT_ALL_LOGITS && out) ? out + (size_t)i * D.out_rows : S.logits;
            NH_TRY(product(m->head, &a, 1, y, D.out_rows, nullptr, st), "head");
            if (i == rows - 1 && y != S.logits)
                NH_TRY(hipMemcpyAsync(S.logits, y, (size_t)D.out_rows * 4, hipMemcpyDeviceToDevice, st), "logits");
        }
        if (out && !logits)
            NH_TRY(hipMemcpyAsync(out, S.hid, (size_t)rows * d * 4, hipMemcpyDeviceToDevice, st), "hidden");
        if (out && outputs == NH_OUT_LAST_LOGITS)
            NH_TRY(hipMemcpyAsync(out, S.logits, (size_t)D.out_rows * 4, hipMemcpyDeviceToDevice, st), "logits");
        // (the head's input kernel writes the last row's hidden state to S.last_hid as well)
        s->have_logits = logits;
        s->have_hidden = true;
    } else {
        s->have_logits = false;
    }
    // the host mirrors, chunk by chunk: the history rows and their trim
    // (chunk.rs:319-329), the RoPE list and its trim (rope_rows,
    // infer.rs:1740-1745)
    s->len = p0 + t;
    const int keep = D.taps - 1 + nh::ROLLBACK;
    for (int c = 0; c < t; c += nh::FWD_ROWS) {
        const int tc = std::min(nh::FWD_ROWS, t - c);
        s->hrows += tc;
        if (s->hrows > 2 * keep) s->hrows = keep;
        s->rope_n += tc;
        if (s->rope_n > 2 * (nh::ROLLBACK + 1)) s->rope_n = nh::ROLLBACK + 1;
    }
    return rows;
}

// Back to an empty session, keeping the attention span and cell tracking
// the caller set.
void clear(nh_session* s) {
    s->len = 0;
    s->have_logits = s->have_hidden = false;
    s->hrows = s->rope_n = 0;
    s->slot_pos.clear();
    s->toks.clear();
    s->ncells = 0;
}

// The session's status word (bounded in-kernel waits that gave up).  A call
// that feeds ends by queueing a copy of the word to pinned host memory and
// an event behind it (post_status); the next call reads that copy if the
// event has completed (wait: waits for it) and otherwise leaves the check
// to a later call, so a feed never waits for the previous one's work.  A
// failure is reported by the first call made after the stream has passed
// the copy (any call after a synchronization).  An error when set (the word
// is cleared and the session reset, its caches being unreliable).
int check_status(nh_session* s, hipStream_t st, bool wait) {
    if (!s->status_pending) return NH_OK;
    const hipError_t q = wait ? hipEventSynchronize(s->ev_status) : hipEventQuery(s->ev_status);
    if (q == hipErrorNotReady) return NH_OK;
    NH_TRY(q, "status");
    s->status_pending = false;
    if (*s->h_status == 0) return NH_OK;
    const int32_t zero = 0;
    NH_TRY(hipMemcpyAsync(s->S.status, &zero, 4, hipMemcpyHostToDevice, st), "status");
    NH_TRY(hipStreamSynchronize(st), "status");
    clear(s);
    return fail(NH_EDEVICE, "a bounded wait in the layer kernel gave up (the session was reset)");
}

int post_status(nh_session* s, hipStream_t st) {
    NH_TRY(hipMemcpyAsync(s->h_status, s->S.status, 4, hipMemcpyDeviceToHost, st), "status");
    NH_TRY(hipEventRecord(s->ev_status, st), "status");
    s->status_pending = true;
    return NH_OK;
}

// A feed that failed part way: the device caches hold part of it (the
// reference would have panicked), so the session starts over rather than
// keep them.
int reset_after(nh_session* s, int rc) {
    const std::string msg = nh_last_error();
    clear(s);
    return fail(rc, msg + " (the session was reset)");
}

// Session::cells.truncate(len * (L+1) * d) (model.rs:108-110,118-121,
// infer.rs:1096-1099).
void truncate_cells(nh_session* s, int len) { s->ncells = std::min(s->ncells, len); }

// A ring shorter than a chunk takes only feeds that fit it: two rows of a
// longer chunk would share a KV slot (the reference's members race there)
// and a row could see no key at all (attend_head_ref's step_by(0) panics).
int check_ring(const nh_session* s, int n) {
    if (s->ring > 0 && s->ring < nh::FWD_ROWS && n > s->ring)
        return fail(NH_EINVAL, "a feed longer than an attention ring shorter than 32 (two of its rows would share "
                               "a KV slot)");
    return NH_OK;
}

// Model::forward_native (infer.rs:1105-1132) over host token ids: chunks of
// 32, a one-token chunk as a step, LastLogits / LastHidden from the last
// chunk only.  Returns the rows written.  want_cells: the cells are computed
// (forward_inner, model.rs:339-343: requested or tracked; prefill_native
// passes false, infer.rs:1089,1100), into `cells` (device [n][L+1][d], or
// null) and appended to a tracking session's store (step.rs:730-732,
// chunk.rs:353-355).
int forward_ids(nh_session* s, const uint32_t* toks, int n, int outputs, float* out, bool want_cells, float* cells,
                hipStream_t st) {
    if (int rc = check_status(s, st, false)) return rc;
    NH_TRY(hipMemcpyAsync(s->S.tokens + s->len, toks, (size_t)n * 4, hipMemcpyHostToDevice, st), "tokens");
    s->toks.resize(s->len);
    s->toks.insert(s->toks.end(), toks, toks + n);
    const int width = out_width(s, outputs);
    int rows = 0;
    for (int i = 0; i < n;) {
        // whole chunks of 32 together while every chunk has two tokens or
        // more (a one-token chunk is a step) and no attention span (a span's
        // slot map changes chunk by chunk)
        int t = std::min(nh::FWD_ROWS, n - i);
        if (s->ring == 0 && t > 1)
            while (t < nh::BATCH_ROWS && i + t < n && n - (i + t) > 1) t += std::min(nh::FWD_ROWS, n - (i + t));
        const bool last = i + t == n;
        const int want =
            (!last && (outputs == NH_OUT_LAST_LOGITS || outputs == NH_OUT_LAST_HIDDEN)) ? NH_OUT_NONE : outputs;
        const size_t cw = s->cell_floats();
        float* cdst = nullptr;
        if (want_cells) cdst = s->track_cells ? s->d_cells + (size_t)s->ncells * cw : cells ? cells + i * cw : nullptr;
        const int r = feed(s, t, want, out ? out + (size_t)rows * width : nullptr, cdst, st);
        if (r < 0) return reset_after(s, r);
        if (cdst && s->track_cells) {
            if (cells)
                NH_TRY(hipMemcpyAsync(cells + i * cw, cdst, (size_t)t * cw * 4, hipMemcpyDeviceToDevice, st), "cells");
            s->ncells += t;
        }
        rows += r;
        i += t;
    }
    if (int rc = post_status(s, st)) return rc;
    return rows;
}

int check_feed(nh_session* s, const uint32_t* toks, int n, int outputs) {
    if (!s || (n > 0 && !toks) || n < 0) return fail(NH_EINVAL, "bad arguments");
    if (outputs < NH_OUT_NONE || outputs > NH_OUT_LAST_HIDDEN) return fail(NH_EINVAL, "unknown outputs mode");
    if (!nh::ready()) return fail(NH_ESTATE, "nh_init has not been called");
    if (s->len + n > s->dims.cap) return fail(NH_EINVAL, "the tokens do not fit the session's capacity");
    for (int i = 0; i < n; ++i)
        if (toks[i] >= (uint32_t)s->dims.vocab) return fail(NH_EINVAL, "token id outside the vocabulary");
    return NH_OK;
}

int check_cells(const nh_session* s, int n, const float* cells, int64_t cells_cap) {
    if (cells && (int64_t)n * (int64_t)s->cell_floats() > cells_cap)
        return fail(NH_ESMALL, "the cells buffer is too small");
    return NH_OK;
}

int check_out(const nh_session* s, int n, int outputs, const float* out, int64_t out_cap) {
    const int rows = n == 0 ? 0 : out_rows_of(outputs, n);
    if (out && (int64_t)rows * out_width(s, outputs) > out_cap)
        return fail(NH_ESMALL, "the output buffer is too small");
    return NH_OK;
}

}  // namespace

extern "C" {

int nh_model_load(const uint8_t* bytes, uint64_t n, nh_model** out) {
    if (!out) return fail(NH_EINVAL, "null argument");
    *out = nullptr;
    nh::ArchiveSmall sm;
    nh_weights* w = nullptr;
    int rc = nh::load_archive(bytes, n, &w, &sm);
    if (rc != NH_OK) return rc;
    auto* m = new (std::nothrow) nh_model;
    if (!m) {
        nh_weights_free(w);
        return fail(NH_ENOMEM, "out of host memory");
    }
    m->w = w;
    nh_weights_header(w, m->header, 49);
    rc = check_geometry(m, sm);
    if (rc == NH_OK) rc = build_model(m, sm);
    if (rc != NH_OK) {
        delete m;
        return rc;
    }
    *out = m;
    return NH_OK;
}

int nh_model_free(nh_model* m) {
    delete m;
    return NH_OK;
}

int nh_model_weights(const nh_model* m, const nh_weights** w) {
    if (!m || !w) return fail(NH_EINVAL, "null argument");
    *w = m->w;
    return NH_OK;
}

int nh_model_out_rows(const nh_model* m) {
    if (!m) return fail(NH_EINVAL, "null model");
    return m->dims.out_rows;
}

int nh_session_new(const nh_model* m, int cap, nh_session** out) {
    if (!m || !out) return fail(NH_EINVAL, "null argument");
    *out = nullptr;
    if (cap <= 0 || cap > (1 << 20)) return fail(NH_EINVAL, "session capacity out of range");
    auto* s = new (std::nothrow) nh_session;
    if (!s) return fail(NH_ENOMEM, "out of host memory");
    s->m = m;
    nh::Dims& D = s->dims;
    D = m->dims;
    D.cap = cap;
    D.vcap = (int)round_up((size_t)cap + 4, 16);
    int mc = 1;
    for (int n = 1; n <= cap; ++n) mc = std::max(mc, key_chunk_count(n, D.nkv));
    D.max_chunks = mc;
    const size_t d = D.d, L = D.layers, c = cap, E = D.sites, R = nh::BATCH_ROWS, AR = nh::ACT_ROWS;
    const size_t half = D.qk / 2;
    const int Gd = (D.d + nh::GROUP - 1) / nh::GROUP, Ga = (D.nh * D.vd + nh::GROUP - 1) / nh::GROUP;
    Layout Y;
    const size_t o_xs = Y.take(R * 4 * d * 4), o_u = Y.take(R * d * 4), o_x1 = Y.take(R * d * 4);
    const size_t o_p = Y.take(R * 64 * 4), o_proj = Y.take(R * D.nq * 4), o_q = Y.take(R * D.nh * D.qk * 4);
    const size_t o_o = Y.take(R * d * 4), o_ekv = Y.take(E * R * 2 * d * 4), o_ev = Y.take(E * R * d * 4);
    const size_t o_lg = Y.take(round_up(D.out_rows, nh::PANEL_ROWS) * 4);
    const size_t o_rc = Y.take(R * half * 4), o_rs = Y.take(R * half * 4);
    const size_t o_rrc = Y.take(nh::ROPE_RING * half * 4), o_rrs = Y.take(nh::ROPE_RING * half * 4);
    const size_t o_hid = Y.take(R * d * 4), o_lh = Y.take(d * 4), o_tok = Y.take(c * 4);
    const size_t o_po = Y.take(R * D.nh * mc * D.vd * 4), o_pm = Y.take(R * D.nh * mc * 4),
                 o_ps = Y.take(R * D.nh * mc * 4);
    const size_t o_hist = Y.take(L * D.hist_slots * D.W * 4);
    const size_t o_k8 = Y.take(L * c * D.nkv * D.qk), o_ks = Y.take(L * c * D.nkv * 4);
    const size_t o_v8 = Y.take(L * D.nkv * D.vd * D.vcap), o_vs = Y.take(L * c * D.nkv * 4);
    const size_t o_e8 = Y.take(E * c * d), o_es = Y.take(E * c * (d / 32) * 4);
    const size_t o_xi = Y.take(AR * Gd * nh::GROUP), o_si = Y.take(AR * Gd * 4);
    const size_t o_xa = Y.take(AR * Ga * nh::GROUP), o_sa = Y.take(AR * Ga * 4);
    const size_t o_xe = Y.take(E * AR * Gd * nh::GROUP), o_se = Y.take(E * AR * Gd * 4);
    const size_t o_am = Y.take(16), o_st = Y.take(16), o_fl = Y.take(R), o_dc = Y.take(nh::DCOUNT_SLOTS * 4);
    hipError_t e = hipMalloc(&s->d_buf, Y.size);
    if (e == hipSuccess) e = hipMemset(s->d_buf, 0, Y.size);
    if (e == hipSuccess) e = hipHostMalloc((void**)&s->h_status, sizeof(int32_t), hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s->ev_status, hipEventDisableTiming);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        delete s;
        return fail(NH_ENOMEM, std::string("session allocation: ") + hipGetErrorString(e));
    }
    s->bytes = Y.size;
    uint8_t* b = (uint8_t*)s->d_buf;
    nh::SessDev& S = s->S;
    S.xs = (float*)(b + o_xs), S.u = (float*)(b + o_u), S.x1 = (float*)(b + o_x1), S.p = (float*)(b + o_p);
    S.proj = (float*)(b + o_proj), S.qbuf = (float*)(b + o_q), S.o = (float*)(b + o_o);
    S.ekv = (float*)(b + o_ekv), S.evals = (float*)(b + o_ev), S.logits = (float*)(b + o_lg);
    S.rope_c = (float*)(b + o_rc), S.rope_s = (float*)(b + o_rs), S.tokens = (uint32_t*)(b + o_tok);
    S.rope_rc = (float*)(b + o_rrc), S.rope_rs = (float*)(b + o_rrs);
    S.hid = (float*)(b + o_hid), S.last_hid = (float*)(b + o_lh);
    S.po = (float*)(b + o_po), S.pm = (float*)(b + o_pm), S.psum = (float*)(b + o_ps);
    S.hist = (float*)(b + o_hist), S.k8 = (int8_t*)(b + o_k8), S.ks = (float*)(b + o_ks);
    S.v8t = (int8_t*)(b + o_v8), S.vs = (float*)(b + o_vs), S.ev8 = (int8_t*)(b + o_e8), S.evs = (float*)(b + o_es);
    S.xq_in = (int8_t*)(b + o_xi), S.sx_in = (float*)(b + o_si);
    S.xq_att = (int8_t*)(b + o_xa), S.sx_att = (float*)(b + o_sa);
    S.xq_eng = (int8_t*)(b + o_xe), S.sx_eng = (float*)(b + o_se);
    S.argmax = (int32_t*)(b + o_am);
    S.status = (int32_t*)(b + o_st);
    S.flags = (uint8_t*)(b + o_fl);
    S.dcount = (int32_t*)(b + o_dc);
    D.spin_limit = nh::SPIN_LIMIT;
    auto view = [](int8_t* xq, float* sx, int in_dim, int groups) {
        nh_qact a{};
        a.cap_rows = nh::ACT_ROWS;
        a.rows = 1;
        a.in_dim = in_dim;
        a.groups = groups;
        a.d_xq = xq;
        a.d_sx = sx;
        return a;
    };
    s->a_in = view(S.xq_in, S.sx_in, D.d, Gd);
    s->a_att = view(S.xq_att, S.sx_att, D.nh * D.vd, Ga);
    for (int i = 0; i < D.sites; ++i)
        s->a_eng.push_back(view(S.xq_eng + (size_t)i * AR * Gd * nh::GROUP, S.sx_eng + (size_t)i * AR * Gd, D.d, Gd));
    *out = s;
    return NH_OK;
}

int nh_session_free(nh_session* s) {
    delete s;
    return NH_OK;
}

int nh_session_len(const nh_session* s) {
    if (!s) return fail(NH_EINVAL, "null session");
    return s->len;
}

int nh_session_reset(nh_session* s) {
    if (!s) return fail(NH_EINVAL, "null session");
    clear(s);
    s->sink = s->ring = 0;
    s->track_cells = false;
    return NH_OK;
}

int nh_session_track_cells(nh_session* s, int on) {
    if (!s) return fail(NH_EINVAL, "null session");
    if (on && s->len != 0) return fail(NH_EINVAL, "cell tracking starts at an empty session");
    if (on && !s->d_cells) {
        NH_TRY(hipMalloc(&s->d_cells, (size_t)s->dims.cap * s->cell_floats() * 4), "cells allocation");
    }
    s->track_cells = on != 0;
    s->ncells = 0;
    return NH_OK;
}

int nh_session_cell_rows(const nh_session* s) {
    if (!s) return fail(NH_EINVAL, "null session");
    if (!s->track_cells) return fail(NH_EINVAL, "the session does not track cells");
    return s->ncells;
}

int nh_session_cells(const nh_session* s, int row0, int n, float* dst, void* stream) {
    if (!s || row0 < 0 || n < 0 || (n > 0 && !dst)) return fail(NH_EINVAL, "bad arguments");
    if (!s->track_cells) return fail(NH_EINVAL, "the session does not track cells");
    if (row0 + n > s->ncells) return fail(NH_EINVAL, "rows past the tracked cells");
    const size_t cw = s->cell_floats();
    if (n > 0)
        NH_TRY(hipMemcpyAsync(dst, s->d_cells + (size_t)row0 * cw, (size_t)n * cw * 4, hipMemcpyDeviceToDevice,
                              (hipStream_t)stream),
               "cells");
    return n;
}

int nh_session_debug_fail_feed(nh_session* s, int after) {
    if (!s || after < 0) return fail(NH_EINVAL, "bad arguments");
    s->fail_in = after;
    return NH_OK;
}

int nh_session_clone(const nh_session* s, void* stream, nh_session** out) {
    if (!s || !out) return fail(NH_EINVAL, "null argument");
    *out = nullptr;
    nh_session* c = nullptr;
    if (int rc = nh_session_new(s->m, s->dims.cap, &c)) return rc;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e = hipMemcpyAsync(c->d_buf, s->d_buf, s->bytes, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        delete c;
        return hip_fail(e, "session clone");
    }
    c->len = s->len;
    c->have_logits = s->have_logits;
    c->have_hidden = s->have_hidden;
    c->hrows = s->hrows;
    c->rope_n = s->rope_n;
    c->sink = s->sink;
    c->ring = s->ring;
    c->slot_pos = s->slot_pos;
    c->toks = s->toks;
    c->dims.spin_limit = s->dims.spin_limit;
    if (s->track_cells) {
        c->track_cells = true;
        c->ncells = s->ncells;
        e = hipMalloc(&c->d_cells, (size_t)c->dims.cap * c->cell_floats() * 4);
        if (e == hipSuccess && s->ncells > 0)
            e = hipMemcpyAsync(c->d_cells, s->d_cells, (size_t)s->ncells * s->cell_floats() * 4,
                               hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) {
            delete c;
            return hip_fail(e, "session clone (cells)");
        }
    }
    // A bounded wait of the source that gave up and has not been reported
    // yet would travel with the copy: refuse, so the failure is reported by
    // the source's own next feed.
    int32_t word = 0;
    e = hipMemcpyAsync(&word, c->S.status, 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess || word != 0) {
        delete c;
        if (e != hipSuccess) return hip_fail(e, "session clone");
        return fail(NH_EDEVICE, "the source session has a failed bounded wait not yet reported (its next feed reports it)");
    }
    *out = c;
    return NH_OK;
}

int nh_session_sync(nh_session* s, void* stream) {
    if (!s) return fail(NH_EINVAL, "null argument");
    hipStream_t st = (hipStream_t)stream;
    NH_TRY(hipStreamSynchronize(st), "session sync");
    return check_status(s, st, true);
}

int nh_session_debug_spin_limit(nh_session* s, int limit) {
    if (!s || limit < 0) return fail(NH_EINVAL, "bad arguments");
    s->dims.spin_limit = limit > 0 ? limit : 0;
    return NH_OK;
}

int nh_session_set_attend(nh_session* s, int sink, int ring) {
    if (!s || sink < 0 || ring < 0) return fail(NH_EINVAL, "bad arguments");
    // (a ring shorter than a chunk takes only feeds that fit it: check_ring)
    s->sink = ring > 0 ? sink : 0;
    s->ring = ring;
    return NH_OK;
}

int nh_session_rollback(nh_session* s, int n) {
    if (!s || n < 0) return fail(NH_EINVAL, "bad arguments");
    if (n > nh::ROLLBACK) return fail(NH_EINVAL, "rollback of more than 32 positions");
    if (n > s->len) return fail(NH_EINVAL, "rollback past the start of the session");
    if (n == 0) return NH_OK;
    s->len -= n;
    s->hrows = std::max(0, s->hrows - n);
    s->rope_n = std::max(0, s->rope_n - n);
    s->toks.resize(s->len);
    s->have_logits = false;
    truncate_cells(s, s->len);
    return NH_OK;
}

int nh_session_rewind_zeroed(nh_session* s, int len) {
    if (!s || len < 0) return fail(NH_EINVAL, "bad arguments");
    if (len < s->len) {
        s->len = len;
        s->toks.resize(len);
        s->have_logits = false;
    }
    s->hrows = 0;
    s->rope_n = 0;
    truncate_cells(s, len);
    return NH_OK;
}

int nh_session_last_hidden(const nh_session* s, float* h, void* stream) {
    if (!s || !h) return fail(NH_EINVAL, "bad arguments");
    if (!s->have_hidden) return fail(NH_EINVAL, "no hidden state yet (no feed has returned outputs)");
    NH_TRY(hipMemcpyAsync(h, s->S.last_hid, (size_t)s->dims.d * 4, hipMemcpyDeviceToDevice, (hipStream_t)stream),
           "last hidden");
    return NH_OK;
}

int nh_session_head_logits(nh_session* s, float* logits, void* stream) {
    if (!s || !logits) return fail(NH_EINVAL, "bad arguments");
    if (!nh::ready()) return fail(NH_ESTATE, "nh_init has not been called");
    if (!s->have_hidden) return fail(NH_EINVAL, "no hidden state yet (no feed has returned outputs)");
    hipStream_t st = (hipStream_t)stream;
    const nh::Dims& D = s->dims;
    nh_qact a = s->a_in;
    a.bits = s->m->head_bits;
    NH_TRY(nh::launch_act_prep(s->S.last_hid, 1, D.d, a.groups, s->m->head_bits, nullptr, a.d_xq, a.d_sx, st),
           "head A8");
    NH_TRY(product(s->m->head, &a, 1, logits, D.out_rows, nullptr, st), "head");
    return NH_OK;
}

int nh_session_head_logits_sparse(nh_session* s, const uint32_t* ids, int n, float* logits, void* stream) {
    if (!s || !logits || n < 0 || (n > 0 && !ids)) return fail(NH_EINVAL, "bad arguments");
    if (!nh::ready()) return fail(NH_ESTATE, "nh_init has not been called");
    if (!s->have_hidden) return fail(NH_EINVAL, "no hidden state yet (no feed has returned outputs)");
    hipStream_t st = (hipStream_t)stream;
    const nh::Dims& D = s->dims;
    nh_qact a = s->a_in;
    a.rows = 1;
    a.bits = s->m->head_bits;
    NH_TRY(nh::launch_act_prep(s->S.last_hid, 1, D.d, a.groups, s->m->head_bits, nullptr, a.d_xq, a.d_sx, st),
           "head A8");
    return nh_head_logits_sparse(s->m->head, &a, ids, n, D.out_rows, logits, stream);
}

int nh_forward_outputs(nh_session* s, const uint32_t* toks, int n, int outputs, float* out, int64_t out_cap,
                       void* stream) {
    if (int rc = check_feed(s, toks, n, outputs)) return rc;
    if (int rc = check_out(s, n, outputs, out, out_cap)) return rc;
    if (int rc = check_ring(s, n)) return rc;
    if (n == 0) return 0;
    return forward_ids(s, toks, n, outputs, out, s->track_cells, nullptr, (hipStream_t)stream);
}

int nh_forward_cells(nh_session* s, const uint32_t* toks, int n, int outputs, float* out, int64_t out_cap,
                     float* cells, int64_t cells_cap, void* stream) {
    if (int rc = check_feed(s, toks, n, outputs)) return rc;
    if (int rc = check_out(s, n, outputs, out, out_cap)) return rc;
    if (int rc = check_cells(s, n, cells, cells_cap)) return rc;
    if (int rc = check_ring(s, n)) return rc;
    if (n == 0) return 0;
    return forward_ids(s, toks, n, outputs, out, true, cells, (hipStream_t)stream);
}

int nh_prefill(nh_session* s, const uint32_t* toks, int n, int outputs, float* out, int64_t out_cap, void* stream) {
    if (int rc = check_feed(s, toks, n, outputs)) return rc;
    if (int rc = check_out(s, n, outputs, out, out_cap)) return rc;
    // prefill_native (infer.rs:1078-1101): with a span and a slot map, the
    // first position in max(end - ring, sink) .. len whose slot another
    // position holds now starts a re-feed with the conv history zeroed
    const int pos = s->len, end = pos + n;
    if (s->ring > 0 && !s->slot_pos.empty()) {
        for (int p = std::max(end - s->ring, s->sink); p < pos; ++p) {
            if (live(s, p)) continue;
            std::vector<uint32_t> refeed(s->toks.begin() + p, s->toks.begin() + pos);
            refeed.insert(refeed.end(), toks, toks + n);
            if (int rc = check_out(s, (int)refeed.size(), outputs, out, out_cap)) return rc;
            if (int rc = check_ring(s, (int)refeed.size())) return rc;
            nh_session_rewind_zeroed(s, p);
            return forward_ids(s, refeed.data(), (int)refeed.size(), outputs, out, false, nullptr,
                               (hipStream_t)stream);
        }
    }
    if (int rc = check_ring(s, n)) return rc;
    if (n == 0) return 0;
    return forward_ids(s, toks, n, outputs, out, false, nullptr, (hipStream_t)stream);
}

int nh_forward(nh_session* s, const uint32_t* toks, int n, float* logits, void* stream) {
    if (int rc = check_feed(s, toks, n, NH_OUT_LAST_LOGITS)) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (n == 0) {
        // nothing fed: the logits of the last position, when the session has them
        if (!logits) return NH_OK;
        if (!s->have_logits) return fail(NH_EINVAL, "no tokens and no logits of an earlier feed");
    } else {
        if (int rc = check_ring(s, n)) return rc;
        const int r = forward_ids(s, toks, n, NH_OUT_LAST_LOGITS, nullptr, s->track_cells, nullptr, st);
        if (r < 0) return r;
    }
    if (logits)
        NH_TRY(hipMemcpyAsync(logits, s->S.logits, (size_t)s->dims.out_rows * 4, hipMemcpyDeviceToDevice, st),
               "logits");
    return NH_OK;
}

int nh_argmax(const float* x, int n, uint32_t* dst, void* stream) {
    if (!x || !dst || n <= 0) return fail(NH_EINVAL, "bad arguments");
    if (!nh::ready()) return fail(NH_ESTATE, "nh_init has not been called");
    NH_TRY(nh::fwd_argmax(x, n, dst, (hipStream_t)stream), "argmax");
    return NH_OK;
}

int nh_generate_greedy(nh_session* s, int steps, uint32_t* out, float* logits, void* stream) {
    if (!s || steps < 0 || (steps > 0 && !out)) return fail(NH_EINVAL, "bad arguments");
    if (!nh::ready()) return fail(NH_ESTATE, "nh_init has not been called");
    if (!s->have_logits) return fail(NH_EINVAL, "no logits to pick from (nh_forward a prompt first)");
    if (s->len + steps > s->dims.cap) return fail(NH_EINVAL, "the steps do not fit the session's capacity");
    hipStream_t st = (hipStream_t)stream;
    const int len0 = s->len;
    for (int i = 0; i < steps; ++i) {
        // (the step's first kernel picks its token: the argmax of the
        // previous step's logits, stored at S.tokens[len])
        float* cdst = s->track_cells ? s->d_cells + (size_t)s->ncells * s->cell_floats() : nullptr;
        const int r = feed(s, 1, NH_OUT_LAST_LOGITS, nullptr, cdst, st, true);
        if (r < 0) return reset_after(s, r);
        if (cdst) ++s->ncells;
    }
    if (logits)
        NH_TRY(hipMemcpyAsync(logits, s->S.logits, (size_t)s->dims.out_rows * 4, hipMemcpyDeviceToDevice, st),
               "logits");
    if (steps > 0)
        NH_TRY(hipMemcpyAsync(out, s->S.tokens + len0, (size_t)steps * 4, hipMemcpyDeviceToHost, st), "tokens");
    // (the picks are read on the host once the stream has passed the status copy)
    if (int rc = post_status(s, st)) return rc;
    if (int rc = check_status(s, st, true)) return rc;
    if (steps > 0) {
        s->toks.resize(len0);
        s->toks.insert(s->toks.end(), out, out + steps);
    }
    return NH_OK;
}

}  // extern "C"
