// The .cact deployment archive (crates/needle-core/src/cact.rs) read into
// the packed weights of the fast path: QWeights
// (crates/needle-engine/src/weights.rs:136-148) as
// Weights::from_archive_mode builds it with fast = true
// (weights.rs:314-467), every matrix uploaded to HBM.
//
// Two passes.  The plan pass parses the header, codebook and directory with
// the reference's checks (cact.rs:120-131, 213-230, 593-614) and walks the
// canonical record order (weights.rs:318-420), checking every record the
// walk touches; no device call happens before it succeeds, so a malformed
// archive fails the same way with or without a GPU.  The upload pass turns
// each matmul record into a matrix (CQ records as stored, QMat::from_cq,
// qlinear.rs:220-236; f16 / f32 ones through cq_pack, QMat::from_f32,
// weights.rs:112-128) and fuses them as QWeights holds them:
// q | k | v | gate and out per layer, the mHC pre | post | res rows of each
// layer (weights.rs:376-389), key | value per engram site (weights.rs:413).
#include <string.h>

#include <array>
#include <string>
#include <vector>

#include "../../include/needle_hip.h"
#include "nh_internal.h"

namespace {

constexpr uint32_t kTag = 0x05E12A84u;    // cact.rs:18
constexpr uint32_t kTagV2 = 0x05E12A83u;  // cact.rs:19
constexpr size_t kHeaderBytes = 49 * 4;   // cact.rs:21
constexpr size_t kRecSize = 44;           // cact.rs:22
enum : uint8_t { kF16 = 1, kF32 = 2, kCq = 3, kRaw = 4 };  // cact.rs:26-31
constexpr uint64_t kCondRank = 8;         // HADA_COND_RANK (crates/needle-core/src/config.rs:13)
constexpr int kTernaryBits = 5;           // TERNARY_RECORD_BITS (quant.rs:12)

// Header words (cact.rs:80-118).
enum HeaderWord {
    W_TAG = 0,
    W_NUM_TENSORS = 1,
    W_CODEBOOK_LEN = 2,
    W_D_MODEL = 7,
    W_NUM_LAYERS = 10,
    W_MHC_LANES = 15,
    W_QKV_CONV_TAPS = 19,
    W_NUM_ORDERS = 26,
    W_NUM_SITES = 31,
};

uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}

uint64_t rd64(const uint8_t* p) {
    uint64_t v;
    memcpy(&v, p, 8);
    return v;
}

struct Rec {
    uint8_t dtype = 0;
    int ndim = 0;
    uint64_t shape[4] = {0, 0, 0, 0};
    uint64_t offset = 0, nbytes = 0;
    uint32_t group = 0, bits = 0;
};

struct Fail {
    std::string msg;
};

// What the upload pass does: record indices of every matmul weight, and of
// the small tensors (Cursor::next) the decode step reads.
struct Plan {
    uint32_t header[49];
    std::vector<Rec> recs;
    size_t embedding = 0;
    std::vector<std::array<size_t, 5>> layers;  // q, k, v, gate, out
    std::array<size_t, 3> phi{};                // pre, post, res
    std::vector<std::array<size_t, 3>> engrams; // tables, key, value
    std::vector<std::array<long, nh::SMALL_KINDS>> small;  // per layer (-1: absent)
    std::array<size_t, 6> mhc{};                // a_pre, a_post, a_res, b_pre, b_post, b_res
    size_t perm1 = 0, perm2 = 0, final_norm = 0;
    std::vector<size_t> etaps;
};

const char* dtype_name(uint8_t d) {
    switch (d) {
        case kF16: return "F16";
        case kF32: return "F32";
        case kCq: return "Cq";
        default: return "Raw";
    }
}

// hada_blocks (config.rs:315-319).
void hada_blocks(uint64_t n, uint64_t& a, uint64_t& b) {
    int bits = 0;
    while (bits < 64 && ((n - 1) >> bits) != 0) ++bits;
    a = uint64_t(1) << (bits / 2);
    b = n / a;
}

uint64_t next_pow2(uint64_t v) {
    uint64_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

class Walker {
public:
    Walker(const uint8_t* data, uint64_t n, Plan& plan) : d_(data), n_(n), p_(plan) {}

    void parse() {
        // Header::parse (cact.rs:120-131).
        if (n_ < kHeaderBytes) throw Fail{"not a complete .cact archive"};
        for (int i = 0; i < 49; ++i) p_.header[i] = rd32(d_ + 4 * i);
        const uint32_t tag = p_.header[W_TAG];
        if (tag != kTag) {
            char buf[96];
            if (tag == kTagV2)
                snprintf(buf, sizeof buf, "this is a Needle 2 archive; Needle 3 (tag 0x%08x) is required", kTag);
            else
                snprintf(buf, sizeof buf, "unknown .cact format tag 0x%08x", tag);
            throw Fail{buf};
        }
        if (p_.header[W_NUM_ORDERS] > 4 || p_.header[W_NUM_SITES] > 16) throw Fail{"corrupt .cact header"};
        // Archive::parse (cact.rs:593-614): codebook, then the directory.
        uint64_t off = kHeaderBytes;
        const uint64_t cb_bytes = uint64_t(p_.header[W_CODEBOOK_LEN]) * 4;
        if (cb_bytes > n_ - off) throw Fail{"truncated codebook"};
        off += cb_bytes;
        const uint32_t nt = p_.header[W_NUM_TENSORS];
        p_.recs.reserve(nt);
        for (uint32_t i = 0; i < nt; ++i) {
            if (kRecSize > n_ - off) throw Fail{"truncated directory"};
            p_.recs.push_back(parse_rec(d_ + off));
            const Rec& r = p_.recs.back();
            if (r.offset > n_ || r.nbytes > n_ - r.offset) throw Fail{"tensor past the end of the archive"};
            off += kRecSize;
        }
    }

    // The canonical order (weights.rs:318-420).
    void walk() {
        const uint64_t layers = p_.header[W_NUM_LAYERS];
        const uint64_t lanes = p_.header[W_MHC_LANES];
        const bool taps = p_.header[W_QKV_CONV_TAPS] > 0;
        const uint64_t sites = p_.header[W_NUM_SITES];
        const uint64_t hada_n = next_pow2(p_.header[W_D_MODEL]);
        std::vector<std::array<uint64_t, 2>> kron;
        std::vector<uint64_t> cond_u;
        p_.embedding = big();
        for (uint64_t l = 0; l < layers; ++l) {
            std::array<long, nh::SMALL_KINDS> sm;
            sm.fill(-1);
            auto take = [&](int kind) {
                sm[kind] = (long)i_;
                return next();
            };
            take(nh::S_NORM_IN);
            const size_t q = big(), k = big(), v = big();
            if (taps) take(nh::S_Q_TAPS), take(nh::S_K_TAPS), take(nh::S_V_TAPS);
            take(nh::S_Q_NORM), take(nh::S_K_NORM);
            const size_t g = big(), o = big();
            p_.layers.push_back({q, k, v, g, o});
            take(nh::S_POST_NORM);
            if (take(nh::S_ATTN_GATE) < 1)
                throw Fail{"archive tensor " + std::to_string(i_ - 1) + ": attn_gate is empty"};
            take(nh::S_PRE_HADA);
            for (int j = 0; j < 5; ++j) take(nh::S_D1 + j);  // d1, d2, b2, d3, d4
            uint64_t kl[6];
            for (int j = 0; j < 6; ++j) kl[j] = take(nh::S_KRON0 + j);
            kron.push_back({kl[0], kl[1]});
            take(nh::S_COND_V);
            cond_u.push_back(take(nh::S_COND_U));
            p_.small.push_back(sm);
        }
        for (int j = 0; j < 6; ++j) {  // mhc a_pre, a_post, a_res, b_pre, b_post, b_res
            p_.mhc[j] = i_;
            next();
        }
        p_.phi = {big(), big(), big()};
        p_.perm1 = i_;
        const uint64_t perm1 = next();
        p_.perm2 = i_;
        const uint64_t perm2 = next();
        for (uint64_t s = 0; s < sites; ++s) {
            const size_t t = big(), k = big(), v = big();
            p_.etaps.push_back(i_);
            next();  // taps
            p_.engrams.push_back({t, k, v});
        }
        p_.final_norm = i_;
        next();  // final_norm
        // The fast-path checks (weights.rs:460-464), on the lengths the
        // records hold.
        if (perm1 != hada_n || perm2 != hada_n) throw Fail{"Hadamard permutations do not match hada_n"};
        uint64_t ba, bb;
        hada_blocks(hada_n, ba, bb);
        for (auto& kr : kron)
            if (kr[0] != ba * ba || kr[1] != bb * bb) throw Fail{"Hadamard factor shapes"};
        for (uint64_t c : cond_u)
            if (c != kCondRank * hada_n) throw Fail{"cond_u shape"};
        // Fusion and slicing preconditions (QLinear::new's compatibility
        // assert, qlinear.rs:501-519; slice_rows ranges, weights.rs:384-386).
        for (auto& ly : p_.layers) fusable({ly[0], ly[1], ly[2], ly[3]}, "q|k|v|gate");
        if (layers > 0 && lanes == 0) throw Fail{"mhc_lanes is zero"};
        if (rows(p_.phi[0]) < layers * lanes || rows(p_.phi[1]) < layers * lanes ||
            rows(p_.phi[2]) < layers * lanes * lanes)
            throw Fail{"mHC phi rows do not match the depth"};
        if (layers > 0) fusable({p_.phi[0], p_.phi[1], p_.phi[2]}, "mHC pre|post|res");
        for (auto& e : p_.engrams) fusable({e[1], e[2]}, "engram key|value");
    }

private:
    static Rec parse_rec(const uint8_t* b) {
        // Record::parse (cact.rs:213-230).
        Rec r;
        r.ndim = b[1];
        if (r.ndim > 4) throw Fail{"corrupt .cact record"};
        if (b[0] < kF16 || b[0] > kRaw) throw Fail{"unknown .cact tensor dtype " + std::to_string(b[0])};
        r.dtype = b[0];
        for (int i = 0; i < r.ndim; ++i) r.shape[i] = rd32(b + 4 + 4 * i);
        r.offset = rd64(b + 20);
        r.nbytes = rd64(b + 28);
        r.group = rd32(b + 36);
        r.bits = rd32(b + 40);
        return r;
    }

    const Rec& at(size_t i) const {
        if (i >= p_.recs.size())
            throw Fail{"archive tensor " + std::to_string(i) + ": the archive ends before the canonical order does"};
        return p_.recs[i];
    }

    // Archive::cq (cact.rs:617-627) plus QMat::from_cq's preconditions.
    void check_cq(size_t i) const {
        const Rec& r = at(i);
        const std::string at_i = "archive tensor " + std::to_string(i) + ": ";
        if (r.dtype != kCq) throw Fail{at_i + "tensor " + std::to_string(i) + " is " + dtype_name(r.dtype) + ", not CQ"};
        if (r.ndim < 2) throw Fail{at_i + "a CQ record needs an [out, in] shape"};
        if (r.group != (uint32_t)nh::GROUP)
            throw Fail{at_i + "CQ group size " + std::to_string(r.group) + " is not supported"};
        if (r.bits != 2 && r.bits != 4 && r.bits != (uint32_t)kTernaryBits)
            throw Fail{at_i + "CQ records of " + std::to_string(r.bits) + " bits are not supported"};
        const uint64_t out = r.shape[0], in_dim = r.shape[1];
        if (out == 0 || in_dim == 0 || out > 0x7fffffff) throw Fail{at_i + "empty or oversized CQ matrix"};
        if (in_dim > 4096) throw Fail{at_i + "in_dim above 4096 is not supported"};
        const uint64_t groups = (in_dim + nh::GROUP - 1) / nh::GROUP;
        const uint64_t cbits = r.bits == (uint32_t)kTernaryBits ? 2 : r.bits;
        const uint64_t need = out * (groups * nh::GROUP * cbits / 8) + out * groups * 2;
        if (r.nbytes < need) throw Fail{at_i + "CQ blob shorter than its shape"};
    }

    // Cursor::next (weights.rs:106-110): any non-raw tensor; its element
    // count (CQ records dequantize to out x in).
    uint64_t next() {
        const size_t i = i_;
        const Rec& r = at(i);
        ++i_;
        switch (r.dtype) {
            case kF16: return r.nbytes / 2;
            case kF32: return r.nbytes / 4;
            case kCq: check_cq(i); return r.shape[0] * r.shape[1];
            default:
                throw Fail{"archive tensor " + std::to_string(i) + ": tensor " + std::to_string(i) +
                           " is a raw attachment"};
        }
    }

    // Cursor::big (weights.rs:113-128): a matmul weight.
    size_t big() {
        const size_t i = i_;
        const Rec& r = at(i);
        if (r.dtype == kCq) {
            check_cq(i);
            ++i_;
            return i;
        }
        const uint64_t elems = next();
        if (r.ndim < 2 || r.shape[0] == 0 || r.shape[1] == 0 || r.shape[0] > 0x7fffffff)
            throw Fail{"archive tensor " + std::to_string(i) + ": a matmul weight needs an [out, in] shape"};
        if (r.shape[1] > 4096) throw Fail{"archive tensor " + std::to_string(i) + ": in_dim above 4096 is not supported"};
        if (elems < r.shape[0] * r.shape[1])
            throw Fail{"archive tensor " + std::to_string(i) + ": data shorter than its shape"};
        return i;
    }

    uint64_t rows(size_t i) const { return p_.recs[i].shape[0]; }

    // The width a matmul record becomes: CQ records keep theirs (ternary
    // apart), f16 / f32 ones are packed at 4 bits.
    int width(size_t i) const {
        const Rec& r = p_.recs[i];
        return r.dtype == kCq ? (int)r.bits : 4;
    }

    void fusable(std::initializer_list<size_t> parts, const char* what) const {
        const size_t first = *parts.begin();
        for (size_t i : parts)
            if (p_.recs[i].shape[1] != p_.recs[first].shape[1] || width(i) != width(first))
                throw Fail{std::string(what) + ": fused parts must share in_dim and code width"};
    }

    const uint8_t* d_;
    uint64_t n_;
    Plan& p_;
    size_t i_ = 0;
};

// IEEE binary16 -> binary32 (exact).
float half_to_float(uint16_t h) {
    const uint32_t s = uint32_t(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {
            e = 127 - 15 + 1;
            while (!(m & 0x400)) {
                m <<= 1;
                --e;
            }
            bits = s | (e << 23) | ((m & 0x3ff) << 13);
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// One matmul record as a matrix in HBM.
int upload(const uint8_t* data, const Rec& r, nh_qmat** h) {
    const uint8_t* blob = data + r.offset;
    const int out = (int)r.shape[0], in_dim = (int)r.shape[1];
    if (r.dtype == kCq) {
        const int groups = (in_dim + nh::GROUP - 1) / nh::GROUP;
        const int cbits = r.bits == (uint32_t)kTernaryBits ? 2 : (int)r.bits;
        const uint64_t n_packed = (uint64_t)out * groups * nh::GROUP * cbits / 8;
        std::vector<uint16_t> norms((size_t)out * groups);
        memcpy(norms.data(), blob + n_packed, norms.size() * 2);
        return nh_qmat_from_cq(blob, n_packed, norms.data(), norms.size(), out, in_dim, (int)r.bits, nh::GROUP, h);
    }
    std::vector<float> w((size_t)out * in_dim);
    if (r.dtype == kF32) {
        memcpy(w.data(), blob, w.size() * 4);
    } else {
        for (size_t j = 0; j < w.size(); ++j) {
            uint16_t v;
            memcpy(&v, blob + 2 * j, 2);
            w[j] = half_to_float(v);
        }
    }
    return nh_qmat_from_f32(w.data(), out, in_dim, h);
}

}  // namespace

struct nh_weights {
    uint32_t header[49];
    nh_qmat* embedding = nullptr;
    std::vector<nh_qmat*> qkvg, out, phi, engram_tables, engram_kv;

    ~nh_weights() {
        nh_qmat_free(embedding);
        for (auto* v : {&qkvg, &out, &phi, &engram_tables, &engram_kv})
            for (nh_qmat* m : *v) nh_qmat_free(m);
    }
};

namespace {

// Frees the matrices it holds unless released.
struct Held {
    std::vector<nh_qmat*> m;
    ~Held() {
        for (nh_qmat* x : m) nh_qmat_free(x);
    }
    nh_qmat* add(nh_qmat* x) {
        m.push_back(x);
        return x;
    }
};

int fuse(std::initializer_list<nh_qmat*> parts, nh_qmat** h) {
    std::vector<nh_qmat*> v(parts);
    const int rc = nh_qlinear_new(v.data(), (int)v.size(), h);
    if (rc == NH_OK) (*h)->resident = true;  // a model's weights
    return rc;
}

}  // namespace

namespace {

// One small tensor widened to f32.
std::vector<float> small_f32(const uint8_t* data, const Plan& plan, size_t i) {
    const Rec& r = plan.recs[i];
    const uint8_t* blob = data + r.offset;
    std::vector<float> v;
    if (r.dtype == kF32) {
        v.resize(r.nbytes / 4);
        memcpy(v.data(), blob, v.size() * 4);
    } else if (r.dtype == kF16) {
        v.resize(r.nbytes / 2);
        for (size_t j = 0; j < v.size(); ++j) {
            uint16_t h;
            memcpy(&h, blob + 2 * j, 2);
            v[j] = half_to_float(h);
        }
    } else {
        throw Fail{"archive tensor " + std::to_string(i) + ": a CQ record where the decode step reads a small tensor"};
    }
    return v;
}

void read_small(const uint8_t* data, const Plan& plan, nh::ArchiveSmall& sm) {
    sm.layer.clear();
    for (const auto& ly : plan.small) {
        std::vector<std::vector<float>> kinds(nh::SMALL_KINDS);
        for (int k = 0; k < nh::SMALL_KINDS; ++k)
            if (ly[k] >= 0) kinds[k] = small_f32(data, plan, (size_t)ly[k]);
        sm.layer.push_back(std::move(kinds));
    }
    sm.mhc.clear();
    for (size_t i : plan.mhc) sm.mhc.push_back(small_f32(data, plan, i));
    sm.perm1 = small_f32(data, plan, plan.perm1);
    sm.perm2 = small_f32(data, plan, plan.perm2);
    sm.final_norm = small_f32(data, plan, plan.final_norm);
    sm.etaps.clear();
    for (size_t i : plan.etaps) sm.etaps.push_back(small_f32(data, plan, i));
}

}  // namespace

int nh::load_archive(const uint8_t* bytes, uint64_t n, nh_weights** out, nh::ArchiveSmall* small) {
    if (!out) {
        nh::set_error("null argument");
        return NH_EINVAL;
    }
    *out = nullptr;
    if (!bytes && n > 0) {
        nh::set_error("null archive bytes");
        return NH_EINVAL;
    }
    Plan plan;
    try {
        Walker w(bytes, n, plan);
        w.parse();
        w.walk();
        if (small) read_small(bytes, plan, *small);
    } catch (const Fail& f) {
        nh::set_error(f.msg);
        return NH_EINVAL;
    } catch (const std::bad_alloc&) {
        nh::set_error("out of host memory reading the archive");
        return NH_ENOMEM;
    }
    if (!nh::ready()) {
        nh::set_error("nh_init has not been called");
        return NH_ESTATE;
    }
    auto* wts = new (std::nothrow) nh_weights;
    if (!wts) {
        nh::set_error("out of host memory");
        return NH_ENOMEM;
    }
    memcpy(wts->header, plan.header, sizeof wts->header);
    int rc = NH_OK;
    auto put = [&](size_t i, nh_qmat** h) {
        if (rc == NH_OK) rc = upload(bytes, plan.recs[i], h);
        if (rc == NH_OK) (*h)->resident = true;  // a model's weights
        return rc == NH_OK;
    };
    if (put(plan.embedding, &wts->embedding)) {
        for (auto& ly : plan.layers) {
            Held tmp;
            nh_qmat *q = nullptr, *k = nullptr, *v = nullptr, *g = nullptr, *o = nullptr, *f = nullptr;
            if (!put(ly[0], &q)) break;
            tmp.add(q);
            if (!put(ly[1], &k)) break;
            tmp.add(k);
            if (!put(ly[2], &v)) break;
            tmp.add(v);
            if (!put(ly[3], &g)) break;
            tmp.add(g);
            if ((rc = fuse({q, k, v, g}, &f)) != NH_OK) break;
            wts->qkvg.push_back(f);
            if (!put(ly[4], &o)) break;
            wts->out.push_back(o);
        }
    }
    if (rc == NH_OK) {
        Held whole;
        nh_qmat *pre = nullptr, *post = nullptr, *res = nullptr;
        if (put(plan.phi[0], &pre) && whole.add(pre) && put(plan.phi[1], &post) && whole.add(post) &&
            put(plan.phi[2], &res) && whole.add(res)) {
            const int n = (int)plan.header[W_MHC_LANES];
            for (int l = 0; l < (int)plan.header[W_NUM_LAYERS] && rc == NH_OK; ++l) {
                Held parts;
                nh_qmat *a = nullptr, *b = nullptr, *c = nullptr, *f = nullptr;
                if ((rc = nh_qmat_slice_rows(pre, l * n, (l + 1) * n, &a)) != NH_OK) break;
                parts.add(a);
                if ((rc = nh_qmat_slice_rows(post, l * n, (l + 1) * n, &b)) != NH_OK) break;
                parts.add(b);
                if ((rc = nh_qmat_slice_rows(res, l * n * n, (l + 1) * n * n, &c)) != NH_OK) break;
                parts.add(c);
                if ((rc = fuse({a, b, c}, &f)) != NH_OK) break;
                wts->phi.push_back(f);
            }
        }
    }
    if (rc == NH_OK) {
        for (auto& e : plan.engrams) {
            nh_qmat *t = nullptr, *k = nullptr, *v = nullptr, *f = nullptr;
            if (!put(e[0], &t)) break;
            wts->engram_tables.push_back(t);
            Held tmp;
            if (!put(e[1], &k)) break;
            tmp.add(k);
            if (!put(e[2], &v)) break;
            tmp.add(v);
            if ((rc = fuse({k, v}, &f)) != NH_OK) break;
            wts->engram_kv.push_back(f);
        }
    }
    if (rc != NH_OK) {
        delete wts;  // the error text of the failing call stays
        return rc;
    }
    *out = wts;
    return NH_OK;
}

extern "C" {

int nh_weights_load(const uint8_t* bytes, uint64_t n, nh_weights** out) {
    return nh::load_archive(bytes, n, out, nullptr);
}

int nh_weights_free(nh_weights* w) {
    delete w;
    return NH_OK;
}

int nh_weights_header(const nh_weights* w, uint32_t* words, int n) {
    if (!w || (n > 0 && !words) || n < 0) {
        nh::set_error("bad arguments");
        return NH_EINVAL;
    }
    if (n > 0) memcpy(words, w->header, sizeof(uint32_t) * (n < 49 ? n : 49));
    return 49;
}

int nh_weights_count(const nh_weights* w, int kind) {
    if (!w) {
        nh::set_error("null weights");
        return NH_EINVAL;
    }
    switch (kind) {
        case NH_W_EMBEDDING: return 1;
        case NH_W_QKVG: return (int)w->qkvg.size();
        case NH_W_OUT: return (int)w->out.size();
        case NH_W_PHI: return (int)w->phi.size();
        case NH_W_ENGRAM_TABLE: return (int)w->engram_tables.size();
        case NH_W_ENGRAM_KV: return (int)w->engram_kv.size();
        default: nh::set_error("unknown weight kind"); return NH_EINVAL;
    }
}

int nh_weights_get(const nh_weights* w, int kind, int index, const nh_qmat** m) {
    if (!w || !m) {
        nh::set_error("null argument");
        return NH_EINVAL;
    }
    const int count = nh_weights_count(w, kind);
    if (count < 0) return count;
    if (index < 0 || index >= count) {
        nh::set_error("weight index out of range");
        return NH_EINVAL;
    }
    switch (kind) {
        case NH_W_EMBEDDING: *m = w->embedding; break;
        case NH_W_QKVG: *m = w->qkvg[index]; break;
        case NH_W_OUT: *m = w->out[index]; break;
        case NH_W_PHI: *m = w->phi[index]; break;
        case NH_W_ENGRAM_TABLE: *m = w->engram_tables[index]; break;
        default: *m = w->engram_kv[index]; break;
    }
    return NH_OK;
}

int64_t nh_weights_bytes(const nh_weights* w) {
    if (!w) {
        nh::set_error("null weights");
        return NH_EINVAL;
    }
    int64_t b = nh_qmat_bytes(w->embedding);
    for (auto* v : {&w->qkvg, &w->out, &w->phi, &w->engram_tables, &w->engram_kv})
        for (nh_qmat* m : *v) b += nh_qmat_bytes(m);
    return b;
}

}  // extern "C"
