"""Pins of the oracle's Needle-3 step (oracle/forward.c) by what the
mathematics or the reference's own definitions fix, independently of the
restatement's code.

- attend_head (crates/needle-engine/src/infer.rs:1871-2007): one key returns
  that key's dequantized value row; equal scores return the mean of the
  value rows (one chunk and the multi-chunk merge); a score far above the
  rest keeps the digit path bit-identical to that key alone; random keys
  match the float64 softmax(q . k / sqrt(qk)) average of the dequantized
  values within the 21-bit digit precision.  A wrong query scale, digit
  scale or value scale fails the last check.
- the engram hash (infer.rs:1256-1275): a Python restatement from the
  reference's text, a literal known answer, and the input row equals
  QMat::row of each hashed slot at its table's offset (zeros before an
  order is reached).
- the mHC read (infer.rs:1359-1393): the projection equals the float64
  product of the dequantized Phi8 rows with the lanes normalized together,
  within the int8 step; the gates at their own-lane offsets; z = 0 gives
  exactly half of every lane.
- the post gates and the mHC write (infer.rs:1577-1605): z = 0 gives
  hpost = 1 exactly; a permutation hres moves lane pi(a) into lane a
  bit-exactly (which pins the axis hres[a * 4 + b] is read along); a zero
  branch with hres = I keeps the lanes.
- the session (model.rs:81-121, infer.rs:1039-1101,1749-1826): a rollback
  then a feed equals never having fed the dropped tokens; a clone diverges
  independently; rewind_zeroed(0) is a fresh session; with a one-layer,
  one-tap model the last logits depend exactly on the tokens the
  attention span (sink, ring) and the slot map let it see, and the
  prefill re-feed of stale slots equals a fresh feed.
- Outputs (model.rs:150-160): every AllLogits row is head_logits of the
  Hidden row, the Last* modes are the last rows, sparse logits agree with
  the full ones.
"""
import numpy as np
import pytest

import oracle as o
from oracle import cact, forward
from exactf32 import fma32

F = np.float32
K127 = np.frombuffer(np.uint32(0x3C010204).tobytes(), np.float32)[0]
INV_SQRT_QK = np.frombuffer(np.uint32(0x3E13CD3A).tobytes(), np.float32)[0]
Q21 = np.frombuffer(np.uint32(0x49FFFFF8).tobytes(), np.float32)[0]


def lib():
    return forward._lib()


def archive(g, seed):
    ts, _ = cact.needle3_tensors(g, seed=seed, kind=lambda n: ("cq", 4) if n == "embedding" else ("random", 4))
    return cact.pack(ts, g.header())


_models = {}


def model(name):
    """Small models, built once per run."""
    if name not in _models:
        geos = {
            # one global layer, one conv tap, no engram: a position's keys and
            # values come from its own token only
            "one": cact.Geometry(vocab=300, num_layers=1, qkv_conv_taps=1, engram_sites=(), global_layers=(0,),
                                 sliding_window=0, engram_slots=64),
            "one3": cact.Geometry(vocab=300, num_layers=1, qkv_conv_taps=3, engram_sites=(), global_layers=(0,),
                                  sliding_window=0, engram_slots=64),
            "small": cact.Geometry(vocab=300, num_layers=3, engram_slots=64, engram_sites=(1,), global_layers=(1,),
                                   sliding_window=8),
            "wide": cact.Geometry(vocab=300, num_layers=3, engram_slots=64, engram_sites=(1,), global_layers=(1,),
                                  sliding_window=64),
        }
        _models[name] = forward.Forward(archive(geos[name], seed=21 + len(_models)))
    return _models[name]


# ------------------------------------------------------------- attention
def attend(k8, ks, v8, vs, q, nested=False):
    f = model("one")
    s = f.session(max(64, len(ks)))
    return s.attend_test(k8, ks, v8, vs, q, nested)


def exact_query(rng, qk):
    """A query whose int8 codes are exactly q8 (max |q8| = 127)."""
    q8 = rng.integers(-127, 128, size=qk)
    q8[rng.integers(qk)] = 127
    c = F(0.013)
    return (q8.astype(F) * c).astype(F), q8, c


def softmax_ref(q8, c, k8, ks, v8, vs):
    qk = q8.size
    dots = k8.astype(np.int64) @ q8.astype(np.int64)
    sc = dots * ks.astype(np.float64) * float(c) / np.sqrt(qk)
    w = np.exp(sc - sc.max())
    w /= w.sum()
    return w @ (v8.astype(np.float64) * vs.astype(np.float64)[:, None])


def test_attend_single_key_is_its_value_row():
    rng = np.random.default_rng(1)
    q, _, _ = exact_query(rng, 48)
    k8 = rng.integers(-128, 128, size=(1, 48)).astype(np.int8)
    v8 = rng.integers(-128, 128, size=(1, 64)).astype(np.int8)
    ks, vs = np.array([0.02], F), np.array([0.035], F)
    got = attend(k8, ks, v8, vs, q)
    want = v8[0].astype(np.float64) * float(vs[0])
    assert np.abs(got - want).max() <= 4e-6 * np.abs(want).max()


@pytest.mark.parametrize("n,nested", [(7, False), (64, False), (300, False), (300, True)])
def test_attend_equal_scores_is_the_mean(n, nested):
    rng = np.random.default_rng(n)
    q, _, _ = exact_query(rng, 48)
    k8 = np.repeat(rng.integers(-128, 128, size=(1, 48)).astype(np.int8), n, axis=0)
    v8 = rng.integers(-128, 128, size=(n, 64)).astype(np.int8)
    ks, vs = np.full(n, 0.02, F), np.full(n, 0.035, F)
    got = attend(k8, ks, v8, vs, q, nested)
    want = v8.astype(np.float64).mean(axis=0) * float(vs[0])
    assert np.abs(got - want).max() <= 2e-6 * 127 * float(vs[0])


def test_attend_dominant_key_is_bit_identical_to_it_alone():
    rng = np.random.default_rng(2)
    q = np.zeros(48, F)
    q[0] = F(1.0)
    n, hot = 37, 20
    k8 = rng.integers(-128, 128, size=(n, 48)).astype(np.int8)
    k8[:, 0] = -127
    k8[hot, 0] = 127
    ks = np.full(n, 100.0, F)
    v8 = rng.integers(-128, 128, size=(n, 64)).astype(np.int8)
    vs = rng.uniform(0.01, 0.05, size=n).astype(F)
    got = attend(k8, ks, v8, vs, q)
    alone = attend(k8[hot:hot + 1], ks[hot:hot + 1], v8[hot:hot + 1], vs[hot:hot + 1], q)
    assert np.array_equal(got.view(np.uint32), alone.view(np.uint32))


@pytest.mark.parametrize("n,nested", [(5, False), (100, False), (300, False), (300, True)])
def test_attend_matches_float64_softmax(n, nested):
    rng = np.random.default_rng(10 + n)
    q, q8, c = exact_query(rng, 48)
    k8 = rng.integers(-128, 128, size=(n, 48)).astype(np.int8)
    # key scales that spread the scores over several units
    ks = rng.uniform(0.03, 0.08, size=n).astype(F)
    v8 = rng.integers(-128, 128, size=(n, 64)).astype(np.int8)
    vs = rng.uniform(0.01, 0.05, size=n).astype(F)
    got = attend(k8, ks, v8, vs, q, nested)
    want = softmax_ref(q8, c, k8, ks, v8, vs)
    sc = (k8.astype(np.int64) @ q8) * ks * float(c) / np.sqrt(48)
    assert sc.max() - sc.min() > 3.0  # the check sees the temperature
    err = np.abs(got - want).max()
    assert err <= 1e-5 * 127 * float(vs.max()), err
    # the same keys with 1/qk in place of 1/sqrt(qk) would be far off
    wrong = softmax_ref(q8, F(c / np.sqrt(48)), k8, ks, v8, vs)
    assert np.abs(wrong - want).max() > 100 * err


# ---------------------------------------------------------------- engram
SEED, PRIME = 0x9E3779B9, 0x01000193


def engram_hash_py(tokens, pos, oi, h, order, stride, slots, heads):
    """The hash as crates/needle-engine/src/infer.rs:1256-1275 states it."""
    acc = (SEED * (oi * stride + h + 1)) & 0xFFFFFFFF
    for j in range(order):
        t = int(tokens[pos - j]) if pos >= j else 0
        acc = ((acc ^ t) * PRIME) & 0xFFFFFFFF
    acc ^= acc >> 15
    return (oi * heads + h) * slots + acc % slots


def test_engram_hash_known_answer():
    f = model("small")
    cfg = f.cfg
    rng = np.random.default_rng(4)
    tokens = rng.integers(0, 300, size=40).astype(np.uint32)
    rows = np.zeros(16, np.int64)
    for pos in (0, 1, 2, 5, 39):
        lib().nf_engram_rows(f.m, o._p(tokens), pos, o._p(rows))
        for oi in range(cfg.norders):
            order = cfg.orders[oi]
            for h in range(cfg.eheads):
                tbl = oi * cfg.eheads + h
                stride = cfg.seed_heads or cfg.eheads
                want = -1 if pos + 1 < order else engram_hash_py(tokens, pos, oi, h, order, stride,
                                                                  cfg.engram_slots, cfg.eheads)
                assert rows[tbl] == want, (pos, oi, h)
    # a literal: tokens (5, 9), order 2, table 0 of 64 slots, seed factor 1
    assert engram_hash_py([5, 9], 1, 0, 0, 2, 3, 64, 3) == 50
    acc = 0x9E3779B9
    acc = ((acc ^ 9) * 0x01000193) & 0xFFFFFFFF
    acc = ((acc ^ 5) * 0x01000193) & 0xFFFFFFFF
    acc ^= acc >> 15
    assert acc == 0x6D1E0B32 and acc % 64 == 50


def test_engram_input_is_table_rows():
    f = model("small")
    cfg = f.cfg
    d, sub = cfg.d, cfg.engram_sub
    tokens = o.random_tokens(12, 300, seed=5).astype(np.uint32)
    table = f._keep[3][0]  # the site's engram table (OQMat)
    rows = np.zeros(16, np.int64)
    out = np.zeros(d, F)
    for pos in (0, 1, 2, 11):
        lib().nf_engram_input(f.m, 0, o._p(tokens), pos, o._p(out))
        lib().nf_engram_rows(f.m, o._p(tokens), pos, o._p(rows))
        want = np.zeros(d, F)
        for tbl in range(cfg.norders * cfg.eheads):
            if rows[tbl] >= 0:
                want[tbl * sub:(tbl + 1) * sub] = table.row(int(rows[tbl]))
        assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), pos
        if pos == 0:  # no order reaches a single token: the row is zero
            assert not out.any()


# ------------------------------------------------------------------- mHC
def mhc_read(phi_q, phi_s, a_pre, b_pre, lane, x):
    ncols, nc = phi_q.shape
    d = nc // 4
    p = np.zeros(ncols, F)
    u = np.zeros(d, F)
    nx = np.zeros(nc, F)
    nx8 = np.zeros(nc, np.int8)
    lib().nf_mhc_read(o._p(np.ascontiguousarray(phi_q)), o._p(np.ascontiguousarray(phi_s)), ncols, d, float(a_pre),
                      o._p(np.ascontiguousarray(b_pre, F)), lane, o._p(np.ascontiguousarray(x, F)), o._p(p), o._p(u),
                      o._p(nx), o._p(nx8))
    return p, u


def test_mhc_read_projection_and_gates():
    rng = np.random.default_rng(6)
    d = 64
    # lanes of different magnitudes: normalizing per lane would be far off
    x = np.concatenate([rng.normal(size=d) * s for s in (0.5, 1.0, 2.0, 4.0)]).astype(F)
    phi_q = rng.integers(-127, 128, size=(24, 4 * d)).astype(np.int8)
    phi_s = rng.uniform(0.001, 0.01, size=24).astype(F)
    b_pre = rng.normal(size=4).astype(F)
    for lane in range(4):
        p, u = mhc_read(phi_q, phi_s, F(0.7), b_pre, lane, x)
        r = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
        nx = x * r
        phi = phi_q.astype(np.float64) * phi_s[:, None]
        want = phi @ nx
        step = np.abs(nx).max() / 127.0  # the int8 step of the normed lanes
        tol = 0.5 * step * np.abs(phi).sum(axis=1) + 1e-5 * np.abs(want)
        assert (np.abs(p - want) <= tol).all()
        off = np.where(np.arange(4) == lane, 4.0, -4.0)
        hp = 1.0 / (np.exp(-((p[:4].astype(np.float64) * 0.7 + off) + b_pre)) + 1.0)
        wu = sum(hp[b] * x[b * d:(b + 1) * d].astype(np.float64) for b in range(4))
        assert np.abs(u - wu).max() <= 1e-5 * np.abs(wu).max()


def test_mhc_read_zero_gates_halve():
    rng = np.random.default_rng(7)
    d = 64
    x = rng.normal(size=4 * d).astype(F)
    phi_q = np.zeros((24, 4 * d), np.int8)
    phi_s = np.ones(24, F)
    lane = 2
    b_pre = np.where(np.arange(4) == lane, -4.0, 4.0).astype(F)  # z = 0 on every lane
    p, u = mhc_read(phi_q, phi_s, F(1.0), b_pre, lane, x)
    assert not p.any()
    want = x[:d] * F(0.5)
    for b in range(1, 4):
        want = (want + x[b * d:(b + 1) * d] * F(0.5)).astype(F)
    assert np.array_equal(u.view(np.uint32), want.view(np.uint32))


def post_gates(p, a_post, b_post, a_res, b_res, lane):
    hpost, hres = np.zeros(4, F), np.zeros(16, F)
    lib().nf_post_gates(o._p(np.ascontiguousarray(p, F)), float(a_post), o._p(np.ascontiguousarray(b_post, F)),
                        float(a_res), o._p(np.ascontiguousarray(b_res, F)), lane, o._p(hpost), o._p(hres))
    return hpost, hres


def test_post_gates():
    rng = np.random.default_rng(8)
    p = rng.normal(size=24).astype(F)
    b_post, b_res = rng.normal(size=4).astype(F), rng.normal(size=16).astype(F)
    for lane in range(4):
        hpost, hres = post_gates(p, F(0.3), b_post, F(0.2), b_res, lane)
        off = np.where(np.arange(4) == lane, 0.0, -4.0)
        want = 2.0 / (np.exp(-((p[4:8].astype(np.float64) * F(0.3) + off) + b_post)) + 1.0)
        assert np.abs(hpost - want).max() <= 4e-7 * 2
        zres = np.array([fma32(p[8 + k], F(0.2), b_res[k]) for k in range(16)], F)
        sk = np.zeros(16, F)
        lib().nf_sinkhorn64(o._p(zres), o._p(sk))
        assert np.array_equal(hres.view(np.uint32), sk.view(np.uint32))
    # z = 0: hpost = 2 / (1 + 1) = 1 exactly; a constant residual logit: 1/4
    lane = 1
    hpost, hres = post_gates(np.zeros(24, F), F(0.0), np.where(np.arange(4) == lane, 0.0, 4.0).astype(F), F(0.0),
                             np.full(16, 0.5, F), lane)
    assert (hpost == 1.0).all() and (hres == F(0.25)).all()


def mhc_write(y, hpost, hres, x):
    x = np.ascontiguousarray(x, F).copy()
    lib().nf_mhc_write(y.size, o._p(np.ascontiguousarray(y, F)), o._p(np.ascontiguousarray(hpost, F)),
                       o._p(np.ascontiguousarray(hres, F)), o._p(x))
    return x


def test_mhc_write_permutation_and_identity():
    rng = np.random.default_rng(9)
    d = 96
    x = rng.normal(size=4 * d).astype(F)
    y = rng.normal(size=d).astype(F)
    hpost = rng.uniform(0.2, 1.8, size=4).astype(F)
    perm = [2, 0, 3, 1]  # lane a takes old lane perm[a]
    P = np.zeros((4, 4), F)
    for a, b in enumerate(perm):
        P[a, b] = 1.0
    got = mhc_write(y, hpost, P.reshape(-1), x)
    for a in range(4):
        want = ((y * hpost[a]).astype(F) + x[perm[a] * d:(perm[a] + 1) * d]).astype(F)
        assert np.array_equal(got[a * d:(a + 1) * d].view(np.uint32), want.view(np.uint32)), a
    # a zero branch and the identity mixing keep the lanes
    same = mhc_write(np.zeros(d, F), hpost, np.eye(4, dtype=F).reshape(-1), x)
    assert np.array_equal(same.view(np.uint32), x.view(np.uint32))


def test_nexp_at_zero_halves_the_gate():
    assert lib().nf_nexp(0.0) == 1.0  # att / (nexp(-0) + 1) = att / 2


# --------------------------------------------------------------- sessions
def bits(a):
    return np.asarray(a, F).view(np.uint32)


def test_rollback_then_feed_equals_never_fed():
    f = model("small")
    prompt = o.random_tokens(60, 300, seed=30)
    xs = o.random_tokens(25, 300, seed=31)
    ys = o.random_tokens(4, 300, seed=32)
    a = f.session(128)
    a.forward(prompt)
    for t in xs:  # 25 steps: the history is trimmed on the way (rows > 2 keep)
        a.step(int(t))
    a.rollback(25)
    assert len(a) == 60
    b = f.session(128)
    b.forward(prompt)
    for t in ys:
        assert np.array_equal(bits(a.step(int(t))), bits(b.step(int(t))))
    with pytest.raises(ValueError):
        a.rollback(33)


def test_clone_diverges_independently():
    f = model("small")
    prompt = o.random_tokens(40, 300, seed=33)
    a = f.session(64)
    a.forward(prompt)
    b = a.clone()
    la = a.forward([7, 8, 9])
    lb = b.forward([100])
    fresh_a, fresh_b = f.session(64), f.session(64)
    fresh_a.forward(prompt)
    fresh_b.forward(prompt)
    assert np.array_equal(bits(la), bits(fresh_a.forward([7, 8, 9])))
    assert np.array_equal(bits(lb), bits(fresh_b.forward([100])))
    assert len(a) == 43 and len(b) == 41


def test_rewind_zeroed():
    toks = o.random_tokens(50, 300, seed=34)
    # to zero: a fresh session
    f = model("small")
    a = f.session(64)
    a.forward(toks[:30])
    a.rewind_zeroed(0)
    assert len(a) == 0
    assert np.array_equal(bits(a.forward(toks)), bits(f.session(64).forward(toks)))
    # one tap: the conv reads no history, so the re-feed equals a continuous feed
    f1 = model("one")
    c = f1.session(64)
    c.forward(toks[:20])
    c.forward(toks[20:30])
    c.rewind_zeroed(20)
    d = f1.session(64)
    d.forward(toks[:20])
    assert np.array_equal(bits(c.forward(toks[30:50])), bits(d.forward(toks[30:50])))
    # three taps: the zeroed history shows
    f3 = model("one3")
    e = f3.session(64)
    e.forward(toks[:20])
    e.rewind_zeroed(20)
    g = f3.session(64)
    g.forward(toks[:20])
    assert not np.array_equal(bits(e.forward(toks[20:40])), bits(g.forward(toks[20:40])))


def visible_changes(f, feed, pos, sink, ring, n):
    """Whether changing the token at `pos` changes the last logits."""
    toks = o.random_tokens(n, 300, seed=40)
    alt = toks.copy()
    alt[pos] = (int(toks[pos]) + 1) % 300
    outs = []
    for tt in (toks, alt):
        s = f.session(n + 16)
        s.set_attend(sink, ring)
        outs.append(feed(s, tt))
    return not np.array_equal(bits(outs[0]), bits(outs[1]))


def test_attention_span_receptive_field():
    f = model("one")
    sink, ring, n = 4, 32, 80

    def stepwise(s, tt):
        for t in tt[:-1]:
            s.forward([int(t)], forward.OUT_NONE)
        return s.forward([int(tt[-1])])

    def chunk(s, tt):
        return s.forward(tt)  # 32 + 32 + 16

    probe = [0, 2, 3, 4, 5, 20, 46, 47, 48, 49, 60, 79]
    for feed in (stepwise, chunk):
        seen = [p for p in probe if visible_changes(f, feed, p, sink, ring, n)]
        assert seen == [p for p in probe if p < sink or p >= n - ring], (feed.__name__, seen)
    s = f.session(64)
    s.set_attend(4, 16)  # a ring shorter than a chunk takes feeds that fit it
    with pytest.raises(ValueError):
        s.forward(o.random_tokens(17, 300, seed=43))
    assert len(s) == 0


def test_attention_span_wide_is_no_span():
    # The ring part of a span is not cut by a layer's window (key_ranges,
    # infer.rs:1785-1791: b0 has no .max(lo)), so the span covers the no-span
    # keys only where every window covers the ring: windows of 64 here.
    f = model("wide")
    toks = o.random_tokens(40, 300, seed=41)
    a, b = f.session(64), f.session(64)
    a.set_attend(10, 54)  # sink + ring covers every position
    assert np.array_equal(bits(a.forward(toks)), bits(b.forward(toks)))
    for t in o.random_tokens(5, 300, seed=42):
        assert np.array_equal(bits(a.forward([int(t)])), bits(b.forward([int(t)])))


def test_stale_slots_are_skipped_and_prefill_refeeds():
    f = model("one")
    sink, ring = 4, 32
    toks = o.random_tokens(60, 300, seed=43)

    def after_rollback(tt, new):
        s = f.session(96)
        s.set_attend(sink, ring)
        for t in tt:
            s.forward([int(t)], forward.OUT_NONE)
        s.rollback(3)  # 57..59 keep slots 25..27 (positions 25..27 had them)
        return s, s.forward([new])

    s0, base = after_rollback(toks, 5)
    # the step at 57 sees the sink and 26..57 of the ring, less 26 and 27,
    # whose slots the dropped positions 58 and 59 hold
    for p, seen in ((25, False), (26, False), (27, False), (28, True), (2, True), (56, True)):
        alt = toks.copy()
        alt[p] = (int(toks[p]) + 1) % 300
        _, got = after_rollback(alt, 5)
        assert (not np.array_equal(bits(got), bits(base))) == seen, p
    # prefill finds position 26 stale and re-feeds 26..56 and the new token
    s = f.session(96)
    s.set_attend(sink, ring)
    for t in toks:
        s.forward([int(t)], forward.OUT_NONE)
    s.rollback(3)
    got = s.prefill([5])
    fresh = f.session(96)
    fresh.set_attend(sink, ring)
    for t in toks[:26]:
        fresh.forward([int(t)], forward.OUT_NONE)
    want = fresh.forward(np.concatenate([toks[26:57], [5]]))
    assert len(s) == 58 and np.array_equal(bits(got), bits(want))
    # with AllLogits the re-feed returns a row for every position it feeds
    # (two new tokens end the ring at 59, so 27 is the first stale slot: 30
    # again and the two new ones), not only the new tokens'
    s2 = f.session(96)
    s2.set_attend(sink, ring)
    for t in toks:
        s2.forward([int(t)], forward.OUT_NONE)
    s2.rollback(3)
    rows = s2.prefill([5, 6], forward.OUT_ALL_LOGITS)
    fresh = f.session(96)
    fresh.set_attend(sink, ring)
    for t in toks[:27]:
        fresh.forward([int(t)], forward.OUT_NONE)
    want = fresh.forward(np.concatenate([toks[27:57], [5, 6]]), forward.OUT_ALL_LOGITS)
    assert rows.shape == want.shape == (32, 300) and np.array_equal(bits(rows), bits(want))


# ---------------------------------------------------------------- outputs
def test_outputs_rows_agree():
    f = model("small")
    toks = o.random_tokens(40, 300, seed=44)
    runs = {}
    for mode in (forward.OUT_NONE, forward.OUT_LAST_LOGITS, forward.OUT_ALL_LOGITS, forward.OUT_HIDDEN,
                 forward.OUT_LAST_HIDDEN):
        s = f.session(64)
        runs[mode] = (s.forward(toks, mode), s)
    assert runs[forward.OUT_NONE][0].shape[0] == 0
    allr, hid = runs[forward.OUT_ALL_LOGITS][0], runs[forward.OUT_HIDDEN][0]
    assert allr.shape == (40, 300) and hid.shape == (40, f.cfg.d)
    for r in (0, 31, 32, 39):
        assert np.array_equal(bits(f.head_logits(hid[r])), bits(allr[r])), r
    assert np.array_equal(bits(runs[forward.OUT_LAST_LOGITS][0][0]), bits(allr[-1]))
    assert np.array_equal(bits(runs[forward.OUT_LAST_HIDDEN][0][0]), bits(hid[-1]))
    assert np.array_equal(bits(runs[forward.OUT_LAST_HIDDEN][1].last_hidden()), bits(hid[-1]))
    # None advanced the session the same way
    s_none = runs[forward.OUT_NONE][1]
    s_last = runs[forward.OUT_LAST_LOGITS][1]
    assert np.array_equal(bits(s_none.forward([3])), bits(s_last.forward([3])))
    # sparse logits: NEG off the ids, the single-row kernel close to the full ones
    ids = np.array([0, 5, 17, 299], np.uint32)
    sp = f.head_logits_sparse(hid[-1], ids)
    neg = np.frombuffer(np.uint32(0xF149F2CA).tobytes(), np.float32)[0]
    mask = np.ones(300, bool)
    mask[ids] = False
    assert (sp[mask] == neg).all()
    assert np.abs(sp[ids] - allr[-1][ids]).max() <= 1e-5 * np.abs(allr[-1]).max()
