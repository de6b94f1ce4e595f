"""The oracle's Needle-3 decode step (oracle/forward.c), on the CPU.

Helpers, each against what fixes it independently of the restatement:
- nexp: the reference's own test (crates/needle-engine/src/infer.rs:3078-3084);
- mix8: exact on small integers against numpy's matmul, both layouts and a
  tile prefix;
- sinkhorn64: doubly stochastic after 20 rounds, a constant input gives 1/4;
- digits21: the three digits rebuild round(w * qw) exactly;
- chunk_exp: numerators within nexp's bound of exp, the sum within 1e-6;
- cond_weights: the softmax of h2 . cond_v;
- rope_rotate: a rotation (norms kept, angles add).

The step itself is parity unpinned as a whole (no reference fixtures
exist); what pins its structure here: determinism across sessions, and the
attention window.  With every layer windowed and no engram, the logits at a
position cannot depend on a token more than layers x (window + taps) back,
so changing token 0 must leave late logits bit-identical; with a global
layer it must change them.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as o
from oracle import cact, forward

F = np.float32


def lib():
    return forward._lib()


def test_nexp_close_to_exp():
    for i in range(-200, 200):
        x = F(i) * F(0.37)
        a = lib().nf_nexp(float(x))
        b = np.exp(np.float64(x))
        assert abs(a - b) <= 2e-7 * max(b, 1e-30), (x, a, b)


@pytest.mark.parametrize("transpose", [0, 1])
def test_mix8_exact_on_integers(transpose):
    rng = np.random.default_rng(3)
    ct = rng.integers(-4, 5, size=(32, 32)).astype(F)
    rows = rng.integers(-4, 5, size=(32, 32)).astype(F)
    out = np.zeros((32, 32), F)
    lib().nf_mix8(transpose, o._p(ct), 0, o._p(rows), 0, o._p(out), 16)
    want = (ct.astype(np.int64).T @ rows.astype(np.int64)).astype(F)
    assert np.array_equal(out, want.T if transpose else want)
    # a tile prefix writes only its rows
    part = np.full((32, 32), F(7.0))
    lib().nf_mix8(0, o._p(ct), 0, o._p(rows), 0, o._p(part), 12)
    assert np.array_equal(part[:24], want[:24]) and (part[24:] == 7.0).all()
    # f16 coefficients widen exactly
    ct16 = o.f32_to_f16(ct.reshape(-1))
    out16 = np.zeros((32, 32), F)
    lib().nf_mix8(transpose, o._p(ct16), 1, o._p(rows), 0, o._p(out16), 16)
    assert np.array_equal(out16, out)


def test_sinkhorn64():
    rng = np.random.default_rng(4)
    z = rng.uniform(-3, 3, 16).astype(F)
    out = np.zeros(16, F)
    lib().nf_sinkhorn64(o._p(z), o._p(out))
    m = out.reshape(4, 4).astype(np.float64)
    assert (m > 0).all()
    assert np.allclose(m.sum(axis=0), 1.0, atol=1e-6) and np.allclose(m.sum(axis=1), 1.0, atol=1e-3)
    const = np.full(16, F(0.7))
    lib().nf_sinkhorn64(o._p(const), o._p(out))
    assert (out == F(0.25)).all()


def test_digits21_rebuild():
    rng = np.random.default_rng(5)
    w = rng.uniform(0, 1, 1000).astype(F)
    w[0], w[1] = 0.0, 1.0
    qw = F(2097144.0) / F(w.max())
    hi, mid, lo = (np.zeros(1000, np.int8) for _ in range(3))
    lib().nf_digits21(o._p(w), w.size, float(qw), o._p(hi), o._p(mid), o._p(lo))
    x = w.astype(np.float32) * qw
    wq = np.where(x >= 0, np.floor(x.astype(np.float64) + 0.5), np.ceil(x.astype(np.float64) - 0.5)).astype(np.int64)
    assert np.array_equal(16384 * hi.astype(np.int64) + 128 * mid.astype(np.int64) + lo.astype(np.int64), wq)
    assert (mid >= 0).all() and (lo >= 0).all() and (mid < 128).all() and (lo < 128).all()


@pytest.mark.parametrize("l", [1, 3, 4, 7, 8, 13, 16, 37])
def test_chunk_exp(l):
    rng = np.random.default_rng(l)
    s = rng.uniform(-8, 0, l).astype(F)
    m = F(s.max())
    e = s.copy()
    total = lib().nf_chunk_exp(o._p(e), l, float(m))
    ref = np.exp((s - m).astype(np.float64))
    assert np.all(np.abs(e - ref) <= 2.5e-7 * ref + 1e-30)
    assert abs(total - ref.sum()) <= 1e-6 * ref.sum()


def test_cond_weights_softmax():
    rng = np.random.default_rng(6)
    h2 = rng.standard_normal(768).astype(F)
    cv = o.f32_to_f16((rng.standard_normal(768 * 8) * 0.05).astype(F))
    out = np.zeros(8, F)
    lib().nf_cond_weights(o._p(h2), 768, o._p(cv), o._p(out))
    lg = h2.astype(np.float64) @ o.f16_to_f32(cv).reshape(768, 8).astype(np.float64)
    sm = np.exp(lg - lg.max())
    sm /= sm.sum()
    assert np.allclose(out, sm, rtol=1e-5, atol=1e-7) and abs(out.sum() - 1) < 1e-6


def test_rope_rotation():
    rng = np.random.default_rng(7)
    x = rng.standard_normal(48).astype(F)
    a, b = rng.uniform(0, 6, 24).astype(F), rng.uniform(0, 6, 24).astype(F)
    ca, sa, cb, sb = (np.cos(a).astype(F), np.sin(a).astype(F), np.cos(b).astype(F), np.sin(b).astype(F))
    ab = (a.astype(np.float64) + b.astype(np.float64))
    y = x.copy()
    lib().nf_rope_rotate(o._p(y), 48, o._p(ca), o._p(sa))
    lib().nf_rope_rotate(o._p(y), 48, o._p(cb), o._p(sb))
    xc = x[:24].astype(np.complex128) + 1j * x[24:].astype(np.complex128)
    want = xc * np.exp(1j * ab)
    assert np.allclose(y[:24], want.real, atol=1e-5) and np.allclose(y[24:], want.imag, atol=1e-5)
    assert np.allclose(np.abs(y[:24] + 1j * y[24:]), np.abs(xc), rtol=1e-5)


def test_key_chunks():
    # key_chunks (infer.rs:2093-2101) with NATIVE_TEAM 4, nkv 2 (k = 4)
    def kc(n):
        cnt, size = C.c_size_t(), C.c_size_t()
        lib().nf_key_chunks(n, 2, C.byref(cnt), C.byref(size))
        return cnt.value, size.value
    assert kc(1) == (1, 16)
    assert kc(100) == (1, 112)
    assert kc(300) == (4, 80)
    assert kc(2000) == (8, 256)


def _model(global_layers, sites, window, seed=3):
    g = cact.Geometry(vocab=300, num_layers=3, engram_slots=64, engram_sites=sites, global_layers=global_layers,
                      sliding_window=window)
    ts, _ = cact.needle3_tensors(g, seed=seed, kind=lambda n: ("cq", 4) if n == "embedding" else ("random", 4))
    return forward.Forward(cact.pack(ts, g.header()))


def test_step_deterministic():
    f = _model((1,), (1,), 4)
    toks = o.random_tokens(12, 300, seed=2)
    a, b = f.session(32), f.session(32)
    for t in toks:
        la, lb = a.step(t), b.step(t)
        assert np.isfinite(la).all() and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert len(a) == 12


def test_attention_window_bounds_the_receptive_field():
    f = _model((), (), 3)
    toks = o.random_tokens(24, 300, seed=9)
    alt = toks.copy()
    alt[0] = (alt[0] + 1) % 300
    s1, s2 = f.session(32), f.session(32)
    outs = [(s1.step(a), s2.step(b)) for a, b in zip(toks, alt)]
    # 3 layers x (window 3 + 2 taps rows): positions >= 15 cannot see token 0
    assert not np.array_equal(outs[1][0], outs[1][1])
    for p in range(15, 24):
        assert np.array_equal(outs[p][0].view(np.uint32), outs[p][1].view(np.uint32)), p
    # with a global layer the first token is seen everywhere
    fg = _model((1,), (), 3)
    g1, g2 = fg.session(32), fg.session(32)
    last = [(g1.step(a), g2.step(b)) for a, b in zip(toks, alt)][-1]
    assert not np.array_equal(last[0], last[1])


# ------------------------------------------------------------ prompt chunks
# chunk_job (infer/chunk.rs:32-358) is the step's arithmetic row for row
# except the projections (the prefill combine over the chunk's rows), the
# RoPE rows (sincosf per position) and attention (nested chunking).  What
# pins it beyond the shared, step-checked code: a chunk's logits stay
# within the combines' rounding of the step-by-step feed; the same window
# bound; determinism; a chunk fed after steps and steps after a chunk.

def _rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


def test_chunk_close_to_steps():
    f = _model((1,), (1,), 8)
    toks = o.random_tokens(40, 300, seed=21)
    a, b = f.session(48), f.session(48)
    for t in toks:
        la = a.step(t)
    lb = b.feed(toks)   # 32 + 8
    assert len(a) == len(b) == 40
    assert not np.array_equal(la, lb)        # a different combine order
    assert _rel(lb, la) < 2e-2 and int(np.argmax(lb)) == int(np.argmax(la))


def test_chunk_deterministic_and_split_invariant_state():
    f = _model((1,), (1,), 8)
    toks = o.random_tokens(24, 300, seed=22)
    a, b = f.session(40), f.session(40)
    la, lb = a.feed(toks), b.feed(toks)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    # a step after the chunk continues from the chunk's RoPE row and caches
    na, nb = a.step(7), b.step(7)
    assert np.array_equal(na.view(np.uint32), nb.view(np.uint32)) and len(a) == 25


def test_chunk_window_bounds_the_receptive_field():
    f = _model((), (), 3)
    toks = o.random_tokens(24, 300, seed=23)
    alt = toks.copy()
    alt[0] = (alt[0] + 1) % 300
    s1, s2 = f.session(32), f.session(32)
    # tokens 0..15 as one chunk, then 16..23 as one chunk: the last logits
    # (position 23 >= 3 x (3 + 2)) cannot see token 0
    s1.chunk(toks[:16]), s2.chunk(alt[:16])
    l1, l2 = s1.chunk(toks[16:]), s2.chunk(alt[16:])
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))
    fg = _model((1,), (), 3)
    g1, g2 = fg.session(32), fg.session(32)
    assert not np.array_equal(g1.feed(toks), g2.feed(alt))


def test_chunk_rejects_overflow():
    f = _model((1,), (1,), 8)
    s = f.session(8)
    with pytest.raises(ValueError):
        s.chunk(o.random_tokens(9, 300, seed=1))
