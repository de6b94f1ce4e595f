"""Pins of four computations of the oracle's Needle-3 step (oracle/forward.c)
by what the mathematics or the model's structure fixes, independently of
the restatement's code:

- the qkv conv taps (crates/needle-engine/src/infer/step.rs:502-523): the
  helper with a unit impulse at lag j returns the row of pos - j exactly
  (zero where the history does not hold it), and random taps give the
  float64 sum over taps; through a one-layer model, impulse taps at lag j
  leave in the KV slot of position p exactly what impulse taps at lag 0
  leave for the same token fed at p - j (keys after their norm and RoPE at
  p, values as they are), zeros before the start of the history, also
  after rewind_zeroed;
- the engram value history and dilated conv (infer.rs:1283-1325): the
  history of a position is the int8 quantization, in groups of 32, of the
  value matrix's product with the position's engram input row (the value
  half of key | value); the conv equals the float64 sum over taps j < 4 of
  taps_j * deq(v8[pos - j dil]) (a conv without the dilation fails);
- the engram gate (infer.rs:1409-1412): for x = k, alpha = sigmoid(sqrt(d)
  m / (m + 1e-6)) with m = mean(x^2) (and the negative for x = -k), a
  vector orthogonal to k gives 1/2, and random pairs give
  sigmoid(cos(x, k) sqrt(d) (normalisation with the 1e-6 term)) in float64;
- the Hadamard MLP (infer.rs:1610-1694): with identity Kronecker factors
  and permutations, d1..d4 = 1, b2 = 0 and cond_u = 0 it is exactly
  x / (nexp(-x) + 1) of h2 (the SiLU, within 1e-6 of float64); with random
  factors, permutations, scales and conditioning it equals a float64 dense
  restatement from the Kronecker definition (kron(z, A, B) = A^T Z B,
  infer.rs:2322-2330), which fixes which factor serves which pass, where
  perm1 / perm2, d1..d4 and b2 apply, and the SiLU's place;
- RoPE (infer.rs:942-947,1716-1747): freq[i] within 2e-6 of float64
  theta^(-2i/qk), (sd, cd) within an f32 ulp of sin / cos of freq, a
  chunk's rows within an f32 ulp of sin / cos of the f32 product
  freq * pos, and the single-token recurrence within 2e-7 per step of
  float64 cos / sin of its start row's angle plus freq a step, over 100
  steps (a wrong sign fails).
"""
import numpy as np
import pytest

import oracle as o
from oracle import cact, forward

F = np.float32


def bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def f16(x):
    """Values rounded to f16 (exact in f32 and float64)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def tensors(g, seed):
    return cact.needle3_tensors(g, seed=seed, kind=lambda n: ("cq", 4) if n == "embedding" else ("random", 4))[0]


def build(g, ts):
    return forward.Forward(cact.pack(ts, g.header()))


# ------------------------------------------------------------- conv taps
def test_conv_taps_impulse_and_sum():
    rng = np.random.default_rng(1)
    taps, cw = 4, 80
    rows = [rng.standard_normal(cw).astype(F) for _ in range(taps)]
    for j in range(taps):
        w = np.zeros((taps, cw), np.float32)
        w[j] = 1.0
        w16 = o.f32_to_f16(w.reshape(-1)).reshape(taps, cw)
        got = forward.Forward.conv_taps(rows, w16)
        assert np.array_equal(bits(got), bits(rows[j])), j
        if j > 0:
            held = [r if i < j else None for i, r in enumerate(rows)]  # the history stops before pos - j
            assert np.all(forward.Forward.conv_taps(held, w16) == 0.0), j
    w = f16(rng.uniform(-1, 1, (taps, cw)))
    w16 = o.f32_to_f16(w.reshape(-1)).reshape(taps, cw)
    for held in (taps, 2):
        rr = [r if i < held else None for i, r in enumerate(rows)]
        want = sum(w[i].astype(np.float64) * rows[i].astype(np.float64) for i in range(held))
        got = forward.Forward.conv_taps(rr, w16).astype(np.float64)
        scale = sum(np.abs(w[i].astype(np.float64) * rows[i]) for i in range(held))
        assert np.all(np.abs(got - want) <= 1e-6 * scale + 1e-30), held


ONE3 = dict(vocab=300, num_layers=1, qkv_conv_taps=3, engram_sites=(), global_layers=(0,), sliding_window=0,
            engram_slots=64)


def impulse_model(lag, seed=31):
    """A one-layer, three-tap model whose q, k and v taps are a unit impulse at `lag`."""
    g = cact.Geometry(**ONE3)
    ts = tensors(g, seed)
    qd, kd, vdim = g.num_heads * g.qk_head_dim, g.num_kv_heads * g.qk_head_dim, g.num_kv_heads * g.v_head_dim
    for off, cw in ((4, qd), (5, kd), (6, vdim)):  # the layer block's q, k, v tap records
        w = np.zeros((g.qkv_conv_taps, cw), np.float32)
        w[lag] = 1.0
        ts[1 + off] = cact.fp16(w)
    return build(g, ts), g


def test_conv_taps_through_the_model():
    base, g = impulse_model(0)
    n = 24
    toks = o.random_tokens(n, 300, seed=32)
    for lag in (1, 2):
        f, _ = impulse_model(lag)
        a = f.session(64)
        a.forward(toks)  # a chunk of 24
        shifted = np.concatenate([toks[:lag], toks[:n - lag]]).astype(np.uint32)  # token p - lag at p
        b = base.session(64)
        b.forward(shifted)
        for p in range(n):
            ka, ksa, va, vsa = a.kv(0, p)
            if p < lag:  # before the history's first row: a zero row, no key or value
                assert not ka.any() and not va.any(), (lag, p)
                continue
            kb, ksb, vb, vsb = b.kv(0, p)
            assert np.array_equal(ka, kb) and np.array_equal(va, vb), (lag, p)
            assert np.array_equal(bits(ksa), bits(ksb)) and np.array_equal(bits(vsa), bits(vsb)), (lag, p)
        # rewind_zeroed: the history starts over at position 10
        a.rewind_zeroed(10)
        new = o.random_tokens(12, 300, seed=33 + lag)
        a.forward(new)  # positions 10..21
        ref = np.concatenate([toks[:10], new]).astype(np.uint32)
        b2 = base.session(64)
        b2.forward(np.concatenate([ref[:10 + lag], ref[10:22 - lag]]).astype(np.uint32))
        for p in range(10, 22):
            ka, _, va, _ = a.kv(0, p)
            if p < 10 + lag:
                assert not ka.any() and not va.any(), (lag, p)
            else:
                kb, _, vb, _ = b2.kv(0, p)
                assert np.array_equal(ka, kb) and np.array_equal(va, vb), (lag, p)


# ---------------------------------------------------------------- engram
SMALL = dict(vocab=300, num_layers=3, engram_slots=64, engram_sites=(1,), global_layers=(1,), sliding_window=8)


def test_engram_history_and_conv():
    g = cact.Geometry(**SMALL)
    ts = tensors(g, 41)
    data = cact.pack(ts, g.header())
    f = forward.Forward(data)
    a = cact.Archive(data)
    d = g.d_model
    # the site's records: table, key, value, taps (weights.rs canonical order, after the perms)
    per_layer = 27
    i_site = 1 + g.num_layers * per_layer + 6 + 3 + 2
    packed, norms, out, in_dim, bits_ = a.cq(i_site + 2)
    value = o.OQMat.from_cq(packed, norms, out, in_dim, bits_)
    taps = np.frombuffer(a.bytes(i_site + 3), dtype=np.float16).astype(np.float64).reshape(4, d)
    dil = max(g.engram_orders)
    s = f.session(64)
    toks = o.random_tokens(20, 300, seed=42)
    for t in toks:
        s.forward([int(t)], forward.OUT_NONE)  # one row a feed: the decode combine
    for pos in range(20):
        er = np.zeros(d, np.float32)
        forward._lib().nf_engram_input(f.m, 0, o._p(toks), pos, o._p(er))
        v = value.matmul(o.OQAct.new(er, 1, d, value.bits))[0]
        v8, vs = s.engram_hist(0, pos)
        for gi in range(d // 32):
            q, sc = o.quant_i8(v[gi * 32:(gi + 1) * 32])
            assert np.array_equal(q, v8[gi * 32:(gi + 1) * 32]) and np.float32(sc) == vs[gi], (pos, gi)
    for pos in range(20):
        want = np.zeros(d)
        undil = np.zeros(d)
        for j in range(4):
            for acc, step in ((want, dil), (undil, 1)):
                if pos >= j * step:
                    v8, vs = s.engram_hist(0, pos - j * step)
                    acc += taps[j] * (np.repeat(vs.astype(np.float64), 32) * v8)
        got = s.engram_conv(0, pos).astype(np.float64)
        scale = max(np.abs(want).max(), 1e-30)
        assert np.abs(got - want).max() <= 1e-6 * scale, pos
        if pos >= 2:  # (position 0's engram row is all zeros: no order is reached yet)
            assert np.abs(got - undil).max() > 1e-3 * scale, pos  # the dilation matters


def sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def test_engram_gate():
    f = forward.Forward(cact.pack(tensors(cact.Geometry(**SMALL), 43), cact.Geometry(**SMALL).header()))
    rng = np.random.default_rng(44)
    d = 768
    for scale in (0.01, 1.0, 30.0):
        x = (rng.standard_normal(d) * scale).astype(F)
        m = np.mean(x.astype(np.float64) ** 2)
        want = sigmoid(np.sqrt(d) * m / (m + 1e-6))
        assert abs(f.engram_gate(x, x) - want) < 1e-6, scale
        assert abs(f.engram_gate(x, -x) - sigmoid(-np.sqrt(d) * m / (m + 1e-6))) < 1e-6, scale
        k = rng.standard_normal(d)
        k -= k @ x.astype(np.float64) / (x.astype(np.float64) @ x) * x
        assert abs(f.engram_gate(x, k.astype(F)) - 0.5) < 1e-5, scale
    for _ in range(20):
        x = rng.standard_normal(d).astype(F)
        k = (0.5 * x + rng.standard_normal(d)).astype(F)
        x64, k64 = x.astype(np.float64), k.astype(np.float64)
        xn = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6)
        kn = k64 / np.sqrt(np.mean(k64 ** 2) + 1e-6)
        want = sigmoid(xn @ kn / np.sqrt(d))
        assert abs(f.engram_gate(x, k) - want) < 1e-6


# ------------------------------------------------------------------- MLP
def _mlp_model(seed):
    g = cact.Geometry(**SMALL)
    return forward.Forward(cact.pack(tensors(g, seed), g.header())), g


def _silu_nexp(x):
    x = np.asarray(x, np.float32)
    return np.array([F(v) / (F(forward._lib().nf_nexp(float(-v))) + F(1.0)) for v in x], dtype=np.float32)


def test_hada_mlp_identity_is_silu():
    f, g = _mlp_model(45)
    d, hn = g.d_model, g.hada_n
    eye = np.eye(32, dtype=np.float32)
    for k in range(6):
        f.set_layer_f16(0, forward.KRON0 + k, eye)
    for which in (forward.D1, forward.D2, forward.D3, forward.D4):
        f.set_layer_f16(0, which, np.ones(hn, np.float32))
    f.set_layer_f16(0, forward.B2, np.zeros(hn, np.float32))
    f.set_layer_f16(0, forward.COND_U, np.zeros((8, hn), np.float32))
    f.set_perms(np.arange(hn), np.arange(hn))
    rng = np.random.default_rng(46)
    h2 = (rng.standard_normal(d) * 2).astype(F)
    got = f.hada_mlp(0, h2)
    assert np.array_equal(bits(got), bits(_silu_nexp(h2)))
    x = h2.astype(np.float64)
    assert np.abs(got - x * sigmoid(x)).max() <= 1e-6 * np.abs(x).max()


def mlp64(h2, A, B, d1, d2, b2, d3, d4, cond_v, cond_u, perm1, perm2, d):
    """The Hadamard MLP in float64 from its definition: cond softmax, three
    stages T = A^T Z B over Z = the vector as 32 x 32 rows, SiLU after the
    first, perm1 / d2 / b2 / cond into the first, perm2 / d3 into the
    second, d4 on the output."""
    h = h2.astype(np.float64)
    lg = h @ cond_v.astype(np.float64)  # [8]
    w = np.exp(lg - lg.max())
    w /= w.sum()
    hn = 1024
    z = np.zeros(hn)
    z[:d] = h * d1[:d]
    t = (A[0].T @ z.reshape(32, 32) @ B[0]).reshape(-1)
    cond = 1.0 + w @ cond_u.astype(np.float64)
    zs = t[perm1] * cond * d2 + b2
    zs = zs * sigmoid(zs)
    t = (A[1].T @ zs.reshape(32, 32) @ B[1]).reshape(-1)
    zs = t[perm2] * d3
    t = (A[2].T @ zs.reshape(32, 32) @ B[2]).reshape(-1)
    return t[:d] * d4[:d]


def test_hada_mlp_random_matches_the_definition():
    f, g = _mlp_model(47)
    d, hn = g.d_model, g.hada_n
    rng = np.random.default_rng(48)
    A = [f16(rng.uniform(-0.4, 0.4, (32, 32))) for _ in range(3)]
    B = [f16(rng.uniform(-0.4, 0.4, (32, 32))) for _ in range(3)]
    for k in range(3):
        f.set_layer_f16(0, forward.KRON0 + 2 * k, A[k])
        f.set_layer_f16(0, forward.KRON0 + 2 * k + 1, B[k])
    vals = {}
    for which, lo, hi in ((forward.D1, 0.5, 1.5), (forward.D2, 0.5, 1.5), (forward.D3, 0.5, 1.5),
                          (forward.D4, 0.5, 1.5), (forward.B2, -0.5, 0.5)):
        vals[which] = f16(rng.uniform(lo, hi, hn))
        f.set_layer_f16(0, which, vals[which])
    cond_v = f16(rng.uniform(-0.2, 0.2, (d, 8)))
    cond_u = f16(rng.uniform(-0.5, 0.5, (8, hn)))
    f.set_layer_f16(0, forward.COND_V, cond_v)
    f.set_layer_f16(0, forward.COND_U, cond_u)
    perm1, perm2 = rng.permutation(hn), rng.permutation(hn)
    f.set_perms(perm1, perm2)
    for trial in range(3):
        h2 = rng.standard_normal(d).astype(F)
        got = f.hada_mlp(0, h2).astype(np.float64)
        args = (A, B, vals[forward.D1], vals[forward.D2], vals[forward.B2], vals[forward.D3], vals[forward.D4],
                cond_v, cond_u)
        want = mlp64(h2, *args, perm1, perm2, d)
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 1e-4 * scale, (trial, np.abs(got - want).max() / scale)
        # plausible misreadings fail: the factors of a stage swapped, the permutations swapped
        swapped = mlp64(h2, A, [a.T for a in B], *args[2:], perm1, perm2, d)
        assert np.abs(got - swapped).max() > 1e-2 * scale
        assert np.abs(got - mlp64(h2, *args, perm2, perm1, d)).max() > 1e-2 * scale


# ------------------------------------------------------------------ RoPE
def test_rope_tables_and_rows():
    g = cact.Geometry(**SMALL)
    f = forward.Forward(cact.pack(tensors(g, 49), g.header()))
    qk, theta = g.qk_head_dim, g.rope_theta
    half = qk // 2
    fr, sd, cd = f.rope_tables()
    i = np.arange(half)
    want = np.float64(theta) ** (-2.0 * i / qk)
    assert np.all(np.abs(fr - want) <= 2e-6 * want)
    fr64 = fr.astype(np.float64)
    assert np.all(np.abs(sd - np.sin(fr64)) <= np.spacing(np.float32(1.0)))
    assert np.all(np.abs(cd - np.cos(fr64)) <= np.spacing(np.float32(1.0)))
    # a chunk's rows: sincos of the f32 product freq * pos
    s = f.session(160)
    s.forward(o.random_tokens(40, 300, seed=50))
    ulp = np.spacing(np.float32(1.0)) / 2
    for p in range(40):
        c, sn = s.rope(p)
        ang = (fr * np.float32(p)).astype(np.float64)
        assert np.all(np.abs(c - np.cos(ang)) <= ulp) and np.all(np.abs(sn - np.sin(ang)) <= ulp), p
    # single tokens after it: the recurrence from the chunk's last row (the
    # angle f32(freq * 39)), advancing by freq a step and drifting by at most
    # ~2e-7 a step (the tables' and the fmas' roundings)
    a39 = (fr * np.float32(39)).astype(np.float64)

    def ang(p):
        return a39 + (p - 39) * fr64

    for k, t in enumerate(o.random_tokens(100, 300, seed=51)):
        s.forward([int(t)], forward.OUT_NONE)
        p = 40 + k
        c, sn = s.rope(p)
        err = max(np.abs(c - np.cos(ang(p))).max(), np.abs(sn - np.sin(ang(p))).max())
        assert err <= 2e-7 * (k + 1), (k, err)
    # the recurrence's signs: a flipped one drifts off at once
    c0, s0 = s.rope(139)
    cs, sn = f.rope_rows(140, 1, (c0, s0))
    assert np.abs(cs[0] - np.cos(ang(140))).max() <= 2e-7 * 101
    assert np.abs(sn[0] - np.sin(ang(140))).max() <= 2e-7 * 101
    bad = (cd * c0 + sd * s0).astype(np.float64)  # cos(a - b)
    assert np.abs(bad - np.cos(ang(140))).max() > 1e-3
