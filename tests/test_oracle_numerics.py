"""Pins of the oracle's arithmetic against closed forms, brute force and
restatements written from the reference's numerics spec
(docs/engine-rules.md:190-213) rather than from its code.  A dropped term,
a wrong sign or index, or a swapped rounding order fails one of these.
"""
import math

import numpy as np
import pytest

import oracle as o
from exactf32 import F32, f16_to_f32, fma32

K127 = np.uint32(0x3C010204).view(np.float32)


def sylvester(n):
    h = np.ones((1, 1), dtype=np.int64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


@pytest.mark.parametrize("n", [16, 32, 64, 128])
def test_fwht_exact_on_integers(n):
    # Integer inputs keep every partial sum exact in f32, so the butterfly
    # must equal the integer Sylvester product bit for bit.
    rng = np.random.default_rng(n)
    x = rng.integers(-1000, 1000, size=n)
    want = x @ sylvester(n)
    assert np.array_equal(o.fwht(x.astype(np.float32)), want.astype(np.float32))


@pytest.mark.parametrize("n", [16, 128])
def test_rotate_matches_dense(n):
    # crates/needle-core/src/quant.rs:293-304, extended to the group size.
    x = np.sin(np.arange(n, dtype=np.float32) * np.float32(0.37)).astype(np.float32)
    dense = x.astype(np.float64) @ (sylvester(n) / math.sqrt(n))
    assert np.allclose(o.rotate(x), dense, atol=1e-5)
    assert np.allclose(o.hadamard(n), sylvester(n) / math.sqrt(n), atol=0)
    assert int(np.float32(1.0 / math.sqrt(128.0)).view(np.uint32)) == 0x3DB504F3


def spec_quant(x):
    x = np.asarray(x, dtype=np.float32)
    m = np.max(np.abs(x)) if x.size else F32(0)
    s = F32(m * K127) if m > 0 else F32(1.0)
    inv = F32(F32(1.0) / s)
    v = (x * inv).astype(np.float64)  # the f32 products, widened exactly
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).clip(-128, 127).astype(np.int8)
    return q, s


@pytest.mark.parametrize("seed", range(4))
def test_quant_i8_spec(seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(128) * (10.0 ** rng.uniform(-3, 3))).astype(np.float32)
    q, s = o.quant_i8(x)
    wq, ws = spec_quant(x)
    assert s == ws and np.array_equal(q, wq)
    # All zero: scale 1, codes 0.
    q0, s0 = o.quant_i8(np.zeros(128, np.float32))
    assert s0 == 1.0 and not q0.any()


def test_quant_rounds_half_away():
    # Values landing exactly on .5 after scaling: 127 * k/254 with amax 1.
    x = np.zeros(128, np.float32)
    x[0] = 1.0
    inv = F32(1.0) / F32(F32(1.0) * K127)
    # find inputs whose scaled value is an exact half-integer
    cands = [F32(v) for v in np.linspace(-1, 1, 20001, dtype=np.float32) if float(F32(v) * inv) % 1 == 0.5]
    x[1: 1 + min(len(cands), 60)] = cands[:60]
    q, s = o.quant_i8(x)
    wq, ws = spec_quant(x)
    assert np.array_equal(q, wq)


def test_prep_group_layout():
    # act_pos (crates/needle-engine/src/qlinear.rs:145-147): 4-bit
    # (p % 2) * 64 + p / 2.  Group 2 of a 300-long row is zero-padded.
    rng = np.random.default_rng(7)
    x = rng.standard_normal(300).astype(np.float32)
    for g in range(3):
        buf = np.zeros(128, np.float32)
        seg = x[g * 128:(g + 1) * 128]
        buf[:seg.size] = seg
        nat, s = spec_quant(o.rotate(buf))
        q, qs = o.prep_group(x, g, 4)
        assert qs == s
        pos = np.array([(p % 2) * 64 + p // 2 for p in range(128)])
        assert np.array_equal(q[pos], nat)


def test_f16_conversion_matches_ieee():
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(allh.view(np.float16))
    got = o.f16_to_f32(allh[finite])
    assert np.array_equal(got.view(np.uint32), allh[finite].view(np.float16).astype(np.float32).view(np.uint32))
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.3),
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),  # f16 subnormals
        rng.uniform(6e4, 7e4, 500).astype(np.float32),  # overflow edge
    ])
    # exact halfway points between neighbouring f16 values (ties to even)
    h = rng.integers(0, 0x7BFF, 3000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    x = np.concatenate([x, ((lo + hi) / 2).astype(np.float32)])
    assert np.array_equal(o.f32_to_f16(x), x.astype(np.float16).view(np.uint16))


def test_cq_pack_spec():
    # quantize_group (crates/needle-core/src/quant.rs:127-135): rotate, sum of
    # squares in order, sqrt, nearest centroid of v / max(norm, 1e-12) with
    # ties low (argmin's first index); norm stored f16.
    rng = np.random.default_rng(11)
    rows, d = 3, 384
    w = (rng.standard_normal(rows * d) * 0.02).astype(np.float32)
    packed, norms = o.cq_pack(w, d)
    cb = o.codebook(4)
    for r in range(rows):
        codes = o.unpack_lsb(packed[r], 4, d)
        for g in range(d // 128):
            v = o.rotate(w[r * d + g * 128: r * d + (g + 1) * 128])
            acc = F32(0)
            for t in v:
                acc = F32(acc + F32(t * t))
            norm = F32(np.sqrt(acc))
            denom = max(norm, F32(1e-12))
            want = np.argmin(np.abs((v / denom)[:, None] - cb[None, :]), axis=1)
            assert np.array_equal(codes[g * 128:(g + 1) * 128], want)
            assert norms[r, g] == np.float16(norm).view(np.uint16)
            # orthonormal rotation keeps the norm
            assert abs(float(norm) - float(np.linalg.norm(w[r * d + g * 128: r * d + (g + 1) * 128]))) < 1e-5


def test_cq_roundtrip_error_bound():
    # Gaussian weights through CQ-4 keep ~20 dB SNR per group.
    rng = np.random.default_rng(5)
    out, d = 16, 512
    w = (rng.standard_normal(out * d) * 0.02).astype(np.float32).reshape(out, d)
    packed, norms = o.cq_pack(w, d)
    deq = o.cq_unpack(packed, norms, out, d)
    err = np.linalg.norm(deq - w, axis=1) / np.linalg.norm(w, axis=1)
    assert err.max() < 0.15


def ref_case():
    # crates/needle-engine/src/qlinear.rs:978-984
    out, din = 37, 384
    i = np.arange(out * din)
    w = (((i * 7919 % 1000).astype(np.float32) / F32(500.0) - F32(1.0)) * F32(0.05)).astype(np.float32)
    x = ((np.arange(din) * 31 % 97).astype(np.float32) / F32(48.0) - F32(1.0)).astype(np.float32)
    return out, din, w, x


def nibbles(q):
    c = q.codes
    return np.stack([c & 15, c >> 4], axis=-1).reshape(q.out, -1)


def brute_lanes(q, xq_row, bits=4):
    """Decode lanes by brute force: lane (p % 32) / 8, act at act_pos."""
    codes = nibbles(q) if bits == 4 else None
    vals = q.vals.astype(np.int64)
    g = q.groups
    out = np.zeros((q.out, g, 4), dtype=np.int64)
    pos = np.array([(p % 2) * 64 + p // 2 for p in range(128)])
    lane = np.array([(p % 32) // 8 for p in range(128)])
    for gi in range(g):
        x = xq_row[gi][pos].astype(np.int64)
        prod = vals[codes[:, gi * 128:(gi + 1) * 128]] * x[None, :]
        for l in range(4):
            out[:, gi, l] = prod[:, lane == l].sum(axis=1)
    return out


def spec_decode(lanes, sx, cbs, norms16):
    norms = f16_to_f32(norms16)
    y = []
    for r in range(lanes.shape[0]):
        acc = [F32(0)] * 4
        for g in range(lanes.shape[1]):
            sc = F32(F32(sx[g] * cbs) * norms[r, g])
            acc = [fma32(F32(lanes[r, g, l]), sc, acc[l]) for l in range(4)]
        y.append(F32(F32(acc[0] + acc[1]) + F32(acc[2] + acc[3])))
    return np.array(y, dtype=np.float32)


def spec_prefill(totals, sx, cbs, norms16, rows):
    # totals [rows, out, groups]
    norms = f16_to_f32(norms16)
    blocked = rows // 4 * 4
    y = np.zeros((rows, totals.shape[1]), dtype=np.float32)
    for t in range(rows):
        for r in range(totals.shape[1]):
            acc = F32(0)
            for g in range(totals.shape[2]):
                s = sx[t, g]
                sc = F32(F32(norms[r, g] * cbs) * s) if t < blocked else F32(norms[r, g] * F32(cbs * s))
                acc = fma32(F32(totals[t, r, g]), sc, acc)
            y[t, r] = acc
    return y


def test_reference_kernels_case_decode():
    # crates/needle-engine/src/qlinear.rs:976-990,1002-1005
    out, din, w, x = ref_case()
    q = o.OQMat.from_f32(w, out, din)
    p, nrm = o.cq_pack(w, din)
    deq = o.cq_unpack(p, nrm, out, din)
    a = o.OQAct.new(x, 1, din)
    y = q.matmul(a)[0]
    want = (x[None, :] * deq).sum(axis=1, dtype=np.float32)
    assert np.all(np.abs(y - want) < 0.02 * (1.0 + np.abs(want)))
    lanes = brute_lanes(q, a.xq[0])
    assert np.array_equal(q.all_lane_sums(a), lanes)
    assert np.array_equal(y.view(np.uint32), spec_decode(lanes, a.sx[0], q.cbs, q.norms).view(np.uint32))
    for r in range(out):
        assert y[r] == q.decode_row_ref(r, a)
    row = q.row(5)
    assert np.all(np.abs(row - deq[5]) < 1e-5)


@pytest.mark.parametrize("rows", [2, 3, 5, 9, 13, 17])
def test_reference_kernels_case_prefill(rows):
    # crates/needle-engine/src/qlinear.rs:991-1001
    out, din, w, _ = ref_case()
    q = o.OQMat.from_f32(w, out, din)
    xs = np.sin(np.arange(rows * din, dtype=np.float32) * F32(0.37)).astype(np.float32)
    a = o.OQAct.new(xs, rows, din)
    y = q.matmul(a)
    tot = q.all_totals(a)
    brute = np.stack([brute_lanes(q, a.xq[t]).sum(axis=2) for t in range(rows)])
    assert np.array_equal(tot, brute)
    want = spec_prefill(tot, a.sx, q.cbs, q.norms, rows)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_two_bit_reference_case():
    # crates/needle-engine/src/qlinear.rs:1008-1029: lane (p % 64) / 16,
    # act_pos (p % 4) * 32 + p / 4.
    out, din = 9, 256
    groups = din // 128
    codes = np.array([(i * 37) % 251 for i in range(out * din // 4)], dtype=np.uint8)
    norms = np.array([np.float16(np.float32(0.5) + np.float32(i) * np.float32(0.01)) for i in range(out * groups)],
                     dtype=np.float16).view(np.uint16)
    q = o.OQMat.build(out, din, 2, o.codebook(2), codes, norms)
    xs = np.cos(np.arange(5 * din, dtype=np.float32) * F32(0.21)).astype(np.float32)
    a1 = o.OQAct.new(xs[:din], 1, din, 2)
    y = q.matmul(a1)[0]
    # brute-force 2-bit lanes
    cz = np.stack([(codes >> (2 * k)) & 3 for k in range(4)], axis=-1).reshape(out, din)
    vals = q.vals.astype(np.int64)
    pos = np.array([(p % 4) * 32 + p // 4 for p in range(128)])
    lane = np.array([(p % 64) // 16 for p in range(128)])
    lanes = np.zeros((out, groups, 4), np.int64)
    for g in range(groups):
        x = a1.xq[0][g][pos].astype(np.int64)
        prod = vals[cz[:, g * 128:(g + 1) * 128]] * x[None, :]
        for l in range(4):
            lanes[:, g, l] = prod[:, lane == l].sum(axis=1)
    assert np.array_equal(q.all_lane_sums(a1), lanes)
    assert np.array_equal(y.view(np.uint32), spec_decode(lanes, a1.sx[0], q.cbs, q.norms).view(np.uint32))
    a5 = o.OQAct.new(xs, 5, din, 2)
    y5 = q.matmul(a5)
    want = spec_prefill(q.all_totals(a5), a5.sx, q.cbs, q.norms, 5)
    assert np.array_equal(y5.view(np.uint32), want.view(np.uint32))


def spec_dot16(x, y):
    a = [[F32(0)] * 4 for _ in range(4)]
    for c in range(x.size // 16):
        for j in range(4):
            for l in range(4):
                i = c * 16 + j * 4 + l
                a[j][l] = fma32(x[i], y[i], a[j][l])
    t = [F32(F32(F32(a[2][l] + a[3][l]) + a[1][l]) + a[0][l]) for l in range(4)]
    return F32(F32(t[0] + t[1]) + F32(t[2] + t[3]))


def test_norms_spec():
    # docs/engine-rules.md:199-201; crates/needle-engine/src/infer.rs:369-473
    rng = np.random.default_rng(2)
    x = rng.standard_normal(768).astype(np.float32)
    s16 = (rng.standard_normal(768) * 0.1).astype(np.float16).view(np.uint16)
    ss = o.dot16(x, x)
    assert ss == spec_dot16(x, x)
    assert abs(float(ss) - float(np.dot(x.astype(np.float64), x))) < 1e-4 * float(ss)
    r = F32(F32(1.0) / np.sqrt(F32(F32(ss / F32(768)) + F32(1e-6))))
    assert o.rinv(float(ss), 768) == r
    s = f16_to_f32(s16)
    want = np.array([fma32(F32(v * r), sv, F32(v * r)) for v, sv in zip(x, s)], dtype=np.float32)
    assert np.array_equal(o.zcn16(x, s16).view(np.uint32), want.view(np.uint32))


def test_qlinear_merge():
    # QLinear::new merges neighbours with the same codebook
    # (crates/needle-engine/src/qlinear.rs:501-519); output side by side.
    rng = np.random.default_rng(9)
    parts_w = [(rng.standard_normal(n * 256) * 0.02).astype(np.float32) for n in (24, 8, 40)]
    parts = [o.OQMat.from_f32(w, w.size // 256, 256) for w in parts_w]
    lin = o.OQLinear(parts)
    assert lin.nparts == 1 and lin.out == 72
    x = rng.standard_normal(3 * 256).astype(np.float32)
    a = o.OQAct.new(x, 3, 256)
    y = lin.matmul(a)
    cols = np.concatenate([p.matmul(a) for p in parts], axis=1)
    assert np.array_equal(y, cols)


def argmax_ref(x):
    """generate::argmax (crates/needle-engine/src/generate.rs:42-50) as written."""
    best = 0
    for i, v in enumerate(x):
        if v > x[best]:
            best = i
    return best


def argmax_cases():
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    rng = np.random.default_rng(17)
    base = rng.normal(size=5000).astype(np.float32)
    cases = [base.copy()]
    for spots in ([0], [1], [3000], [0, 4999], list(range(0, 5000, 7))):
        c = base.copy()
        c[spots] = nan
        cases.append(c)
    ties = np.zeros(3000, np.float32)
    ties[[17, 1800, 2999]] = 2.0
    cases += [ties, np.full(100, -inf, np.float32), np.array([nan, nan, 3.0], np.float32),
              np.array([-inf, nan, -inf], np.float32), np.array([1.0, inf, nan, inf], np.float32)]
    return cases


def test_argmax_rule():
    for x in argmax_cases():
        assert o.argmax(x) == argmax_ref(list(x))
