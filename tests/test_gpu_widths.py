"""GPU parity for the other CQ record widths and group counts.

2-bit and ternary records (crates/needle-core/src/quant.rs:12,51-60,286;
crates/needle-engine/src/qlinear.rs:142-147,218-265,325-337): upload with
the ternary code remap, the 2-bit activation layout, the decode lanes
(p % 64) / 16, the prefill combine, row lookups and single rows, each
bit-exact against the oracle.  Also group counts outside the common
shapes (in_dim 896, 1664, 200) on both widths.
"""
import sys

import numpy as np
import pytest
import torch

import oracle as o

pytestmark = pytest.mark.gpu
F = np.float32


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bits_equal(a, b):
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def report(got, want):
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    return f"max_abs={d.max():.3e} mismatches={(got != want).sum()}"


def random_record(out, in_dim, bits, seed):
    """Random archive bytes and f16 norms for a `bits`-bit record (5 =
    ternary, packed at 2 bits)."""
    rng = np.random.default_rng(seed)
    groups = (in_dim + 127) // 128
    cbits = 2 if bits == 5 else bits
    packed = rng.integers(0, 256, size=(out, groups * 128 * cbits // 8), dtype=np.uint8)
    norms = np.float16(rng.uniform(0.2, 3.0, size=(out, groups))).view(np.uint16)
    return packed, norms


def check_product(nh, packed, norms, out, in_dim, bits, M, seed):
    q = nh.QMat.from_cq(packed, norms, out, in_dim, bits)
    oq = o.OQMat.from_cq(packed, norms, out, in_dim, bits)
    abits = q.act_bits()
    assert abits == (2 if bits in (2, 5) else 4)
    x = o.seeded_normals([M * in_dim], seed)[0]
    a = nh.QAct.new(dev(x), M, in_dim, abits)
    oa = o.OQAct.new(x, M, in_dim, abits)
    xq, sx = a.download()
    assert np.array_equal(xq.reshape(-1), oa.xq.reshape(-1)) and bits_equal(sx.reshape(-1), oa.sx.reshape(-1))
    y = q.matmul(a).cpu().numpy()
    want = oq.matmul(oa)
    assert bits_equal(y, want), report(y, want)
    part = q.partials(a).cpu().numpy()
    if M == 1:
        assert np.array_equal(part, oq.all_lane_sums(oa))
    else:
        assert np.array_equal(part, oq.all_totals(oa))
    return q, oq, a, oa


def test_two_bit_reference_case(nh):
    # crates/needle-engine/src/qlinear.rs:1003-1029: out 9, in 256, codes
    # (i * 37) % 251, norms 0.5 + 0.01 i, x = cos(0.21 i).
    say("2-bit reference case out=9 in=256")
    out, din = 9, 256
    codes = np.array([(i * 37) % 251 for i in range(out * din // 4)], dtype=np.uint8).reshape(out, din // 4)
    norms = np.array([np.float16(F(0.5) + F(i) * F(0.01)) for i in range(out * din // 128)],
                     dtype=np.float16).view(np.uint16).reshape(out, din // 128)
    q = nh.QMat.from_cq(codes, norms, out, din, 2)
    oq = o.OQMat.build(out, din, 2, o.codebook(2), codes.reshape(-1), norms.reshape(-1))
    xs = np.cos(np.arange(5 * din, dtype=F) * F(0.21)).astype(F)
    a1 = nh.QAct.new(dev(xs[:din]), 1, din, 2)
    a5 = nh.QAct.new(dev(xs), 5, din, 2)
    o1 = o.OQAct.new(xs[:din], 1, din, 2)
    o5 = o.OQAct.new(xs, 5, din, 2)
    assert bits_equal(q.matmul(a1).cpu().numpy()[0], oq.matmul(o1)[0])
    assert np.array_equal(q.partials(a1).cpu().numpy(), oq.all_lane_sums(o1))
    assert bits_equal(q.matmul(a5).cpu().numpy(), oq.matmul(o5))
    assert np.array_equal(q.partials(a5).cpu().numpy(), oq.all_totals(o5))


@pytest.mark.parametrize("bits", [2, 5])
@pytest.mark.parametrize("M", [1, 3, 8, 17, 64, 200])
def test_narrow_records(nh, bits, M):
    say(f"{'ternary' if bits == 5 else '2-bit'} record out=1000 in=768 M={M}")
    packed, norms = random_record(1000, 768, bits, seed=20 + M)
    check_product(nh, packed, norms, 1000, 768, bits, M, seed=30 + M)


@pytest.mark.parametrize("bits", [2, 5])
def test_narrow_large_products(nh, bits):
    say(f"{'ternary' if bits == 5 else '2-bit'} record out=3072 in=768 M=1024 and out=8192 in=2048 M=1")
    packed, norms = random_record(3072, 768, bits, seed=40)
    check_product(nh, packed, norms, 3072, 768, bits, 1024, seed=41)
    packed, norms = random_record(8192, 2048, bits, seed=42)
    check_product(nh, packed, norms, 8192, 2048, bits, 1, seed=43)


@pytest.mark.parametrize("bits", [2, 4, 5])
@pytest.mark.parametrize("in_dim", [896, 1664, 200, 4096])
def test_group_counts(nh, bits, in_dim):
    say(f"group count in={in_dim} bits={bits}")
    packed, norms = random_record(77, in_dim, bits, seed=50 + in_dim)
    for M in (1, 6, 40):
        check_product(nh, packed, norms, 77, in_dim, bits, M, seed=60 + M)


@pytest.mark.parametrize("bits", [2, 5])
def test_narrow_rows_and_single_rows(nh, bits):
    say(f"{'ternary' if bits == 5 else '2-bit'} rows and single rows")
    out, K = 4096, 768
    packed, norms = random_record(out, K, bits, seed=70)
    q = nh.QMat.from_cq(packed, norms, out, K, bits)
    oq = o.OQMat.from_cq(packed, norms, out, K, bits)
    ids = o.random_tokens(64, out, seed=71)
    rows = q.rows(dev(ids.astype(np.int32))).cpu().numpy()
    want = np.stack([oq.row(int(r)) for r in ids])
    assert bits_equal(rows, want), report(rows, want)
    x = o.seeded_normals([K], 72)[0]
    a = nh.QAct.new(dev(x), 1, K, 2)
    oa = o.OQAct.new(x, 1, K, 2)
    vals = q.single_rows(dev(ids.astype(np.int32)), a).cpu().numpy()
    want = np.array([oq.single_row(int(r), oa) for r in ids], dtype=np.float32)
    assert bits_equal(vals, want), report(vals, want)


def test_width_mismatch_and_fusion(nh):
    say("width checks and 2-bit fusion")
    packed2, norms2 = random_record(40, 256, 2, seed=80)
    packed4, norms4 = random_record(40, 256, 4, seed=81)
    q2 = nh.QMat.from_cq(packed2, norms2, 40, 256, 2)
    q4 = nh.QMat.from_cq(packed4, norms4, 40, 256, 4)
    x = o.seeded_normals([256], 82)[0]
    with pytest.raises(nh.NeedleHipError):
        q2.matmul(nh.QAct.new(dev(x), 1, 256, 4))
    with pytest.raises(nh.NeedleHipError):
        nh.QLinear([q2, q4])
    with pytest.raises(nh.NeedleHipError) as e:
        nh.QMat.from_cq(packed4, norms4, 40, 256, 3)
    assert e.value.code == -1
    qt = nh.QMat.from_cq(packed2, norms2, 40, 256, 5)
    with pytest.raises(nh.NeedleHipError):
        nh.QLinear([q2, qt])  # different codebooks
    # fused 2-bit parts
    packed2b, norms2b = random_record(24, 256, 2, seed=83)
    lin = nh.QLinear([q2, nh.QMat.from_cq(packed2b, norms2b, 24, 256, 2)])
    olin = o.OQLinear([o.OQMat.from_cq(packed2, norms2, 40, 256, 2), o.OQMat.from_cq(packed2b, norms2b, 24, 256, 2)])
    for M in (1, 5):
        xs = o.seeded_normals([M * 256], 84)[0]
        y = lin.matmul(nh.QAct.new(dev(xs), M, 256, 2)).cpu().numpy()
        assert bits_equal(y, olin.matmul(o.OQAct.new(xs, M, 256, 2)))
    # archive bytes come back as uploaded
    p, n = q2.download()
    assert np.array_equal(p, packed2) and np.array_equal(n, norms2)
    assert q2.bytes() == 40 * 2 * 32 + 40 * 2 * 2


@pytest.mark.parametrize("bits", [2, 4])
def test_slice_rows(nh, bits):
    # QMat::slice_rows (qlinear.rs:268-276) as weights.rs:383-388 uses it.
    say(f"slice_rows bits={bits}")
    out, K = 96, 384
    packed, norms = random_record(out, K, bits, seed=90)
    q = nh.QMat.from_cq(packed, norms, out, K, bits)
    s = q.slice_rows(24, 72)
    assert (s.out, s.in_dim, s.bits) == (48, K, bits)
    p, n = s.download()
    assert np.array_equal(p, packed[24:72]) and np.array_equal(n, norms[24:72])
    x = o.seeded_normals([3 * K], 91)[0]
    a = nh.QAct.new(dev(x), 3, K, bits)
    y = s.matmul(a).cpu().numpy()
    want = o.OQMat.from_cq(packed[24:72], norms[24:72], 48, K, bits).matmul(o.OQAct.new(x, 3, K, bits))
    assert bits_equal(y, want)
    with pytest.raises(nh.NeedleHipError):
        q.slice_rows(50, 40)
