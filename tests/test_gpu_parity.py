"""GPU parity: the gfx950 kernels through the C ABI against the oracle.

Bar: int8 codes, int32 partial sums and f32 outputs bit-exact (every float
step of the reference is a fixed-order IEEE operation), argmax identical.
Inputs follow the seeded recipe (threefry normal, rand.rs:205-217):
weights 0.02 * N(0, 1) through cq_pack, activations N(0, 1).
"""
import sys

import numpy as np
import pytest
import torch

import oracle as o

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def seeded(out, in_dim, rows, seed=0):
    w, x = o.seeded_normals([out * in_dim, rows * in_dim], seed)
    w = (w * np.float32(0.02)).astype(np.float32)
    return w, x


def pair(nh, w, out, in_dim):
    packed, norms = o.cq_pack(w, in_dim)
    return nh.QMat.from_cq(packed, norms, out, in_dim), o.OQMat.from_cq(packed, norms, out, in_dim)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bits_equal(a, b):
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def report(got, want):
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    return f"max_abs={d.max():.3e} max_rel={(d / np.maximum(np.abs(want), 1e-30)).max():.3e} mismatches={(got != want).sum()}"


@pytest.mark.parametrize("rows,in_dim", [(1, 2048), (3, 768), (37, 384), (64, 3072), (5, 200)])
def test_act_prep_bit_exact(nh, rows, in_dim):
    say(f"act_prep rows={rows} in_dim={in_dim}")
    x = o.seeded_normals([rows * in_dim], 1)[0]
    x[: in_dim // 2] *= 1e3  # a wide dynamic range in one row
    a = nh.QAct.new(dev(x), rows, in_dim)
    xq, sx = a.download()
    ref = o.OQAct.new(x, rows, in_dim)
    assert np.array_equal(xq, ref.xq)
    assert bits_equal(sx, ref.sx)


@pytest.mark.parametrize("rows", [1, 32])
def test_act_prep_fused_norm(nh, rows):
    say(f"act_prep+zcn16 rows={rows}")
    d = 768
    x, s = o.seeded_normals([rows * d, d], 2)
    s16 = (s * np.float32(0.1)).astype(np.float16).view(np.uint16)
    h = np.stack([o.zcn16(x[r * d:(r + 1) * d], s16) for r in range(rows)])
    ref = o.OQAct.new(h, rows, d)
    a = nh.QAct.new(dev(x), rows, d, norm_scale=dev(s16.view(np.int16)))
    xq, sx = a.download()
    assert np.array_equal(xq, ref.xq)
    assert bits_equal(sx, ref.sx)


def ref_case():
    out, din = 37, 384
    i = np.arange(out * din)
    f = np.float32
    w = (((i * 7919 % 1000).astype(f) / f(500.0) - f(1.0)) * f(0.05)).astype(f)
    x = ((np.arange(din) * 31 % 97).astype(f) / f(48.0) - f(1.0)).astype(f)
    return out, din, w, x


def test_reference_case_decode(nh):
    # crates/needle-engine/src/qlinear.rs:976-990
    say("reference case decode out=37 in=384")
    out, din, w, x = ref_case()
    q, oq = pair(nh, w, out, din)
    a = nh.QAct.new(dev(x), 1, din)
    y = q.matmul(a).cpu().numpy()[0]
    oa = o.OQAct.new(x, 1, din)
    want = oq.matmul(oa)[0]
    assert bits_equal(y, want), report(y, want)
    lanes = q.partials(a).cpu().numpy()
    assert np.array_equal(lanes, oq.all_lane_sums(oa))


@pytest.mark.parametrize("rows", [2, 3, 5, 9, 13, 17])
def test_reference_case_prefill(nh, rows):
    # crates/needle-engine/src/qlinear.rs:991-1001
    say(f"reference case prefill rows={rows}")
    out, din, w, _ = ref_case()
    q, oq = pair(nh, w, out, din)
    xs = np.sin(np.arange(rows * din, dtype=np.float32) * np.float32(0.37)).astype(np.float32)
    a = nh.QAct.new(dev(xs), rows, din)
    y = q.matmul(a).cpu().numpy()
    oa = o.OQAct.new(xs, rows, din)
    want = oq.matmul(oa)
    assert bits_equal(y, want), report(y, want)
    tot = q.partials(a).cpu().numpy()
    assert np.array_equal(tot, oq.all_totals(oa))


def test_gemv_c1_full_size(nh):
    # K = 2048, N = 8192, one token, seed 0.
    say("gemv C1 K=2048 N=8192")
    K, N = 2048, 8192
    w, x = seeded(N, K, 1, seed=0)
    q, oq = pair(nh, w, N, K)
    a = nh.QAct.new(dev(x), 1, K)
    y = q.matmul(a).cpu().numpy()[0]
    oa = o.OQAct.new(x, 1, K)
    want = oq.matmul(oa)[0]
    assert bits_equal(y, want), report(y, want)
    lanes = q.partials(a).cpu().numpy()
    assert np.array_equal(lanes, oq.all_lane_sums(oa))
    # Invariant: the product approximates x . dequant(w) (no oracle).
    i = np.arange(0, N, 257)
    p, nrm = oq.codes, oq.norms
    deq = o.cq_unpack(p[i], nrm[i], len(i), K)
    approx = deq @ x
    assert np.all(np.abs(y[i] - approx) < 0.02 * (1 + np.abs(approx)))


@pytest.mark.parametrize("K", [256, 768])
def test_gemv_tall_streaming(nh, K):
    # Past 8 tiles per resident workgroup (8192 16-row tiles on 256 CUs) the
    # decode GEMV runs as a persistent streaming grid; rows not a multiple
    # of 16.
    N = 131112
    say(f"gemv streaming K={K} N={N}")
    w, x = seeded(N, K, 1, seed=3)
    q, oq = pair(nh, w, N, K)
    a = nh.QAct.new(dev(x), 1, K)
    y = q.matmul(a).cpu().numpy()[0]
    want = oq.matmul(o.OQAct.new(x, 1, K))[0]
    assert bits_equal(y, want), report(y, want)


C2 = [(M, K, N) for M in (64, 256, 1024) for (K, N) in ((768, 2304), (768, 3072), (3072, 768))]


@pytest.mark.parametrize("M,K,N", C2)
def test_gemm_c2_shapes(nh, M, K, N):
    say(f"gemm C2 M={M} K={K} N={N}")
    w, x = seeded(N, K, M, seed=0)
    q, oq = pair(nh, w, N, K)
    a = nh.QAct.new(dev(x), M, K)
    y = q.matmul(a).cpu().numpy()
    oa = o.OQAct.new(x, M, K)
    want = oq.matmul(oa)
    assert bits_equal(y, want), report(y, want)
    if M == 64:
        tot = q.partials(a).cpu().numpy()
        assert np.array_equal(tot, oq.all_totals(oa))


@pytest.mark.parametrize("M", [1, 8, 64])
def test_lm_head_c5(nh, M):
    say(f"lm head C5 K=768 N=32768 M={M}")
    K, N = 768, 32768
    w, x = seeded(N, K, M, seed=0)
    q, oq = pair(nh, w, N, K)
    a = nh.QAct.new(dev(x), M, K)
    y = q.matmul(a).cpu().numpy()
    want = oq.matmul(o.OQAct.new(x, M, K))
    assert bits_equal(y, want), report(y, want)
    for t in range(M):
        assert o.argmax(y[t]) == o.argmax(want[t])


def test_batched_chunk_flags(nh):
    # A 118-token prompt fed as chunks of 32, 32, 32, 22 (infer.rs:1106):
    # each token's block flag is its in-chunk index < len / 4 * 4.
    say("flags 118 tokens K=768 N=1568")
    K, N, T = 768, 1568, 118
    w, x = seeded(N, K, T, seed=3)
    q, oq = pair(nh, w, N, K)
    flags = []
    for start in range(0, T, 32):
        n = min(32, T - start)
        flags += [1 if i < n // 4 * 4 else 0 for i in range(n)]
    flags = np.array(flags, dtype=np.uint8)
    a = nh.QAct.new(dev(x), T, K)
    y = q.matmul_flags(a, dev(flags)).cpu().numpy()
    oa = o.OQAct.new(x, T, K)
    want = oq.prefill_flags(oa, flags)
    assert bits_equal(y, want), report(y, want)
    # Chunk by chunk through matmul gives the same bits.
    for start in range(0, T, 32):
        n = min(32, T - start)
        ac = nh.QAct.new(dev(x[start * K:(start + n) * K]), n, K)
        yc = q.matmul(ac).cpu().numpy()
        assert bits_equal(yc, want[start:start + n])


def test_single_rows_and_sparse_logits(nh):
    say("single rows / sparse logits K=768 N=8192")
    K, N = 768, 8192
    w, x = seeded(N, K, 1, seed=4)
    q, oq = pair(nh, w, N, K)
    ids = o.random_tokens(300, N, seed=4)
    a = nh.QAct.new(dev(x), 1, K)
    oa = o.OQAct.new(x, 1, K)
    vals = q.single_rows(dev(ids.astype(np.int32)), a).cpu().numpy()
    want = np.array([oq.single_row(int(r), oa) for r in ids], dtype=np.float32)
    assert bits_equal(vals, want), report(vals, want)
    logits = nh.head_logits_sparse(q, a, dev(ids.astype(np.int32)), N).cpu().numpy()
    assert bits_equal(logits, oq.head_logits_sparse(oa, ids, N))


def test_row_dequant(nh):
    say("row dequant K=768 N=4096")
    K, N = 768, 4096
    w, _ = seeded(N, K, 1, seed=5)
    q, oq = pair(nh, w, N, K)
    ids = o.random_tokens(64, N, seed=5)
    rows = q.rows(dev(ids.astype(np.int32))).cpu().numpy()
    want = np.stack([oq.row(int(r)) for r in ids])
    assert bits_equal(rows, want), report(rows, want)


@pytest.mark.parametrize("out,in_dim", [(1024, 768), (37, 384), (16, 200)])
def test_gpu_cq_pack(nh, out, in_dim):
    say(f"cq_pack on GPU out={out} in={in_dim}")
    w, _ = seeded(out, in_dim, 1, seed=6)
    q = nh.QMat.from_f32(w, out, in_dim)
    packed, norms = q.download()
    wp, wn = o.cq_pack(w, in_dim)
    assert np.array_equal(norms, wn)
    assert np.array_equal(packed, wp)


def test_qlinear_fused_qkvg(nh):
    # q | k | v | gate (crates/needle-engine/src/weights.rs:484-490).
    say("qlinear q|k|v|gate 576+96+128+768 x 768")
    K = 768
    sizes = (576, 96, 128, 768)
    ws = o.seeded_normals([n * K for n in sizes], 7)
    parts, oparts = [], []
    for n, wv in zip(sizes, ws):
        g, og = pair(nh, (wv * np.float32(0.02)).astype(np.float32), n, K)
        parts.append(g)
        oparts.append(og)
    lin = nh.QLinear(parts)
    olin = o.OQLinear(oparts)
    assert lin.out == 1568
    for M in (1, 5):
        x = o.seeded_normals([M * K], 8)[0]
        y = lin.matmul(nh.QAct.new(dev(x), M, K)).cpu().numpy()
        want = olin.matmul(o.OQAct.new(x, M, K))
        assert bits_equal(y, want), report(y, want)
    # QLinear::apply (qlinear.rs:555-557): A8 and the products in one call
    for M in (1, 3, 70):
        x = o.seeded_normals([M * K], 9 + M)[0]
        y = lin.apply(dev(x), M).cpu().numpy()
        want = olin.matmul(o.OQAct.new(x, M, K))
        assert bits_equal(y, want), report(y, want)


def test_edge_cases(nh):
    say("edge cases")
    K, N = 256, 48
    w, _ = seeded(N, K, 1, seed=9)
    q, oq = pair(nh, w, N, K)
    # all-zero activations: scale 1, codes 0, outputs 0
    z = np.zeros(K, np.float32)
    y = q.matmul(nh.QAct.new(dev(z), 1, K)).cpu().numpy()[0]
    assert bits_equal(y, oq.matmul(o.OQAct.new(z, 1, K))[0])
    # matmul_into with ldy/col0 side by side
    x = o.seeded_normals([2 * K], 10)[0]
    a = nh.QAct.new(dev(x), 2, K)
    ybig = torch.full((2, 3 * N), 7.0, device="cuda")
    q.matmul_into(a, ybig, 3 * N, N)
    yb = ybig.cpu().numpy()
    want = oq.matmul(o.OQAct.new(x, 2, K))
    assert bits_equal(yb[:, N:2 * N], want)
    assert np.all(yb[:, :N] == 7.0) and np.all(yb[:, 2 * N:] == 7.0)
    # errors become negative returns, not aborts
    with pytest.raises(nh.NeedleHipError) as e:
        nh.QMat.from_cq(np.zeros((1, 32), np.uint8), np.zeros((1, 1), np.uint16), 1, 64, 4, 64)
    assert e.value.code == -1
    other = nh.QAct.new(dev(np.zeros(512, np.float32)), 1, 512)
    with pytest.raises(nh.NeedleHipError):
        q.matmul(other)
    small = nh.QAct(2, K)
    with pytest.raises(nh.NeedleHipError):
        small.prep(dev(np.zeros(70 * K, np.float32)), 70)


def test_read_floors(nh):
    """The measurement-only read floors run in the product's grid and write nothing but
    mode 2's one float per row."""
    say("read floors")
    K, N = 2048, 40
    w, x = seeded(N, K, 1, seed=11)
    q, _ = pair(nh, w, N, K)
    a = nh.QAct.new(dev(x), 1, K)
    y = torch.full((N + 8,), 7.0, device="cuda")
    q.read_floor(a, 0)
    q.read_floor(a, 1)
    q.read_floor(a, 2, y)
    yh = y.cpu().numpy()
    # the stored bits have bit 30 clear: finite, below 2, never the 7.0 sentinel
    assert np.all(np.isfinite(yh[:N])) and np.all(np.abs(yh[:N]) < 2.0)
    assert np.all(yh[N:] == 7.0)
    with pytest.raises(ValueError):
        q.read_floor(a, 2, y[:N - 1])
    with pytest.raises(nh.NeedleHipError):
        q.read_floor(a, 3)


def test_repeatable(nh):
    say("determinism")
    K, N, M = 768, 2304, 64
    w, x = seeded(N, K, M, seed=11)
    q, _ = pair(nh, w, N, K)
    a = nh.QAct.new(dev(x), M, K)
    y1 = q.matmul(a).cpu().numpy()
    y2 = q.matmul(a).cpu().numpy()
    assert bits_equal(y1, y2)


def test_device_argmax_rule(nh):
    """generate::argmax on the device: the first maximum, NaNs never win, a NaN
    first element gives 0 (the reference's loop), over cases that cross the
    kernel's thread, wavefront and batch boundaries."""
    from test_oracle_numerics import argmax_cases
    cases = argmax_cases()
    rng = np.random.default_rng(5)
    big = rng.normal(size=40000).astype(np.float32)
    big[[5, 1029, 33000]] = np.float32(9.0)
    big[[3, 20000]] = np.float32(np.nan)
    cases.append(big)
    for x in cases:
        assert nh.argmax(torch.from_numpy(x).cuda()) == o.argmax(x)
