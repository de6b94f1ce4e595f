"""The oracle reproduces the committed golden vectors (tests/golden/,
written by tests/golden/make_golden.py) bit for bit."""
import hashlib
import json
import os

import numpy as np

import oracle as o

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F = np.float32


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def ref_case():
    out, din = 37, 384
    i = np.arange(out * din)
    w = (((i * 7919 % 1000).astype(F) / F(500.0) - F(1.0)) * F(0.05)).astype(F)
    x = ((np.arange(din) * 31 % 97).astype(F) / F(48.0) - F(1.0)).astype(F)
    return out, din, w, x


def seeded(out, in_dim, rows, seed=0):
    w, x = o.seeded_normals([out * in_dim, rows * in_dim], seed)
    return (w * F(0.02)).astype(F), x


def test_codebook_fixture():
    g = json.load(open(os.path.join(GOLD, "codebook4.json")))
    cb = o.codebook(4)
    cb8, cbs = o.int8_codebook(cb)
    assert [int(v) for v in cb.view(np.uint32)] == g["cb_bits"]
    assert [int(v) for v in cb8] == g["cb8"]
    assert int(np.float32(cbs).view(np.uint32)) == g["cbs_bits"]


def test_reference_case_fixture():
    g = load("ref_case_4bit.npz")
    out, din, w, x = ref_case()
    q = o.OQMat.from_f32(w, out, din)
    a = o.OQAct.new(x, 1, din)
    assert np.array_equal(q.codes, g["codes"]) and np.array_equal(q.norms, g["norms"])
    assert np.array_equal(a.xq, g["xq"]) and np.array_equal(bits(a.sx), bits(g["sx"]))
    assert np.array_equal(q.all_lane_sums(a), g["lanes"])
    assert np.array_equal(bits(q.matmul(a)[0]), bits(g["y"]))
    for rows in (2, 3, 5, 9, 13, 17):
        xs = np.sin(np.arange(rows * din, dtype=F) * F(0.37)).astype(F)
        ar = o.OQAct.new(xs, rows, din)
        assert np.array_equal(bits(q.matmul(ar)), bits(g[f"prefill_{rows}"]))
        assert np.array_equal(q.all_totals(ar), g[f"totals_{rows}"])


def test_two_bit_fixture():
    g = load("two_bit_case.npz")
    out, din = 9, 256
    codes = np.array([(i * 37) % 251 for i in range(out * din // 4)], dtype=np.uint8)
    norms = np.array([np.float16(F(0.5) + F(i) * F(0.01)) for i in range(out * din // 128)],
                     dtype=np.float16).view(np.uint16)
    q = o.OQMat.build(out, din, 2, o.codebook(2), codes, norms)
    xs = np.cos(np.arange(5 * din, dtype=F) * F(0.21)).astype(F)
    a1 = o.OQAct.new(xs[:din], 1, din, 2)
    a5 = o.OQAct.new(xs, 5, din, 2)
    assert np.array_equal(bits(q.matmul(a1)[0]), bits(g["y1"]))
    assert np.array_equal(q.all_lane_sums(a1), g["lanes1"])
    assert np.array_equal(bits(q.matmul(a5)), bits(g["y5"]))
    assert np.array_equal(q.all_totals(a5), g["totals5"])


def test_gemv_full_size_fixture():
    g = load("gemv_k2048_n8192.npz")
    K, N = 2048, 8192
    w, x = seeded(N, K, 1, seed=0)
    packed, nrm = o.cq_pack(w, K)
    q = o.OQMat.from_cq(packed, nrm, N, K)
    a = o.OQAct.new(x, 1, K)
    y = q.matmul(a)[0]
    lanes = q.all_lane_sums(a)
    assert list(g["hashes"]) == [sha(packed), sha(nrm), sha(a.xq), sha(a.sx), sha(lanes), sha(y)]
    assert np.array_equal(bits(y[::128]), bits(g["y_slice"]))


def test_gemm_m64_fixture():
    g = load("gemm_m64_k768_n2304.npz")
    M, K, N = 64, 768, 2304
    w, x = seeded(N, K, M, seed=0)
    packed, nrm = o.cq_pack(w, K)
    q = o.OQMat.from_cq(packed, nrm, N, K)
    a = o.OQAct.new(x, M, K)
    y = q.matmul(a)
    tot = q.all_totals(a)
    assert list(g["hashes"]) == [sha(packed), sha(nrm), sha(a.xq), sha(a.sx), sha(tot), sha(y)]


def test_norm_prep_fixture():
    g = load("norm_prep_768.npz")
    h = o.zcn16(g["x"], g["s16"])
    assert np.array_equal(bits(h), bits(g["h"]))
    a = o.OQAct.new(h, 1, 768)
    assert np.array_equal(a.xq, g["xq"]) and np.array_equal(bits(a.sx), bits(g["sx"]))
