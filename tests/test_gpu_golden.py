"""The GPU path reproduces the committed golden vectors (tests/golden/)."""
import hashlib
import os

import numpy as np
import pytest
import torch

import oracle as o

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F = np.float32


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_gpu_reference_case_fixture(nh):
    print("golden: reference case", flush=True)
    g = load("ref_case_4bit.npz")
    out, din = 37, 384
    q = nh.QMat.from_cq(g["codes"], g["norms"], out, din)
    x = ((np.arange(din) * 31 % 97).astype(F) / F(48.0) - F(1.0)).astype(F)
    a = nh.QAct.new(dev(x), 1, din)
    xq, sx = a.download()
    assert np.array_equal(xq, g["xq"]) and np.array_equal(bits(sx), bits(g["sx"]))
    assert np.array_equal(q.partials(a).cpu().numpy(), g["lanes"])
    assert np.array_equal(bits(q.matmul(a).cpu().numpy()[0]), bits(g["y"]))
    for rows in (2, 3, 5, 9, 13, 17):
        xs = np.sin(np.arange(rows * din, dtype=F) * F(0.37)).astype(F)
        ar = nh.QAct.new(dev(xs), rows, din)
        assert np.array_equal(bits(q.matmul(ar).cpu().numpy()), bits(g[f"prefill_{rows}"]))
        assert np.array_equal(q.partials(ar).cpu().numpy(), g[f"totals_{rows}"])


def test_gpu_gemv_full_size_fixture(nh):
    print("golden: gemv K=2048 N=8192", flush=True)
    g = load("gemv_k2048_n8192.npz")
    K, N = 2048, 8192
    w, x = o.seeded_normals([N * K, K], 0)
    w = (w * F(0.02)).astype(F)
    q = nh.QMat.from_f32(w, N, K)  # cq_pack on the GPU
    packed, nrm = q.download()
    a = nh.QAct.new(dev(x), 1, K)
    xq, sx = a.download()
    y = q.matmul(a).cpu().numpy()[0]
    lanes = q.partials(a).cpu().numpy()
    assert list(g["hashes"]) == [sha(packed), sha(nrm), sha(xq), sha(sx), sha(lanes), sha(y)]


def test_gpu_gemm_m64_fixture(nh):
    print("golden: gemm M=64 K=768 N=2304", flush=True)
    g = load("gemm_m64_k768_n2304.npz")
    M, K, N = 64, 768, 2304
    w, x = o.seeded_normals([N * K, M * K], 0)
    w = (w * F(0.02)).astype(F)
    q = nh.QMat.from_f32(w, N, K)
    packed, nrm = q.download()
    a = nh.QAct.new(dev(x), M, K)
    xq, sx = a.download()
    y = q.matmul(a).cpu().numpy()
    tot = q.partials(a).cpu().numpy()
    assert list(g["hashes"]) == [sha(packed), sha(nrm), sha(xq), sha(sx), sha(tot), sha(y)]


def test_gpu_norm_prep_fixture(nh):
    print("golden: fused norm + A8, 768", flush=True)
    g = load("norm_prep_768.npz")
    a = nh.QAct.new(dev(g["x"]), 1, 768, norm_scale=dev(g["s16"].view(np.int16)))
    xq, sx = a.download()
    assert np.array_equal(xq, g["xq"]) and np.array_equal(bits(sx), bits(g["sx"]))
