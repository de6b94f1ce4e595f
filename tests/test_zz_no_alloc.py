"""GPU: nh_qlinear_apply_static, the entry point that allocates nothing,
against nh_qlinear_apply (QLinear::apply, qlinear.rs:555-557) on the same
matrices and activations: bit-identical outputs over consecutive calls whose
inputs shrink (the static staging keeps the previous call's contents), on
the decode (one row) and prefill (more rows) paths, 4- and 2-bit matrices,
and the row limit refused.
"""
import numpy as np
import pytest
import torch

import oracle as o

pytestmark = pytest.mark.gpu


def mat(nh, n, k, seed, bits=4):
    w = (o.seeded_normals([n * k], seed)[0] * np.float32(0.02)).astype(np.float32)
    packed, norms = o.cq_pack(w, k, bits=bits)
    return nh.QLinear([nh.QMat.from_cq(packed, norms, n, k, bits)])


def check(nh, lin, rows, seed):
    x = torch.from_numpy(o.seeded_normals([rows * lin.in_dim], seed)[0]).cuda()
    want = lin.apply(x, rows)
    y = torch.full((rows, lin.out), float("nan"), dtype=torch.float32, device="cuda")
    got = lin.apply_static(x, rows, y)
    torch.cuda.synchronize()
    g, w = got.cpu().numpy(), want.cpu().numpy()
    assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (rows, float(np.abs(g - w).max()))


def test_static_apply_matches_apply(nh):
    print("nh_qlinear_apply_static vs nh_qlinear_apply", flush=True)
    qkvg = mat(nh, 1568, 768, 31)
    # two calls in a row, the second smaller: prefill then decode, and
    # 64 rows then 5
    check(nh, qkvg, 37, 1)
    check(nh, qkvg, 1, 2)
    wide = mat(nh, 768, 3072, 32)
    check(nh, wide, 64, 3)
    check(nh, wide, 5, 4)
    two = mat(nh, 200, 1024, 33, bits=2)
    check(nh, two, 17, 5)
    check(nh, two, 1, 6)
    # the limits
    x = torch.zeros(65 * 768, dtype=torch.float32, device="cuda")
    y = torch.zeros((65, 1568), dtype=torch.float32, device="cuda")
    with pytest.raises(nh.NeedleHipError, match="64 rows"):
        qkvg.apply_static(x, 65, y)
    with pytest.raises(nh.NeedleHipError, match="no rows"):
        qkvg.apply_static(x, 0, y)
    # (in_dim above 4096 cannot reach it: no matrix that wide uploads)
    torch.cuda.synchronize()
