"""Write the golden vectors under tests/golden/ from the oracle.

    python tests/golden/make_golden.py

The vectors pin regressions of both the oracle and the GPU path; the
oracle itself is pinned by the reference's known answers
(tests/test_oracle_kat.py) and the spec restatements
(tests/test_oracle_numerics.py).  Inputs follow the reference's own
generators (crates/needle-engine/src/qlinear.rs:976-1029) or the seeded
threefry recipe (crates/needle-train/src/rand.rs:205-217).
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as o  # noqa: E402

F = np.float32


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def ref_case():
    out, din = 37, 384
    i = np.arange(out * din)
    w = (((i * 7919 % 1000).astype(F) / F(500.0) - F(1.0)) * F(0.05)).astype(F)
    x = ((np.arange(din) * 31 % 97).astype(F) / F(48.0) - F(1.0)).astype(F)
    return out, din, w, x


def seeded(out, in_dim, rows, seed=0):
    w, x = o.seeded_normals([out * in_dim, rows * in_dim], seed)
    return (w * F(0.02)).astype(F), x


def main():
    # (1) int8 codebook KAT
    cb = o.codebook(4)
    cb8, cbs = o.int8_codebook(cb)
    with open(os.path.join(HERE, "codebook4.json"), "w") as f:
        json.dump({"cb_bits": [int(v) for v in cb.view(np.uint32)], "cb8": [int(v) for v in cb8],
                   "cbs_bits": int(np.float32(cbs).view(np.uint32))}, f, indent=1)

    # (2) the reference's kernels_match_reference case (4-bit)
    out, din, w, x = ref_case()
    q = o.OQMat.from_f32(w, out, din)
    a = o.OQAct.new(x, 1, din)
    d = {"codes": q.codes, "norms": q.norms, "xq": a.xq, "sx": a.sx, "lanes": q.all_lane_sums(a),
         "y": q.matmul(a)[0]}
    for rows in (2, 3, 5, 9, 13, 17):
        xs = np.sin(np.arange(rows * din, dtype=F) * F(0.37)).astype(F)
        ar = o.OQAct.new(xs, rows, din)
        d[f"prefill_{rows}"] = q.matmul(ar)
        d[f"totals_{rows}"] = q.all_totals(ar)
    np.savez_compressed(os.path.join(HERE, "ref_case_4bit.npz"), **d)

    # (3) the reference's two-bit case
    out2, din2 = 9, 256
    codes = np.array([(i * 37) % 251 for i in range(out2 * din2 // 4)], dtype=np.uint8)
    norms = np.array([np.float16(F(0.5) + F(i) * F(0.01)) for i in range(out2 * din2 // 128)],
                     dtype=np.float16).view(np.uint16)
    q2 = o.OQMat.build(out2, din2, 2, o.codebook(2), codes, norms)
    xs = np.cos(np.arange(5 * din2, dtype=F) * F(0.21)).astype(F)
    a1 = o.OQAct.new(xs[:din2], 1, din2, 2)
    a5 = o.OQAct.new(xs, 5, din2, 2)
    np.savez_compressed(os.path.join(HERE, "two_bit_case.npz"), y1=q2.matmul(a1)[0], lanes1=q2.all_lane_sums(a1),
                        y5=q2.matmul(a5), totals5=q2.all_totals(a5))

    # (4) the K=2048, N=8192 decode GEMV at full size: hashes + a 64-row slice
    K, N = 2048, 8192
    w, x = seeded(N, K, 1, seed=0)
    packed, nrm = o.cq_pack(w, K)
    qc = o.OQMat.from_cq(packed, nrm, N, K)
    ac = o.OQAct.new(x, 1, K)
    y = qc.matmul(ac)[0]
    lanes = qc.all_lane_sums(ac)
    np.savez_compressed(os.path.join(HERE, "gemv_k2048_n8192.npz"), rows=np.arange(0, N, 128),
                        y_slice=y[::128], lanes_slice=lanes[::128],
                        hashes=np.array([sha(packed), sha(nrm), sha(ac.xq), sha(ac.sx), sha(lanes), sha(y)]))

    # (5) one prefill shape, M = 64, K = 768, N = 2304: hashes + slice
    M, K, N = 64, 768, 2304
    w, x = seeded(N, K, M, seed=0)
    packed, nrm = o.cq_pack(w, K)
    qm = o.OQMat.from_cq(packed, nrm, N, K)
    am = o.OQAct.new(x, M, K)
    y = qm.matmul(am)
    tot = qm.all_totals(am)
    np.savez_compressed(os.path.join(HERE, "gemm_m64_k768_n2304.npz"), y_slice=y[:, ::64], totals_slice=tot[:, ::64],
                        hashes=np.array([sha(packed), sha(nrm), sha(am.xq), sha(am.sx), sha(tot), sha(y)]))

    # (6) the fused norm -> A8 of one 768-wide row
    d = 768
    xn, s = o.seeded_normals([d, d], 2)
    s16 = (s * F(0.1)).astype(np.float16).view(np.uint16)
    h = o.zcn16(xn, s16)
    an = o.OQAct.new(h, 1, d)
    np.savez_compressed(os.path.join(HERE, "norm_prep_768.npz"), x=xn, s16=s16, h=h, xq=an.xq, sx=an.sx)
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()
