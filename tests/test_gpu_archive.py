"""GPU: nh_weights_load reads a .cact archive into QWeights
(crates/needle-engine/src/weights.rs:314-467, 480-495).

Every matrix comes back as the records hold it: the fused ones are the
row concatenation of their parts (q|k|v|gate, engram key|value), the mHC
matrices the per-layer slices pre[4l..4l+4] | post[4l..4l+4] |
res[16l..16l+16] (weights.rs:376-389); f16 / f32 matmul records are packed
at 4 bits as QMat::from_f32 does (weights.rs:119-125).  Products over the
loaded matrices are bit-exact against the oracle built from the same
records, and bytes() is QWeights::bytes.
"""
import sys

import numpy as np
import pytest
import torch

import oracle as o
from oracle import cact

pytestmark = pytest.mark.gpu

SMALL = cact.Geometry(vocab=300, d_model=256, num_heads=4, num_kv_heads=1, num_layers=2, qk_head_dim=32,
                      v_head_dim=64, mhc_lanes=4, qkv_conv_taps=3, engram_orders=(2, 3), engram_slots=32,
                      engram_sites=(1,), global_layers=(1,), sliding_window=64)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bits_equal(a, b):
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def part_codes(m: cact.Matmul, rows=None):
    """(packed, norms, bits) of one part as the loader stores it."""
    if m.w is not None:
        packed, norms = o.cq_pack(m.w, m.in_dim, 4)
        bits = 4
    else:
        packed, norms, bits = m.packed, m.norms, m.bits
    if rows is not None:
        packed, norms = packed[rows[0]:rows[1]], norms[rows[0]:rows[1]]
    return np.asarray(packed), np.asarray(norms), bits


def expected(parts):
    codes = [part_codes(m, r) for m, r in parts]
    packed = np.concatenate([c[0] for c in codes])
    norms = np.concatenate([c[1] for c in codes])
    return packed, norms, codes[0][2], parts[0][0].in_dim


def check_matrix(q, parts, label):
    packed, norms, bits, in_dim = expected(parts)
    assert (q.out, q.in_dim) == (packed.shape[0], in_dim), label
    assert q.bits == (2 if bits == 5 else bits), label
    p, n = q.download()
    assert np.array_equal(p, packed), label
    assert np.array_equal(n, norms), label
    return packed, norms, bits, in_dim


def check_product(nh, q, packed, norms, bits, in_dim, seed, label):
    oq = o.OQMat.from_cq(packed, norms, packed.shape[0], in_dim, bits)
    abits = q.act_bits()
    for M in (1, 5):
        x = o.seeded_normals([M * in_dim], seed + M)[0]
        y = q.matmul(nh.QAct.new(dev(x), M, in_dim, abits)).cpu().numpy()
        want = oq.matmul(o.OQAct.new(x, M, in_dim, abits))
        assert bits_equal(y, want), (label, M)


def small_kind(name):
    if name == "embedding" or name.startswith("engram_key") or name.startswith("engram_value"):
        return ("cq", 4)
    if name.startswith("phi"):
        return ("random", 5)
    if name.startswith("engram_table"):
        return ("random", 2)
    if name == "out.0":
        return ("f16", 4)
    if name == "out.1":
        return ("f32", 4)
    layer = int(name.split(".")[1])
    return ("random", 4 if layer == 0 else 2)


def test_small_mixed_archive(nh):
    say("small mixed-width archive: load, compare every matrix, products")
    ts, mats = cact.needle3_tensors(SMALL, seed=5, kind=small_kind)
    data = cact.pack(ts, SMALL.header())
    w = nh.QWeights.from_archive(data)
    h = w.header
    assert (h["tag"], h["num_tensors"], h["d_model"], h["num_layers"], h["mhc_lanes"]) == \
        (cact.TAG, len(ts), 256, 2, 4)
    assert h["rope_theta"] == 100000.0
    fz = cact.fused(mats, SMALL)
    groups = {"embedding": [w.embedding], "qkvg": w.qkvg, "out": w.out, "phi": w.phi,
              "engram_tables": w.engram_tables, "engram_kv": w.engram_kv}
    total = 0
    for key, mats_of in groups.items():
        assert len(mats_of) == len(fz[key]), key
        for i, (q, parts) in enumerate(zip(mats_of, fz[key])):
            packed, norms, bits, in_dim = check_matrix(q, parts, f"{key}[{i}]")
            total += packed.nbytes + norms.nbytes
            assert q.bytes() == packed.nbytes + norms.nbytes
            if key in ("qkvg", "out", "phi", "engram_kv"):
                check_product(nh, q, packed, norms, bits, in_dim, seed=100 + 10 * i, label=f"{key}[{i}]")
    assert w.bytes() == total
    assert w.qkvg[0].out == 128 + 32 + 64 + 256 and w.phi[1].out == 24 and w.engram_kv[0].out == 512


def test_loader_errors_after_init(nh):
    say("malformed archives with a device: same errors, nothing kept")
    ts, _ = cact.needle3_tensors(SMALL, seed=6)
    good = cact.pack(ts, SMALL.header())
    with pytest.raises(nh.NeedleHipError) as e:
        nh.QWeights.from_archive(good[:1000])
    assert e.value.code == -1 and "past the end" in str(e.value)
    bad = bytearray(good)
    bad[0:4] = (0x05E12A83).to_bytes(4, "little")
    with pytest.raises(nh.NeedleHipError) as e:
        nh.QWeights.from_archive(bytes(bad))
    assert "Needle 2" in str(e.value)
    # a loaded archive is independent of its bytes afterwards
    w = nh.QWeights.from_archive(bytearray(good))
    p0, _ = w.qkvg[0].download()
    del good
    assert np.array_equal(w.qkvg[0].download()[0], p0)


def test_full_needle3_archive(nh):
    say("full Needle-3 geometry archive (random records): shapes, bytes, samples")
    g = cact.Geometry()
    ts, mats = cact.needle3_tensors(g, seed=7)
    data = cact.pack(ts, g.header())
    assert len(ts) == 573
    w = nh.QWeights.from_archive(data)
    assert (w.embedding.out, w.embedding.in_dim) == (16384, 768)
    assert len(w.qkvg) == len(w.out) == len(w.phi) == 20 and len(w.engram_tables) == len(w.engram_kv) == 5
    assert all((q.out, q.in_dim) == (1568, 768) for q in w.qkvg)
    assert all((q.out, q.in_dim) == (768, 768) for q in w.out)
    assert all((q.out, q.in_dim) == (24, 3072) for q in w.phi)
    assert all((q.out, q.in_dim) == (6 * 18432, 128) for q in w.engram_tables)
    assert all((q.out, q.in_dim) == (1536, 768) for q in w.engram_kv)
    fz = cact.fused(mats, g)
    total = 0
    for key, lst in fz.items():
        for parts in lst:
            packed, norms, _, _ = expected(parts)
            total += packed.nbytes + norms.nbytes
    assert w.bytes() == total
    for key, idx in (("qkvg", 13), ("phi", 19), ("engram_kv", 4), ("out", 0)):
        q = getattr(w, key)[idx]
        packed, norms, bits, in_dim = check_matrix(q, fz[key][idx], f"{key}[{idx}]")
        check_product(nh, q, packed, norms, bits, in_dim, seed=300 + idx, label=f"{key}[{idx}]")
