"""The product's archive writer (needle_hip/archive.py) read back by the
oracle's independent reader (oracle/cact.py), on the CPU: the header words,
the codebook block (nh_codebook against the oracle's Lloyd-Max codebooks,
crates/needle-core/src/quant.rs:17-68), record layout, 64-byte alignment and
blob contents; and the C ABI loader's walk over a written archive.
"""
import ctypes as C

import numpy as np

import needle_hip
from needle_hip import archive as W
import oracle as o
from oracle import cact


def test_codebooks_match_the_oracle():
    for bits in (2, 3, 4, 5):
        got = needle_hip.codebook(bits)
        want = o.codebook(bits)
        assert got.dtype == np.float32 and np.array_equal(got.view(np.uint32), want.view(np.uint32)), bits


def _small_records(g, rng):
    """Records in the export order with random CQ blobs (no GPU)."""
    w = W._Writer()
    d, L, n = g.d_model, g.num_layers, g.mhc_lanes
    qk, vd = g.qk_head_dim, g.v_head_dim
    qd, kd, vdim = g.num_heads * qk, g.num_kv_heads * qk, g.num_kv_heads * vd
    hn = g.hada_n
    ba, bb = W._hada_blocks(hn)
    tables = len(g.engram_orders) * g.engram_heads

    def mat(out, in_dim):
        groups = -(-in_dim // 128)
        w.cq(rng.integers(0, 256, (out, groups * 64), dtype=np.uint8),
             rng.integers(0, 0x3c00, (out, groups), dtype=np.uint16), out, in_dim)

    def row(*shape):
        w.f16(rng.uniform(-1, 1, shape))

    mat(g.vocab, d)
    for _ in range(L):
        row(d)
        mat(qd, d), mat(kd, d), mat(vdim, d)
        row(g.qkv_conv_taps, qd), row(g.qkv_conv_taps, kd), row(g.qkv_conv_taps, vdim)
        row(qk), row(qk)
        mat(g.num_heads * vd, d), mat(d, g.num_heads * vd)
        row(d)
        w.f16(rng.uniform(-1, 1, 1), [1])
        row(d)
        for _ in range(5):
            row(hn)
        for _ in range(3):
            row(ba, ba), row(bb, bb)
        row(d, 8), row(8, hn)
    for _ in range(3):
        row(L)
    row(L, n), row(L, n), row(L, n * n)
    mat(L * n, n * d), mat(L * n, n * d), mat(L * n * n, n * d)
    for s in W.PERM_SEEDS:
        w.f32(np.random.RandomState(s).permutation(hn).astype(np.float32))
    for _ in g.engram_sites:
        mat(tables * g.engram_slots, g.engram_sub_dim), mat(d, d), mat(d, d)
        row(4, d)
    row(d)
    return w.records


def test_writer_read_back_by_the_oracle():
    g = W.Needle3(vocab=300, num_layers=2, engram_slots=32, engram_sites=(1,), global_layers=(0,), sliding_window=16)
    recs = _small_records(g, np.random.default_rng(1))
    cb = np.concatenate([needle_hip.codebook(b) for b in W.CB_BITS])
    data = W.pack(recs, g, cb)
    a = cact.Archive(data)
    h = a.header
    og = cact.Geometry(vocab=300, num_layers=2, engram_slots=32, engram_sites=(1,), global_layers=(0,),
                       sliding_window=16)
    want = og.header()
    want.num_tensors, want.codebook_len = len(recs), 28
    assert h == want
    assert np.array_equal(a.codebook, cact.codebook_block())
    assert len(a.records) == len(recs) == 1 + 2 * 27 + 6 + 3 + 2 + 4 + 1
    for i, (r, (dtype, shape, blob, group, bits)) in enumerate(zip(a.records, recs)):
        assert (r.dtype, list(r.shape), r.group, r.bits) == (dtype, list(shape), group, bits), i
        assert r.offset % 64 == 0 and a.bytes(i) == blob, i
    # the perms are the reference's seeded permutations
    assert np.array_equal(np.frombuffer(a.bytes(2 * 27 + 10), np.float32), cact.hada_perm(11, 1024))
    # the C ABI walk accepts it (and stops at the missing device)
    import torch
    if not torch.cuda.is_available():
        lib = needle_hip.load_library()
        buf = np.frombuffer(data, dtype=np.uint8)
        h = C.c_void_p()
        assert lib.nh_model_load(buf.ctypes.data_as(C.c_void_p), buf.nbytes, C.byref(h)) == -5
