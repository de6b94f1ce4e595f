"""The .cact archive format and the loader's checks, on the CPU.

Layout pins (crates/needle-core/src/cact.rs): the 196-byte header with its
word positions (80-118), the 44-byte directory record (199-211), 64-byte
blob alignment and the 2/3/4-bit codebook block (398-475); the export order
of a Needle-3 geometry (274-343); the Hadamard permutation generator against
the reference's own known answer (crates/needle-core/src/rng.rs:94-98).

The C ABI's nh_weights_load parses and walks an archive completely before
touching a device, so every malformed archive below fails with NH_EINVAL and
the reference's message here, without a GPU; a well-formed one gets as far
as NH_ESTATE (nh_init not called).
"""
import ctypes as C
import struct

import numpy as np
import pytest

import needle_hip
import oracle as o
from oracle import cact

SMALL = cact.Geometry(vocab=300, d_model=256, num_heads=4, num_kv_heads=1, num_layers=2, qk_head_dim=32,
                      v_head_dim=64, mhc_lanes=4, qkv_conv_taps=3, engram_orders=(2, 3), engram_slots=32,
                      engram_sites=(1,), global_layers=(1,), sliding_window=64)


def small_archive(kind=lambda name: ("random", 4), mutate=None, seed=1):
    ts, mats = cact.needle3_tensors(SMALL, seed=seed, kind=kind)
    if mutate:
        mutate(ts)
    return cact.pack(ts, SMALL.header()), ts, mats


def test_header_layout():
    h = cact.Geometry().header()
    h.num_tensors, h.codebook_len = 7, 28
    b = h.to_bytes()
    assert len(b) == cact.HEADER_BYTES == 196
    w = struct.unpack("<48I", b[:192])
    assert w[0] == 0x05E12A84 and w[1] == 7 and w[2] == 28
    assert (w[5], w[7], w[8], w[9], w[10], w[11], w[12]) == (16384, 768, 12, 2, 20, 48, 64)
    assert w[14] == 1024 and w[15] == 4 and w[19] == 3
    assert w[17] | (w[18] << 32) == (1 << 4) | (1 << 9) | (1 << 14) | (1 << 19)
    # engram geometry: 2 orders x 3 heads of 128, dilation = max order
    assert (w[20], w[21], w[22], w[23], w[24]) == (18432, 128, 6, 4, 3)
    assert w[26] == 2 and w[27:31] == (2, 3, 0, 0)
    assert w[31] == 5 and w[32:37] == (3, 7, 11, 15, 19) and w[37:48] == (0,) * 11
    assert struct.unpack("<f", b[192:196])[0] == 100000.0
    assert cact.Header.parse(b) == h


def test_record_layout():
    r = cact.Record(cact.CQ, [1568, 768], 4096, 123456, 128, 5)
    b = r.to_bytes()
    assert len(b) == cact.REC_SIZE == 44
    assert b[0] == 3 and b[1] == 2
    assert struct.unpack_from("<4I", b, 4) == (1568, 768, 0, 0)
    assert struct.unpack_from("<QQII", b, 20) == (4096, 123456, 128, 5)
    assert cact.Record.parse(b) == r


def test_hada_helpers():
    # rng.rs:94-98: np.random.RandomState(11).permutation(16)
    assert cact.hada_perm(11, 16).tolist() == [8, 3, 6, 10, 15, 4, 5, 14, 2, 13, 12, 7, 1, 11, 0, 9]
    assert cact.hada_blocks(1024) == (32, 32)
    assert cact.hada_blocks(512) == (16, 32)
    assert cact.hada_blocks(256) == (16, 16)
    g = cact.Geometry()
    assert (g.hada_n, g.engram_heads, g.engram_sub_dim, g.num_engram_tables) == (1024, 3, 128, 6)


def test_pack_layout_and_roundtrip():
    data, ts, _ = small_archive()
    a = cact.Archive(data)
    assert a.header.num_tensors == len(ts)
    cb = np.concatenate([o.codebook(2), o.codebook(3), o.codebook(4)]).astype(np.float32)
    assert a.header.codebook_len == 28 and np.array_equal(a.codebook, cb)
    dir_end = cact.HEADER_BYTES + 28 * 4 + len(ts) * cact.REC_SIZE
    prev = dir_end
    for t, r in zip(ts, a.records):
        assert r.offset % 64 == 0 and r.offset >= prev and r.offset - prev < 64
        assert a.bytes(a.records.index(r)) == t.blob and r.dtype == t.dtype and r.shape == t.shape
        prev = r.offset + r.nbytes
    assert prev == len(data)
    # canonical order: 1 + L * 27 + 6 + 3 + 2 + 4 * sites + 1 records
    assert len(ts) == 1 + 2 * 27 + 6 + 3 + 2 + 4 + 1


def test_needle3_export_count():
    # Needle 3: 20 layers with conv taps, 5 engram sites (cact.rs:274-343).
    g = cact.Geometry()
    n = 1 + g.num_layers * 27 + 6 + 3 + 2 + 4 * len(g.engram_sites) + 1
    assert n == 573


def _load_rc(data: bytes):
    lib = needle_hip.load_library()
    buf = np.frombuffer(data, dtype=np.uint8)
    h = C.c_void_p()
    rc = lib.nh_weights_load(buf.ctypes.data_as(C.c_void_p), buf.nbytes, C.byref(h))
    return rc, lib.nh_last_error().decode()


def _patch(data: bytes, off: int, fmt: str, *vals) -> bytes:
    b = bytearray(data)
    struct.pack_into(fmt, b, off, *vals)
    return bytes(b)


def _rec_off(i: int) -> int:
    return cact.HEADER_BYTES + 28 * 4 + i * cact.REC_SIZE


def _minimal_truncated_directory() -> bytes:
    """A header claiming two tensors, the codebook, and one record (an empty
    blob at offset 0): the second record is missing."""
    h = SMALL.header()
    h.num_tensors, h.codebook_len = 2, 28
    return h.to_bytes() + cact.codebook_block().tobytes() + cact.Record(cact.F16, [0], 0, 0).to_bytes()


def _bad_cases():
    good, ts, _ = small_archive()
    n = len(ts)
    last = cact.Archive(good).records[-1]
    cases = [
        ("short", good[:100], "not a complete .cact archive"),
        ("needle2", _patch(good, 0, "<I", cact.TAG_V2),
         "this is a Needle 2 archive; Needle 3 (tag 0x05e12a84) is required"),
        ("tag", _patch(good, 0, "<I", 0x12345678), "unknown .cact format tag 0x12345678"),
        ("orders", _patch(good, 26 * 4, "<I", 5), "corrupt .cact header"),
        ("sites", _patch(good, 31 * 4, "<I", 17), "corrupt .cact header"),
        ("codebook", _patch(good, 2 * 4, "<I", 1 << 28), "truncated codebook"),
        ("directory", _minimal_truncated_directory(), "truncated directory"),
        ("past end", _patch(good, _rec_off(3) + 28, "<Q", len(good)), "tensor past the end of the archive"),
        ("offset", _patch(good, _rec_off(3) + 20, "<Q", 1 << 62), "tensor past the end of the archive"),
        ("dtype", _patch(good, _rec_off(5), "<B", 9), "unknown .cact tensor dtype 9"),
        ("ndim", _patch(good, _rec_off(5) + 1, "<B", 5), "corrupt .cact record"),
        ("group", _patch(good, _rec_off(2) + 36, "<I", 64), "CQ group size 64 is not supported"),
        ("bits", _patch(good, _rec_off(2) + 40, "<I", 3), "CQ records of 3 bits are not supported"),
        ("raw", _patch(good, _rec_off(0), "<B", cact.RAW), "tensor 0 is a raw attachment"),
        # a CQ blob read as f16 values holds fewer than [300, 256]
        ("cq as f16", _patch(good, _rec_off(0), "<B", cact.F16), "data shorter than its shape"),
        ("short blob", _patch(good, _rec_off(2) + 28, "<Q", 100), "CQ blob shorter than its shape"),
        ("ends early", _patch(good, 4, "<I", n - 1), "the archive ends before the canonical order does"),
        # cut inside the directory: record 0's blob now lies past the end
        ("dropped dir", good[:_rec_off(n - 1)], "tensor past the end of the archive"),
        ("last blob", good[:last.offset + 10], "tensor past the end of the archive"),
    ]

    def mutated(name, fn, msg):
        data, _, _ = small_archive(mutate=fn)
        return (name, data, msg)

    # Records the walk finds by position (export order, small geometry):
    # 0 embedding; layer l base 1 + 27 l: norm 0, q 1, k 2, v 3, taps 4-6,
    # norms 7-8, gate 9, out 10, post 11, gate scalar 12, pre 13, d1..d4 14-18,
    # kron 19-24, cond_v 25, cond_u 26; then 55 + (6 mhc vectors), 61-63 phi,
    # 64-65 perms, 66-69 engram site 0, 70 final norm.
    def set_tensor(i, t):
        def f(ts):
            ts[i] = t
        return f

    cases += [
        mutated("perm", set_tensor(64, cact.f32(np.arange(255, dtype=np.float32))),
                "Hadamard permutations do not match hada_n"),
        mutated("kron", set_tensor(1 + 27 + 19, cact.fp16(np.zeros((16, 15), np.float32))),
                "Hadamard factor shapes"),
        mutated("cond_u", set_tensor(1 + 26, cact.fp16(np.zeros((8, 255), np.float32))), "cond_u shape"),
        mutated("attn_gate", set_tensor(1 + 12, cact.fp16(np.zeros(0, np.float32), [0])), "attn_gate is empty"),
    ]
    data, _, _ = small_archive(kind=lambda name: ("random", 2) if name == "k.1" else ("random", 4))
    cases.append(("fusion", data, "q|k|v|gate: fused parts must share in_dim and code width"))

    def short_phi(ts):
        packed = np.zeros((20, 1024 * 4 // 8), np.uint8)
        ts[63] = cact.cq_tensor(packed, np.zeros((20, 8), np.uint16), 20, 1024, 4)

    cases.append(mutated("phi rows", short_phi, "mHC phi rows do not match the depth"))
    return cases


@pytest.mark.parametrize("case", _bad_cases(), ids=lambda c: c[0])
def test_loader_rejects_malformed_archives(case):
    name, data, msg = case
    rc, err = _load_rc(data)
    assert rc == -1, (name, rc, err)
    assert msg in err, (name, err)


def test_loader_accepts_well_formed_archive_before_init():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is visible: the load would upload")
    for kind in (lambda n: ("random", 4), lambda n: ("random", 2) if n.startswith("phi") else ("random", 4),
                 lambda n: ("f16", 4) if n.startswith("out") else ("random", 5 if n.startswith("engram_t") else 4)):
        data, _, _ = small_archive(kind=kind)
        rc, err = _load_rc(data)
        assert rc == -5 and "nh_init" in err, (rc, err)


def test_weights_accessors_reject_null():
    lib = needle_hip.load_library()
    m = C.c_void_p()
    assert lib.nh_weights_get(None, 0, 0, C.byref(m)) == -1
    assert lib.nh_weights_count(None, 0) == -1
    assert lib.nh_weights_bytes(None) == -1
    assert lib.nh_weights_free(None) == 0
    rc = lib.nh_weights_load(None, 0, None)
    assert rc == -1
