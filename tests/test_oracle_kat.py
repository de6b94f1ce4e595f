"""Known-answer tests that pin the oracle to the reference's own vectors.

Every expected value here is copied from a test in the reference (cited);
none is produced by the oracle itself.
"""
import numpy as np
import pytest

import oracle as o


def test_threefry_random123_kat():
    # crates/needle-train/src/rand.rs:224-227 (Random123 threefry2x32_20 KAT)
    assert o.threefry2x32([0x13198A2E, 0x03707344], [0x243F6A88, 0x85A308D3]) == [0xC4923A9C, 0x483DF7A0]


def test_jax_split_and_normal():
    # crates/needle-train/src/rand.rs:236-245
    k, s = o.split(o.prng_key(0))
    assert k == [0x6B200159, 0x99BA4EFE]
    assert s == [0x375F238F, 0xCDDB151D]
    want = np.array([-2.4424558, -2.0356805, 0.20554423, -0.3535502, -0.76197404, -1.1785518], dtype=np.float32)
    got = o.normal(s, 6)
    assert np.all(np.abs(got - want) <= 2e-6 * np.maximum(np.abs(want), 1.0))


def test_numpy_seed_sequence_and_permutations():
    # crates/needle-train/src/rand.rs:229-234
    assert o.seed_sequence_u64(0, 4) == [0xDB2CD7E7B0F478BE, 0xABF4641A2C71BA49, 0x20C6ED6D9D7B8D41,
                                        0x2C4099DE223C39D4]
    assert o.NpRng(0).permutation(12) == [9, 2, 7, 4, 5, 11, 0, 3, 6, 10, 8, 1]
    assert o.NpRng(5).permutation(7) == [1, 4, 2, 3, 6, 5, 0]


def test_codebook_closed_form():
    # crates/needle-core/src/quant.rs:30-47,65-68: centroid / sqrt(group) in
    # f64 rounded to f32.  The f64 bit patterns restated independently here.
    lm4 = [0xC005AE0F408928FB, 0xC0005B0B8A516D54, 0xBFF9841FF0758FC8, 0xBFF3BBBEBADAC679, 0xBFED82C6DD21F59E,
           0xBFE47717151708B5, 0xBFD7D9B9E4B565FA, 0xBFBD4CA474B8559B, 0x3FC2683E9154FCE2, 0x3FD9DAF49368793A,
           0x3FE586B43E57D29D, 0x3FEEC3D50CBC3B33, 0x3FF4688DB93B85F1, 0x3FFA3164906B428F, 0x4000ACE7BBDE2442,
           0x4005ED98D06F2A4A]
    c = np.array(lm4, dtype=np.uint64).view(np.float64)
    want = (c / np.sqrt(128.0)).astype(np.float32)
    assert np.array_equal(o.codebook(4).view(np.uint32), want.view(np.uint32))
    # Sampled Lloyd-Max centroids: sorted, and symmetric up to sampling noise.
    assert np.all(np.diff(c) > 0)
    assert np.allclose(c, -c[::-1], atol=5e-2)


def test_int8_codebook_kat():
    # crates/needle-engine/src/qlinear.rs:40,211-216: cbs = max|cb| * K127
    # (K127 = 0x3c010204), cb8 = round-half-away(cb / cbs).  Closed form in
    # float64 from the f32 codebook.
    cb = o.codebook(4)
    cb8, cbs = o.int8_codebook(cb)
    k127 = np.uint32(0x3C010204).view(np.float32)
    m = np.float32(np.max(np.abs(cb)))
    assert np.float32(m * k127) == cbs
    inv = np.float32(np.float32(1.0) / cbs)
    v = (cb * inv).astype(np.float64)
    want = (np.sign(v) * np.floor(np.abs(v) + 0.5)).clip(-128, 127).astype(np.int8)
    assert np.array_equal(cb8, want)
    assert cb8.tolist() == [-126, -95, -74, -57, -43, -30, -17, -5, 7, 19, 31, 45, 59, 76, 97, 127]
    assert int(np.float32(cbs).view(np.uint32)) == 0x3AFA0AAE


def test_nearest_ties_low():
    # crates/needle-core/src/quant.rs:314-321
    cb = np.array([-1.0, 0.0, 1.0], dtype=np.float32)
    assert o.nearest(0.5, cb) == 1
    assert o.nearest(-0.5, cb) == 0
    assert o.nearest(5.0, cb) == 2
    assert o.nearest(-5.0, cb) == 0


def test_pack_round_trips():
    # crates/needle-core/src/quant.rs:306-312
    idx = np.array([(i * 7) % 16 for i in range(256)], dtype=np.uint8)
    assert np.array_equal(o.unpack_lsb(o.pack_lsb(idx, 4), 4, 256), idx)
    idx3 = np.array([(i * 5) % 8 for i in range(256)], dtype=np.uint8)
    assert np.array_equal(o.unpack_lsb(o.pack_lsb(idx3, 3), 3, 256), idx3)
    idx2 = np.array([(i * 3) % 4 for i in range(256)], dtype=np.uint8)
    assert np.array_equal(o.unpack_lsb(o.pack_lsb(idx2, 2), 2, 256), idx2)
    # LSB-first: byte j of a 4-bit row is code 2j | code 2j+1 << 4.
    p = o.pack_lsb(idx, 4)
    assert np.array_equal(p, (idx[0::2] | (idx[1::2] << 4)).astype(np.uint8))


def test_neg_constant():
    # crates/needle-engine/src/infer.rs:36
    assert np.float32(o.neg()).view(np.uint32) == 0xF149F2CA


def test_argmax_first_max():
    # crates/needle-engine/src/generate.rs:42-50
    assert o.argmax(np.array([1, 3, 3, 2], dtype=np.float32)) == 1
    assert o.argmax(np.array([-1, -1], dtype=np.float32)) == 0


@pytest.mark.parametrize("seed", [0, 1])
def test_random_tokens_in_range(seed):
    # numpy masked rejection interval (rand.rs:105-119): ids uniform in
    # [0, vocab - 1] and reproducible.
    t = o.random_tokens(500, 8192, seed)
    assert t.min() >= 0 and t.max() <= 8191
    assert np.array_equal(t, o.random_tokens(500, 8192, seed))
    assert len(np.unique(t)) > 400
