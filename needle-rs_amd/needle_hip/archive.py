"""Writing .cact archives (crates/needle-core/src/cact.rs:274-475) for a
random-init Needle-3 model, the input of benchmarks and examples without a
trained checkpoint.

The records follow the export order of cact.rs:278-351 (no probe heads, no
tokenizer): every matmul weight is 0.02 * N(0, 1) packed to CQ-W4 on the
GPU with QMat::from_f32 (nh_qmat_from_f32) and stored as cact::cq stores it
(packed codes, then f16 norms, cact.rs:265-270); the small tensors are
seeded uniform(-1, 1) in f16 (fp16, cact.rs:255-258); the Hadamard
permutations are the reference's seeded ones (seeds 11 and 13,
crates/needle-core/src/config.rs:14, MT19937 Fisher-Yates as numpy's
RandomState.permutation).  The header, codebook block, 44-byte directory
records and 64-byte blob alignment are cact::pack's (cact.rs:398-475).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

TAG = 0x05E12A84   # cact.rs:18
F16, F32, CQ = 1, 2, 3
GROUP = 128
ALIGN = 64
REC_SIZE = 44
CB_BITS = (2, 3, 4)
ENGRAM_CONV_TAPS = 4
PERM_SEEDS = (11, 13)


@dataclass
class Needle3:
    """The Config fields the export reads (crates/needle-core/src/config.rs:61-100 defaults)."""
    vocab: int = 16384
    d_model: int = 768
    num_heads: int = 12
    num_kv_heads: int = 2
    num_layers: int = 20
    qk_head_dim: int = 48
    v_head_dim: int = 64
    max_seq_len: int = 4096
    mhc_lanes: int = 4
    qkv_conv_taps: int = 3
    engram_orders: tuple = (2, 3)
    engram_slots: int = 18432
    engram_sites: tuple = (3, 7, 11, 15, 19)
    global_layers: tuple = (4, 9, 14, 19)
    sliding_window: int = 1024
    rope_theta: float = 100000.0
    out_vocab: int = 0
    extra: dict = field(default_factory=dict)

    @property
    def engram_heads(self) -> int:
        # engram_geometry (config.rs:274-279) with engram_heads unset
        return max(self.d_model // (len(self.engram_orders) * GROUP), 1)

    @property
    def engram_sub_dim(self) -> int:
        return self.d_model // (len(self.engram_orders) * self.engram_heads)

    @property
    def hada_n(self) -> int:
        n = 1
        while n < self.d_model:
            n *= 2
        return n


def _hada_blocks(n: int):
    # hada_blocks (config.rs:315-319)
    bits = (n - 1).bit_length()
    a = 1 << (bits // 2)
    return a, n // a


class _Writer:
    def __init__(self):
        self.records = []  # (dtype, shape, blob, group, bits)

    def f16(self, values: np.ndarray, shape=None):
        v = np.asarray(values, dtype=np.float32)
        self.records.append((F16, list(shape if shape is not None else v.shape),
                             v.astype(np.float16).tobytes(), 0, 0))

    def f32(self, values: np.ndarray):
        v = np.ascontiguousarray(values, dtype=np.float32)
        self.records.append((F32, list(v.shape), v.tobytes(), 0, 0))

    def cq(self, packed: np.ndarray, norms: np.ndarray, out: int, in_dim: int, bits: int = 4):
        blob = np.ascontiguousarray(packed).tobytes() + np.ascontiguousarray(norms, dtype=np.uint16).tobytes()
        self.records.append((CQ, [out, in_dim], blob, GROUP, bits))


def _header(g: Needle3, num_tensors: int, codebook_len: int) -> bytes:
    orders = list(g.engram_orders) + [0] * (4 - len(g.engram_orders))
    sites = list(g.engram_sites) + [0] * (16 - len(g.engram_sites))
    gmask = 0
    for l in g.global_layers:
        gmask |= 1 << l
    words = [TAG, num_tensors, codebook_len, 0, 8, g.vocab, g.out_vocab, g.d_model, g.num_heads, g.num_kv_heads,
             g.num_layers, g.qk_head_dim, g.v_head_dim, g.max_seq_len, g.hada_n, g.mhc_lanes, g.sliding_window,
             gmask & 0xFFFFFFFF, gmask >> 32, g.qkv_conv_taps, g.engram_slots, g.engram_sub_dim,
             len(g.engram_orders) * g.engram_heads, ENGRAM_CONV_TAPS, max(g.engram_orders, default=0), 0,
             len(g.engram_orders), *orders, len(g.engram_sites), *sites]
    assert len(words) == 48
    return struct.pack("<48I", *words) + struct.pack("<f", g.rope_theta)


def pack(records, g: Needle3, codebook: np.ndarray) -> bytes:
    """cact::pack's layout (cact.rs:416-475) for records already made."""
    buf = bytearray(_header(g, len(records), codebook.size))
    buf += codebook.astype(np.float32).tobytes()
    pos = len(buf) + len(records) * REC_SIZE
    offsets = []
    for r in records:
        pos = (pos + ALIGN - 1) & ~(ALIGN - 1)
        offsets.append(pos)
        pos += len(r[2])
    for (dtype, shape, blob, group, bits), off in zip(records, offsets):
        dims = list(shape) + [0] * (4 - len(shape))
        buf += struct.pack("<BB2x4IQQII", dtype, len(shape), *dims, off, len(blob), group, bits)
    for (_, _, blob, _, _), off in zip(records, offsets):
        buf += bytes(off - len(buf))
        buf += blob
    return bytes(buf)


def random_needle3(nh, g: Needle3 | None = None, seed: int = 0) -> bytes:
    """The archive of a random-init model of geometry g (Needle-3 by
    default): matmul weights 0.02 * N(0, 1) through CQ-W4, seeded."""
    g = g or Needle3()
    rng = np.random.default_rng(seed)
    w = _Writer()
    d, L, n = g.d_model, g.num_layers, g.mhc_lanes
    qk, vd = g.qk_head_dim, g.v_head_dim
    qd, kd, vdim = g.num_heads * qk, g.num_kv_heads * qk, g.num_kv_heads * vd
    hn = g.hada_n
    ba, bb = _hada_blocks(hn)
    tables = len(g.engram_orders) * g.engram_heads

    def mat(out, in_dim):
        x = rng.standard_normal((out, in_dim), dtype=np.float32)
        x *= np.float32(0.02)
        q = nh.QMat.from_f32(x, out, in_dim)
        packed, norms = q.download()
        w.cq(packed, norms, out, in_dim)

    def row(*shape):
        w.f16(rng.uniform(-1.0, 1.0, size=shape).astype(np.float32))

    mat(g.vocab, d)
    for _ in range(L):
        row(d)
        mat(qd, d)
        mat(kd, d)
        mat(vdim, d)
        if g.qkv_conv_taps > 0:
            row(g.qkv_conv_taps, qd)
            row(g.qkv_conv_taps, kd)
            row(g.qkv_conv_taps, vdim)
        row(qk)
        row(qk)
        mat(g.num_heads * vd, d)   # gate
        mat(d, g.num_heads * vd)   # out
        row(d)
        w.f16(rng.uniform(-1.0, 1.0, size=1), [1])  # attn_gate
        row(d)
        for _ in range(5):         # d1, d2, b2, d3, d4
            row(hn)
        for _ in range(3):         # w1a, w1b, w2a, w2b, w3a, w3b
            row(ba, ba)
            row(bb, bb)
        row(d, 8)                  # cond_v
        row(8, hn)                 # cond_u
    for _ in range(3):             # mhc a_pre, a_post, a_res
        row(L)
    row(L, n)
    row(L, n)
    row(L, n * n)
    mat(L * n, n * d)              # phi pre, post, res
    mat(L * n, n * d)
    mat(L * n * n, n * d)
    for s in PERM_SEEDS:
        w.f32(np.random.RandomState(s).permutation(hn).astype(np.float32))
    for _ in g.engram_sites:
        mat(tables * g.engram_slots, g.engram_sub_dim)
        mat(d, d)                  # key
        mat(d, d)                  # value
        row(ENGRAM_CONV_TAPS, d)
    row(d)                         # final_norm
    cb = np.concatenate([nh.codebook(b) for b in CB_BITS]).astype(np.float32)
    return pack(w.records, g, cb)
