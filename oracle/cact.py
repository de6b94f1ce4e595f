"""The .cact archive format (crates/needle-core/src/cact.rs), restated for the
tests.  TEST INFRASTRUCTURE: only tests/ may use it; the product reads
archives in C++ (needle-rs_amd/csrc/nh_archive.cpp).

- `Header`, `Record`: the byte layouts (cact.rs:80-131, 199-230).
- `pack`: the archive bytes for a list of tensors (cact.rs:398-475): header,
  the 2/3/4-bit codebooks, the 44-byte directory, blobs 64-byte aligned.
- `Archive`: the reader with the reference's checks (cact.rs:593-627).
- `needle3_tensors`: tensors in the canonical export order (cact.rs:274-343,
  the order weights.rs:318-420 reads) for a model geometry, with seeded
  synthetic contents, and the fused matrices QWeights builds from them
  (weights.rs:372-389, 413, 480-495).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

from . import codebook, cq_pack, f32_to_f16

TAG = 0x05E12A84     # cact.rs:18
TAG_V2 = 0x05E12A83  # cact.rs:19
ALIGN = 64           # cact.rs:20
HEADER_BYTES = 49 * 4
REC_SIZE = 44
F16, F32, CQ, RAW = 1, 2, 3, 4  # cact.rs:26-31
CB_BITS = (2, 3, 4)  # quant.rs:13
TERNARY = 5          # quant.rs:12
GROUP = 128


class ArchiveError(ValueError):
    pass


@dataclass
class Header:
    """cact.rs:47-78; `to_bytes` / `parse` follow cact.rs:80-165."""
    num_tensors: int = 0
    codebook_len: int = 0
    kv_window: int = 0
    kv_bits: int = 8
    vocab: int = 0
    out_vocab: int = 0
    d_model: int = 0
    num_heads: int = 0
    num_kv_heads: int = 0
    num_layers: int = 0
    qk_head_dim: int = 0
    v_head_dim: int = 0
    max_seq_len: int = 0
    hada_n: int = 0
    mhc_lanes: int = 0
    sliding_window: int = 0
    global_mask: int = 0
    qkv_conv_taps: int = 0
    engram_slots: int = 0
    engram_sub_dim: int = 0
    num_engram_tables: int = 0
    engram_conv_taps: int = 4
    engram_conv_dilation: int = 0
    engram_seed_heads: int = 0
    engram_orders: list = field(default_factory=list)
    engram_sites: list = field(default_factory=list)
    rope_theta: float = 100000.0
    tag: int = TAG

    def words(self) -> list:
        orders = list(self.engram_orders) + [0] * (4 - len(self.engram_orders))
        sites = list(self.engram_sites) + [0] * (16 - len(self.engram_sites))
        return [self.tag, self.num_tensors, self.codebook_len, self.kv_window, self.kv_bits, self.vocab,
                self.out_vocab, self.d_model, self.num_heads, self.num_kv_heads, self.num_layers, self.qk_head_dim,
                self.v_head_dim, self.max_seq_len, self.hada_n, self.mhc_lanes, self.sliding_window,
                self.global_mask & 0xFFFFFFFF, self.global_mask >> 32, self.qkv_conv_taps, self.engram_slots,
                self.engram_sub_dim, self.num_engram_tables, self.engram_conv_taps, self.engram_conv_dilation,
                self.engram_seed_heads, len(self.engram_orders), *orders, len(self.engram_sites), *sites]

    def to_bytes(self) -> bytes:
        w = self.words()
        assert len(w) == 48
        return struct.pack("<48I", *w) + struct.pack("<f", self.rope_theta)

    @classmethod
    def parse(cls, b: bytes) -> "Header":
        if len(b) < HEADER_BYTES:
            raise ArchiveError("not a complete .cact archive")
        u = struct.unpack_from("<48I", b, 0)
        if u[0] != TAG:
            if u[0] == TAG_V2:
                raise ArchiveError(f"this is a Needle 2 archive; Needle 3 (tag 0x{TAG:08x}) is required")
            raise ArchiveError(f"unknown .cact format tag 0x{u[0]:08x}")
        n_orders, n_sites = u[26], u[31]
        if n_orders > 4 or n_sites > 16:
            raise ArchiveError("corrupt .cact header")
        return cls(num_tensors=u[1], codebook_len=u[2], kv_window=u[3], kv_bits=u[4], vocab=u[5], out_vocab=u[6],
                   d_model=u[7], num_heads=u[8], num_kv_heads=u[9], num_layers=u[10], qk_head_dim=u[11],
                   v_head_dim=u[12], max_seq_len=u[13], hada_n=u[14], mhc_lanes=u[15], sliding_window=u[16],
                   global_mask=u[17] | (u[18] << 32), qkv_conv_taps=u[19], engram_slots=u[20],
                   engram_sub_dim=u[21], num_engram_tables=u[22], engram_conv_taps=u[23],
                   engram_conv_dilation=u[24], engram_seed_heads=u[25], engram_orders=list(u[27:27 + n_orders]),
                   engram_sites=list(u[32:32 + n_sites]), rope_theta=struct.unpack_from("<f", b, 192)[0],
                   tag=u[0])


@dataclass
class Record:
    """A directory entry (cact.rs:189-230)."""
    dtype: int
    shape: list
    offset: int
    nbytes: int
    group: int = 0
    bits: int = 0

    def to_bytes(self) -> bytes:
        b = bytearray(REC_SIZE)
        b[0] = self.dtype
        b[1] = len(self.shape)
        for i, d in enumerate(self.shape[:4]):
            struct.pack_into("<I", b, 4 + 4 * i, d)
        struct.pack_into("<QQII", b, 20, self.offset, self.nbytes, self.group, self.bits)
        return bytes(b)

    @classmethod
    def parse(cls, b: bytes) -> "Record":
        ndim = b[1]
        if ndim > 4:
            raise ArchiveError("corrupt .cact record")
        if b[0] not in (F16, F32, CQ, RAW):
            raise ArchiveError(f"unknown .cact tensor dtype {b[0]}")
        shape = list(struct.unpack_from(f"<{ndim}I", b, 4))
        offset, nbytes, group, bits = struct.unpack_from("<QQII", b, 20)
        return cls(b[0], shape, offset, nbytes, group, bits)


@dataclass
class Tensor:
    """A tensor about to be written (cact.rs:233-240)."""
    dtype: int
    shape: list
    blob: bytes
    group: int = 0
    bits: int = 0


def fp16(x, shape=None) -> Tensor:
    x = np.asarray(x, dtype=np.float32)
    return Tensor(F16, list(shape if shape is not None else x.shape), f32_to_f16(x.reshape(-1)).tobytes())


def f32(x, shape=None) -> Tensor:
    x = np.asarray(x, dtype=np.float32)
    return Tensor(F32, list(shape if shape is not None else x.shape), x.tobytes())


def cq_tensor(packed: np.ndarray, norms: np.ndarray, out: int, in_dim: int, bits: int) -> Tensor:
    """A CQ blob: packed rows, then f16 norms (cact.rs:261-268)."""
    blob = np.ascontiguousarray(packed, np.uint8).tobytes() + np.ascontiguousarray(norms, np.uint16).tobytes()
    return Tensor(CQ, [out, in_dim], blob, GROUP, bits)


def align(n: int) -> int:
    return (n + ALIGN - 1) & ~(ALIGN - 1)


def codebook_block() -> np.ndarray:
    """The header's codebooks: 2-, 3- and 4-bit, group 128 (cact.rs:412)."""
    return np.concatenate([codebook(b, GROUP) for b in CB_BITS]).astype(np.float32)


def pack(tensors: list, header: Header) -> bytes:
    """cact::pack's layout (cact.rs:398-475) for tensors already made."""
    cb = codebook_block()
    header.num_tensors = len(tensors)
    header.codebook_len = cb.size
    buf = bytearray(header.to_bytes())
    assert len(buf) == HEADER_BYTES
    buf += cb.tobytes()
    pos = len(buf) + len(tensors) * REC_SIZE
    recs = []
    for t in tensors:
        pos = align(pos)
        recs.append(Record(t.dtype, t.shape, pos, len(t.blob), t.group, t.bits))
        pos += len(t.blob)
    for r in recs:
        buf += r.to_bytes()
    for t, r in zip(tensors, recs):
        buf += bytes(r.offset - len(buf))
        buf += t.blob
    return bytes(buf)


class Archive:
    """The reader (cact.rs:593-627)."""

    def __init__(self, data: bytes):
        self.data = data
        self.header = Header.parse(data)
        off = HEADER_BYTES
        n = self.header.codebook_len
        if off + 4 * n > len(data):
            raise ArchiveError("truncated codebook")
        self.codebook = np.frombuffer(data, dtype=np.float32, count=n, offset=off)
        off += 4 * n
        self.records = []
        for _ in range(self.header.num_tensors):
            if off + REC_SIZE > len(data):
                raise ArchiveError("truncated directory")
            r = Record.parse(data[off:off + REC_SIZE])
            if r.offset + r.nbytes > len(data):
                raise ArchiveError("tensor past the end of the archive")
            self.records.append(r)
            off += REC_SIZE

    def bytes(self, i: int) -> bytes:
        r = self.records[i]
        return self.data[r.offset:r.offset + r.nbytes]

    def cq(self, i: int):
        """-> (packed u8 [out, row_bytes], norms u16 [out, groups], out, in_dim, bits) (cact.rs:617-627)."""
        r = self.records[i]
        if r.dtype != CQ:
            raise ArchiveError(f"tensor {i} is not CQ")
        out, in_dim = r.shape[0], r.shape[1]
        groups = -(-in_dim // r.group)
        cbits = 2 if r.bits == TERNARY else r.bits
        row_bytes = groups * r.group * cbits // 8
        blob = np.frombuffer(self.bytes(i), dtype=np.uint8)
        packed = blob[:out * row_bytes].reshape(out, row_bytes)
        norms = blob[out * row_bytes:out * row_bytes + out * groups * 2].view(np.uint16).reshape(out, groups)
        return packed, norms, out, in_dim, r.bits


# ----------------------------------------------------------------- geometry

@dataclass
class Geometry:
    """The fields of crates/needle-core/src/config.rs that fix the export
    order and shapes (defaults: Needle 3, config.rs:61-100)."""
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

    @property
    def engram_heads(self) -> int:
        """engram_geometry (config.rs:274-279) with engram_heads unset."""
        return max(self.d_model // (len(self.engram_orders) * 128), 1)

    @property
    def engram_sub_dim(self) -> int:
        return self.d_model // (len(self.engram_orders) * self.engram_heads)

    @property
    def num_engram_tables(self) -> int:
        return len(self.engram_orders) * self.engram_heads

    @property
    def hada_n(self) -> int:
        """config.rs:291-293: d_model rounded up to a power of two."""
        n = 1
        while n < self.d_model:
            n *= 2
        return n

    def header(self) -> Header:
        """The header cact::pack writes for this geometry (cact.rs:416-447)."""
        return Header(kv_window=0, kv_bits=8, vocab=self.vocab, out_vocab=0, d_model=self.d_model,
                      num_heads=self.num_heads, num_kv_heads=self.num_kv_heads, num_layers=self.num_layers,
                      qk_head_dim=self.qk_head_dim, v_head_dim=self.v_head_dim, max_seq_len=self.max_seq_len,
                      hada_n=self.hada_n, mhc_lanes=self.mhc_lanes, sliding_window=self.sliding_window,
                      global_mask=sum(1 << g for g in self.global_layers), qkv_conv_taps=self.qkv_conv_taps,
                      engram_slots=self.engram_slots, engram_sub_dim=self.engram_sub_dim,
                      num_engram_tables=self.num_engram_tables, engram_conv_taps=4,
                      engram_conv_dilation=max(self.engram_orders) if self.engram_orders else 0,
                      engram_seed_heads=0, engram_orders=list(self.engram_orders),
                      engram_sites=list(self.engram_sites), rope_theta=self.rope_theta)


def hada_blocks(n: int):
    """config.rs:315-319."""
    bits = (n - 1).bit_length()
    a = 1 << (bits // 2)
    return a, n // a


def hada_perm(seed: int, n: int) -> np.ndarray:
    """Mt19937(seed).permutation(n) = np.random.RandomState(seed).permutation(n)
    (crates/needle-core/src/rng.rs:77-88,94-98)."""
    return np.random.RandomState(seed).permutation(n)


@dataclass
class Matmul:
    """One matmul record: the matrix a loader makes of it (CQ blob as stored,
    or f32 values it packs at 4 bits)."""
    out: int
    in_dim: int
    bits: int = 4
    packed: np.ndarray | None = None
    norms: np.ndarray | None = None
    w: np.ndarray | None = None  # f32 [out, in] for an f16/f32 record


def _matmul_record(rng, out: int, in_dim: int, bits: int, kind: str):
    """A matmul record and its Matmul: 'cq' packs seeded N(0, 0.02) weights
    with cq_pack (4-bit, as cact::cq does, cact.rs:261-268); 'random' writes
    seeded code bytes and norms (any width, fast at full size); 'f16' / 'f32'
    store the weights unpacked."""
    groups = -(-in_dim // GROUP)
    if kind == "cq":
        w = (rng.standard_normal((out, in_dim)) * 0.02).astype(np.float32)
        packed, norms = cq_pack(w, in_dim, 4)
        return cq_tensor(packed, norms, out, in_dim, 4), Matmul(out, in_dim, 4, packed, norms)
    if kind == "random":
        cbits = 2 if bits == TERNARY else bits
        packed = rng.integers(0, 256, size=(out, groups * GROUP * cbits // 8), dtype=np.uint8)
        norms = f32_to_f16(rng.uniform(0.2, 3.0, size=out * groups).astype(np.float32)).reshape(out, groups)
        return cq_tensor(packed, norms, out, in_dim, bits), Matmul(out, in_dim, bits, packed, norms)
    w = (rng.standard_normal((out, in_dim)) * 0.02).astype(np.float32)
    if kind == "f16":
        t = fp16(w)
        w = np.frombuffer(f32_to_f16(w.reshape(-1)).tobytes(), dtype=np.float16).astype(np.float32).reshape(w.shape)
        return t, Matmul(out, in_dim, 4, w=w)
    return f32(w), Matmul(out, in_dim, 4, w=w)


def needle3_tensors(g: Geometry, seed: int = 0, kind=lambda name: ("random", 4)):
    """Tensors in the export order of cact.rs:274-343 (no probe heads, no
    tokenizer) with seeded contents, and the matmuls by name.

    `kind(name)` -> (record kind, bits) for each matmul record: names are
    'embedding', 'q.l', 'k.l', 'v.l', 'gate.l', 'out.l', 'phi_pre',
    'phi_post', 'phi_res', 'engram_table.s', 'engram_key.s', 'engram_value.s'."""
    rng = np.random.default_rng(seed)
    d, L, n = g.d_model, g.num_layers, g.mhc_lanes
    qk, vd = g.qk_head_dim, g.v_head_dim
    qd, kd, vdim = g.num_heads * qk, g.num_kv_heads * qk, g.num_kv_heads * vd
    hn = g.hada_n
    ba, bb = hada_blocks(hn)
    ts, mats = [], {}

    def mm(name, out, in_dim):
        k, bits = kind(name)
        t, m = _matmul_record(rng, out, in_dim, bits, k)
        ts.append(t)
        mats[name] = m

    def row(*shape):
        ts.append(fp16(rng.uniform(-1.0, 1.0, size=shape).astype(np.float32)))

    mm("embedding", g.vocab, d)
    for i in range(L):
        row(d)  # ZCRMSNorm_0/scale
        mm(f"q.{i}", qd, d)
        mm(f"k.{i}", kd, d)
        mm(f"v.{i}", vdim, d)
        if g.qkv_conv_taps > 0:
            row(g.qkv_conv_taps, qd)
            row(g.qkv_conv_taps, kd)
            row(g.qkv_conv_taps, vdim)
        row(qk)  # q_norm
        row(qk)  # k_norm
        mm(f"gate.{i}", g.num_heads * vd, d)
        mm(f"out.{i}", d, g.num_heads * vd)
        row(d)  # post_attn_norm
        ts.append(fp16(rng.uniform(-1.0, 1.0, size=1).astype(np.float32), [1]))  # attn_gate
        row(d)  # pre_hada_norm
        for _ in ("d1", "d2", "b2", "d3", "d4"):
            row(hn)
        for _ in range(3):
            row(ba, ba)
            row(bb, bb)
        row(d, 8)   # cond_v
        row(8, hn)  # cond_u
    for _ in ("a_pre", "a_post", "a_res"):
        row(L)
    row(L, n)      # b_pre
    row(L, n)      # b_post
    row(L, n * n)  # b_res
    mm("phi_pre", L * n, n * d)
    mm("phi_post", L * n, n * d)
    mm("phi_res", L * n * n, n * d)
    for s in (11, 13):  # HADA_PERM_SEEDS (config.rs:14)
        ts.append(f32(hada_perm(s, hn).astype(np.float32)))
    for s in range(len(g.engram_sites)):
        mm(f"engram_table.{s}", g.num_engram_tables * g.engram_slots, g.engram_sub_dim)
        mm(f"engram_key.{s}", d, d)
        mm(f"engram_value.{s}", d, d)
        row(4, d)  # taps
    row(d)  # final_norm
    return ts, mats


def fused(mats: dict, g: Geometry) -> dict:
    """QWeights' matrices as lists of (part Matmul, row range) (weights.rs:372-389,
    413, 480-495)."""
    L, n = g.num_layers, g.mhc_lanes
    out = {"embedding": [[(mats["embedding"], None)]],
           "qkvg": [[(mats[f"{p}.{i}"], None) for p in ("q", "k", "v", "gate")] for i in range(L)],
           "out": [[(mats[f"out.{i}"], None)] for i in range(L)],
           "phi": [[(mats["phi_pre"], (l * n, (l + 1) * n)), (mats["phi_post"], (l * n, (l + 1) * n)),
                    (mats["phi_res"], (l * n * n, (l + 1) * n * n))] for l in range(L)],
           "engram_tables": [[(mats[f"engram_table.{s}"], None)] for s in range(len(g.engram_sites))],
           "engram_kv": [[(mats[f"engram_key.{s}"], None), (mats[f"engram_value.{s}"], None)]
                         for s in range(len(g.engram_sites))]}
    return out
