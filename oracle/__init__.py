"""CPU oracle for needle-rs's packed CQ runtime (test infrastructure).

Loads ``oracle/_build/libcq_oracle.so`` (the C restatement in
``cq_oracle.c``) and exposes numpy-friendly wrappers.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import
this module; the product package never does.

Parity of every function here is pinned by the tests in
``tests/test_oracle_*.py`` (known-answer vectors from the reference's own
tests, closed forms and brute force); see the header of ``cq_oracle.h``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libcq_oracle.so")
GROUP = 128

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc, host only)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class QAct(C.Structure):
    _fields_ = [("rows", C.c_size_t), ("groups", C.c_size_t), ("bits", C.c_uint8),
                ("xq", C.POINTER(C.c_int8)), ("sx", C.POINTER(C.c_float))]


class QMat(C.Structure):
    _fields_ = [("out", C.c_size_t), ("in_dim", C.c_size_t), ("groups", C.c_size_t), ("bits", C.c_uint8),
                ("codes", C.POINTER(C.c_uint8)), ("norms", C.POINTER(C.c_uint16)),
                ("tables", (C.c_int8 * 16) * 2), ("vals", C.c_int8 * 16), ("cbs", C.c_float),
                ("fvals", C.c_float * 16)]


class QLinear(C.Structure):
    _fields_ = [("nparts", C.c_size_t), ("out", C.c_size_t), ("in_dim", C.c_size_t),
                ("parts", C.POINTER(C.POINTER(QMat)))]


P = C.c_void_p
SZ = C.c_size_t
F = C.c_float
PQA = C.POINTER(QAct)
PQM = C.POINTER(QMat)
PQL = C.POINTER(QLinear)


def _declare(l):
    sig = {
        "cq_f32_to_f16": (C.c_uint16, [F]),
        "cq_f16_to_f32": (F, [C.c_uint16]),
        "cq_k127": (F, []),
        "cq_neg": (F, []),
        "cq_lloyd_max": (C.c_int, [C.c_uint32, P]),
        "cq_codebook": (C.c_int, [C.c_uint32, SZ, P]),
        "cq_hadamard_scale": (F, [SZ]),
        "cq_hadamard": (None, [SZ, P]),
        "cq_fwht": (None, [P, SZ]),
        "cq_rotate": (None, [P, SZ]),
        "cq_nearest": (SZ, [F, P, SZ]),
        "cq_pack_lsb": (SZ, [P, SZ, C.c_uint32, P]),
        "cq_unpack_lsb_into": (None, [P, SZ, C.c_uint32, P, SZ]),
        "cq_packed_row_bytes": (SZ, [SZ, C.c_uint32]),
        "cq_pack": (None, [P, SZ, SZ, C.c_uint32, SZ, P, P, C.c_int]),
        "cq_unpack": (None, [P, P, SZ, SZ, C.c_uint32, SZ, P]),
        "cq_quant_i8": (F, [P, SZ, P]),
        "cq_quant_scale": (F, [P, SZ]),
        "cq_quant_with": (None, [P, SZ, F, P]),
        "cq_act_pos": (SZ, [SZ, C.c_uint8]),
        "cq_prep_group": (F, [P, SZ, SZ, P, C.c_uint8]),
        "cq_int8_codebook": (None, [P, SZ, P, P]),
        "cq_qact_new": (PQA, [P, SZ, SZ, C.c_uint8, C.c_int]),
        "cq_qact_empty_rows": (PQA, [SZ, SZ, C.c_uint8]),
        "cq_qact_free": (None, [PQA]),
        "cq_qmat_build": (PQM, [SZ, SZ, C.c_uint8, P, SZ, C.c_int, P, P]),
        "cq_qmat_from_cq": (PQM, [P, P, SZ, SZ, C.c_uint32, SZ]),
        "cq_qmat_from_f32": (PQM, [P, SZ, SZ, C.c_int]),
        "cq_qmat_free": (None, [PQM]),
        "cq_qmat_bytes": (SZ, [PQM]),
        "cq_qmat_row": (None, [PQM, SZ, P]),
        "cq_lane_sums": (None, [PQM, SZ, SZ, PQA, SZ, P]),
        "cq_decode_row_ref": (F, [PQM, SZ, PQA]),
        "cq_prefill_row_ref": (F, [PQM, SZ, PQA, SZ, C.c_int]),
        "cq_single_row": (F, [PQM, SZ, PQA]),
        "cq_matmul_into": (None, [PQM, PQA, P, SZ, SZ, C.c_int]),
        "cq_prefill_rows_flags": (None, [PQM, PQA, P, P, SZ, SZ, C.c_int]),
        "cq_head_logits_sparse": (None, [PQM, PQA, P, SZ, SZ, P]),
        "cq_all_lane_sums": (None, [PQM, PQA, SZ, P, C.c_int]),
        "cq_all_totals": (None, [PQM, PQA, P, C.c_int]),
        "cq_matmul_rows": (None, [PQM, PQA, P, P, SZ, SZ, SZ, SZ, C.c_int]),
        "cq_qlinear_new": (PQL, [P, SZ]),
        "cq_qlinear_free": (None, [PQL]),
        "cq_qlinear_matmul": (None, [PQL, PQA, P, C.c_int]),
        "cq_dot16": (F, [P, P, SZ]),
        "cq_rinv": (F, [F, SZ]),
        "cq_zcn16": (None, [P, P, SZ, P]),
        "cq_norm_apply16": (None, [P, P, F, P, SZ]),
        "cq_argmax": (SZ, [P, SZ]),
        "cq_threefry2x32": (None, [P, P, P]),
        "cq_prng_key": (None, [C.c_uint64, P]),
        "cq_split": (None, [P, P, P]),
        "cq_erfinv_f32": (F, [F]),
        "cq_normal": (None, [P, SZ, P, C.c_int]),
        "cq_seed_sequence_u64": (None, [C.c_uint64, SZ, P]),
        "cq_nprng_new": (P, [C.c_uint64]),
        "cq_nprng_free": (None, [P]),
        "cq_nprng_next_u64": (C.c_uint64, [P]),
        "cq_nprng_next_u32": (C.c_uint32, [P]),
        "cq_nprng_interval": (C.c_uint64, [P, C.c_uint64]),
        "cq_nprng_permutation": (None, [P, SZ, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def default_threads() -> int:
    env = os.environ.get("NEEDLE_THREADS")
    if env:
        return int(env)
    return len(os.sched_getaffinity(0))


# ---------------------------------------------------------------- scalars
def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([lib().cq_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    return np.array([lib().cq_f16_to_f32(int(v)) for v in h], dtype=np.float32)


def k127() -> float:
    return lib().cq_k127()


def neg() -> float:
    return lib().cq_neg()


# ---------------------------------------------------------------- quant.rs
def lloyd_max(bits: int) -> np.ndarray:
    out = np.zeros(16, dtype=np.float64)
    n = lib().cq_lloyd_max(bits, _p(out))
    return out[:n]


def codebook(bits: int, group: int = GROUP) -> np.ndarray:
    out = np.zeros(16, dtype=np.float32)
    n = lib().cq_codebook(bits, group, _p(out))
    return out[:n]


def hadamard(n: int) -> np.ndarray:
    out = np.zeros((n, n), dtype=np.float32)
    lib().cq_hadamard(n, _p(out))
    return out


def fwht(x: np.ndarray) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    lib().cq_fwht(_p(y), y.size)
    return y


def rotate(x: np.ndarray) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    lib().cq_rotate(_p(y), y.size)
    return y


def nearest(x: float, cb: np.ndarray) -> int:
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    return lib().cq_nearest(x, _p(cb), cb.size)


def pack_lsb(idx: np.ndarray, bits: int) -> np.ndarray:
    idx = np.ascontiguousarray(idx, dtype=np.uint8)
    out = np.zeros((idx.size + 7) // 8 * bits, dtype=np.uint8)
    n = lib().cq_pack_lsb(_p(idx), idx.size, bits, _p(out))
    return out[:n]


def unpack_lsb(packed: np.ndarray, bits: int, n: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros(n, dtype=np.uint8)
    lib().cq_unpack_lsb_into(_p(packed), packed.size, bits, _p(out), n)
    return out


def cq_pack(w: np.ndarray, d: int, bits: int = 4, group: int = GROUP, threads: int | None = None):
    """-> (packed u8 [rows, in_pad*bits/8], norms f16-bits u16 [rows, in_pad/group])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows = w.size // d
    in_pad = (d + group - 1) // group * group
    packed = np.zeros((rows, in_pad * bits // 8), dtype=np.uint8)
    norms = np.zeros((rows, in_pad // group), dtype=np.uint16)
    lib().cq_pack(_p(w), rows, d, bits, group, _p(packed), _p(norms), threads or default_threads())
    return packed, norms


def cq_unpack(packed, norms, out: int, in_dim: int, bits: int = 4, group: int = GROUP) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    norms = np.ascontiguousarray(norms, dtype=np.uint16)
    w = np.zeros((out, in_dim), dtype=np.float32)
    lib().cq_unpack(_p(packed), _p(norms), out, in_dim, bits, group, _p(w))
    return w


# -------------------------------------------------------------- qlinear.rs
def quant_i8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(x.size, dtype=np.int8)
    s = lib().cq_quant_i8(_p(x), x.size, _p(q))
    return q, np.float32(s)


def act_pos(p: int, bits: int) -> int:
    return lib().cq_act_pos(p, bits)


def prep_group(x: np.ndarray, g: int, bits: int = 4):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(GROUP, dtype=np.int8)
    s = lib().cq_prep_group(_p(x), x.size, g, _p(q), bits)
    return q, np.float32(s)


def int8_codebook(cb: np.ndarray):
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    cb8 = np.zeros(cb.size, dtype=np.int8)
    s = np.zeros(1, dtype=np.float32)
    lib().cq_int8_codebook(_p(cb), cb.size, _p(cb8), _p(s))
    return cb8, s[0]


class OQAct:
    """QAct (crates/needle-engine/src/qlinear.rs:65-72, 166-208)."""

    def __init__(self, ptr):
        self.ptr = ptr

    @classmethod
    def new(cls, x: np.ndarray, rows: int, in_dim: int, bits: int = 4, threads: int | None = None):
        x = np.ascontiguousarray(x, dtype=np.float32)
        assert x.size == rows * in_dim
        return cls(lib().cq_qact_new(_p(x), rows, in_dim, bits, threads or 1))

    @property
    def rows(self):
        return self.ptr.contents.rows

    @property
    def groups(self):
        return self.ptr.contents.groups

    @property
    def xq(self) -> np.ndarray:
        c = self.ptr.contents
        return np.ctypeslib.as_array(c.xq, shape=(c.rows, c.groups, GROUP)).copy()

    @property
    def sx(self) -> np.ndarray:
        c = self.ptr.contents
        return np.ctypeslib.as_array(c.sx, shape=(c.rows, c.groups)).copy()

    def __del__(self):
        if getattr(self, "ptr", None) and _lib is not None:
            _lib.cq_qact_free(self.ptr)
            self.ptr = None


class OQMat:
    """QMat (crates/needle-engine/src/qlinear.rs:43-61, 218-488)."""

    def __init__(self, ptr):
        if not ptr:
            raise ValueError("oracle QMat construction failed")
        self.ptr = ptr

    @classmethod
    def from_f32(cls, w: np.ndarray, out: int, in_dim: int, threads: int | None = None):
        w = np.ascontiguousarray(w, dtype=np.float32)
        return cls(lib().cq_qmat_from_f32(_p(w), out, in_dim, threads or default_threads()))

    @classmethod
    def from_cq(cls, packed, norms, out: int, in_dim: int, bits: int = 4, group: int = GROUP):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        norms = np.ascontiguousarray(norms, dtype=np.uint16)
        return cls(lib().cq_qmat_from_cq(_p(packed), _p(norms), out, in_dim, bits, group))

    @classmethod
    def build(cls, out: int, in_dim: int, bits: int, cb: np.ndarray, codes, norms, ternary: bool = False):
        cb = np.ascontiguousarray(cb, dtype=np.float32)
        codes = np.ascontiguousarray(codes, dtype=np.uint8)
        norms = np.ascontiguousarray(norms, dtype=np.uint16)
        return cls(lib().cq_qmat_build(out, in_dim, bits, _p(cb), cb.size, int(ternary), _p(codes), _p(norms)))

    @property
    def out(self):
        return self.ptr.contents.out

    @property
    def in_dim(self):
        return self.ptr.contents.in_dim

    @property
    def groups(self):
        return self.ptr.contents.groups

    @property
    def bits(self):
        return self.ptr.contents.bits

    @property
    def cbs(self) -> np.float32:
        return np.float32(self.ptr.contents.cbs)

    @property
    def vals(self) -> np.ndarray:
        return np.array(list(self.ptr.contents.vals), dtype=np.int8)

    @property
    def codes(self) -> np.ndarray:
        c = self.ptr.contents
        return np.ctypeslib.as_array(c.codes, shape=(c.out, c.groups * GROUP * c.bits // 8)).copy()

    @property
    def norms(self) -> np.ndarray:
        c = self.ptr.contents
        return np.ctypeslib.as_array(c.norms, shape=(c.out, c.groups)).copy()

    def bytes(self) -> int:
        return lib().cq_qmat_bytes(self.ptr)

    def row(self, r: int) -> np.ndarray:
        out = np.zeros(self.in_dim, dtype=np.float32)
        lib().cq_qmat_row(self.ptr, r, _p(out))
        return out

    def lane_sums(self, r: int, g: int, a: OQAct, t: int) -> np.ndarray:
        s = np.zeros(4, dtype=np.int32)
        lib().cq_lane_sums(self.ptr, r, g, a.ptr, t, _p(s))
        return s

    def all_lane_sums(self, a: OQAct, t: int = 0, threads: int | None = None) -> np.ndarray:
        """int32 [out, groups, 4] decode lanes for token t."""
        out = np.zeros((self.out, self.groups, 4), dtype=np.int32)
        lib().cq_all_lane_sums(self.ptr, a.ptr, t, _p(out), threads or default_threads())
        return out

    def all_totals(self, a: OQAct, threads: int | None = None) -> np.ndarray:
        """int32 [rows, out, groups] prefill group totals."""
        out = np.zeros((a.rows, self.out, self.groups), dtype=np.int32)
        lib().cq_all_totals(self.ptr, a.ptr, _p(out), threads or default_threads())
        return out

    def matmul_rows(self, a: OQAct, r0: int, r1: int, block: np.ndarray | None = None,
                    threads: int | None = None) -> np.ndarray:
        """Columns [r0, r1) of matmul (or of the flagged prefill): [rows, r1 - r0]."""
        y = np.zeros((a.rows, r1 - r0), dtype=np.float32)
        bp = None
        if block is not None:
            block = np.ascontiguousarray(block, dtype=np.uint8)
            bp = _p(block)
        # col0 = -r0 places row r at column r - r0 of a width-(r1 - r0) buffer.
        base = y.ctypes.data - r0 * 4
        lib().cq_matmul_rows(self.ptr, a.ptr, bp, C.c_void_p(base), r1 - r0, 0, r0, r1, threads or default_threads())
        return y

    def decode_row_ref(self, r: int, a: OQAct) -> np.float32:
        return np.float32(lib().cq_decode_row_ref(self.ptr, r, a.ptr))

    def prefill_row_ref(self, r: int, a: OQAct, t: int, block: bool) -> np.float32:
        return np.float32(lib().cq_prefill_row_ref(self.ptr, r, a.ptr, t, int(block)))

    def single_row(self, r: int, a: OQAct) -> np.float32:
        return np.float32(lib().cq_single_row(self.ptr, r, a.ptr))

    def matmul(self, a: OQAct, threads: int | None = None) -> np.ndarray:
        y = np.zeros((a.rows, self.out), dtype=np.float32)
        lib().cq_matmul_into(self.ptr, a.ptr, _p(y), self.out, 0, threads or default_threads())
        return y

    def matmul_into(self, a: OQAct, y: np.ndarray, ldy: int, col0: int, threads: int | None = None):
        lib().cq_matmul_into(self.ptr, a.ptr, _p(y), ldy, col0, threads or default_threads())

    def prefill_flags(self, a: OQAct, block: np.ndarray, threads: int | None = None) -> np.ndarray:
        block = np.ascontiguousarray(block, dtype=np.uint8)
        y = np.zeros((a.rows, self.out), dtype=np.float32)
        lib().cq_prefill_rows_flags(self.ptr, a.ptr, _p(block), _p(y), self.out, 0, threads or default_threads())
        return y

    def head_logits_sparse(self, a: OQAct, ids: np.ndarray, out_rows: int) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros(out_rows, dtype=np.float32)
        lib().cq_head_logits_sparse(self.ptr, a.ptr, _p(ids), ids.size, out_rows, _p(out))
        return out

    def __del__(self):
        if getattr(self, "ptr", None) and _lib is not None:
            _lib.cq_qmat_free(self.ptr)
            self.ptr = None


class OQLinear:
    """QLinear (crates/needle-engine/src/qlinear.rs:493-574)."""

    def __init__(self, parts):
        arr = (C.POINTER(QMat) * len(parts))(*[p.ptr for p in parts])
        self.ptr = lib().cq_qlinear_new(C.cast(arr, C.c_void_p), len(parts))

    @property
    def out(self):
        return self.ptr.contents.out

    @property
    def nparts(self):
        return self.ptr.contents.nparts

    def matmul(self, a: OQAct, threads: int | None = None) -> np.ndarray:
        y = np.zeros((a.rows, self.out), dtype=np.float32)
        lib().cq_qlinear_matmul(self.ptr, a.ptr, _p(y), threads or default_threads())
        return y

    def __del__(self):
        if getattr(self, "ptr", None) and _lib is not None:
            _lib.cq_qlinear_free(self.ptr)
            self.ptr = None


# ------------------------------------------------------------------- norms
def dot16(x, y) -> np.float32:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    return np.float32(lib().cq_dot16(_p(x), _p(y), x.size))


def rinv(ss: float, n: int) -> np.float32:
    return np.float32(lib().cq_rinv(ss, n))


def zcn16(x, s_f16) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    s = np.ascontiguousarray(s_f16, dtype=np.uint16)
    out = np.zeros_like(x)
    lib().cq_zcn16(_p(x), _p(s), x.size, _p(out))
    return out


def argmax(x) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().cq_argmax(_p(x), x.size)


# ------------------------------------------------------------------ rand.rs
def threefry2x32(key, x):
    k = np.array(key, dtype=np.uint32)
    xx = np.array(x, dtype=np.uint32)
    out = np.zeros(2, dtype=np.uint32)
    lib().cq_threefry2x32(_p(k), _p(xx), _p(out))
    return [int(out[0]), int(out[1])]


def prng_key(seed: int):
    out = np.zeros(2, dtype=np.uint32)
    lib().cq_prng_key(seed, _p(out))
    return [int(out[0]), int(out[1])]


def split(key):
    k = np.array(key, dtype=np.uint32)
    a = np.zeros(2, dtype=np.uint32)
    b = np.zeros(2, dtype=np.uint32)
    lib().cq_split(_p(k), _p(a), _p(b))
    return [int(a[0]), int(a[1])], [int(b[0]), int(b[1])]


def normal(key, n: int, threads: int | None = None) -> np.ndarray:
    k = np.array(key, dtype=np.uint32)
    out = np.zeros(n, dtype=np.float32)
    lib().cq_normal(_p(k), n, _p(out), threads or default_threads())
    return out


def seed_sequence_u64(seed: int, n: int):
    out = np.zeros(n, dtype=np.uint64)
    lib().cq_seed_sequence_u64(seed, n, _p(out))
    return [int(v) for v in out]


class NpRng:
    """numpy Generator(PCG64(seed)) (crates/needle-train/src/rand.rs:68-130)."""

    def __init__(self, seed: int):
        self.ptr = lib().cq_nprng_new(seed)

    def next_u64(self) -> int:
        return lib().cq_nprng_next_u64(self.ptr)

    def next_u32(self) -> int:
        return lib().cq_nprng_next_u32(self.ptr)

    def interval(self, mx: int) -> int:
        return lib().cq_nprng_interval(self.ptr, mx)

    def permutation(self, n: int):
        out = np.zeros(n, dtype=np.uint64)
        lib().cq_nprng_permutation(self.ptr, n, _p(out))
        return [int(v) for v in out]

    def __del__(self):
        if getattr(self, "ptr", None) and _lib is not None:
            _lib.cq_nprng_free(self.ptr)
            self.ptr = None


# ------------------------------------------------------- seeded workloads
def seeded_normals(sizes, seed: int = 0, threads: int | None = None):
    """The workload recipe: key = prng_key(seed); per tensor in order,
    (key, sub) = split(key) and normal(sub, n)."""
    key = prng_key(seed)
    outs = []
    for n in sizes:
        key, sub = split(key)
        outs.append(normal(sub, n, threads))
    return outs


def random_tokens(n: int, vocab: int, seed: int = 0):
    r = NpRng(seed)
    return np.array([r.interval(vocab - 1) for _ in range(n)], dtype=np.uint32)
