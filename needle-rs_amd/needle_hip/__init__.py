"""Host-side mirror of needle-rs's packed CQ runtime over the MI355X C ABI.

The classes follow crates/needle-engine/src/qlinear.rs (QMat, QAct,
QLinear) method by method; every call goes through
``libneedle_hip.so`` (include/needle_hip.h), whose gfx950 kernels do the
work.  Device buffers are torch tensors on ``cuda:0`` (plumbing only).
There is no CPU fallback: without a built library or a gfx950 device every
entry point raises ``NeedleHipError``.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import torch  # loaded first so the library binds to torch's HIP runtime

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libneedle_hip.so")
GROUP = 128
NEG = np.frombuffer(np.uint32(0xF149F2CA).tobytes(), dtype=np.float32)[0]

# Outputs (crates/needle-engine/src/model.rs:150-160)
OUT_NONE, OUT_LAST_LOGITS, OUT_ALL_LOGITS, OUT_HIDDEN, OUT_LAST_HIDDEN = range(5)

# Every exported symbol of include/needle_hip.h, with (restype, argtypes).
P = C.c_void_p
I = C.c_int
SIGNATURES = {
    "nh_init": (I, [I]),
    "nh_last_error": (C.c_char_p, []),
    "nh_version": (I, []),
    "nh_qmat_from_cq": (I, [P, C.c_uint64, P, C.c_uint64, I, I, I, I, P]),
    "nh_qmat_from_f32": (I, [P, I, I, P]),
    "nh_qlinear_new": (I, [P, I, P]),
    "nh_qmat_slice_rows": (I, [P, I, I, P]),
    "nh_qmat_free": (I, [P]),
    "nh_qmat_shape": (I, [P, P, P, P]),
    "nh_qmat_bytes": (C.c_int64, [P]),
    "nh_qmat_download": (I, [P, P, C.c_uint64, P, C.c_uint64]),
    "nh_qmat_rows": (I, [P, P, I, P, P]),
    "nh_qact_new": (I, [I, I, I, P]),
    "nh_qact_free": (I, [P]),
    "nh_act_prep": (I, [P, P, I, I, P, P]),
    "nh_qact_rows": (I, [P]),
    "nh_qact_download": (I, [P, P, C.c_uint64, P, C.c_uint64]),
    "nh_matmul": (I, [P, P, P, I, I, P]),
    "nh_qlinear_apply": (I, [P, P, I, P, P]),
    "nh_qlinear_apply_static": (I, [P, P, I, P, P]),
    "nh_matmul_flags": (I, [P, P, P, P, I, I, P]),
    "nh_single_rows": (I, [P, P, P, I, P, P]),
    "nh_head_logits_sparse": (I, [P, P, P, I, I, P, P]),
    "nh_debug_partials": (I, [P, P, P, P]),
    "nh_weights_load": (I, [P, C.c_uint64, P]),
    "nh_weights_free": (I, [P]),
    "nh_weights_header": (I, [P, P, I]),
    "nh_weights_count": (I, [P, I]),
    "nh_weights_get": (I, [P, I, I, P]),
    "nh_weights_bytes": (C.c_int64, [P]),
    "nh_codebook": (I, [I, P]),
    "nh_model_load": (I, [P, C.c_uint64, P]),
    "nh_model_free": (I, [P]),
    "nh_model_weights": (I, [P, P]),
    "nh_model_out_rows": (I, [P]),
    "nh_session_new": (I, [P, I, P]),
    "nh_session_free": (I, [P]),
    "nh_session_len": (I, [P]),
    "nh_session_reset": (I, [P]),
    "nh_forward": (I, [P, P, I, P, P]),
    "nh_forward_outputs": (I, [P, P, I, I, P, C.c_int64, P]),
    "nh_forward_cells": (I, [P, P, I, I, P, C.c_int64, P, C.c_int64, P]),
    "nh_debug_read_floor": (I, [P, P, I, P, P]),
    "nh_session_track_cells": (I, [P, I]),
    "nh_session_cell_rows": (I, [P]),
    "nh_session_cells": (I, [P, I, I, P, P]),
    "nh_session_debug_fail_feed": (I, [P, I]),
    "nh_prefill": (I, [P, P, I, I, P, C.c_int64, P]),
    "nh_session_clone": (I, [P, P, P]),
    "nh_session_set_attend": (I, [P, I, I]),
    "nh_session_rollback": (I, [P, I]),
    "nh_session_debug_spin_limit": (I, [P, I]),
    "nh_session_sync": (I, [P, P]),
    "nh_session_rewind_zeroed": (I, [P, I]),
    "nh_session_last_hidden": (I, [P, P, P]),
    "nh_session_head_logits": (I, [P, P, P]),
    "nh_session_head_logits_sparse": (I, [P, P, I, P, P]),
    "nh_generate_greedy": (I, [P, I, P, P, P]),
    "nh_argmax": (I, [P, I, P, P]),
    "nh_normal": (I, [C.c_uint32, C.c_uint32, C.c_uint64, P]),
    "nh_split": (I, [C.c_uint32, C.c_uint32, P]),
}


class NeedleHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"needle_hip error {code}: {msg}")
        self.code = code


_lib = None
_ready = False


def load_library():
    """dlopen libneedle_hip.so (no device work)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NeedleHipError(-3, f"{LIB_PATH} is not built (run __graft_entry__.build())")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _check(rc: int) -> int:
    if rc < 0:
        raise NeedleHipError(rc, _lib.nh_last_error().decode(errors="replace"))
    return rc


def init(device: int = 0):
    """Select the gfx950 device (nh_init)."""
    global _ready
    lib = load_library()
    if not _ready:
        if not torch.cuda.is_available():
            raise NeedleHipError(-3, "no HIP device visible")
        torch.cuda.set_device(device)
        _check(lib.nh_init(device))
        _ready = True
    return lib


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _dptr(t: torch.Tensor):
    assert t.is_cuda and t.is_contiguous()
    return C.c_void_p(t.data_ptr())


def _hptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


class QAct:
    """Rotated int8 activations in HBM (qlinear.rs:63-72, 166-208)."""

    def __init__(self, rows: int, in_dim: int, bits: int = 4):
        lib = init()
        h = C.c_void_p()
        _check(lib.nh_qact_new(rows, in_dim, bits, C.byref(h)))
        self.h = h
        self.cap = rows
        self.in_dim = in_dim
        self.bits = bits
        self.groups = (in_dim + GROUP - 1) // GROUP

    @classmethod
    def empty_rows(cls, rows: int, in_dim: int, bits: int = 4) -> "QAct":
        return cls(rows, in_dim, bits)

    @classmethod
    def new(cls, x: torch.Tensor, rows: int, in_dim: int, bits: int = 4, norm_scale: torch.Tensor | None = None,
            stream=None) -> "QAct":
        """QAct::new(x, rows, in_dim, bits); with ``norm_scale`` (f16 [in_dim])
        the zero-centred RMSNorm is fused in front (zcn16)."""
        a = cls(rows, in_dim, bits)
        a.prep(x, rows, norm_scale, stream)
        return a

    def prep(self, x: torch.Tensor, rows: int | None = None, norm_scale: torch.Tensor | None = None, stream=None):
        rows = rows if rows is not None else x.numel() // self.in_dim
        assert x.dtype == torch.float32 and x.numel() >= rows * self.in_dim
        ns = None
        if norm_scale is not None:
            assert norm_scale.dtype in (torch.float16, torch.int16, torch.uint16) and norm_scale.numel() == self.in_dim
            ns = _dptr(norm_scale)
        _check(_lib.nh_act_prep(self.h, _dptr(x), rows, self.in_dim, ns, _stream(stream)))
        return self

    @property
    def rows(self) -> int:
        return _check(_lib.nh_qact_rows(self.h))

    def download(self):
        """(xq int8 [rows, groups, 128] in act_pos order, sx f32 [rows, groups])."""
        rows = self.rows
        xq = np.zeros((rows, self.groups, GROUP), dtype=np.int8)
        sx = np.zeros((rows, self.groups), dtype=np.float32)
        _check(_lib.nh_qact_download(self.h, _hptr(xq), xq.nbytes, _hptr(sx), sx.size))
        return xq, sx

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.nh_qact_free(self.h)
            self.h = None


class QMat:
    """A CQ matrix (2- or 4-bit codes, or a ternary record) resident in HBM
    (qlinear.rs:43-61, 218-488)."""

    def __init__(self, h, owner=None):
        # A matrix owned by another handle (QWeights) keeps that handle
        # alive and is not freed here.
        self.h = h
        self._owner = owner
        out, ind, bits = C.c_int(), C.c_int(), C.c_int()
        _check(_lib.nh_qmat_shape(h, C.byref(out), C.byref(ind), C.byref(bits)))
        self.out, self.in_dim, self.bits = out.value, ind.value, bits.value
        self.groups = (self.in_dim + GROUP - 1) // GROUP

    @classmethod
    def from_cq(cls, packed: np.ndarray, norms: np.ndarray, out: int, in_dim: int, bits: int = 4,
                group: int = GROUP) -> "QMat":
        """QMat::from_cq over a CqView blob: packed u8 [out, row_bytes], norms f16 bits;
        bits 2, 4 or 5 (ternary)."""
        lib = init()
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        norms = np.ascontiguousarray(norms, dtype=np.uint16)
        h = C.c_void_p()
        _check(lib.nh_qmat_from_cq(_hptr(packed), packed.nbytes, _hptr(norms), norms.size, out, in_dim, bits, group,
                                   C.byref(h)))
        return cls(h)

    @classmethod
    def from_f32(cls, w: np.ndarray, out: int, in_dim: int) -> "QMat":
        """QMat::from_f32: cq_pack on the GPU, then upload."""
        lib = init()
        w = np.ascontiguousarray(w, dtype=np.float32)
        assert w.size == out * in_dim
        h = C.c_void_p()
        _check(lib.nh_qmat_from_f32(_hptr(w), out, in_dim, C.byref(h)))
        return cls(h)

    def bytes(self) -> int:
        return _check(_lib.nh_qmat_bytes(self.h))

    def slice_rows(self, r0: int, r1: int) -> "QMat":
        """QMat::slice_rows: rows r0..r1 as their own matrix."""
        h = C.c_void_p()
        _check(_lib.nh_qmat_slice_rows(self.h, r0, r1, C.byref(h)))
        return QMat(h)

    def act_bits(self) -> int:
        return self.bits

    def download(self):
        """(packed u8 [out, groups*128*bits/8], norms u16 [out, groups]) in archive layout."""
        packed = np.zeros((self.out, self.groups * GROUP * self.bits // 8), dtype=np.uint8)
        norms = np.zeros((self.out, self.groups), dtype=np.uint16)
        _check(_lib.nh_qmat_download(self.h, _hptr(packed), packed.nbytes, _hptr(norms), norms.size))
        return packed, norms

    def matmul_into(self, a: QAct, y: torch.Tensor, ldy: int, col0: int, stream=None):
        _check(_lib.nh_matmul(self.h, a.h, _dptr(y), ldy, col0, _stream(stream)))

    def matmul(self, a: QAct, stream=None) -> torch.Tensor:
        y = torch.empty((a.rows, self.out), dtype=torch.float32, device="cuda")
        self.matmul_into(a, y, self.out, 0, stream)
        return y

    def matmul_flags(self, a: QAct, block: torch.Tensor, stream=None) -> torch.Tensor:
        """The prefill combine with an explicit block flag per token."""
        y = torch.empty((a.rows, self.out), dtype=torch.float32, device="cuda")
        assert block.dtype == torch.uint8 and block.numel() >= a.rows
        _check(_lib.nh_matmul_flags(self.h, a.h, _dptr(block), _dptr(y), self.out, 0, _stream(stream)))
        return y

    def single_rows(self, ids: torch.Tensor, a: QAct, stream=None) -> torch.Tensor:
        assert ids.dtype == torch.int32 or ids.dtype == torch.uint32
        out = torch.empty(ids.numel(), dtype=torch.float32, device="cuda")
        _check(_lib.nh_single_rows(self.h, a.h, _dptr(ids), ids.numel(), _dptr(out), _stream(stream)))
        return out

    def single_row(self, r: int, a: QAct) -> float:
        ids = torch.tensor([r], dtype=torch.int32, device="cuda")
        return float(self.single_rows(ids, a).cpu()[0])

    def rows(self, ids: torch.Tensor, stream=None) -> torch.Tensor:
        out = torch.empty((ids.numel(), self.in_dim), dtype=torch.float32, device="cuda")
        _check(_lib.nh_qmat_rows(self.h, _dptr(ids), ids.numel(), _dptr(out), _stream(stream)))
        return out

    def row(self, r: int) -> torch.Tensor:
        return self.rows(torch.tensor([r], dtype=torch.int32, device="cuda"))[0]

    def read_floor(self, a: QAct, mode: int, y: torch.Tensor | None = None, stream=None):
        """Measurement: the decode product's loads with no arithmetic (mode 0, its grid), a plain
        stream of its code and norm bytes (mode 1), or mode 0 ending as the product does, with a
        workgroup barrier and one float stored per row to y (mode 2; y: float32, at least out)."""
        if mode == 2 and (y is None or y.dtype != torch.float32 or y.numel() < self.out or not y.is_cuda):
            raise ValueError("mode 2 stores one float32 per row to a device tensor y")
        _check(_lib.nh_debug_read_floor(self.h, a.h, int(mode), _dptr(y) if mode == 2 else None,
                                        _stream(stream)))

    def partials(self, a: QAct, stream=None) -> torch.Tensor:
        """int32 lanes [out, groups, 4] (one token) or totals [rows, out, groups]."""
        shape = (self.out, self.groups, 4) if a.rows == 1 else (a.rows, self.out, self.groups)
        out = torch.empty(shape, dtype=torch.int32, device="cuda")
        _check(_lib.nh_debug_partials(self.h, a.h, _dptr(out), _stream(stream)))
        return out

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None and getattr(self, "_owner", None) is None:
            _lib.nh_qmat_free(self.h)
        self.h = None


class QLinear:
    """Fused projections (qlinear.rs:493-574): parts concatenated by rows."""

    def __init__(self, parts):
        lib = init()
        arr = (C.c_void_p * len(parts))(*[p.h.value for p in parts])
        h = C.c_void_p()
        _check(lib.nh_qlinear_new(C.cast(arr, C.c_void_p), len(parts), C.byref(h)))
        self.fused = QMat(h)
        self.out = self.fused.out
        self.in_dim = self.fused.in_dim
        self.part_rows = [p.out for p in parts]

    def act_bits(self) -> int:
        return self.fused.bits

    def matmul(self, a: QAct, stream=None) -> torch.Tensor:
        return self.fused.matmul(a, stream)

    def rows_into(self, a: QAct, y: torch.Tensor, ldy: int, stream=None):
        self.fused.matmul_into(a, y, ldy, 0, stream)

    def apply(self, x: torch.Tensor, rows: int, stream=None) -> torch.Tensor:
        """QLinear::apply (qlinear.rs:555-557): A8 of x [rows][in_dim] and the
        products, in one call (nh_qlinear_apply)."""
        y = torch.empty((rows, self.out), dtype=torch.float32, device="cuda")
        _check(_lib.nh_qlinear_apply(self.fused.h, _dptr(x), int(rows), _dptr(y), _stream(stream)))
        return y

    def apply_static(self, x: torch.Tensor, rows: int, y: torch.Tensor, stream=None) -> torch.Tensor:
        """nh_qlinear_apply_static: QLinear::apply into a caller's y [rows][out]
        with no allocation (a per-GPU static staging; at most 64 rows)."""
        _check(_lib.nh_qlinear_apply_static(self.fused.h, _dptr(x), int(rows), _dptr(y), _stream(stream)))
        return y

    def bytes(self) -> int:
        return self.fused.bytes()


# Header words of a .cact archive (crates/needle-core/src/cact.rs:80-118).
HEADER_WORDS = ("tag", "num_tensors", "codebook_len", "kv_window", "kv_bits", "vocab", "out_vocab", "d_model",
                "num_heads", "num_kv_heads", "num_layers", "qk_head_dim", "v_head_dim", "max_seq_len", "hada_n",
                "mhc_lanes", "sliding_window", "global_mask_lo", "global_mask_hi", "qkv_conv_taps", "engram_slots",
                "engram_sub_dim", "num_engram_tables", "engram_conv_taps", "engram_conv_dilation",
                "engram_seed_heads", "num_engram_orders")
W_EMBEDDING, W_QKVG, W_OUT, W_PHI, W_ENGRAM_TABLE, W_ENGRAM_KV = range(6)


class QWeights:
    """QWeights (crates/needle-engine/src/weights.rs:136-148): every matmul
    weight of a .cact archive, packed in HBM, as
    Weights::from_archive_mode(fast = true) reads them (weights.rs:314-467).
    embedding; qkvg / out per layer (q|k|v|gate fused); phi per layer (mHC
    pre|post|res rows fused); engram_tables and engram_kv (key|value fused)
    per site."""

    def __init__(self, h, owner=None):
        self.h = h
        self._owner = owner  # a Model that owns these weights (not freed here)
        words = (C.c_uint32 * 49)()
        _check(_lib.nh_weights_header(h, C.cast(words, C.c_void_p), 49))
        self.header_words = list(words)
        self.header = dict(zip(HEADER_WORDS, self.header_words))
        self.header["rope_theta"] = float(np.frombuffer(np.uint32(words[48]).tobytes(), dtype=np.float32)[0])

        def kind(k):
            n = _lib.nh_weights_count(h, k)
            _check(n)
            out = []
            for i in range(n):
                m = C.c_void_p()
                _check(_lib.nh_weights_get(h, k, i, C.byref(m)))
                out.append(QMat(m, owner=self))
            return out

        self.embedding = kind(W_EMBEDDING)[0]
        self.qkvg = kind(W_QKVG)
        self.out = kind(W_OUT)
        self.phi = kind(W_PHI)
        self.engram_tables = kind(W_ENGRAM_TABLE)
        self.engram_kv = kind(W_ENGRAM_KV)

    @classmethod
    def from_archive(cls, data) -> "QWeights":
        """Read the archive bytes (bytes or a u8 array); they are borrowed for
        the call only."""
        lib = init()
        buf = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray)) else \
            np.ascontiguousarray(data, dtype=np.uint8)
        h = C.c_void_p()
        _check(lib.nh_weights_load(_hptr(buf), buf.nbytes, C.byref(h)))
        return cls(h)

    def bytes(self) -> int:
        """QWeights::bytes (weights.rs:151-155)."""
        n = _lib.nh_weights_bytes(self.h)
        _check(int(n) if n < 0 else 0)
        return int(n)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None and getattr(self, "_owner", None) is None:
            _lib.nh_weights_free(self.h)
        self.h = None


class Model:
    """Model::quantized with the native tables (crates/needle-engine/src/model.rs:248-262,
    crates/needle-engine/src/infer.rs:869-960) for the decode step, in HBM."""

    def __init__(self, h):
        self.h = h
        self.out_rows = _check(_lib.nh_model_out_rows(h))
        w = C.c_void_p()
        _check(_lib.nh_model_weights(h, C.byref(w)))
        words = np.zeros(49, dtype=np.uint32)
        _check(_lib.nh_weights_header(w.value, _hptr(words), 49))
        self.d_model = int(words[7])  # the header's d_model word (cact.rs:80-118)
        self.layers = int(words[10])  # num_layers

    @property
    def weights(self) -> "QWeights":
        """The model's matmul weights (they keep the model alive)."""
        w = C.c_void_p()
        _check(_lib.nh_model_weights(self.h, C.byref(w)))
        return QWeights(w.value, owner=self)

    @classmethod
    def from_archive(cls, data) -> "Model":
        """nh_model_load over archive bytes, borrowed for the call only."""
        lib = init()
        buf = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray)) else \
            np.ascontiguousarray(data, dtype=np.uint8)
        h = C.c_void_p()
        _check(lib.nh_model_load(_hptr(buf), buf.nbytes, C.byref(h)))
        return cls(h.value)

    def session(self, cap: int = 4096) -> "Session":
        """Model::session (model.rs:264-280) with room for `cap` positions."""
        return Session(self, cap)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.nh_model_free(self.h)
        self.h = None


class Session:
    """Session (crates/needle-engine/src/model.rs:55-121): one sequence's
    decoding state (KV caches, tap and engram histories) in HBM."""

    def __init__(self, model: Model, cap: int, handle=None):
        self.model = model
        if handle is None:
            h = C.c_void_p()
            _check(_lib.nh_session_new(model.h, int(cap), C.byref(h)))
            handle = h.value
        self.h = handle
        self.cap = cap

    def __len__(self):
        return _check(_lib.nh_session_len(self.h))

    def reset(self):
        _check(_lib.nh_session_reset(self.h))

    def _width(self, outputs):
        return self.model.d_model if outputs in (OUT_HIDDEN, OUT_LAST_HIDDEN) else self.model.out_rows

    def _feed(self, fn, tokens, outputs, stream):
        toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))
        # a prefill may re-feed up to the session's length before the tokens
        rows = (toks.size + (len(self) if fn is _lib.nh_prefill else 0)) if outputs in (OUT_ALL_LOGITS, OUT_HIDDEN) \
            else (1 if outputs != OUT_NONE else 0)
        width = self._width(outputs)
        out = torch.empty(max(rows, 1) * width, dtype=torch.float32, device="cuda")
        r = _check(fn(self.h, _hptr(toks), toks.size, int(outputs), _dptr(out), out.numel(), _stream(stream)))
        return out[:r * width].view(r, width)

    def forward(self, tokens, outputs: int | None = None, stream=None) -> torch.Tensor:
        """Model::forward (model.rs:304-306) as forward_native feeds it
        (infer.rs:1105-1132): chunks of 32 tokens (chunk_job), a single token
        as a step.  Without `outputs`: the last token's logits [out_rows];
        with an Outputs mode: the rows it returns, [rows][width] (device)."""
        if outputs is None:
            toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))
            logits = torch.empty(self.model.out_rows, dtype=torch.float32, device="cuda")
            _check(_lib.nh_forward(self.h, _hptr(toks), toks.size, _dptr(logits), _stream(stream)))
            return logits
        return self._feed(_lib.nh_forward_outputs, tokens, outputs, stream)

    def forward_cells(self, tokens, outputs: int = OUT_NONE, stream=None):
        """Model::forward_cells (model.rs:330-345): (the rows `outputs` selects,
        [rows][width], the feed's cells [n][L+1][d]), both on the device."""
        toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))
        rows = toks.size if outputs in (OUT_ALL_LOGITS, OUT_HIDDEN) else (1 if outputs != OUT_NONE else 0)
        width = self._width(outputs)
        out = torch.empty(max(rows, 1) * width, dtype=torch.float32, device="cuda")
        cw = (self.model.layers + 1) * self.model.d_model
        cells = torch.empty(max(toks.size, 1) * cw, dtype=torch.float32, device="cuda")
        r = _check(_lib.nh_forward_cells(self.h, _hptr(toks), toks.size, int(outputs), _dptr(out), out.numel(),
                                         _dptr(cells), cells.numel(), _stream(stream)))
        return out[:r * width].view(r, width), cells[:toks.size * cw].view(toks.size, self.model.layers + 1,
                                                                            self.model.d_model)

    def track_cells(self, on: bool = True):
        """Session::cells = Some(vec![]) (on, at an empty session) or None (model.rs:60-62)."""
        _check(_lib.nh_session_track_cells(self.h, int(bool(on))))

    def cells(self, stream=None) -> torch.Tensor:
        """Session::cells: the tracked rows [rows][L+1][d] (device)."""
        n = _check(_lib.nh_session_cell_rows(self.h))
        cw = (self.model.layers + 1) * self.model.d_model
        out = torch.empty(max(n, 1) * cw, dtype=torch.float32, device="cuda")
        _check(_lib.nh_session_cells(self.h, 0, n, _dptr(out), _stream(stream)))
        return out[:n * cw].view(n, self.model.layers + 1, self.model.d_model)

    def debug_fail_feed(self, after: int):
        """Test hook: the `after`-th feed from now fails before it launches (0: off)."""
        _check(_lib.nh_session_debug_fail_feed(self.h, int(after)))

    def prefill(self, tokens, outputs: int = OUT_LAST_LOGITS, stream=None) -> torch.Tensor:
        """Model::prefill on the native path (prefill_native, infer.rs:1078-1101)."""
        return self._feed(_lib.nh_prefill, tokens, outputs, stream)

    def clone(self, stream=None) -> "Session":
        """Session::clone (model.rs:53-55)."""
        h = C.c_void_p()
        _check(_lib.nh_session_clone(self.h, _stream(stream), C.byref(h)))
        return Session(self.model, self.cap, handle=h.value)

    def set_attend(self, sink: int, ring: int):
        """Session::attend = Some((sink, ring)) (model.rs:62-66); ring 0: None."""
        _check(_lib.nh_session_set_attend(self.h, int(sink), int(ring)))

    def debug_spin_limit(self, limit: int):
        """Test hook: the polls a bounded in-kernel wait makes before giving up."""
        _check(_lib.nh_session_debug_spin_limit(self.h, int(limit)))

    def sync(self, stream=None):
        """Wait for the session's queued work and report a bounded wait that gave
        up in its feeds (raises, and the session is reset); no reference
        counterpart (its calls are synchronous)."""
        _check(_lib.nh_session_sync(self.h, _stream(stream)))

    def rollback(self, n: int):
        """Session::rollback (model.rs:81-113)."""
        _check(_lib.nh_session_rollback(self.h, int(n)))

    def rewind_zeroed(self, length: int):
        """Session::rewind_zeroed (model.rs:115-121)."""
        _check(_lib.nh_session_rewind_zeroed(self.h, int(length)))

    def last_hidden(self, stream=None) -> torch.Tensor:
        """NatState::last_hidden (infer.rs:1014-1016)."""
        h = torch.empty(self.model.d_model, dtype=torch.float32, device="cuda")
        _check(_lib.nh_session_last_hidden(self.h, _dptr(h), _stream(stream)))
        return h

    def head_logits(self, stream=None) -> torch.Tensor:
        """Model::head_logits (infer.rs:1135-1141) of the last hidden state."""
        out = torch.empty(self.model.out_rows, dtype=torch.float32, device="cuda")
        _check(_lib.nh_session_head_logits(self.h, _dptr(out), _stream(stream)))
        return out

    def head_logits_sparse(self, ids: torch.Tensor, stream=None) -> torch.Tensor:
        """Model::head_logits_sparse (infer.rs:1145-1166) of the last hidden state."""
        out = torch.empty(self.model.out_rows, dtype=torch.float32, device="cuda")
        _check(_lib.nh_session_head_logits_sparse(self.h, _dptr(ids), ids.numel(), _dptr(out), _stream(stream)))
        return out

    def generate_greedy(self, steps: int, stream=None):
        """The greedy loop of generate (crates/needle-engine/src/generate.rs:87-139)
        on the device: (token ids [steps], the last step's logits)."""
        out = np.zeros(max(1, steps), dtype=np.uint32)
        logits = torch.empty(self.model.out_rows, dtype=torch.float32, device="cuda")
        _check(_lib.nh_generate_greedy(self.h, int(steps), _hptr(out), _dptr(logits), _stream(stream)))
        return out[:steps].copy(), logits

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.nh_session_free(self.h)
        self.h = None


def head_logits_sparse(embedding: QMat, a: QAct, ids: torch.Tensor, out_rows: int, stream=None) -> torch.Tensor:
    """Model::head_logits_sparse (crates/needle-engine/src/infer.rs:1145-1166)."""
    logits = torch.empty(out_rows, dtype=torch.float32, device="cuda")
    _check(_lib.nh_head_logits_sparse(embedding.h, a.h, _dptr(ids), ids.numel(), out_rows, _dptr(logits),
                                      _stream(stream)))
    return logits


def head_logits(embedding: QMat, h: torch.Tensor, out_rows: int) -> torch.Tensor:
    """Model::head_logits (crates/needle-engine/src/infer.rs:1135-1141)."""
    a = QAct.new(h, 1, h.numel(), embedding.act_bits())
    return embedding.matmul(a)[0, :out_rows]


def argmax(x: torch.Tensor, stream=None) -> int:
    """generate::argmax (crates/needle-engine/src/generate.rs:42-50) on the device."""
    dst = torch.zeros(1, dtype=torch.int32, device="cuda")
    _check(_lib.nh_argmax(_dptr(x), x.numel(), _dptr(dst), _stream(stream)))
    return int(dst.item())


def codebook(bits: int) -> np.ndarray:
    """quant::codebook(bits, 128) (crates/needle-core/src/quant.rs:52-68)."""
    out = np.zeros(16, dtype=np.float32)
    n = _check(load_library().nh_codebook(int(bits), _hptr(out)))
    return out[:n].copy()


# ------------------------------------------------------------- seeded inputs
def split(key):
    """jax.random.split (crates/needle-train/src/rand.rs:161-163)."""
    lib = load_library()
    out = np.zeros(4, dtype=np.uint32)
    _check(lib.nh_split(int(key[0]), int(key[1]), _hptr(out)))
    return [int(out[0]), int(out[1])], [int(out[2]), int(out[3])]


def normal(key, n: int) -> np.ndarray:
    """jax.random.normal float32 (crates/needle-train/src/rand.rs:205-217)."""
    lib = load_library()
    out = np.zeros(n, dtype=np.float32)
    _check(lib.nh_normal(int(key[0]), int(key[1]), n, _hptr(out)))
    return out


def seeded_normals(sizes, seed: int = 0):
    """key = prng_key(seed); per tensor: (key, sub) = split(key); normal(sub, n)."""
    key = [(seed >> 32) & 0xFFFFFFFF, seed & 0xFFFFFFFF]
    outs = []
    for n in sizes:
        key, sub = split(key)
        outs.append(normal(sub, n))
    return outs
