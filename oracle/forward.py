"""The Needle-3 decode step on the CPU (oracle/forward.c), loaded from a
.cact archive the way Weights::from_archive_mode(fast = true) reads one
(crates/needle-engine/src/weights.rs:314-467) plus the native tables
(Tables::new, crates/needle-engine/src/infer.rs:935-960: Phi8 of the
dequantized mHC rows, the small weights in f16).

TEST INFRASTRUCTURE: only tests/ (and a CPU baseline) may use it.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import OQLinear, OQMat, _p, default_threads, f16_to_f32, lib
from .cact import CQ, F16, F32, Archive, hada_blocks

P = C.c_void_p

# Outputs (crates/needle-engine/src/model.rs:150-160)
OUT_NONE, OUT_LAST_LOGITS, OUT_ALL_LOGITS, OUT_HIDDEN, OUT_LAST_HIDDEN = range(5)

(KRON0, KRON1, KRON2, KRON3, KRON4, KRON5, COND_V, COND_U, D1, D2, B2, D3, D4, NORM_IN, POST_NORM, PRE_HADA, Q_TAPS,
 K_TAPS, V_TAPS, Q_NORM, K_NORM) = range(21)


class Config(C.Structure):
    """nf_config (oracle/forward.h)."""
    _fields_ = [("d", C.c_int), ("nh", C.c_int), ("nkv", C.c_int), ("qk", C.c_int), ("vd", C.c_int),
                ("layers", C.c_int), ("lanes", C.c_int), ("taps", C.c_int), ("out_rows", C.c_int),
                ("sliding_window", C.c_int), ("global_mask", C.c_uint64), ("sites", C.c_int),
                ("site_layers", C.c_int * 16), ("norders", C.c_int), ("orders", C.c_int * 4), ("eheads", C.c_int),
                ("seed_heads", C.c_int), ("engram_slots", C.c_int), ("engram_sub", C.c_int),
                ("dilation", C.c_int), ("rope_theta", C.c_float)]


_declared = False


def _lib():
    global _declared
    l = lib()
    if not _declared:
        sig = {
            "nf_model_new": (P, [P]),
            "nf_model_free": (None, [P]),
            "nf_set_layer_f16": (None, [P, C.c_int, C.c_int, P, C.c_size_t]),
            "nf_set_layer_scalars": (None, [P, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float, P, P, P]),
            "nf_set_phi": (None, [P, C.c_int, P, C.c_size_t, C.c_size_t]),
            "nf_set_matrices": (None, [P, P, P, P, P, P]),
            "nf_set_engram_taps": (None, [P, C.c_int, P, C.c_size_t]),
            "nf_set_globals": (None, [P, P, P, P]),
            "nf_session_new": (P, [P, C.c_size_t]),
            "nf_session_free": (None, [P, P]),
            "nf_session_len": (C.c_size_t, [P]),
            "nf_step": (C.c_int, [P, P, C.c_uint32, P, C.c_int]),
            "nf_chunk": (C.c_int, [P, P, P, C.c_size_t, P, C.c_int]),
            "nf_nexp": (C.c_float, [C.c_float]),
            "nf_rope_rotate": (None, [P, C.c_size_t, P, P]),
            "nf_cond_weights": (None, [P, C.c_size_t, P, P]),
            "nf_mix8": (None, [C.c_int, P, C.c_int, P, C.c_int, P, C.c_int]),
            "nf_sinkhorn64": (None, [P, P]),
            "nf_chunk_exp": (C.c_float, [P, C.c_size_t, C.c_float]),
            "nf_digits21": (None, [P, C.c_size_t, C.c_float, P, P, P]),
            "nf_key_chunks": (None, [C.c_size_t, C.c_size_t, P, P]),
            "nf_session_clone": (P, [P, P]),
            "nf_session_set_attend": (C.c_int, [P, C.c_size_t, C.c_size_t]),
            "nf_session_rollback": (C.c_int, [P, P, C.c_size_t]),
            "nf_session_rewind_zeroed": (C.c_int, [P, P, C.c_size_t]),
            "nf_session_last_hidden": (C.c_int, [P, P, P]),
            "nf_forward": (C.c_int, [P, P, P, C.c_size_t, C.c_int, P, C.c_int]),
            "nf_prefill": (C.c_int, [P, P, P, C.c_size_t, C.c_int, P, C.c_int]),
            "nf_forward_cells": (C.c_int, [P, P, P, C.c_size_t, C.c_int, P, P, C.c_int]),
            "nf_conv_taps": (None, [P, C.c_int, P, C.c_int, P]),
            "nf_engram_conv": (None, [P, P, C.c_int, C.c_size_t, P]),
            "nf_engram_gate": (C.c_float, [P, P, C.c_int]),
            "nf_hada_mlp": (None, [P, C.c_int, P, P]),
            "nf_rope_rows": (None, [P, C.c_size_t, C.c_size_t, P, P, P, P]),
            "nf_rope_tables": (None, [P, P, P, P]),
            "nf_session_rope": (C.c_int, [P, C.c_size_t, P, P, C.c_int]),
            "nf_session_kv": (C.c_int, [P, P, C.c_int, C.c_size_t, P, P, P, P]),
            "nf_session_engram_hist": (C.c_int, [P, P, C.c_int, C.c_size_t, P, P]),
            "nf_session_track_cells": (C.c_int, [P, P, C.c_int]),
            "nf_session_cells": (C.c_int, [P, P, C.c_size_t, C.c_size_t, P]),
            "nf_head_logits": (None, [P, P, P, C.c_int]),
            "nf_head_logits_sparse": (C.c_int, [P, P, P, C.c_size_t, P]),
            "nf_attend_test": (C.c_int, [P, P, P, P, P, P, C.c_size_t, P, C.c_int, P]),
            "nf_engram_rows": (None, [P, P, C.c_size_t, P]),
            "nf_engram_input": (None, [P, C.c_int, P, C.c_size_t, P]),
            "nf_mhc_read": (None, [P, P, C.c_int, C.c_int, C.c_float, P, C.c_int, P, P, P, P, P]),
            "nf_post_gates": (None, [P, C.c_float, P, C.c_float, P, C.c_int, P, P]),
            "nf_mhc_write": (None, [C.c_int, P, P, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _declared = True
    return l


def _f16(a: Archive, i: int) -> np.ndarray:
    r = a.records[i]
    if r.dtype != F16:
        raise ValueError(f"tensor {i} is not f16")
    return np.frombuffer(a.bytes(i), dtype=np.uint16).copy()


def _f32(a: Archive, i: int) -> np.ndarray:
    r = a.records[i]
    if r.dtype == F16:
        return f16_to_f32(_f16(a, i))
    if r.dtype == F32:
        return np.frombuffer(a.bytes(i), dtype=np.float32).copy()
    raise ValueError(f"tensor {i} is neither f16 nor f32")


def _mat(a: Archive, i: int) -> OQMat:
    """Cursor::big (weights.rs:113-128): CQ records as stored, others packed."""
    r = a.records[i]
    if r.dtype == CQ:
        packed, norms, out, in_dim, bits = a.cq(i)
        return OQMat.from_cq(packed, norms, out, in_dim, bits)
    w = _f32(a, i)
    return OQMat.from_f32(w[:r.shape[0] * r.shape[1]], r.shape[0], r.shape[1])


class Forward:
    """A Needle-3 model on the oracle's decode step (step_native)."""

    def __init__(self, data: bytes, threads: int | None = None):
        l = _lib()
        a = Archive(data)
        h = a.header
        self.threads = threads or default_threads()
        orders = list(h.engram_orders)
        eheads = h.num_engram_tables // len(orders) if orders else 0
        cfg = Config()
        cfg.d, cfg.nh, cfg.nkv = h.d_model, h.num_heads, h.num_kv_heads
        cfg.qk, cfg.vd, cfg.layers, cfg.lanes, cfg.taps = h.qk_head_dim, h.v_head_dim, h.num_layers, h.mhc_lanes, \
            h.qkv_conv_taps
        cfg.out_rows = h.out_vocab if h.out_vocab > 0 else h.vocab
        cfg.sliding_window, cfg.global_mask = h.sliding_window, h.global_mask
        cfg.sites = len(h.engram_sites)
        for i, s in enumerate(h.engram_sites):
            cfg.site_layers[i] = s
        cfg.norders = len(orders)
        for i, o in enumerate(orders):
            cfg.orders[i] = o
        cfg.eheads, cfg.seed_heads = eheads, h.engram_seed_heads
        cfg.engram_slots, cfg.engram_sub = h.engram_slots, h.engram_sub_dim
        cfg.dilation = max(orders) if orders else 1
        cfg.rope_theta = h.rope_theta
        self.cfg = cfg
        self.vocab = h.vocab
        m = l.nf_model_new(C.byref(cfg))
        self.m = m
        keep = []  # the oracle matrices the model points at

        # The canonical order (weights.rs:318-420).
        i = 0

        def take():
            nonlocal i
            i += 1
            return i - 1

        emb = _mat(a, take())
        keep.append(emb)
        qkvg, outs, scal = [], [], []
        for layer in range(h.num_layers):
            def f16(which, idx=None):
                t = _f16(a, take() if idx is None else idx)
                l.nf_set_layer_f16(m, layer, which, _p(t), t.size)

            f16(NORM_IN)
            q, k, v = _mat(a, take()), _mat(a, take()), _mat(a, take())
            if h.qkv_conv_taps > 0:
                f16(Q_TAPS)
                f16(K_TAPS)
                f16(V_TAPS)
            f16(Q_NORM)
            f16(K_NORM)
            g, o = _mat(a, take()), _mat(a, take())
            keep += [q, k, v, g, o]
            qkvg.append(OQLinear([q, k, v, g]))
            outs.append(OQLinear([o]))
            f16(POST_NORM)
            attn_gate = float(_f32(a, take())[0])
            f16(PRE_HADA)
            for which in (D1, D2, B2, D3, D4):
                f16(which)
            for which in (KRON0, KRON1, KRON2, KRON3, KRON4, KRON5):
                f16(which)
            f16(COND_V)
            f16(COND_U)
            scal.append(attn_gate)
        a_pre, a_post, a_res = _f32(a, take()), _f32(a, take()), _f32(a, take())
        b_pre, b_post, b_res = _f32(a, take()), _f32(a, take()), _f32(a, take())
        phi_pre, phi_post, phi_res = _mat(a, take()), _mat(a, take()), _mat(a, take())
        n = h.mhc_lanes
        nc = n * h.d_model
        for layer in range(h.num_layers):
            bp = np.ascontiguousarray(b_pre[layer * n:(layer + 1) * n], dtype=np.float32)
            bq = np.ascontiguousarray(b_post[layer * n:(layer + 1) * n], dtype=np.float32)
            br = np.ascontiguousarray(b_res[layer * n * n:(layer + 1) * n * n], dtype=np.float32)
            l.nf_set_layer_scalars(m, layer, float(a_pre[layer]), float(a_post[layer]), float(a_res[layer]),
                                   scal[layer], _p(bp), _p(bq), _p(br))
            # QLinear::new(pre | post | res slices).dequantize() (weights.rs:380-389,492)
            rows = [phi_pre.row(r) for r in range(layer * n, (layer + 1) * n)]
            rows += [phi_post.row(r) for r in range(layer * n, (layer + 1) * n)]
            rows += [phi_res.row(r) for r in range(layer * n * n, (layer + 1) * n * n)]
            w = np.ascontiguousarray(np.stack(rows), dtype=np.float32)
            l.nf_set_phi(m, layer, _p(w), w.shape[0], nc)
        perm1 = _f32(a, take()).astype(np.int32)
        perm2 = _f32(a, take()).astype(np.int32)
        hn = 1
        while hn < h.d_model:
            hn *= 2
        if perm1.size != hn or perm2.size != hn or hada_blocks(hn) != (32, 32):
            raise ValueError("the decode step covers the shipped geometry (hada_n 1024)")
        etables, ekv = [], []
        for s in range(len(h.engram_sites)):
            t, kk, vv = _mat(a, take()), _mat(a, take()), _mat(a, take())
            keep += [t, kk, vv]
            etables.append(t)
            ekv.append(OQLinear([kk, vv]))
            taps = np.ascontiguousarray(_f32(a, take()), dtype=np.float32)
            l.nf_set_engram_taps(m, s, _p(taps), taps.size)
        final_norm = np.ascontiguousarray(_f32(a, take()), dtype=np.float32)
        l.nf_set_globals(m, _p(final_norm), _p(perm1), _p(perm2))
        self.final_norm, self.perm1, self.perm2 = final_norm, perm1, perm2

        def arr(objs):
            return (C.c_void_p * max(1, len(objs)))(*[C.cast(x.ptr, C.c_void_p).value for x in objs])

        self._arrs = (arr(qkvg), arr(outs), arr(etables), arr(ekv))
        l.nf_set_matrices(m, C.cast(emb.ptr, C.c_void_p), *[C.cast(x, C.c_void_p) for x in self._arrs])
        self._keep = (keep, qkvg, outs, etables, ekv, emb)

    # -- the helpers the step is built from, for their own checks
    def set_layer_f16(self, layer: int, which: int, values):
        """Replace a small per-layer tensor (values in f32, stored as f16)."""
        from . import f32_to_f16
        v = np.ascontiguousarray(f32_to_f16(np.asarray(values, dtype=np.float32).reshape(-1)), dtype=np.uint16)
        _lib().nf_set_layer_f16(self.m, int(layer), int(which), _p(v), v.size)

    def set_perms(self, perm1, perm2):
        """Replace the Hadamard MLP's permutations."""
        self.perm1 = np.ascontiguousarray(perm1, dtype=np.int32)
        self.perm2 = np.ascontiguousarray(perm2, dtype=np.int32)
        _lib().nf_set_globals(self.m, _p(self.final_norm), _p(self.perm1), _p(self.perm2))

    @staticmethod
    def conv_taps(rows, w) -> np.ndarray:
        """nf_conv_taps: rows[j] the pre-tap row of pos - j (None: not held), w [taps][cw] f16 bits."""
        w = np.ascontiguousarray(w, dtype=np.uint16)
        taps, cw = w.shape
        keep = [None if r is None else np.ascontiguousarray(r, dtype=np.float32) for r in rows]
        ptrs = (C.c_void_p * taps)(*[None if r is None else r.ctypes.data for r in keep])
        out = np.zeros(cw, dtype=np.float32)
        _lib().nf_conv_taps(ptrs, taps, _p(w), cw, _p(out))
        return out

    def engram_gate(self, x, k) -> float:
        x = np.ascontiguousarray(x, dtype=np.float32)
        k = np.ascontiguousarray(k, dtype=np.float32)
        return float(_lib().nf_engram_gate(_p(x), _p(k), x.size))

    def hada_mlp(self, layer: int, h2) -> np.ndarray:
        h2 = np.ascontiguousarray(h2, dtype=np.float32)
        out = np.zeros(self.cfg.d, dtype=np.float32)
        _lib().nf_hada_mlp(self.m, int(layer), _p(h2), _p(out))
        return out

    def rope_tables(self):
        half = self.cfg.qk // 2
        fr, sd, cd = (np.zeros(half, dtype=np.float32) for _ in range(3))
        _lib().nf_rope_tables(self.m, _p(fr), _p(sd), _p(cd))
        return fr, sd, cd

    def rope_rows(self, p0: int, t: int, prev=None):
        """nf_rope_rows: (cos, sin) [t][qk/2]; prev = (cos, sin) of position p0 - 1 for the recurrence."""
        half = self.cfg.qk // 2
        cs, sn = np.zeros((t, 32), np.float32), np.zeros((t, 32), np.float32)
        c0 = s0 = None
        if prev is not None:
            c0 = np.zeros(32, np.float32)
            s0 = np.zeros(32, np.float32)
            c0[:half], s0[:half] = prev
        _lib().nf_rope_rows(self.m, int(p0), int(t), None if c0 is None else _p(c0), None if s0 is None else _p(s0),
                            _p(cs), _p(sn))
        return cs[:, :half], sn[:, :half]

    def session(self, cap: int = 256) -> "Session":
        return Session(self, cap)

    def head_logits(self, h) -> np.ndarray:
        """Model::head_logits (infer.rs:1135-1141)."""
        h = np.ascontiguousarray(h, dtype=np.float32)
        out = np.zeros(self.cfg.out_rows, dtype=np.float32)
        _lib().nf_head_logits(self.m, _p(h), _p(out), self.threads)
        return out

    def head_logits_sparse(self, h, ids) -> np.ndarray:
        """Model::head_logits_sparse (infer.rs:1145-1166)."""
        h = np.ascontiguousarray(h, dtype=np.float32)
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32).reshape(-1))
        out = np.zeros(self.cfg.out_rows, dtype=np.float32)
        if _lib().nf_head_logits_sparse(self.m, _p(h), _p(ids), ids.size, _p(out)) != 0:
            raise ValueError("id past out_rows")
        return out

    def __del__(self):
        if getattr(self, "m", None) and lib is not None:
            _lib().nf_model_free(self.m)
            self.m = None


class Session:
    """The decoding state of one sequence (Session with NatState,
    crates/needle-engine/src/model.rs:53-121, infer.rs:966-1071)."""

    def __init__(self, f: Forward, cap: int, handle=None):
        self.f = f
        self.s = handle if handle is not None else _lib().nf_session_new(f.m, cap)
        self.cap = cap

    def step(self, tok: int) -> np.ndarray:
        """step_native for one token: the logits [out_rows]."""
        out = np.zeros(self.f.cfg.out_rows, dtype=np.float32)
        rc = _lib().nf_step(self.f.m, self.s, int(tok), _p(out), self.f.threads)
        if rc != 0:
            raise ValueError("step outside the session's capacity or geometry")
        return out

    def chunk(self, toks) -> np.ndarray:
        """One chunk of <= 32 tokens (chunk_job, infer/chunk.rs:32-358; one
        token is a step): the last row's logits."""
        t = np.ascontiguousarray(np.asarray(toks, dtype=np.uint32).reshape(-1))
        out = np.zeros(self.f.cfg.out_rows, dtype=np.float32)
        rc = _lib().nf_chunk(self.f.m, self.s, _p(t), t.size, _p(out), self.f.threads)
        if rc != 0:
            raise ValueError("chunk outside the session's capacity or geometry")
        return out

    def _width(self, outputs):
        return self.f.cfg.d if outputs in (OUT_HIDDEN, OUT_LAST_HIDDEN) else self.f.cfg.out_rows

    def _run(self, fn, toks, outputs):
        t = np.ascontiguousarray(np.asarray(toks, dtype=np.uint32).reshape(-1))
        # a prefill's re-feed returns rows for the positions it feeds again
        # too (infer.rs:1090-1100): up to the session's length more
        rows_max = t.size + (len(self) if fn is _lib().nf_prefill else 0) \
            if outputs in (OUT_ALL_LOGITS, OUT_HIDDEN) else 1
        out = np.zeros((max(rows_max, 1), self._width(outputs)), dtype=np.float32)
        r = fn(self.f.m, self.s, _p(t), t.size, int(outputs), _p(out), self.f.threads)
        assert r <= out.shape[0], "the oracle wrote past its output rows"
        if r < 0:
            raise ValueError("feed outside the session's capacity, geometry or key runs")
        return out[:r]

    def forward(self, toks, outputs: int = OUT_LAST_LOGITS) -> np.ndarray:
        """Model::forward on the native path (forward_native,
        infer.rs:1105-1132): the rows `outputs` selects, [rows][width]."""
        return self._run(_lib().nf_forward, toks, outputs)

    def prefill(self, toks, outputs: int = OUT_LAST_LOGITS) -> np.ndarray:
        """Model::prefill on the native path (prefill_native, infer.rs:1078-1101)."""
        return self._run(_lib().nf_prefill, toks, outputs)

    def forward_cells(self, toks, outputs: int = OUT_NONE):
        """Model::forward_cells (model.rs:330-345): (the rows `outputs`
        selects, the feed's cells [t][L+1][d])."""
        t = np.ascontiguousarray(np.asarray(toks, dtype=np.uint32).reshape(-1))
        rows_max = t.size if outputs in (OUT_ALL_LOGITS, OUT_HIDDEN) else 1
        out = np.zeros((max(rows_max, 1), self._width(outputs)), dtype=np.float32)
        cells = np.zeros((t.size, self.f.cfg.layers + 1, self.f.cfg.d), dtype=np.float32)
        r = _lib().nf_forward_cells(self.f.m, self.s, _p(t), t.size, int(outputs), _p(out), _p(cells),
                                    self.f.threads)
        if r < 0:
            raise ValueError("feed outside the session's capacity, geometry or key runs")
        return out[:r], cells

    def track_cells(self, on: bool = True):
        """Session::cells = Some(vec![]) (on, at an empty session) or None."""
        if _lib().nf_session_track_cells(self.f.m, self.s, int(bool(on))) != 0:
            raise ValueError("cell tracking starts at an empty session")

    def cells(self) -> np.ndarray:
        """Session::cells: the tracked rows [rows][L+1][d]."""
        l = _lib()
        n = l.nf_session_cells(self.f.m, self.s, 0, 0, None)
        if n < 0:
            raise ValueError("the session does not track cells")
        out = np.zeros((n, self.f.cfg.layers + 1, self.f.cfg.d), dtype=np.float32)
        if n and l.nf_session_cells(self.f.m, self.s, 0, n, _p(out)) < 0:
            raise ValueError("the session does not track cells")
        return out

    def feed(self, toks) -> np.ndarray:
        """Model::forward with Outputs::LastLogits: the last row's logits."""
        return self.forward(toks, OUT_LAST_LOGITS)[0]

    def set_attend(self, sink: int, ring: int):
        """Session::attend = Some((sink, ring)) (ring 0: None)."""
        if _lib().nf_session_set_attend(self.s, int(sink), int(ring)) != 0:
            raise ValueError("bad attention span")

    def rollback(self, n: int):
        if _lib().nf_session_rollback(self.f.m, self.s, int(n)) != 0:
            raise ValueError("rollback past ROLLBACK or the length")

    def rewind_zeroed(self, length: int):
        _lib().nf_session_rewind_zeroed(self.f.m, self.s, int(length))

    def clone(self) -> "Session":
        return Session(self.f, self.cap, handle=_lib().nf_session_clone(self.f.m, self.s))

    def last_hidden(self) -> np.ndarray:
        out = np.zeros(self.f.cfg.d, dtype=np.float32)
        if _lib().nf_session_last_hidden(self.f.m, self.s, _p(out)) != 0:
            raise ValueError("no hidden state yet")
        return out

    def attend_test(self, k8, ks, v8, vs, q, nested=False) -> np.ndarray:
        """attend_head over keys written into layer 0's slots 0..n-1 (kv head 0)."""
        k8 = np.ascontiguousarray(k8, dtype=np.int8)
        v8 = np.ascontiguousarray(v8, dtype=np.int8)
        ks = np.ascontiguousarray(ks, dtype=np.float32)
        vs = np.ascontiguousarray(vs, dtype=np.float32)
        q = np.ascontiguousarray(q, dtype=np.float32)
        out = np.zeros(self.f.cfg.vd, dtype=np.float32)
        if _lib().nf_attend_test(self.f.m, self.s, _p(k8), _p(ks), _p(v8), _p(vs), ks.size, _p(q), int(nested),
                                 _p(out)) != 0:
            raise ValueError("bad key count")
        return out

    def rope(self, pos: int):
        """The RoPE row (cos, sin) [qk/2] the session computed for a position."""
        half = self.f.cfg.qk // 2
        c, s = np.zeros(half, np.float32), np.zeros(half, np.float32)
        if _lib().nf_session_rope(self.s, int(pos), _p(c), _p(s), half) != 0:
            raise ValueError("position not fed")
        return c, s

    def kv(self, layer: int, slot: int):
        """A KV slot: (k8 [nkv][qk], ks [nkv], v8 [nkv][vd], vs [nkv])."""
        c = self.f.cfg
        k8 = np.zeros((c.nkv, c.qk), np.int8)
        v8 = np.zeros((c.nkv, c.vd), np.int8)
        ks, vs = np.zeros(c.nkv, np.float32), np.zeros(c.nkv, np.float32)
        if _lib().nf_session_kv(self.f.m, self.s, int(layer), int(slot), _p(k8), _p(ks), _p(v8), _p(vs)) != 0:
            raise ValueError("slot out of range")
        return k8, ks, v8, vs

    def engram_hist(self, site: int, pos: int):
        """The int8 engram value history of a site at a position: (v8 [d], vs [d / 32])."""
        d = self.f.cfg.d
        v8, vs = np.zeros(d, np.int8), np.zeros(d // 32, np.float32)
        if _lib().nf_session_engram_hist(self.f.m, self.s, int(site), int(pos), _p(v8), _p(vs)) != 0:
            raise ValueError("position not fed")
        return v8, vs

    def engram_conv(self, site: int, pos: int) -> np.ndarray:
        out = np.zeros(self.f.cfg.d, np.float32)
        _lib().nf_engram_conv(self.f.m, self.s, int(site), int(pos), _p(out))
        return out

    def __len__(self):
        return _lib().nf_session_len(self.s)

    def __del__(self):
        # At interpreter exit the model may be finalized first; its session
        # memory then goes with the process.
        if getattr(self, "s", None) and lib is not None and getattr(self.f, "m", None):
            _lib().nf_session_free(self.f.m, self.s)
        self.s = None
