"""Pins of the oracle's per-depth cells (Model::forward_cells and a tracking
session, crates/needle-engine/src/model.rs:60-62,108-123,330-345;
infer/step.rs:240-243,672-714; infer/chunk.rs:69-70,310,353-356;
infer.rs:1096-1130), by what the model's structure fixes:

- depth k of a row is the lane mean after k layers: a model cut to its first
  k layers (the same tensors, stacked records sliced) gives bit-identical
  cells at depths 0..k, and its final normed hidden state (the output path,
  not the cell code) is the zero-centred RMSNorm of that depth's cell, in
  float64 within 1e-5;
- depth 0 is the mean of the four equal embedding lanes: within an ulp of
  row * sqrt(d);
- the cells do not depend on the Outputs mode;
- a tracking session's store is the concatenation of its feeds' cells;
  rollback and rewind_zeroed truncate it to the session's length; a prefill
  appends nothing (prefill_native runs with want_cells = false) and its
  re-feed truncates it; a clone carries it;
- tracking starts at an empty session only.

And the attention span with a ring shorter than a chunk (model.rs:62-66):
feeds that fit the ring are taken, stepwise logits depend exactly on the
positions p < sink or p >= n - ring, and a longer feed is refused.
"""
import numpy as np
import pytest

import oracle as o
from oracle import cact, forward

F = np.float32


def bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


GEO = dict(vocab=300, num_layers=3, engram_slots=64, engram_sites=(1,), global_layers=(1,), sliding_window=8)


def tensors(g, seed):
    return cact.needle3_tensors(g, seed=seed, kind=lambda n: ("cq", 4) if n == "embedding" else ("random", 4))[0]


def _rows16(t, rows):
    """The first `rows` rows of a stacked f16 record."""
    w = int(np.prod(t.shape[1:])) if len(t.shape) > 1 else 1
    return cact.Tensor(t.dtype, [rows] + list(t.shape[1:]), t.blob[:rows * w * 2])


def _rows_cq(t, rows):
    """The first `rows` rows of a CQ record: packed rows, then f16 norms."""
    out, in_dim = t.shape
    groups = -(-in_dim // 128)
    rb = groups * 128 * (2 if t.bits == 5 else t.bits) // 8
    packed, norms = t.blob[:out * rb], t.blob[out * rb:]
    return cact.Tensor(t.dtype, [rows, in_dim], packed[:rows * rb] + norms[:rows * groups * 2], t.group, t.bits)


def truncated(g, ts, k):
    """The archive of the first k layers of (g, ts): per-layer blocks kept,
    the stacked mHC records sliced to k layers, sites past k dropped."""
    per_layer = 27 if g.qkv_conv_taps > 0 else 24
    n = g.mhc_lanes
    L = g.num_layers
    head = ts[:1 + k * per_layer]
    i = 1 + L * per_layer
    stacked = [_rows16(t, k) for t in ts[i:i + 6]]  # a_pre, a_post, a_res, b_pre, b_post, b_res
    i += 6
    phi = [_rows_cq(ts[i], k * n), _rows_cq(ts[i + 1], k * n), _rows_cq(ts[i + 2], k * n * n)]
    i += 3
    perms = ts[i:i + 2]
    i += 2
    sites = []
    keep = []
    for s, layer in enumerate(g.engram_sites):
        if layer < k:
            sites.append(layer)
            keep += ts[i + 4 * s:i + 4 * s + 4]
    i += 4 * len(g.engram_sites)
    final = ts[i:]
    gk = cact.Geometry(**{**GEO, "num_layers": k, "engram_sites": tuple(sites),
                          "global_layers": tuple(x for x in g.global_layers if x < k)})
    return cact.pack(head + stacked + phi + perms + keep + final, gk.header())


def zcn64(x, s):
    """zc_rms_norm in float64: x / sqrt(mean(x^2) + 1e-6) * (1 + s)."""
    x = x.astype(np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x) + 1e-6)
    return x * r * (1.0 + s.astype(np.float64))


def final_norm(ts):
    return np.frombuffer(ts[-1].blob, dtype=np.float16).astype(np.float32) if ts[-1].dtype == cact.F16 else \
        np.frombuffer(ts[-1].blob, dtype=np.float32)


def test_cells_depth_is_the_lane_mean_after_k_layers():
    g = cact.Geometry(**GEO)
    ts = tensors(g, seed=91)
    full = forward.Forward(cact.pack(ts, g.header()))
    toks = o.random_tokens(37, 300, seed=92)  # a chunk of 32 and one of 5
    _, cells = full.session(64).forward_cells(toks)
    assert cells.shape == (37, g.num_layers + 1, g.d_model)
    fn = final_norm(ts)
    for k in range(1, g.num_layers + 1):
        part = forward.Forward(truncated(g, ts, k))
        hid, ck = part.session(64).forward_cells(toks, forward.OUT_HIDDEN)
        assert np.array_equal(bits(ck), bits(cells[:, :k + 1])), k
        for i in (0, 5, 31, 32, 36):
            want = zcn64(ck[i, k], fn)
            err = np.abs(hid[i].astype(np.float64) - want).max() / np.abs(want).max()
            assert err < 1e-5, (k, i, err)
    # the stepwise path records the same depths
    s = full.session(64)
    for t in toks[:3]:
        _, c1 = s.forward_cells([int(t)], forward.OUT_LAST_HIDDEN)
        assert c1.shape == (1, g.num_layers + 1, g.d_model)


def test_cells_depth0_is_the_embedding_row():
    g = cact.Geometry(**GEO)
    ts = tensors(g, seed=93)
    f = forward.Forward(cact.pack(ts, g.header()))
    a = cact.Archive(cact.pack(ts, g.header()))
    packed, norms, out, in_dim, _ = a.cq(0)
    emb = o.OQMat.from_cq(packed, norms, out, in_dim)
    toks = o.random_tokens(9, 300, seed=94)
    _, cells = f.session(16).forward_cells(toks)
    scale = F(np.sqrt(F(g.d_model)))
    for i, t in enumerate(toks):
        e = (emb.row(int(t)) * scale).astype(F)
        c = cells[i, 0]
        assert np.all(np.abs(c - e) <= np.spacing(np.abs(e))), i


def test_cells_do_not_depend_on_outputs():
    f = forward.Forward(cact.pack(tensors(cact.Geometry(**GEO), 95), cact.Geometry(**GEO).header()))
    toks = o.random_tokens(40, 300, seed=96)
    ref = None
    for mode in (forward.OUT_NONE, forward.OUT_LAST_LOGITS, forward.OUT_ALL_LOGITS, forward.OUT_HIDDEN,
                 forward.OUT_LAST_HIDDEN):
        out, cells = f.session(64).forward_cells(toks, mode)
        plain = f.session(64).forward(toks, mode)
        assert np.array_equal(bits(out), bits(plain)), mode
        if ref is None:
            ref = cells
        assert np.array_equal(bits(cells), bits(ref)), mode


def test_cells_tracking_store():
    g = cact.Geometry(**GEO)
    f = forward.Forward(cact.pack(tensors(g, 97), g.header()))
    toks = o.random_tokens(90, 300, seed=98)
    s = f.session(128)
    s.track_cells()
    assert s.cells().shape == (0, g.num_layers + 1, g.d_model)
    parts = []
    parts.append(f.session(128).forward_cells(toks[:40])[1])  # the same feeds on an untracked session ...
    s.forward(toks[:40])
    assert np.array_equal(bits(s.cells()), bits(parts[0]))
    s2 = f.session(128)
    s2.forward(toks[:40])
    for t in toks[40:44]:
        parts.append(s2.forward_cells([int(t)])[1])
        s.forward([int(t)])
    want = np.concatenate(parts)
    assert np.array_equal(bits(s.cells()), bits(want))
    # rollback and rewind truncate
    s.rollback(3)
    assert np.array_equal(bits(s.cells()), bits(want[:41]))
    c = s.clone()
    s.rewind_zeroed(30)
    assert np.array_equal(bits(s.cells()), bits(want[:30]))
    assert np.array_equal(bits(c.cells()), bits(want[:41]))
    # forward_cells on a tracking session appends what it returns
    _, fc = c.forward_cells(toks[44:50])
    assert np.array_equal(bits(c.cells()[41:]), bits(fc))
    # a prefill appends nothing
    n = len(c.cells())
    c.prefill(toks[50:55])
    assert len(c.cells()) == n and len(c) == n + 5
    with pytest.raises(ValueError):
        c.track_cells()  # not at an empty session
    c.track_cells(False)
    with pytest.raises(ValueError):
        c.cells()


def test_cells_prefill_refeed_truncates():
    g = cact.Geometry(**GEO)
    f = forward.Forward(cact.pack(tensors(g, 99), g.header()))
    toks = o.random_tokens(80, 300, seed=100)
    s = f.session(128)
    s.set_attend(4, 32)
    s.track_cells()
    for t in toks[:45]:
        s.forward([int(t)])
    # positions 36..44 took the slots of 4..12 (ring 32 past a sink of 4);
    # rolled back to 25, they leave positions 4..12 stale
    s.rollback(20)
    assert len(s.cells()) == 25
    # a prefill whose keys reach position 4 re-feeds from it, with the
    # cells cut there and none appended
    s.prefill(toks[45:55])
    assert len(s) == 35
    assert len(s.cells()) == 4


def test_short_ring_receptive_field():
    f = forward.Forward(cact.pack(tensors(cact.Geometry(vocab=300, num_layers=1, qkv_conv_taps=1, engram_sites=(),
                                                        global_layers=(0,), sliding_window=0, engram_slots=64),
                                          21),
                                  cact.Geometry(vocab=300, num_layers=1, qkv_conv_taps=1, engram_sites=(),
                                                global_layers=(0,), sliding_window=0, engram_slots=64).header()))
    sink, ring, n = 3, 8, 30
    toks = o.random_tokens(n, 300, seed=101)

    def last(tt):
        s = f.session(64)
        s.set_attend(sink, ring)
        s.forward(tt[:5])  # one feed that fits the ring
        for t in tt[5:-1]:
            s.forward([int(t)], forward.OUT_NONE)
        return s.forward([int(tt[-1])])

    base = last(toks)
    seen = []
    for p in range(n):
        alt = toks.copy()
        alt[p] = (int(toks[p]) + 1) % 300
        if not np.array_equal(bits(last(alt)), bits(base)):
            seen.append(p)
    assert seen == [p for p in range(n) if p < sink or p >= n - ring]
    s = f.session(64)
    s.set_attend(sink, ring)
    with pytest.raises(ValueError):
        s.forward(toks[:9])  # a chunk longer than the ring
    assert len(s) == 0
    s.forward(toks[:8])
    assert len(s) == 8
