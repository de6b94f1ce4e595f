"""GPU: the session operations of the model boundary against the oracle doing
the same operations on the same archive (bit-identical at every step).

- Outputs (crates/needle-engine/src/model.rs:150-160): None, LastLogits,
  AllLogits, Hidden, LastHidden over prompts of several chunks;
- Session::rollback / rewind_zeroed / clone (model.rs:81-121,
  infer.rs:1039-1071), including a rollback across the history trim;
- Session::attend = (sink, ring) with the KV slot ring and the slot map
  (infer.rs:1749-1826), stale slots after a rollback and prefill_native's
  re-feed (infer.rs:1078-1101), stepwise and in chunks, a ring shorter than
  the sequence;
- the session heads: last_hidden, head_logits, head_logits_sparse
  (infer.rs:1135-1166, agent.rs:398-409);
- the conv tap counts 1, 2, 4, 6 (the exact and the clamped unit kernels),
  with a one-token prompt and a prompt past one chunk;
- a geometry with more taps than the kernels take is refused at load;
- a ring shorter than a chunk (feeds that fit it; a longer one refused);
- cells (Model::forward_cells and a tracking session, model.rs:60-62,
  108-123,330-345): fresh-session cells of a batched feed, steps and chunks
  in every Outputs mode, the tracked store across rollback, clone, rewind,
  prefill and the greedy loop;
- failure paths: a greedy step or a feed that fails part way (injected from
  the host) resets the session and keeps its span; a clone of a session
  whose failed wait is unreported is refused.
"""
import sys

import numpy as np
import pytest
import torch

import oracle as o
from oracle import cact, forward

pytestmark = pytest.mark.gpu

REL_TOL = 2e-3


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def archive(g, seed):
    ts, _ = cact.needle3_tensors(g, seed=seed, kind=lambda n: ("cq", 4) if n == "embedding" else ("random", 4))
    return cact.pack(ts, g.header())


def same(label, got, want, stats):
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    assert got.shape == want.shape, (label, got.shape, want.shape)
    stats["n"] = stats.get("n", 0) + 1
    if want.size == 0:
        stats["exact"] = stats.get("exact", 0) + 1
        return
    assert np.isfinite(got).all() and np.isfinite(want).all(), label
    scale = max(float(np.abs(want).max()), 1e-30)
    err = float(np.abs(got - want).max()) / scale
    stats["max_rel"] = max(stats.get("max_rel", 0.0), err)
    stats["exact"] = stats.get("exact", 0) + int(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
    assert err <= REL_TOL, (label, err)


class Pair:
    """A device session and an oracle session driven by the same script."""

    def __init__(self, nh, data, cap):
        self.f = forward.Forward(data)
        self.m = nh.Model.from_archive(data)
        self.g, self.o = self.m.session(cap), self.f.session(cap)
        self.stats = {}

    def fwd(self, toks, outputs=forward.OUT_LAST_LOGITS, label="forward"):
        got = self.g.forward(toks, outputs).cpu().numpy()
        same(label, got, self.o.forward(toks, outputs), self.stats)
        return got

    def prefill(self, toks, outputs=forward.OUT_LAST_LOGITS, label="prefill"):
        got = self.g.prefill(toks, outputs).cpu().numpy()
        same(label, got, self.o.prefill(toks, outputs), self.stats)
        return got

    def steps(self, toks, outputs=forward.OUT_LAST_LOGITS, label="step"):
        for i, t in enumerate(toks):
            self.fwd([int(t)], outputs, f"{label} {i}")

    def rollback(self, n):
        self.g.rollback(n)
        self.o.rollback(n)
        assert len(self.g) == len(self.o)

    def rewind_zeroed(self, n):
        self.g.rewind_zeroed(n)
        self.o.rewind_zeroed(n)
        assert len(self.g) == len(self.o)

    def attend(self, sink, ring):
        self.g.set_attend(sink, ring)
        self.o.set_attend(sink, ring)

    def clone(self):
        c = Pair.__new__(Pair)
        c.f, c.m, c.stats = self.f, self.m, self.stats
        c.g, c.o = self.g.clone(), self.o.clone()
        return c

    def heads(self, ids):
        h = self.o.last_hidden()
        same("last_hidden", self.g.last_hidden().cpu().numpy(), h, self.stats)
        same("head_logits", self.g.head_logits().cpu().numpy(), self.f.head_logits(h), self.stats)
        dev_ids = torch.from_numpy(np.asarray(ids, dtype=np.int32)).cuda()
        same("head_logits_sparse", self.g.head_logits_sparse(dev_ids).cpu().numpy(),
             self.f.head_logits_sparse(h, ids), self.stats)

    def done(self, label):
        say(f"{label}: {self.stats['exact']}/{self.stats['n']} bit-identical, "
            f"max rel {self.stats.get('max_rel', 0.0):.3g}")
        assert self.stats["exact"] == self.stats["n"], self.stats


SMALL = dict(vocab=300, num_layers=3, engram_slots=64, engram_sites=(1,), global_layers=(1,), sliding_window=8)


def test_outputs_modes(nh):
    say("Outputs modes over a 40-token prompt (32 + 8) and steps")
    data = archive(cact.Geometry(**SMALL), seed=51)
    toks = o.random_tokens(40, 300, seed=51)
    for mode in (forward.OUT_NONE, forward.OUT_LAST_LOGITS, forward.OUT_ALL_LOGITS, forward.OUT_HIDDEN,
                 forward.OUT_LAST_HIDDEN):
        p = Pair(nh, data, 64)
        got = p.fwd(toks, mode, f"mode {mode} prompt")
        rows = {forward.OUT_NONE: 0, forward.OUT_ALL_LOGITS: 40, forward.OUT_HIDDEN: 40}.get(mode, 1)
        assert got.shape[0] == rows
        p.steps(o.random_tokens(3, 300, seed=52), mode, f"mode {mode} step")
        if mode != forward.OUT_NONE:
            p.heads([0, 7, 150, 299])
        p.done(f"outputs mode {mode}")


def test_rollback_clone_rewind(nh):
    say("rollback (across the history trim), clone, rewind_zeroed")
    data = archive(cact.Geometry(**SMALL), seed=52)
    p = Pair(nh, data, 160)
    p.fwd(o.random_tokens(60, 300, seed=53))
    p.steps(o.random_tokens(25, 300, seed=54))
    p.rollback(25)
    p.steps(o.random_tokens(4, 300, seed=55), label="after rollback")
    p.rollback(3)
    p.rollback(1)
    c = p.clone()
    p.fwd(o.random_tokens(9, 300, seed=56), label="original")
    c.fwd(o.random_tokens(33, 300, seed=57), label="clone")
    c.steps(o.random_tokens(2, 300, seed=58), label="clone step")
    p.rewind_zeroed(50)
    p.fwd(o.random_tokens(40, 300, seed=59), label="after rewind")
    p.steps(o.random_tokens(2, 300, seed=60), label="after rewind step")
    p.heads([3, 4, 5])
    p.done("rollback / clone / rewind")
    with pytest.raises(nh.NeedleHipError, match="32"):
        p.g.rollback(33)


@pytest.mark.parametrize("stepwise", [True, False])
def test_attention_span(nh, stepwise):
    say(f"attention span (sink 6, ring 32), {'steps' if stepwise else 'chunks'}, with rollbacks and prefill")
    data = archive(cact.Geometry(**SMALL), seed=61)
    p = Pair(nh, data, 160)
    p.attend(6, 32)
    toks = o.random_tokens(70, 300, seed=62)
    if stepwise:
        p.steps(toks[:40])
    else:
        p.fwd(toks[:40])
    p.rollback(5)  # leaves stale slots
    p.steps(toks[40:43], label="after rollback")
    p.prefill(toks[43:50], label="prefill re-feed")
    p.rollback(2)
    p.prefill(toks[50:70], forward.OUT_ALL_LOGITS, label="prefill all rows")
    p.steps(o.random_tokens(3, 300, seed=63), label="tail")
    p.heads([1, 2, 3])
    p.done(f"attention span {'steps' if stepwise else 'chunks'}")
    q = Pair(nh, data, 64)
    q.attend(6, 16)  # a ring shorter than a chunk takes only feeds that fit it
    with pytest.raises(nh.NeedleHipError, match="longer than an attention ring"):
        q.g.forward(toks[:17])
    assert len(q.g) == 0


def test_attention_span_long(nh):
    say("attention span over 300 positions (sink 20, ring 256: two key chunks), chunks and steps")
    g = cact.Geometry(vocab=300, num_layers=2, engram_slots=64, engram_sites=(1,), global_layers=(0,),
                      sliding_window=64)
    p = Pair(nh, archive(g, seed=64), 320)
    p.attend(20, 256)
    p.fwd(o.random_tokens(290, 300, seed=65))
    p.steps(o.random_tokens(6, 300, seed=66))
    p.done("attention span long")


def test_attention_span_agent(nh):
    say("attention span as the agent sets it (sink 118, ring 256): a 118-token prefix, 300 more, then greedy steps "
        "past 418 positions (374 keys: four key chunks), every step against the oracle")
    g = cact.Geometry(vocab=300, num_layers=3, engram_slots=64, engram_sites=(1,), global_layers=(0, 2),
                      sliding_window=64)
    p = Pair(nh, archive(g, seed=67), 448)
    p.attend(118, 256)
    toks = o.random_tokens(418, 300, seed=68)
    p.prefill(toks[:118], forward.OUT_NONE, label="prefix")
    p.prefill(toks[118:418], label="fill")
    want = p.o.forward(o.random_tokens(1, 300, seed=69))[0]
    p.g.forward(o.random_tokens(1, 300, seed=69))
    picks, logits = p.g.generate_greedy(12)
    for i, k in enumerate(picks):
        assert int(k) == int(np.argmax(want)), i
        want = p.o.forward([int(k)])[0]
    same("greedy logits", logits.cpu().numpy(), want, p.stats)
    p.rollback(5)
    p.steps(o.random_tokens(8, 300, seed=70), label="after rollback")
    p.done("attention span (118, 256)")


@pytest.mark.parametrize("taps", [1, 2, 4, 6])
def test_conv_taps(nh, taps):
    say(f"qkv conv taps {taps}: a one-token prompt, steps, a 40-token prompt, steps")
    g = cact.Geometry(vocab=300, num_layers=3, engram_slots=64, engram_sites=(1,), global_layers=(1,),
                      sliding_window=8, qkv_conv_taps=taps)
    data = archive(g, seed=70 + taps)
    p = Pair(nh, data, 96)
    p.fwd(o.random_tokens(1, 300, seed=71))
    p.steps(o.random_tokens(5, 300, seed=72))
    p.fwd(o.random_tokens(40, 300, seed=73))
    p.steps(o.random_tokens(3, 300, seed=74))
    p.done(f"taps {taps}")


def test_too_many_taps_refused(nh):
    say("an archive with 9 conv taps is refused, naming the limit")
    g = cact.Geometry(vocab=300, num_layers=2, engram_slots=64, engram_sites=(1,), global_layers=(1,),
                      sliding_window=8, qkv_conv_taps=9)
    with pytest.raises(nh.NeedleHipError, match="at most 8"):
        nh.Model.from_archive(archive(g, seed=79))
    torch.cuda.synchronize()


def test_forward_empty(nh):
    say("forward of no tokens")
    data = archive(cact.Geometry(**SMALL), seed=80)
    m = nh.Model.from_archive(data)
    s = m.session(16)
    with pytest.raises(nh.NeedleHipError, match="no tokens"):
        s.forward([])
    a = s.forward([5, 6]).cpu().numpy()
    b = s.forward([]).cpu().numpy()  # the logits the session holds
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert s.forward([], forward.OUT_HIDDEN).shape[0] == 0


def test_bounded_wait_gives_up_and_reports(nh):
    say("the layer kernel's bounded wait: a spin limit of 0 forced from the host")
    data = archive(cact.Geometry(**SMALL), seed=81)
    m = nh.Model.from_archive(data)
    s = m.session(32)
    s.debug_spin_limit(0)  # every mixer wait gives up at once; the kernels still end
    s.forward([1, 2])  # layers 1 and 2 (and the head's input) run the wait
    torch.cuda.synchronize()  # the stream has passed the feed's status copy
    with pytest.raises(nh.NeedleHipError, match="gave up"):
        s.forward([3])  # reported by the first call after that
    assert len(s) == 0  # reset
    s.debug_spin_limit(1 << 20)
    got = s.forward([5, 6, 7]).cpu().numpy()
    want = forward.Forward(data).session(32).feed([5, 6, 7])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a clone of a session whose failed wait is not yet reported is refused,
    # and the source's next feed reports it
    s.debug_spin_limit(0)
    s.forward([8, 9])
    with pytest.raises(nh.NeedleHipError, match="not yet reported"):
        s.clone()
    s.debug_spin_limit(1 << 20)
    torch.cuda.synchronize()
    with pytest.raises(nh.NeedleHipError, match="gave up"):
        s.forward([3])
    assert len(s) == 0
    # an explicit sync attributes the failure to the feed that caused it
    s.sync()  # nothing pending: no error
    s.debug_spin_limit(0)
    s.forward([4, 5])
    with pytest.raises(nh.NeedleHipError, match="gave up"):
        s.sync()
    assert len(s) == 0
    s.debug_spin_limit(1 << 20)
    s.forward([5, 6, 7])
    s.sync()
    assert len(s) == 3


def test_failed_greedy_step_resets(nh):
    say("a greedy step that fails part way (injected from the host) resets the session, keeping its span; "
        "a prefill and steps then match a fresh oracle session")
    data = archive(cact.Geometry(**SMALL), seed=84)
    p = Pair(nh, data, 128)
    p.attend(6, 32)
    toks = o.random_tokens(60, 300, seed=85)
    p.fwd(toks[:40])
    p.g.debug_fail_feed(3)
    with pytest.raises(nh.NeedleHipError, match="on purpose"):
        p.g.generate_greedy(5)
    assert len(p.g) == 0
    p.o = p.f.session(128)
    p.o.set_attend(6, 32)
    p.prefill(toks[:40], label="prefill after the reset")
    p.steps(toks[40:50], label="step after the reset")  # past the ring: the span was kept
    p.g.debug_fail_feed(1)
    with pytest.raises(nh.NeedleHipError, match="on purpose"):
        p.g.forward(toks[50:53])
    assert len(p.g) == 0
    p.o = p.f.session(128)
    p.o.set_attend(6, 32)
    p.fwd(toks[:45], label="forward after the reset")
    p.done("failed feeds")


def test_short_ring(nh):
    say("attention span with a ring of 8 (sink 3): feeds that fit the ring, steps, rollbacks, prefill re-feed")
    data = archive(cact.Geometry(**SMALL), seed=86)
    p = Pair(nh, data, 96)
    p.attend(3, 8)
    toks = o.random_tokens(60, 300, seed=87)
    p.fwd(toks[:6])
    p.steps(toks[6:30])
    p.fwd(toks[30:38], forward.OUT_ALL_LOGITS, label="a feed of 8")
    p.rollback(4)
    p.steps(toks[38:41], label="after rollback")
    p.prefill(toks[41:44], label="prefill")
    p.steps(toks[44:50], label="tail")
    p.heads([1, 2, 3])
    with pytest.raises(nh.NeedleHipError, match="longer than an attention ring"):
        p.g.forward(toks[50:59])
    p.done("short ring")


def test_cells(nh):
    say("cells: forward_cells on a fresh session (a batched feed of 101 rows, Outputs None), steps and chunks "
        "with outputs, a tracking session across rollback, clone, rewind, prefill and the greedy loop")
    data = archive(cact.Geometry(**SMALL), seed=88)
    p = Pair(nh, data, 200)
    toks = o.random_tokens(140, 300, seed=89)
    go, gc = p.g.forward_cells(toks[:101])
    wo, wc = p.o.forward_cells(toks[:101])
    assert go.shape[0] == 0 and gc.shape == wc.shape
    same("cells of a batched feed", gc.cpu().numpy(), wc, p.stats)
    for i, t in enumerate(toks[101:104]):
        go, gc = p.g.forward_cells([int(t)], forward.OUT_LAST_LOGITS)
        wo, wc = p.o.forward_cells([int(t)], forward.OUT_LAST_LOGITS)
        same(f"step {i} logits", go.cpu().numpy(), wo, p.stats)
        same(f"step {i} cells", gc.cpu().numpy(), wc, p.stats)
    for mode in (forward.OUT_ALL_LOGITS, forward.OUT_HIDDEN, forward.OUT_LAST_HIDDEN):
        go, gc = p.g.forward_cells(toks[104:111], mode)
        wo, wc = p.o.forward_cells(toks[104:111], mode)
        same(f"chunk mode {mode}", go.cpu().numpy(), wo, p.stats)
        same(f"chunk mode {mode} cells", gc.cpu().numpy(), wc, p.stats)
        p.rollback(7)
    p.done("forward_cells")

    q = Pair(nh, data, 200)
    q.g.track_cells()
    q.o.track_cells()

    def cells(label, pair=None):
        pair = pair or q
        same(label, pair.g.cells().cpu().numpy(), pair.o.cells(), q.stats)

    q.fwd(toks[:70])  # one batched feed of 70 rows (chunks of 32, 32 and 6)
    q.steps(toks[70:75])
    cells("tracked after feeds")
    q.rollback(3)
    cells("tracked after rollback")
    c = q.clone()
    q.rewind_zeroed(50)
    cells("tracked after rewind")
    cells("clone", c)
    c.prefill(toks[75:80])  # appends nothing
    cells("clone after prefill", c)
    q.fwd(toks[80:84])
    want = q.o.forward(toks[84:86])[0]
    q.g.forward(toks[84:86])
    picks, _ = q.g.generate_greedy(4)
    for k in picks:
        assert int(k) == int(np.argmax(want))
        want = q.o.forward([int(k)])[0]
    cells("tracked after the greedy loop")
    q.done("tracked cells")


def test_greedy_picks_into_pinned_memory(nh):
    say("greedy picks into pinned host memory (C ABI), then a rollback and a prefill whose re-feed replays them")
    import ctypes

    data = archive(cact.Geometry(**SMALL), seed=82)
    p = Pair(nh, data, 96)
    p.attend(4, 32)
    want = p.fwd(o.random_tokens(40, 300, seed=83))
    steps = 12
    out = torch.zeros(steps, dtype=torch.int32, pin_memory=True)
    logits = torch.empty(p.m.out_rows, dtype=torch.float32, device="cuda")
    rc = nh._lib.nh_generate_greedy(p.g.h, steps, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(logits.data_ptr()),
                                    None)
    assert rc == 0, nh._lib.nh_last_error()
    picks = out.numpy().astype(np.uint32)
    for i, t in enumerate(picks):
        assert int(t) == int(np.argmax(want)), (i, int(t))
        want = p.o.forward([int(t)])
    same("greedy logits", logits.cpu().numpy(), np.asarray(want).reshape(-1), p.stats)
    assert len(p.g) == len(p.o) == 52
    # positions 47..51 held slots 15..19; after the rollback a 3-token prefill
    # (end 50) sees 18 and 19 as stale and re-feeds from 18 through the
    # greedy picks at 40..46
    p.rollback(5)
    p.prefill(o.random_tokens(3, 300, seed=84), label="prefill re-feed over greedy picks")
    p.steps(o.random_tokens(2, 300, seed=85), label="after re-feed")
    p.done("greedy picks into pinned memory")


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 5])
def test_random_session_scripts(nh, seed):
    """A seeded random script of feeds (every Outputs mode, lengths across the
    chunk and batch boundaries), prefills, single steps, rollbacks within the
    last feeds, clones, rewinds and, for some seeds, an attention span and
    tracked cells (compared after every rollback, clone and rewind and at the
    end); every result bit-identical to the oracle running the same script."""
    rng = np.random.default_rng(1000 + seed)
    geoms = [SMALL, dict(vocab=300, num_layers=2, engram_slots=64, engram_sites=(0,), global_layers=(0,),
                         sliding_window=48, qkv_conv_taps=4)]
    g = cact.Geometry(**geoms[seed % 2])
    data = archive(g, seed=90 + seed)
    cap = 260
    p = Pair(nh, data, cap)
    if seed in (1, 4):
        p.attend(int(rng.integers(2, 9)), int(rng.choice([32, 48, 64])))
    track = seed != 0
    if track:
        p.g.track_cells()
        p.o.track_cells()

    def check_cells(label):
        if track:
            same(f"cells {label}", p.g.cells().cpu().numpy(), p.o.cells(), p.stats)
    since = 0  # positions fed since the last rollback or rewind (what a rollback may drop)
    hidden = False
    say(f"random session script, seed {seed}")
    for op in range(40):
        kind = rng.choice(["feed", "prefill", "steps", "rollback", "clone", "rewind", "heads"],
                          p=[0.3, 0.15, 0.2, 0.15, 0.07, 0.05, 0.08])
        room = cap - len(p.g)
        if kind in ("feed", "prefill"):
            n = int(rng.choice([1, 2, 5, 31, 32, 33, 64, 70, 97]))
            if n > room:
                continue
            mode = int(rng.integers(0, 5))
            toks = rng.integers(0, 300, n).astype(np.uint32)
            (p.fwd if kind == "feed" else p.prefill)(toks, mode, f"{kind} {n} mode {mode} at op {op}")
            since += n
            hidden = hidden or mode != forward.OUT_NONE
        elif kind == "steps":
            n = int(rng.integers(1, 5))
            if n > room:
                continue
            p.steps(rng.integers(0, 300, n), forward.OUT_LAST_LOGITS, f"step at op {op}")
            since += n
            hidden = True
        elif kind == "rollback":
            n = int(min(since, rng.integers(1, 33)))
            if n < 1:
                continue
            p.rollback(n)
            since -= n
            check_cells(f"after rollback {n} at op {op}")
        elif kind == "clone":
            p = p.clone()
            check_cells(f"of a clone at op {op}")
        elif kind == "rewind":
            length = int(rng.integers(0, len(p.g) + 1))
            p.rewind_zeroed(length)
            since = 0
            check_cells(f"after rewind to {length} at op {op}")
        elif kind == "heads" and hidden:
            p.heads(rng.integers(0, 300, 5))
    check_cells("at the end")
    p.done(f"random session script {seed}")
