"""GPU: the Needle-3 decode step (nh_model_load / nh_session_* / nh_forward /
nh_generate_greedy) against the oracle's step_native (oracle/forward.c) on
the same archives and tokens.

Every float operation of the device step follows the reference's order, and
the libm functions are f64 ones rounded once as the reference computes them
off Apple targets (crates/needle-engine/src/infer.rs:84-101): the device
library's f64 exp against glibc's, both within an f64 ulp.  The logits must
therefore be bit-identical at every step; the only way two correct sides
could differ is an f32 rounding boundary falling between the two f64 exp
results (about 2^-29 of calls).  The statistics are printed per test, and a
relative-error bound is checked first so that a failure shows its size.

Covered: window and global layers (sliding_window small enough to slide),
engram sites (hash rows appear once a position reaches each order), the
multi-chunk attention merge (more than 256 keys), the tap history ring,
mixed code widths, the greedy loop, session reset and the error paths.
"""
import sys

import numpy as np
import pytest
import torch

import oracle as o
from oracle import cact, forward

pytestmark = pytest.mark.gpu

# Max |gpu - oracle| / max(|oracle|) per step.
REL_TOL = 2e-3


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def archive(g, seed, kind=lambda name: ("cq", 4) if name == "embedding" else ("random", 4)):
    ts, _ = cact.needle3_tensors(g, seed=seed, kind=kind)
    return cact.pack(ts, g.header())


def compare(label, got, want, stats):
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    assert got.shape == want.shape and np.isfinite(want).all(), label
    assert np.isfinite(got).all(), label
    scale = float(np.abs(want).max())
    err = float(np.abs(got - want).max()) / max(scale, 1e-30)
    stats["max_rel"] = max(stats.get("max_rel", 0.0), err)
    stats["steps"] = stats.get("steps", 0) + 1
    stats["exact"] = stats.get("exact", 0) + int(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
    assert err <= REL_TOL, (label, err)
    top = np.sort(want)[-2:]
    if top[1] - top[0] > 2 * REL_TOL * scale:
        assert int(np.argmax(got)) == int(np.argmax(want)), label


def run_pair(nh, data, tokens, cap, label):
    f = forward.Forward(data)
    m = nh.Model.from_archive(data)
    s, os_ = m.session(cap), f.session(cap)
    stats = {}
    want = None
    for i, t in enumerate(tokens):
        got = s.forward([int(t)]).cpu().numpy()
        want = os_.step(int(t))
        compare(f"{label} step {i}", got, want, stats)
    assert len(s) == len(tokens)
    say(f"{label}: {stats['steps']} steps, {stats['exact']} bit-identical, max rel {stats['max_rel']:.3g}")
    assert stats["exact"] == stats["steps"], stats
    return m, s, os_, want


SMALL = dict(vocab=300, num_layers=3, engram_slots=64, engram_sites=(1,), global_layers=(1,), sliding_window=8)


def test_decode_small_window_engram(nh):
    say("decode step: 3 layers (window 8, one global), one engram site, 40 tokens")
    g = cact.Geometry(**SMALL)
    data = archive(g, seed=11)
    run_pair(nh, data, o.random_tokens(40, g.vocab, seed=3), 64, "small")


def test_decode_two_sites_mixed_widths(nh):
    say("decode step: 4 layers, two engram sites, 2-bit / ternary / f16 records")
    g = cact.Geometry(vocab=300, num_layers=4, engram_slots=64, engram_sites=(0, 3), global_layers=(2,),
                      sliding_window=5)

    def kind(name):
        if name == "embedding":
            return ("cq", 4)
        if name.startswith("engram_table"):
            return ("random", 2)
        if name.startswith("phi"):
            return ("random", 5)
        if name == "out.1":
            return ("f16", 4)
        layer = int(name.split(".")[1]) if "." in name and name.split(".")[1].isdigit() else 0
        return ("random", 2 if layer == 2 else 4)

    data = archive(g, seed=12, kind=kind)
    run_pair(nh, data, o.random_tokens(24, g.vocab, seed=4), 32, "mixed")


def test_decode_long_context_chunks(nh):
    say("decode step: 2 layers (one global), 300 tokens (4 key chunks past 256)")
    g = cact.Geometry(vocab=300, num_layers=2, engram_slots=64, engram_sites=(1,), global_layers=(0,),
                      sliding_window=64)
    data = archive(g, seed=13)
    run_pair(nh, data, o.random_tokens(300, g.vocab, seed=5), 320, "long")


def test_greedy_loop(nh):
    say("greedy loop on the device against the oracle fed the same picks")
    g = cact.Geometry(**SMALL)
    data = archive(g, seed=14)
    prompt = o.random_tokens(10, g.vocab, seed=6)
    m, s, ref, last = run_pair(nh, data, prompt, 64, "prompt")
    picks, logits = s.generate_greedy(20)
    assert len(s) == 30 and picks.shape == (20,)
    # each pick is the argmax of the oracle's logits of the previous step,
    # the oracle fed the same picks
    for i, t in enumerate(picks):
        top = np.sort(last)[-2:]
        if top[1] - top[0] > 2 * REL_TOL * float(np.abs(last).max()):
            assert int(t) == int(np.argmax(last)), (i, int(t), int(np.argmax(last)))
        last = ref.step(int(t))
    stats = {}
    compare("greedy last logits", logits.cpu().numpy(), last, stats)
    say(f"greedy: picks {picks[:8].tolist()}..., last logits max rel {stats['max_rel']:.3g}")
    assert stats["exact"] == 1
    # reset starts the sequence over (the prompt now as one chunk)
    s.reset()
    assert len(s) == 0
    again = s.forward(prompt).cpu().numpy()
    l2 = forward.Forward(data).session(64).feed(prompt)
    st2 = {}
    compare("after reset", again, l2, st2)
    assert st2["exact"] == 1


def test_full_needle3_geometry(nh):
    say("decode step: the full Needle-3 geometry (20 layers, vocab 16384, 5 engram sites), 6 tokens")
    g = cact.Geometry()
    data = archive(g, seed=15)
    run_pair(nh, data, o.random_tokens(6, g.vocab, seed=7), 16, "needle3")


def test_session_errors(nh):
    say("session error paths")
    g = cact.Geometry(**SMALL)
    m = nh.Model.from_archive(archive(g, seed=16))
    s = m.session(4)
    with pytest.raises(nh.NeedleHipError, match="no logits"):
        s.generate_greedy(1)
    with pytest.raises(nh.NeedleHipError, match="vocabulary"):
        s.forward([g.vocab])
    with pytest.raises(nh.NeedleHipError, match="capacity"):
        s.forward([1, 2, 3, 4, 5])
    assert len(s) == 0
    s.forward([1, 2, 3])
    with pytest.raises(nh.NeedleHipError, match="capacity"):
        s.generate_greedy(2)
    s.generate_greedy(1)
    assert len(s) == 4
    # unsupported geometry is named
    small = cact.Geometry(vocab=300, d_model=256, num_heads=4, num_kv_heads=1, num_layers=2, qk_head_dim=32,
                          v_head_dim=64, engram_slots=32, engram_sites=(1,), global_layers=(1,), sliding_window=64)
    with pytest.raises(nh.NeedleHipError, match="d_model"):
        nh.Model.from_archive(archive(small, seed=17))
    torch.cuda.synchronize()


def test_product_archive_writer(nh):
    say("the product's random-init archive writer, decoded against the oracle")
    from needle_hip import archive as W
    g = W.Needle3(vocab=300, num_layers=2, engram_slots=64, engram_sites=(1,), global_layers=(0,), sliding_window=16)
    data = W.random_needle3(nh, g, seed=3)
    run_pair(nh, data, o.random_tokens(12, g.vocab, seed=8), 16, "written")


# ---------------------------------------------------------- prompt chunks
def run_feed(nh, data, prompt, cap, label, then_steps=0):
    f = forward.Forward(data)
    m = nh.Model.from_archive(data)
    s, os_ = m.session(cap), f.session(cap)
    stats = {}
    got = s.forward(prompt).cpu().numpy()
    want = os_.feed(prompt)
    compare(f"{label} prompt", got, want, stats)
    toks = o.random_tokens(then_steps, 300, seed=31)
    for i, t in enumerate(toks):
        compare(f"{label} step {i}", s.forward([int(t)]).cpu().numpy(), os_.step(int(t)), stats)
    say(f"{label}: prompt of {len(prompt)} + {then_steps} steps: {stats['exact']}/{stats['steps']} bit-identical")
    assert stats["exact"] == stats["steps"], stats
    return m, s


def test_prefill_chunks_then_steps(nh):
    say("prompt chunks (32 + 8) then steps, 3 layers with a window and an engram site")
    g = cact.Geometry(**SMALL)
    run_feed(nh, archive(g, seed=41), o.random_tokens(40, g.vocab, seed=9), 64, "chunks", then_steps=6)


def test_prefill_single_token_tail(nh):
    say("a 33-token prompt: one chunk of 32 and a single-token step")
    g = cact.Geometry(**SMALL)
    run_feed(nh, archive(g, seed=42), o.random_tokens(33, g.vocab, seed=10), 40, "tail", then_steps=2)


def test_prefill_long_nested_chunks(nh):
    say("a 300-token prompt in 10 chunks (rows past 256 keys attend in 2 nested chunks)")
    g = cact.Geometry(vocab=300, num_layers=2, engram_slots=64, engram_sites=(1,), global_layers=(0,),
                      sliding_window=64)
    run_feed(nh, archive(g, seed=43), o.random_tokens(300, g.vocab, seed=11), 320, "long prompt", then_steps=3)


def test_prefill_mixed_widths(nh):
    say("prompt chunks over 2-bit / ternary / f16 records and two engram sites")
    g = cact.Geometry(vocab=300, num_layers=4, engram_slots=64, engram_sites=(0, 3), global_layers=(2,),
                      sliding_window=5)

    def kind(name):
        if name == "embedding":
            return ("cq", 4)
        if name.startswith("engram_table"):
            return ("random", 2)
        if name.startswith("phi"):
            return ("random", 5)
        layer = int(name.split(".")[1]) if "." in name and name.split(".")[1].isdigit() else 0
        return ("random", 2 if layer == 1 else 4)

    run_feed(nh, archive(g, seed=44, kind=kind), o.random_tokens(45, g.vocab, seed=12), 64, "mixed prompt",
             then_steps=2)


def test_prefill_full_needle3(nh):
    say("the full Needle-3 geometry: a 37-token prompt (32 + 5) then 2 steps")
    g = cact.Geometry()
    run_feed(nh, archive(g, seed=45), o.random_tokens(37, g.vocab, seed=13), 48, "needle3 prompt", then_steps=2)


@pytest.mark.parametrize("window", [0, 24])
def test_prefill_feeds_at_offsets(nh, window):
    # Feeds of 37, 63, 2, 200 and 1 tokens in one session (positions 0, 37,
    # 100, 102, 302): odd and even row counts, feeds that start mid-session,
    # rows of one key chunk and of two (past 256 keys), and a one-token step.
    # With every layer global the feed attention pairs consecutive rows in a
    # workgroup where their chunks allow: the odd feeds leave the last
    # workgroup's second row empty, and the 200-row feed pairs rows across
    # the 256-key boundary ((258, 257) keys: two chunks of 144 each).  A
    # window makes consecutive rows start at different keys, so those layers
    # keep one row per workgroup.
    say(f"feeds of 37, 63, 2, 200 and 1 tokens at positions 0 .. 302, window {window}")
    g = cact.Geometry(vocab=300, num_layers=2, engram_slots=64, engram_sites=(1,),
                      global_layers=(0, 1) if window == 0 else (0,), sliding_window=max(window, 8))
    data = archive(g, seed=61 + window)
    f = forward.Forward(data)
    m = nh.Model.from_archive(data)
    s, os_ = m.session(320), f.session(320)
    toks = o.random_tokens(303, g.vocab, seed=62)
    stats = {}
    at = 0
    for n in (37, 63, 2, 200, 1):
        part = toks[at:at + n]
        compare(f"feed of {n} at {at}", s.forward(part).cpu().numpy(), os_.feed(part), stats)
        at += n
    say(f"window {window}: {stats['exact']}/{stats['steps']} feeds bit-identical, max rel {stats['max_rel']:.3g}")
    assert stats["exact"] == stats["steps"], stats


def test_widest_model(nh):
    # d = 1024, the widest the layer kernel takes: a Phi8 row is four 1 KB
    # chunks per wavefront, the layer kernel's form that narrower models
    # (three chunks or fewer) do not use
    say("d_model 1024: a 100-token prompt (three whole chunks together, then a 4-token chunk), steps")
    g = cact.Geometry(vocab=300, d_model=1024, num_layers=2, engram_slots=64, engram_sites=(1,), global_layers=(0,),
                      sliding_window=48)
    data = archive(g, seed=61)
    run_feed(nh, data, o.random_tokens(100, g.vocab, seed=15), 140, "d_model 1024", then_steps=3)


@pytest.mark.parametrize("heads,kv,qk,vd", [(8, 2, 32, 48), (8, 1, 48, 32), (6, 3, 16, 20)])
def test_head_geometries(nh, heads, kv, qk, vd):
    say(f"{heads} heads over {kv} kv heads, qk {qk}, vd {vd}: a 300-token prompt (rows past 256 keys attend in 2 "
        f"chunks), a chunk, steps")
    g = cact.Geometry(vocab=300, num_layers=2, num_heads=heads, num_kv_heads=kv, qk_head_dim=qk, v_head_dim=vd,
                      engram_slots=64, engram_sites=(1,), global_layers=(0,), sliding_window=40)
    data = archive(g, seed=46 + heads + qk)
    m, s = run_feed(nh, data, o.random_tokens(300, g.vocab, seed=14), 340, f"heads {heads}/{kv} qk {qk} vd {vd}",
                    then_steps=3)
