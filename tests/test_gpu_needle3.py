"""GPU: the Needle-3 workloads at full geometry (20 layers, d 768, 12 heads,
2 kv heads, 5 engram sites; random-init CQ-W4 weights from the product's
archive writer, seed 0) against the oracle on the same archive.

- decode: a 118-token prompt (32 + 32 + 32 + 22 chunks), then 64 greedy
  steps (argmax, first maximum, crates/needle-engine/src/generate.rs:42-50)
  fed one token at a time; every step's logits are compared;
- prefill: one sequence of 512 random tokens (16 chunks of 32) and its last
  logits, then one step;
- cells: the per-depth lane means of a 70-token prompt and two steps
  (Model::forward_cells, crates/needle-engine/src/model.rs:330-345).

The logits must be bit-identical (the device follows the reference's float
order; see test_gpu_forward.py), the greedy picks equal; the max-abs and
max-rel errors are printed for the record.
"""
import sys

import numpy as np
import pytest

import oracle as o
from oracle import forward

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


_data = {}


def needle3(nh):
    if "a" not in _data:
        from needle_hip import archive as W
        _data["a"] = W.random_needle3(nh, seed=0)
    return _data["a"]


class Err:
    def __init__(self):
        self.abs = self.rel = 0.0
        self.n = self.exact = 0

    def add(self, got, want):
        got = np.asarray(got, np.float32)
        want = np.asarray(want, np.float32)
        d = float(np.abs(got - want).max())
        self.abs = max(self.abs, d)
        self.rel = max(self.rel, d / max(float(np.abs(want).max()), 1e-30))
        self.n += 1
        self.exact += int(np.array_equal(got.view(np.uint32), want.view(np.uint32)))

    def __str__(self):
        return f"{self.exact}/{self.n} bit-identical, max abs {self.abs:.3g}, max rel {self.rel:.3g}"


def test_needle3_decode_118_plus_64(nh):
    say("Needle-3 decode: 118-token prompt then 64 greedy steps, every step against the oracle")
    data = needle3(nh)
    m = nh.Model.from_archive(data)
    f = forward.Forward(data)
    vocab = m.out_rows
    prompt = np.random.default_rng(0).integers(0, vocab, 118).astype(np.uint32)
    s, os_ = m.session(256), f.session(256)
    e = Err()
    got = s.forward(prompt).cpu().numpy()
    want = os_.feed(prompt)
    e.add(got, want)
    say(f"prompt: {e}")
    picks = []
    for i in range(64):
        t = int(np.argmax(got))
        assert t == int(np.argmax(want)), (i, t, int(np.argmax(want)))
        picks.append(t)
        got = s.forward([t]).cpu().numpy()
        want = os_.step(t)
        e.add(got, want)
        if i % 16 == 15:
            say(f"step {i + 1}: {e}")
    say(f"decode 118 + 64: {e}; picks {picks[:8]}...")
    assert e.exact == e.n, str(e)


def test_needle3_prefill_512(nh):
    say("Needle-3 prefill: one 512-token sequence (16 chunks), last logits and one step")
    data = needle3(nh)
    m = nh.Model.from_archive(data)
    f = forward.Forward(data)
    vocab = m.out_rows
    seq = np.random.default_rng(1).integers(0, vocab, 512).astype(np.uint32)
    s, os_ = m.session(520), f.session(520)
    e = Err()
    got = s.forward(seq).cpu().numpy()
    want = os_.feed(seq)
    e.add(got, want)
    assert int(np.argmax(got)) == int(np.argmax(want))
    t = int(np.argmax(want))
    e.add(s.forward([t]).cpu().numpy(), os_.step(t))
    say(f"prefill 512 + 1: {e}")
    assert e.exact == e.n, str(e)


def test_needle3_cells(nh):
    say("Needle-3 cells (heads::cells: a fresh session, Outputs None) of a 70-token prompt, then 2 steps")
    data = needle3(nh)
    m = nh.Model.from_archive(data)
    f = forward.Forward(data)
    toks = np.random.default_rng(2).integers(0, m.out_rows, 72).astype(np.uint32)
    s, os_ = m.session(128), f.session(128)
    e = Err()
    _, gc = s.forward_cells(toks[:70])
    _, wc = os_.forward_cells(toks[:70])
    e.add(gc.cpu().numpy(), wc)
    for t in toks[70:]:
        go, gc = s.forward_cells([int(t)], forward.OUT_LAST_LOGITS)
        wo, wc = os_.forward_cells([int(t)], forward.OUT_LAST_LOGITS)
        e.add(go.cpu().numpy(), wo)
        e.add(gc.cpu().numpy(), wc)
    say(f"cells 70 + 2: {e}")
    assert e.exact == e.n, str(e)
