"""Benchmark: W4A8 decode GEMV (K=2048, N=8192, one token) on one MI355X.

A step is one sweep of the decode GEMV over `--copies` distinct HBM-resident
weight copies (>= 64 => > 512 MiB, so bytes come from HBM, not the 256 MiB
Infinity Cache): `copies` dependent launches of the full K=2048 N=8192
product, captured once as a HIP graph.  Exactly `--steps` replays are
timed, bracketed by torch.cuda.synchronize() and timed with HIP events on
the stream the kernels run on; `value` is the algorithmic bytes of one
launch over the mean time of one launch.  Algorithmic bytes per launch =
codes N*K/2 + norms N*(K/128)*2 + int8 activations K + scales (K/128)*4 +
f32 output N*4 = 8,685,632 B.

The CPU baseline leg times the oracle (the reference's portable x86-64
decode path restated in C, OpenMP row split as the reference's team splits
it) on the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "needle-rs_amd"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
K, N, GROUP = 2048, 8192, 128
# The published Needle 3's vocabulary (its logits are [t, 8192]): with it the
# Config::default geometry (20 layers, d 768) has 121M parameters.
NEEDLE3_VOCAB = 8192


def host_cpu() -> str:
    """The host's CPU as /proc/cpuinfo describes it: the model name, its
    family / model / stepping numbers (which identify the core generation
    when a virtual machine shortens the name), the logical CPUs and the
    vector extensions the oracle's compiler may use."""
    info = {}
    cpus = 0
    try:
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                continue
            k, v = (x.strip() for x in line.split(":", 1))
            if k == "processor":
                cpus += 1
            info.setdefault(k, v)
    except OSError:
        return "unknown"
    flags = set(info.get("flags", "").split())
    vec = [f for f in ("avx2", "avx512f", "avx512_vnni", "avx512_bf16") if f in flags]
    return (f"{info.get('model name', 'unknown')} (family {info.get('cpu family', '?')}, model {info.get('model', '?')}, "
            f"stepping {info.get('stepping', '?')}; {cpus} logical CPUs; {'/'.join(vec) or 'no AVX2'})")


def logits_err(got, want):
    """(bit-identical, max |got - want|, that over max |want|) of two logit rows."""
    import numpy as np

    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    d = float(np.abs(got - want).max())
    return bool(np.array_equal(got.view(np.uint32), want.view(np.uint32))), d, d / max(float(np.abs(want).max()), 1e-30)


class ErrStats:
    def __init__(self):
        self.n = self.exact = 0
        self.abs = self.rel = 0.0

    def add(self, got, want):
        e, a, r = logits_err(got, want)
        self.n += 1
        self.exact += int(e)
        self.abs = max(self.abs, a)
        self.rel = max(self.rel, r)

    def json(self):
        return {"logit_rows_compared": self.n, "bit_identical": self.exact, "max_abs": float(f"{self.abs:.3g}"),
                "max_rel": float(f"{self.rel:.3g}")}


def progress(msg: str):
    """A progress line on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(M: int, K: int, N: int) -> int:
    G = K // GROUP
    return N * K // 2 + N * G * 2 + M * K + M * G * 4 + M * N * 4


def read_traffic(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (profiles/*.md)."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    return float(m.group(1)) if m else None


def time_graph(fn_sweep, reps: int, warmup: int, torch):
    """Capture fn_sweep (a list of launches) in a graph; return ms per replay."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn_sweep()  # eager warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn_sweep()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            g.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def launch_floors(args, nh, torch):
    """What bounds one dependent launch of the GEMV's size: µs per launch, in the same graph replay of
    `copies` launches over distinct buffers, for a one-element fill (the launch itself), a write of the
    GEMV's algorithmic bytes, a copy of them (read + write), the GEMV's own loads with no arithmetic in
    its grid (nh_debug_read_floor mode 0), a plain grid-stride read of its code and norm bytes (mode 1),
    the loads in its grid ending as the GEMV ends (a workgroup barrier, then one float stored per row:
    mode 2), and the GEMV."""
    nbytes = algorithmic_bytes(1, K, N)
    n4 = nbytes // 4
    tiny = [torch.empty(1, device="cuda") for _ in range(args.copies)]
    dst = [torch.empty(n4, device="cuda") for _ in range(args.copies)]
    src = [torch.ones(n4, device="cuda") for _ in range(args.copies)]

    def us(sweep):
        return round(time_graph(sweep, max(1, args.steps), max(1, args.warmup), torch) / args.copies * 1e3, 4)

    out = {"bytes": nbytes, "launches_per_replay": args.copies,
           "fill_1_float_us": us(lambda: [x.fill_(1.0) for x in tiny]),
           "fill_bytes_us": us(lambda: [x.fill_(1.0) for x in dst]),
           "copy_bytes_us": us(lambda: [d.copy_(s_) for d, s_ in zip(dst, src)])}
    del tiny, dst, src
    gpu = gpu_gemv(args, nh, torch)
    mats, a = gpu["mats"], gpu["a"]
    out["read_gemv_grid_us"] = us(lambda: [m.read_floor(a, 0) for m in mats])
    out["read_stream_us"] = us(lambda: [m.read_floor(a, 1) for m in mats])
    out["read_gemv_grid_store_us"] = us(lambda: [m.read_floor(a, 2, gpu["y"]) for m in mats])
    out["gemv_us"] = round(gpu["ms_launch"] * 1e3, 4)
    out["gemv_again_us"] = round(time_graph(lambda: [m.matmul_into(a, gpu["y"], N, 0) for m in mats],
                                            max(1, args.steps), max(1, args.warmup), torch) / args.copies * 1e3, 4)
    for k in ("read_gemv_grid_us", "read_stream_us", "read_gemv_grid_store_us", "gemv_us"):
        out[k.replace("_us", "_tb_s")] = round(nbytes / out[k] / 1e6, 3)
    return out


def gpu_gemv(args, nh, torch):
    G = K // GROUP
    w, x = nh.seeded_normals([N * K, K], 0)
    w *= 0.02
    q0 = nh.QMat.from_f32(w, N, K)
    packed, norms = q0.download()
    mats = [q0] + [nh.QMat.from_cq(packed, norms, N, K) for _ in range(args.copies - 1)]
    xd = torch.from_numpy(x).cuda()
    a = nh.QAct.new(xd, 1, K)
    y = torch.empty(N, dtype=torch.float32, device="cuda")

    def sweep():
        for m in mats:
            m.matmul_into(a, y, N, 0)

    reps, warm = max(1, args.steps), max(1, args.warmup)
    ms_sweep = time_graph(sweep, reps, warm, torch)
    ms_launch = ms_sweep / len(mats)
    # sanity: the graph's result equals an eager launch (no oracle here)
    ref = mats[-1].matmul(a)[0]
    torch.cuda.synchronize()
    if not torch.equal(ref, y):
        raise SystemExit("graph replay and eager GEMV disagree")
    if not torch.isfinite(y).all():
        raise SystemExit("non-finite GEMV output")
    nbytes = algorithmic_bytes(1, K, N)
    gbs = nbytes / (ms_launch * 1e-3) / 1e9
    return {"ms_launch": ms_launch, "ms_sweep": ms_sweep, "gbs": gbs, "bytes": nbytes, "launches": reps * len(mats),
            "x": x, "packed": packed, "norms": norms, "G": G, "a": a, "mats": mats, "y": y}


def gpu_gemv_steady(gpu, copies, nh, torch):
    """The decode GEMV over the copies fused by row (one launch reads
    copies * 8.7 MB), so the fixed per-dispatch cost is amortised: the
    streaming rate (at this height the product runs as its persistent
    streaming grid)."""
    import numpy as np

    nbig = N * copies
    big = nh.QMat.from_cq(np.tile(gpu["packed"], (copies, 1)), np.tile(gpu["norms"], (copies, 1)), nbig, K)
    y = torch.empty(nbig, dtype=torch.float32, device="cuda")
    a = gpu["a"]

    def sweep():
        for _ in range(8):
            big.matmul_into(a, y, nbig, 0)

    ms = time_graph(sweep, 20, 2, torch) / 8
    nbytes = algorithmic_bytes(1, K, nbig)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": f"one launch of the decode GEMV (its persistent streaming grid) over N={nbig} rows (the "
                        f"{copies} copies fused by row), K={K}", "us_per_launch": round(ms * 1e3, 3),
            "bytes_per_launch": nbytes,
            "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


SWEEP_WEIGHT_BYTES = 320 * 2 ** 20


def gpu_sweeps(nh, torch):
    """Secondary lines: the prefill GEMM sweep and the LM-head shapes."""
    out = []
    shapes = [(M, k, n) for M in (64, 256, 1024) for (k, n) in ((768, 2304), (768, 3072), (3072, 768))]
    shapes += [(M, 768, 32768) for M in (1, 8, 64)]
    for M, k, n in shapes:
        w, x = nh.seeded_normals([n * k, M * k], 0)
        w *= 0.02
        # Enough distinct weight copies that one replay reads more weight
        # bytes than the 256 MB memory-side cache holds, so every product's
        # weights come from HBM: the int8 copy (n * k) above 16 tokens, the
        # 4-bit codes (n * k / 2) up to 16.
        copies = -(-SWEEP_WEIGHT_BYTES // (n * k if M > 16 else n * k // 2))
        mats = [nh.QMat.from_f32(w, n, k)]
        p, nr = mats[0].download()
        mats += [nh.QMat.from_cq(p, nr, n, k) for _ in range(copies - 1)]
        a = nh.QAct.new(torch.from_numpy(x).cuda(), M, k)
        y = torch.empty((M, n), dtype=torch.float32, device="cuda")

        # >= 64 launches per graph so replay submission never starves the GPU
        order = [mats[i % len(mats)] for i in range(max(64, copies))]

        def sweep():
            for m in order:
                m.matmul_into(a, y, n, 0)

        ms = time_graph(sweep, 10, 2, torch) / len(order)
        ops = 2.0 * M * n * k
        nbytes = algorithmic_bytes(M, k, n)
        tops = ops / (ms * 1e-3) / 1e12
        gbs = nbytes / (ms * 1e-3) / 1e9
        ai = ops / nbytes
        roof = min(INT8_PEAK_TOPS, ai * HBM_PEAK_GBS / 1e3)
        del mats
        out.append({"M": M, "K": k, "N": n, "weight_copies": copies, "us": round(ms * 1e3, 3), "TOPS": round(tops, 2),
                    "GBs": round(gbs, 1), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                    "frac_min_roofline": round(tops / roof, 4)})
    return out


def needle3_products(nh, torch):
    """Secondary line: the CQ-W4 x A8 products of the Needle-3 forward at its
    default geometry (crates/needle-core/src/config.rs:61-100: d 768, 20
    layers, vocab 8192, q|k|v|gate 576+96+128+768, 5 engram sites), with
    random-init weights 0.02*N(0,1) packed to CQ-W4 and fused as QWeights
    holds them (crates/needle-engine/src/weights.rs:480-495).

    Products only: attention, mHC, the engram conv and the MLP are not on
    this path, so these times are the products' share of a step, not the
    model's tokens/s.  Decode, per token (infer/step.rs:364,481,575,727):
    engram key|value at each site, q|k|v|gate (RMSNorm fused into its A8
    prep) and out per layer, the tied head over the whole embedding; every
    product behind its A8 prep.  Prefill, per 512-token sequence
    (infer/chunk.rs:197,274,350): the same products, each over all 512 rows
    at once as the forward feeds a prompt's whole 32-token chunks together,
    the head once."""
    import numpy as np

    d, layers, vocab, sites, seq = 768, 20, NEEDLE3_VOCAB, 5, 512
    parts = (576, 96, 128, 768)
    seed = [1000]

    def mat(n, k):
        seed[0] += 1
        (w,) = nh.seeded_normals([n * k], seed[0])
        w *= 0.02
        return nh.QMat.from_f32(w, n, k)

    head = mat(vocab, d)
    qkvg = [nh.QLinear([mat(n, d) for n in parts]) for _ in range(layers)]
    outp = [mat(d, parts[3]) for _ in range(layers)]
    ekv = [nh.QLinear([mat(d, d), mat(d, d)]) for _ in range(sites)]
    xs = nh.seeded_normals([seq * d], 77)[0]
    x = torch.from_numpy(xs).cuda()
    ns = torch.from_numpy(np.float16(1.0 + 0.1 * xs[:d]).view(np.uint16).astype(np.int16)).cuda()
    nq = sum(parts)

    def products(rows, a, ys):
        for e in ekv:
            a.prep(x, rows)
            e.rows_into(a, ys["e"], 2 * d)
        for lq, lo in zip(qkvg, outp):
            a.prep(x, rows, ns)
            lq.rows_into(a, ys["q"], nq)
            a.prep(x, rows)
            lo.matmul_into(a, ys["o"], d, 0)

    def buffers(rows):
        return {"e": torch.empty((rows, 2 * d), device="cuda"), "q": torch.empty((rows, nq), device="cuda"),
                "o": torch.empty((rows, d), device="cuda"), "h": torch.empty(vocab, device="cuda")}

    a1, y1 = nh.QAct(1, d), buffers(1)

    def token():
        products(1, a1, y1)
        a1.prep(x, 1, ns)
        head.matmul_into(a1, y1["h"], vocab, 0)

    ac, yc = nh.QAct(seq, d), buffers(seq)

    def sequence():
        products(seq, ac, yc)
        a1.prep(x, 1, ns)
        head.matmul_into(a1, y1["h"], vocab, 0)

    dec_ms = time_graph(token, 50, 3, torch)
    pre_ms = time_graph(sequence, 10, 2, torch)
    launches = 2 * (sites + 2 * layers + 1)
    return {"workload": "Needle-3 CQ-W4 x A8 products only (random-init weights; attention, mHC, engram conv and "
                        "MLP not included): decode per token; prefill per 512-token sequence, each product over "
                        "the sequence's 512 rows at once (the forward feeds whole 32-token chunks together)",
            "products_only": True, "launches_per_token": launches,
            "decode_us_per_token": round(dec_ms * 1e3, 2),
            "decode_products_tok_s": round(1e3 / dec_ms, 1),
            "decode_us_per_launch": round(dec_ms * 1e3 / launches, 3),
            "prefill_us_per_seq512": round(pre_ms * 1e3, 1),
            "prefill_products_tok_s": round(seq * 1e3 / pre_ms, 1)}


DECODE_PROMPT, DECODE_STEPS = 118, 64


def needle3_decode(nh, torch, cpu_seconds: float, with_cpu: bool):
    """The full Needle-3 decode (crates/needle-core/src/config.rs:61-100:
    20 layers, d 768, 5 engram sites; vocab 8192, 121M parameters) from random-init weights
    0.02*N(0,1) through CQ-W4 (needle_hip.archive.random_needle3, seed 0):
    a prompt of 118 uniform random token ids fed as forward_native feeds it
    (chunks of 32 through chunk_job), then 64 greedy decode steps on the
    device (argmax, step_native, no host round trip), the KV cache and every
    activation in HBM.  decode_tok_s counts the 64 greedy steps over their
    HIP-event time on the launch stream.

    The CPU leg runs the oracle's step_native (oracle/forward.c, OpenMP over
    the products' rows) on the same archive and tokens, for as many steps
    as fit the time bound, and checks its logits' argmax against every
    device pick it reaches."""
    import numpy as np

    from needle_hip import archive

    t0 = time.perf_counter()
    data = archive.random_needle3(nh, archive.Needle3(vocab=NEEDLE3_VOCAB), seed=0)
    build_s = time.perf_counter() - t0
    model = nh.Model.from_archive(data)
    vocab = model.out_rows
    prompt = np.random.default_rng(0).integers(0, vocab, DECODE_PROMPT).astype(np.uint32)
    sess = model.session(DECODE_PROMPT + DECODE_STEPS)
    progress(f"Needle-3 archive built in {build_s:.1f} s ({len(data) / 2**20:.1f} MiB)")
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    runs = []
    picks = None
    for r in range(4):  # the first run warms up
        sess.reset()
        torch.cuda.synchronize()
        ev[0].record(stream)
        sess.forward(prompt)
        ev[1].record(stream)
        picks, _ = sess.generate_greedy(DECODE_STEPS)
        ev[2].record(stream)
        torch.cuda.synchronize()
        if r > 0:
            runs.append((ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2])))
    prompt_ms = min(a for a, _ in runs)
    decode_ms = min(b for _, b in runs)
    layers = 20
    out = {"workload": "Needle-3 random-init decode: 118 random prompt tokens fed together (32-token chunks "
                       "32 + 32 + 32 + 22, each with its own block flags), then 64 greedy steps on the device",
           "prompt_tokens": DECODE_PROMPT, "decode_steps": DECODE_STEPS,
           "decode_tok_s": round(DECODE_STEPS * 1e3 / decode_ms, 1),
           "decode_ms_per_token": round(decode_ms / DECODE_STEPS, 4),
           "prompt_tok_s": round(DECODE_PROMPT * 1e3 / prompt_ms, 1),
           # begin (which also picks the step's token: the argmax of the
           # previous logits), batched engram key | value, engram history;
           # per layer the layer boundary, q|k|v|gate, decode attention,
           # out; head input, head (positions below 256 keys)
           "runs": len(runs), "launches_per_token": 3 + 4 * layers + 2,
           "first_picks": [int(t) for t in picks[:8]]}
    progress(f"Needle-3 decode: {out['decode_ms_per_token'] * 1e3:.1f} us per token")
    out["span"] = needle3_decode_span(nh, torch, model, prompt)
    progress(f"Needle-3 decode under the agent's span: {out['span']['decode_ms_per_token'] * 1e3:.1f} us per token")
    if with_cpu:
        import oracle as o
        from oracle import forward

        # The oracle fed the same prompt and the device's picks; the device
        # re-fed step by step (outside the timed runs) so that every step's
        # logits can be compared.  Only the oracle's time counts for its rate.
        f = forward.Forward(data)
        ses = f.session(DECODE_PROMPT + DECODE_STEPS)
        err = ErrStats()
        sess.reset()
        t1 = time.perf_counter()
        last = ses.feed(prompt)
        t_prompt = time.perf_counter() - t1
        err.add(sess.forward(prompt).cpu().numpy(), last)
        agree, steps, t_dec = 0, 0, 0.0
        for t in picks:
            agree += int(int(np.argmax(last)) == int(t))
            t2 = time.perf_counter()
            last = ses.step(int(t))
            t_dec += time.perf_counter() - t2
            err.add(sess.forward([int(t)]).cpu().numpy(), last)
            steps += 1
            if t_dec >= cpu_seconds:
                break
        out["cpu_baseline"] = {"value": round(steps / t_dec, 2), "unit": "tok/s", "cores": o.default_threads(),
                               "cpu": host_cpu(), "kind": "port",
                               "sample": f"the oracle's step_native: the 118-token prompt ({t_prompt:.1f} s), then "
                                         f"{steps} of the 64 decode steps fed the device's picks ({t_dec:.1f} s)"}
        out["parity"] = {"greedy_picks_checked": steps, "oracle_argmax_agrees": agree, **err.json()}
        out["gpu_over_cpu"] = round(out["decode_tok_s"] / out["cpu_baseline"]["value"], 1)
    return out


SPAN_SINK, SPAN_RING, SPAN_FILL = DECODE_PROMPT, 256, 300


def needle3_decode_span(nh, torch, model, prompt):
    """The decode as the agent runs it (agent.rs:207-209,584-588): attend =
    (sink, ring) with the 118-token prompt as the static prefix and the
    published kv_window of 256 as the ring; 300 more tokens fed as a prefill,
    then 64 greedy steps at positions 418..481, each query seeing the sink
    and the last 256 positions (374 keys: four key chunks)."""
    import numpy as np

    fill = np.random.default_rng(3).integers(0, model.out_rows, SPAN_FILL).astype(np.uint32)
    sess = model.session(DECODE_PROMPT + SPAN_FILL + DECODE_STEPS)
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    runs = []
    for r in range(3):  # the first run warms up
        sess.reset()
        sess.set_attend(SPAN_SINK, SPAN_RING)
        sess.prefill(prompt, 0)
        sess.prefill(fill)
        torch.cuda.synchronize()
        ev[0].record(stream)
        picks, _ = sess.generate_greedy(DECODE_STEPS)
        ev[1].record(stream)
        torch.cuda.synchronize()
        if r > 0:
            runs.append(ev[0].elapsed_time(ev[1]))
    ms = min(runs)
    return {"workload": f"attend = (sink {SPAN_SINK}, ring {SPAN_RING}) as the agent sets it: the 118-token prompt, "
                        f"{SPAN_FILL} more tokens, then {DECODE_STEPS} greedy steps at positions "
                        f"{DECODE_PROMPT + SPAN_FILL}..{DECODE_PROMPT + SPAN_FILL + DECODE_STEPS - 1} "
                        f"({SPAN_SINK + SPAN_RING} keys a query)",
            "decode_tok_s": round(DECODE_STEPS * 1e3 / ms, 1), "decode_ms_per_token": round(ms / DECODE_STEPS, 4),
            "runs": len(runs), "first_picks": [int(t) for t in picks[:8]]}


PREFILL_SEQS, PREFILL_LEN = 16, 512


def needle3_prefill(nh, torch, cpu_seconds: float, with_cpu: bool):
    """The prefill-heavy run: 16 independent sequences of 512 uniform random
    token ids, one sequence at a time, each fed as forward_native feeds a
    prompt (16 chunks of 32 through chunk_job: every product over the
    chunk's rows on the W4A8 GEMM, the prefill combine) into a fresh
    session, Outputs::LastLogits.  Same random-init archive as the decode
    run.  prefill_tok_s = 16 x 512 tokens over the HIP-event time of the
    16 sequences on the launch stream.

    The CPU leg feeds the oracle's chunk_job the same sequences for as many
    chunks as fit the time bound, and checks its last logits' argmax at the
    end of every whole sequence it reaches."""
    import numpy as np

    from needle_hip import archive

    data = archive.random_needle3(nh, archive.Needle3(vocab=NEEDLE3_VOCAB), seed=0)
    model = nh.Model.from_archive(data)
    rng = np.random.default_rng(1)
    seqs = [rng.integers(0, model.out_rows, PREFILL_LEN).astype(np.uint32) for _ in range(PREFILL_SEQS)]
    sess = model.session(PREFILL_LEN)
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    runs, last = [], []
    for r in range(3):  # the first run warms up
        last = []
        torch.cuda.synchronize()
        ev0.record(stream)
        for q in seqs:
            sess.reset()
            last.append(sess.forward(q))
        ev1.record(stream)
        torch.cuda.synchronize()
        if r > 0:
            runs.append(ev0.elapsed_time(ev1))
    ms = min(runs)
    picks = [int(torch.argmax(x).item()) for x in last]
    out = {"workload": "Needle-3 random-init prefill: 16 sequences x 512 random tokens, one at a time, each fed "
                       "as its 16 whole 32-token chunks together (512 rows per layer launch, the products as "
                       "M=512 W4A8 GEMMs)",
           "sequences": PREFILL_SEQS, "tokens_per_sequence": PREFILL_LEN,
           "prefill_tok_s": round(PREFILL_SEQS * PREFILL_LEN * 1e3 / ms, 1),
           "ms_per_sequence": round(ms / PREFILL_SEQS, 3), "runs": len(runs)}
    progress(f"Needle-3 prefill: {out['ms_per_sequence']:.2f} ms per 512-token sequence")
    if with_cpu:
        import oracle as o
        from oracle import forward

        f = forward.Forward(data)
        err = ErrStats()
        tokens, agree, whole, t0 = 0, 0, 0, time.perf_counter()
        for q, pick, got in zip(seqs, picks, last):
            ses = f.session(PREFILL_LEN)
            lg = None
            for i in range(0, PREFILL_LEN, 32):
                lg = ses.chunk(q[i:i + 32])
                tokens += 32
                if time.perf_counter() - t0 >= cpu_seconds:
                    break
            if len(ses) == PREFILL_LEN:
                whole += 1
                agree += int(int(np.argmax(lg)) == pick)
                err.add(got.cpu().numpy(), lg)
            if time.perf_counter() - t0 >= cpu_seconds:
                break
        el = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(tokens / el, 1), "unit": "tok/s", "cores": o.default_threads(),
                               "cpu": host_cpu(), "kind": "port",
                               "sample": f"the oracle's chunk_job over {tokens} tokens of the same sequences "
                                         f"({el:.1f} s)"}
        out["parity"] = {"sequences_checked": whole, "oracle_argmax_agrees": agree, **err.json()}
        out["gpu_over_cpu"] = round(out["prefill_tok_s"] / out["cpu_baseline"]["value"], 1)
    return out


def gemm_shape(spec: str, launches: int, nh, torch):
    """One prefill product M x K x N (seeded as the sweep), `launches` eager
    launches timed with HIP events on the launch stream: the command the
    GEMM profiles are taken from."""
    M, k, n = (int(v) for v in spec.split(","))
    w, x = nh.seeded_normals([n * k, M * k], 0)
    w *= 0.02
    q = nh.QMat.from_f32(w, n, k)
    a = nh.QAct.new(torch.from_numpy(x).cuda(), M, k)
    y = torch.empty((M, n), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    for _ in range(3):
        q.matmul_into(a, y, n, 0)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(launches):
        q.matmul_into(a, y, n, 0)
    end.record(stream)
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / launches
    ops = 2.0 * M * n * k
    return {"gemm": {"M": M, "K": k, "N": n}, "launches": launches, "us_per_launch": round(us, 3),
            "TOPS": round(ops / (us * 1e-6) / 1e12, 2), "frac_int8_peak": round(ops / (us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4)}


def cpu_baseline(gpu, seconds: float):
    """The oracle's decode GEMV (reference x86-64 portable path) on the host."""
    import numpy as np

    import oracle as o

    threads = o.default_threads()
    q = o.OQMat.from_cq(gpu["packed"], gpu["norms"], N, K)
    a = o.OQAct.new(gpu["x"], 1, K)
    y = np.zeros((1, N), dtype=np.float32)
    q.matmul_into(a, y, N, 0, threads)  # warm-up
    calls, t0 = 0, time.perf_counter()
    while True:
        q.matmul_into(a, y, N, 0, threads)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds or calls >= 2000:
            break
    per = el / calls
    return {"value": round(gpu["bytes"] / per / 1e9, 3), "unit": "GB/s", "cores": threads, "cpu": host_cpu(),
            "kind": "port",
            "sample": f"{calls} full K=2048 N=8192 decode GEMVs over {el:.1f} s (one weight copy, host-resident)",
            "ms_per_call": round(per * 1e3, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed sweeps of the copies (graph replays)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--copies", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device-to-device copy of BYTES (scales rocprofv3 byte counters)")
    ap.add_argument("--gemm-shape", default="", metavar="M,K,N",
                    help="only run one prefill product shape, eagerly (for GEMM profiles)")
    ap.add_argument("--launches", type=int, default=200, help="launches for --gemm-shape")
    ap.add_argument("--floors", action="store_true",
                    help="only time the single-launch floors beside the GEMV (launch, write, copy)")
    ap.add_argument("--needle3-only", action="store_true",
                    help="only run the Needle-3 decode and prefill lines (for model profiles)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch

        src = torch.ones(args.copy_calibration // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": args.copy_calibration, "launches": 5}))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "the library runs on one GPU; --gpus above 1 is not supported "
                                   "(the W4A8 products would shard by output rows)"}))
        sys.exit(2)
    if args.copies < 1:
        raise SystemExit("--copies must be >= 1")

    import torch

    import needle_hip as nh

    nh.init(0)
    torch.cuda.synchronize()
    if args.gemm_shape:
        print(json.dumps(gemm_shape(args.gemm_shape, args.launches, nh, torch)))
        return
    if args.floors:
        print(json.dumps(launch_floors(args, nh, torch)))
        return
    if args.needle3_only:
        print(json.dumps({"needle3_decode": needle3_decode(nh, torch, args.cpu_seconds * 2, not args.no_cpu),
                          "needle3_prefill": needle3_prefill(nh, torch, args.cpu_seconds * 2, not args.no_cpu)}))
        return
    gpu = gpu_gemv(args, nh, torch)
    progress(f"decode GEMV: {gpu['ms_launch'] * 1e3:.3f} us per launch")
    steps = args.steps
    line = {
        "metric": "W4A8 GEMV HBM GB/s (K=2048, N=8192, decode combine)",
        "value": round(gpu["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_sweep"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4(cq codebook)/a8 int8, i32 accumulate, f32 combine",
        "data": "synthetic seeded: W=0.02*N(0,1) (threefry, seed 0) through CQ-W4 group 128; x=N(0,1)",
        "config": {"workload": "single W4A8 decode GEMV, K=2048 N=8192 M=1, rotating "
                               f"{args.copies} HBM-resident weight copies", "K": K, "N": N, "M": 1,
                   "copies": args.copies, "bytes_per_launch": gpu["bytes"],
                   "step": f"one sweep of {args.copies} dependent launches, one per weight copy",
                   "us_per_launch": round(gpu["ms_launch"] * 1e3, 4), "launches_timed": gpu["launches"]},
        "roofline": {"bound": "hbm", "achieved": round(gpu["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gpu["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic("gemv_decode_k2048_n8192_pmc.md")},
    }
    if not args.no_sweep:
        line["steady_state"] = gpu_gemv_steady(gpu, args.copies, nh, torch)
        progress("steady state done")
        line["secondary"] = gpu_sweeps(nh, torch)
        progress("GEMM sweep done")
        line["needle3_products"] = needle3_products(nh, torch)
        progress("Needle-3 products done")
        line["needle3_decode"] = needle3_decode(nh, torch, args.cpu_seconds * 2, not args.no_cpu)
        progress("Needle-3 decode done")
        line["needle3_prefill"] = needle3_prefill(nh, torch, args.cpu_seconds * 2, not args.no_cpu)
        progress("Needle-3 prefill done")
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(gpu, args.cpu_seconds)
        line["cpu_baseline"]["gpu_over_cpu"] = round(gpu["gbs"] / line["cpu_baseline"]["value"], 1)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
