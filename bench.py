#!/usr/bin/env python
"""Benchmark: µs per 4-row MTP verify sampling step at V = 248,320 on one MI355X.

Workload (one step): 4 rows x 248,320 f32 logits already resident in HBM (1 main + 3 draft positions, each row
N(0,1.5) plus 50 head ids at N(8,2)), 3 drafts, temperature 0.6, top-k 20, top-p 0.95, per-row uniforms; each
row is sampled and the accepted-prefix length computed, as klein's verify loop (src/engine.cpp:563-575) with
src/sampler.cpp per row. A step is one kls_verify call: one hipGraph launch, results (tokens, and the accepted
count formed on the device) read back through pinned memory. `value` is the mean host wall-clock time per step
over the timed steps (launch to results on the host); every timed step's tokens and accepted count are checked
against an untimed launch with the same uniforms.

Also reported:
  latency       per-step host latencies: the first 25 timed steps, median and p99 of the timed steps, and of
                1,000 more steps (hot), and of 200 steps with HBM cold (a 512 MiB buffer written between steps);
  roofline      the verify kernel's device time per launch (HIP events around a graph of back-to-back copies of
                the captured step, on the step's stream) and the HBM rate of its algorithmic bytes (every logit
                read once: 4 x 993,280 B + drafts and uniforms); traffic from the committed PMC profile when its
                kernel source hash matches the built one;
  handle        per-request cost (klein builds one Sampler per request): create, first verify step (graph
                capture and instantiation), destroy;
  batched       64 independent rows x 248,320 with per-row 16,384-id Zipf histories, penalties (repetition 1.1,
                presence 0.5, frequency 0.2), top-k 64, top-p 0.9: device time per batch, hot (same input every
                launch) and cold (8 input sets rotated, 509 MB, more than the 256 MB last-level cache), every
                launch's tokens checked;
  next_rows     the MTP draft argmax (Engine::mtp_draft_token, 1 row: std::max_element), one pass of the
                perplexity / KL loop (src/main.cpp:308-327: 64 rows plus base log-probabilities), and the
                recurrent-state rollback of a rejected draft (State::rollback_recurrent, 48 DeltaNet layers of a
                27B-class model, f16 snapshots), with their HBM rates;
  cpu_baseline  the reference's own sampler.cpp (oracle/_ref, built -O3 from its sources) on the host: one core
                for every workload (greedy row, top-k/top-p row, penalized row, verify step, 64-row batch) and
                all host cores (up to 16) for the 64-row batch, with the host's CPU, nproc and library versions.
"""
import argparse
import ctypes as C
import hashlib
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "µs per 4-row MTP verify sampling step @V=248,320; achieved HBM GB/s"
HBM_PEAK_GBS = 8000.0
V = 248_320
STEP_BYTES = 4 * V * 4 + 3 * 4 + 4 * 8          # logits + drafts + uniforms = 3,973,164
BATCH_BYTES = 64 * (V * 4 + 16384 * 4)           # logits + raw history ids = 67,764,224
# recurrent state of a 27B-class model: 48 DeltaNet layers, conv rows (4 - 1) x 10,240 f32, ssm rows 128 x 128 x 48
RB_LAYERS, RB_CONV, RB_SSM = 48, 30720, 786432
ROLLBACK_BYTES = RB_LAYERS * (2 * RB_CONV * 4 + RB_SSM * (2 + 4))  # conv slot read + write, f16 row read, f32 write


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=24.0, help="bound of the whole CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batched", action="store_true")
    ap.add_argument("--no-next", action="store_true", help="skip the draft-argmax, ppl and rollback measurements")
    ap.add_argument("--no-extra", action="store_true", help="skip the latency distributions and handle costs")
    return ap.parse_args()


def pct(xs, q):
    s = sorted(xs)
    return s[min(len(s) - 1, (len(s) * q) // 100)]


def kernel_source_hash():
    h = hashlib.sha256()
    for f in ("kls_kernels.hip", "kls_internal.h"):
        h.update(open(os.path.join(ROOT, "klein_amd", "csrc", f), "rb").read())
    return h.hexdigest()[:16]


def traffic_from_profile():
    """HBM bytes per launch of the verify kernel from the committed rocprofv3 PMC summary, when it was measured on
    the kernel source built now (else None: the figure would be stale)."""
    path = os.path.join(ROOT, "profiles", "traffic_verify_4x248320.json")
    if not os.path.exists(path):
        return None, "no profile"
    d = json.load(open(path))
    if d.get("kernel_source_sha16") != kernel_source_hash():
        return None, "profile measured on other kernel source"
    return d.get("hbm_bytes_per_launch"), f"rocprofv3 PMC (FETCH_SIZE, WRITE_SIZE), {path[len(ROOT) + 1:]}"


def copy_probe(torch, stream):
    """A plain device copy of 256 MiB (torch's copy kernel): its measured rate."""
    n = 256 * 1024 * 1024 // 4
    a = torch.empty(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1.0)
    for _ in range(3):
        b.copy_(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(10):
        b.copy_(a)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / 10
    del a, b
    return {"bytes_read": n * 4, "bytes_written": n * 4, "us": round(us, 2),
            "GBps_read_plus_write": round(2 * n * 4 / (us * 1e-6) / 1e9, 1)}


def graph_us(torch, launch, n):
    """Device µs per launch: n launches captured in one graph (no host work between them), the replay timed
    with stream events. launch(stream_ptr) enqueues one call on the given stream."""
    cs = torch.cuda.Stream()
    launch(C.c_void_p(cs.cuda_stream))  # (first call outside the capture)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for _ in range(n):
            launch(C.c_void_p(cs.cuda_stream))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 5
    with torch.cuda.stream(cs):  # (replays run on the current stream)
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        e0.record(cs)
        for _ in range(reps):
            g.replay()
        e1.record(cs)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * n)


def next_rows(torch, klein_amd, W):
    import numpy as np
    from klein_amd import _lib
    L = _lib.lib()
    rng = np.random.default_rng(77)
    res = {}
    S = klein_amd.Sampler(W.Params(temperature=0.0), n_vocab=V, max_rows=64)
    h = S._h
    p = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    # draft argmax: one MTP row (the greedy workload's logits), as called once per draft
    g = W.greedy()
    d1 = torch.from_numpy(g.logits).cuda()
    o1 = torch.zeros(1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()  # (buffers made on torch's stream, used on others: ready before any launch)
    us = graph_us(torch, lambda sp: _lib.check(L.kls_argmax(h, p(d1), 1, V, p(o1), sp), "kls_argmax"), 200)
    assert int(o1.item()) == g.expected_greedy
    res["draft_argmax"] = {"workload": "1 row x 248,320 f32 (std::max_element)", "us": round(us, 2),
                           "GBps": round(V * 4 / (us * 1e-6) / 1e9, 1)}
    # ppl: the loop's default pass of 64 rows with a KL base, 4 input sets (254 MB each way) rotated
    sets = []
    for _ in range(4):
        x = torch.randn((64, V), device="cuda", dtype=torch.float32) * 2.0
        b = torch.log_softmax(torch.randn((64, V), device="cuda", dtype=torch.float32) * 3.0, dim=1)
        sets.append((x, b))
    tg = torch.from_numpy(rng.integers(0, V, 64).astype(np.int32)).cuda()
    outs = [torch.empty(64, dtype=torch.float64, device="cuda") for _ in range(4)]
    tops = [torch.empty(64, dtype=torch.int32, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    k = [0]

    def ppl(sp):
        x, b = sets[k[0] % 4]
        k[0] += 1
        _lib.check(L.kls_ppl_scores(h, p(x), 64, V, p(tg), p(b), V, p(outs[0]), p(outs[1]), p(tops[0]),
                                    p(outs[2]), p(outs[3]), p(tops[1]), sp), "kls_ppl_scores")

    us = graph_us(torch, ppl, 40)
    pbytes = 2 * 64 * V * 4 + 64 * 4
    res["ppl_pass"] = {"workload": "64 rows x 248,320 logits + base log-probabilities, per-token lse/nll/KL",
                       "algorithmic_bytes": pbytes, "us_cold": round(us, 2),
                       "GBps": round(pbytes / (us * 1e-6) / 1e9, 1),
                       "frac": round(pbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del sets
    S.close()
    # rollback of 2 rejected drafts over a 27B-class recurrent state (f16 snapshots, 4 slots)
    conv = [torch.zeros((4, RB_CONV), dtype=torch.float32, device="cuda") for _ in range(RB_LAYERS)]
    ssm = [torch.zeros(RB_SSM, dtype=torch.float32, device="cuda") for _ in range(RB_LAYERS)]
    snap = [torch.zeros((3, RB_SSM), dtype=torch.int16, device="cuda") for _ in range(RB_LAYERS)]
    P = C.c_void_p * RB_LAYERS
    arrs = [P(*[t.data_ptr() for t in ts]) for ts in (conv, ssm, snap)]
    desc = _lib.KlsRecurrentDesc(RB_LAYERS, 4, RB_CONV, RB_SSM, 4 * RB_CONV, 2 * RB_SSM, _lib.KLS_SNAP_F16,
                                 *[C.cast(a, C.POINTER(C.c_void_p)) for a in arrs])
    rh = C.c_void_p()
    _lib.check(L.kls_recurrent_create(C.byref(desc), C.byref(rh)), "kls_recurrent_create")
    acc = torch.tensor([1], dtype=torch.int32, device="cuda")  # accepted 1 of 3 drafts: s = 2
    torch.cuda.synchronize()
    us = graph_us(torch, lambda sp: _lib.check(L.kls_rollback_recurrent(rh, p(acc), 4, sp), "kls_rollback"), 20)
    L.kls_recurrent_destroy(rh)
    res["rollback"] = {"workload": "48 DeltaNet layers (conv 30,720 f32 slot copy, ssm 786,432 f16 -> f32), s = 2",
                       "algorithmic_bytes": ROLLBACK_BYTES, "us": round(us, 2),
                       "GBps": round(ROLLBACK_BYTES / (us * 1e-6) / 1e9, 1),
                       "frac": round(ROLLBACK_BYTES / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del conv, ssm, snap
    return res


def topk_above_64(torch, klein_amd, W):
    """Top-k above 64 (src/sampler.cpp:42-51 with larger k), which no headline config uses: the verify step's
    workload with k = 256 and 1,024 on the mid path (one kernel, captured in the step's graph) and without a limit
    on the wide path (keys, a device-wide sort, the tail: several kernels, captured in the step's graph), the
    64-row batch at k = 256, and one row without a limit launched directly.
    Every timed call is checked against its first (untimed) result."""
    import numpy as np
    from klein_amd import _lib
    L = _lib.lib()
    I32P, F64P = C.POINTER(C.c_int32), C.POINTER(C.c_double)
    v = W.verify()
    d = torch.from_numpy(v.logits).cuda()
    dptr = C.c_void_p(d.data_ptr())
    drafts = np.ascontiguousarray(v.drafts, dtype=np.int32)
    u = np.ascontiguousarray(v.u, dtype=np.float64)
    res = {}
    for k in (256, 1024, 0):
        path = "mid" if k else "wide"
        S = klein_amd.Sampler(W.Params(temperature=0.6, top_k=k, top_p=0.95), n_vocab=V, max_rows=4)
        assert S.path == path
        h, sp = S._h, None
        t0, a0 = np.zeros(4, np.int32), C.c_int32()
        _lib.check(L.kls_verify(h, dptr, 4, drafts.ctypes.data_as(I32P), u.ctypes.data_as(F64P),
                                t0.ctypes.data_as(I32P), C.byref(a0), sp), "kls_verify")
        tk, ac = np.zeros(4, np.int32), C.c_int32()
        lat = []
        for i in range(300):
            x0 = time.perf_counter_ns()
            st = L.kls_verify(h, dptr, 4, drafts.ctypes.data_as(I32P), u.ctypes.data_as(F64P),
                              tk.ctypes.data_as(I32P), C.byref(ac), sp)
            lat.append((time.perf_counter_ns() - x0) / 1e3)
            if st:
                _lib.check(st, "kls_verify")
            assert ac.value == a0.value and list(tk[:ac.value + 1]) == list(t0[:a0.value + 1]), f"{path} verify step"
        kus = C.c_double()
        _lib.check(L.kls_debug_time_verify(h, 50, 5, sp, C.byref(kus)), "kls_debug_time_verify")
        res[f"verify_step_k{k}" if k else "verify_step_no_limit"] = {
            "path": path, "median_us": round(pct(lat, 50), 2), "p99_us": round(pct(lat, 99), 2),
            "kernel_us": round(kus.value, 2)}
        S.close()
    # 64 rows at k = 256, no penalties
    wb = W.batched()
    SB = klein_amd.Sampler(W.Params(temperature=1.0, top_k=256, top_p=0.9), n_vocab=V, max_rows=64)
    xb = torch.from_numpy(wb.logits).cuda()
    ub = torch.from_numpy(wb.u).cuda()
    ob = torch.full((64,), -1, dtype=torch.int32, device="cuda")
    first = torch.full((64,), -2, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()  # (made on torch's stream, written on the library's and on another)
    pb = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    _lib.check(L.kls_sample_batch(SB._h, pb(xb), 64, V, None, None, pb(ub), pb(first), None), "kls_sample_batch")
    us_b = graph_us(torch, lambda s: _lib.check(L.kls_sample_batch(SB._h, pb(xb), 64, V, None, None, pb(ub), pb(ob),
                                                                   s), "kls_sample_batch"), 20)
    torch.cuda.synchronize()
    assert torch.equal(ob, first), "mid batch"
    res["batch_64_rows_k256"] = {"path": "mid", "us_hot": round(us_b, 2),
                                 "GBps": round(64 * V * 4 / (us_b * 1e-6) / 1e9, 1)}
    SB.close()
    # one row without a limit (k = V): the wide path, launched directly
    SW = klein_amd.Sampler(W.Params(temperature=1.0, top_k=0, top_p=0.95), n_vocab=V, max_rows=1)
    assert SW.path == "wide"
    o1 = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    f1 = torch.full((1,), -2, dtype=torch.int32, device="cuda")
    cs = torch.cuda.current_stream()
    sc = C.c_void_p(cs.cuda_stream)  # (the events below are recorded on this stream)
    _lib.check(L.kls_sample_batch(SW._h, dptr, 1, V, None, None, pb(ub), pb(f1), sc), "kls_sample_batch")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cs)
    for _ in range(10):
        _lib.check(L.kls_sample_batch(SW._h, dptr, 1, V, None, None, pb(ub), pb(o1), sc), "kls_sample_batch")
    e1.record(cs)
    torch.cuda.synchronize()
    assert torch.equal(o1, f1), "wide row"
    res["one_row_no_limit"] = {"path": "wide", "us": round(e0.elapsed_time(e1) * 1e3 / 10, 1)}
    SW.close()
    return res


def host_info():
    info = {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "machine": platform.machine()}
    try:
        for line in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if line.startswith("Model name:"):
                info["cpu"] = line.split(":", 1)[1].strip()
    except Exception:
        pass
    info["glibc"] = "-".join(platform.libc_ver())
    try:
        gcc = subprocess.run(["g++", "-dumpfullversion"], capture_output=True, text=True, timeout=10).stdout.strip()
        info["libstdcxx"] = f"GCC {gcc}"
    except Exception:
        pass
    for f in ("/opt/rocm/.info/version", "/opt/rocm/.info/version-dev"):
        if os.path.exists(f):
            info["rocm"] = open(f).read().strip()
            break
    return info


def cpu_baseline(W, seconds):
    """The reference sampler (oracle/_ref: src/sampler.cpp built -O3 -DNDEBUG from its sources), or the oracle's
    restatement when the reference build is absent, on bounded samples of every workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle
    ref = oracle.ref_available()
    sink = C.c_int32()
    budget = seconds / 6.0  # per workload (the 64-row batch gets two)
    out = {}

    def fp(a):
        return a.ctypes.data_as(C.POINTER(C.c_float))

    def time_rows(params, logits, hist=None):
        """(seconds per sample() call) cycling over the rows of `logits` with one sampler."""
        rows = logits.shape[0]
        if ref:
            s = oracle.RefSampler(params)
            if hist is not None:
                for t in hist:
                    s.accept(int(t))
            L = oracle.ref()
            run = lambda reps: L.ref_time_rows(s._h, fp(logits), V, rows, reps, C.byref(sink))  # noqa: E731
        else:
            L = oracle.lib()
            ps = oracle.params_struct(params)
            cnt = None if hist is None else np.ascontiguousarray(W.counts_of(hist, V), np.int32)
            run = lambda reps: L.orc_time_rows(fp(logits), V, rows, C.byref(ps),  # noqa: E731
                                               None if cnt is None else cnt.ctypes.data_as(C.POINTER(C.c_int32)),
                                               reps, C.byref(sink))
        run(rows)
        t = run(rows)
        per = t / rows
        reps = max(rows, int(budget / per) // rows * rows)
        t = run(reps)
        return t / reps, reps, t

    g, tk, pen, ver, bat = W.greedy(), W.topk_topp(), W.penalties(), W.verify(), W.batched()
    for name, w, unit_rows in (("greedy_row", g, 1), ("topk_topp_row", tk, 1), ("penalties_row", pen, 1),
                               ("verify_step", ver, 4)):
        lg = np.ascontiguousarray(w.logits, np.float32)
        per, reps, t = time_rows(w.params, lg, w.histories[0] if w.histories else None)
        out[name] = {"us": round(per * unit_rows * 1e6, 1), "samples": reps, "seconds": round(t, 2)}
    # 64-row batch: one sampler per row (its own history); one thread, then all host cores
    lg = np.ascontiguousarray(bat.logits, np.float32)
    if ref:
        L = oracle.ref()
        samplers = [oracle.RefSampler(bat.params) for _ in range(64)]
        for s, hst in zip(samplers, bat.histories):
            for t in hst:
                s.accept(int(t))
        arr = (C.c_void_p * 64)(*[s._h for s in samplers])
        L.ref_time_rows_threads(arr, fp(lg), V, 64, 1, 1)
        t1 = L.ref_time_rows_threads(arr, fp(lg), V, 64, 1, 1)
        reps = max(1, int(budget / t1))
        t1 = L.ref_time_rows_threads(arr, fp(lg), V, 64, reps, 1)
        out["batched_64_rows"] = {"us": round(t1 / reps * 1e6, 1), "samples": reps * 64, "seconds": round(t1, 2)}
        cores = max(1, min(16, len(os.sched_getaffinity(0))))
        tn = L.ref_time_rows_threads(arr, fp(lg), V, 64, 1, cores)
        reps_n = max(1, int(budget / max(tn, 1e-6)))
        tn = L.ref_time_rows_threads(arr, fp(lg), V, 64, reps_n, cores)
        out["batched_64_rows_all_cores"] = {"us": round(tn / reps_n * 1e6, 1), "cores": cores,
                                            "samples": reps_n * 64, "seconds": round(tn, 2)}
        kind, what = "reference", "klein src/sampler.cpp built -O3 -DNDEBUG from its sources (oracle/_ref)"
    else:
        kind, what = "port", "oracle restatement of src/sampler.cpp (reference build absent)"
    v = out["verify_step"]
    return {"value": v["us"], "unit": "us", "cores": 1, "kind": kind,
            "sample": f"{v['samples'] // 4} verify steps x 4 rows x 248,320 f32, sample() per row as engine.cpp:566, "
                      f"{v['seconds']} s on 1 host thread; {what}",
            "workloads": out, "host": host_info()}


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: the sampling path runs on a single MI355X (rows of a step stay on "
              f"one device); --gpus {a.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import klein_amd
    from klein_amd import _lib, workloads as W

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    L = _lib.lib()
    I32P, F64P = C.POINTER(C.c_int32), C.POINTER(C.c_double)

    # ---------------- the verify step
    w = W.verify()
    p = W.Params(**{**w.params.as_dict(), "seed": 1234})
    S = klein_amd.Sampler(p, n_vocab=V)
    d = torch.from_numpy(w.logits).cuda()
    # a dedicated stream: torch's default stream has handle 0, which the C ABI reads as "the library's stream"
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    sp = C.c_void_p(stream.cuda_stream)
    assert sp.value, "expected a non-default stream"
    torch.cuda.synchronize()
    rng = np.random.default_rng(5)
    M = 64
    us = np.ascontiguousarray(rng.random((M, 4)), dtype=np.float64)
    drafts = np.ascontiguousarray(w.drafts, dtype=np.int32)
    h = S._h
    dptr = C.c_void_p(d.data_ptr())
    dr_p = drafts.ctypes.data_as(I32P)
    u_ps = [us[i].ctypes.data_as(F64P) for i in range(M)]
    # expected results per uniform set, from untimed launches
    exp_t = np.zeros((M, 4), np.int32)
    exp_a = np.zeros(M, np.int32)
    acc1 = C.c_int32()
    for i in range(M):
        _lib.check(L.kls_verify(h, dptr, 4, dr_p, u_ps[i], exp_t[i].ctypes.data_as(I32P), C.byref(acc1), sp),
                   "kls_verify")
        exp_a[i] = acc1.value
    n_rec = max(a.steps, a.warmup, 1000 if not a.no_extra else 1, 200)
    rec_t = np.zeros((n_rec, 4), np.int32)
    rec_a = np.zeros(n_rec, np.int32)
    rec_tp = [rec_t[i].ctypes.data_as(I32P) for i in range(n_rec)]
    rec_ap = [C.cast(rec_a.ctypes.data + 4 * i, I32P) for i in range(n_rec)]

    # The timed steps run back to back from C (kls_debug_run_verify_steps: one kls_verify per step, as klein's C++
    # generation loop calls the sampler), so no Python call sits between steps; each step's host wall time
    # (enqueue to tokens on the host) comes back per step, and every step's tokens are checked afterwards.
    I64P = C.POINTER(C.c_int64)
    dr_all = np.ascontiguousarray(np.tile(drafts, (n_rec, 1)), dtype=np.int32)
    step_ns = np.zeros(n_rec, np.int64)

    def run_steps(n, first):
        """Steps first .. first+n-1 (uniform set i % M) into rec_t / rec_a [0, n); returns their ns."""
        u_all = np.ascontiguousarray(us[(np.arange(first, first + n)) % M], dtype=np.float64)
        _lib.check(L.kls_debug_run_verify_steps(h, dptr, 4, n, dr_all.ctypes.data_as(I32P), u_all.ctypes.data_as(F64P),
                                                rec_t.ctypes.data_as(I32P), rec_a.ctypes.data_as(I32P),
                                                step_ns.ctypes.data_as(I64P), sp), "kls_debug_run_verify_steps")
        return step_ns[:n].copy()

    def check_steps(n, first):
        for j in range(n):
            i = first + j
            acc = rec_a[j]
            assert acc == exp_a[i % M] and list(rec_t[j][:acc + 1]) == list(exp_t[i % M][:acc + 1]), \
                f"step {i}: tokens differ from the untimed launch"

    run_steps(a.warmup, 0)
    check_steps(a.warmup, 0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ns = run_steps(a.steps, 0)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    us_step = (t1 - t0) / a.steps * 1e6
    check_steps(a.steps, 0)
    per = [x / 1e3 for x in ns]
    lat = {"first_25_us": [round(x, 1) for x in per[:25]], "median_us": round(pct(per, 50), 2),
           "p99_us": round(pct(per, 99), 2), "steps_checked": a.warmup + a.steps,
           "loop": "C (kls_debug_run_verify_steps)"}
    # the same steps called one by one from Python (one ctypes call per step), for comparison
    pc = time.perf_counter_ns
    py = []
    for j in range(200):
        x0 = pc()
        _lib.check(L.kls_verify(h, dptr, 4, dr_p, u_ps[j % M], rec_tp[j], rec_ap[j], sp), "kls_verify")
        py.append((pc() - x0) / 1e3)
    check_steps(200, 0)
    lat["python_loop_200"] = {"median_us": round(pct(py, 50), 2), "mean_us": round(sum(py) / len(py), 2)}

    if not a.no_extra:
        # 1,000 more steps (hot), then 200 with the last-level cache flushed between steps (cold HBM)
        hot = [x / 1e3 for x in run_steps(1000, 0)]
        check_steps(1000, 0)
        flush = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.float32, device="cuda")
        cold = []
        for j in range(200):
            flush.fill_(float(j))
            torch.cuda.synchronize()
            cold.append(run_steps(1, j)[0] / 1e3)
            check_steps(1, j)
        del flush
        lat["hot_1000"] = {"median_us": round(pct(hot, 50), 2), "p99_us": round(pct(hot, 99), 2),
                           "mean_us": round(sum(hot) / len(hot), 2)}
        lat["cold_200"] = {"median_us": round(pct(cold, 50), 2), "p99_us": round(pct(cold, 99), 2),
                           "mean_us": round(sum(cold) / len(cold), 2)}

    # the verify kernel's device time per launch, as the captured step runs it (events on the step's stream)
    kus = C.c_double()
    _lib.check(L.kls_debug_time_verify(h, 100, 10, sp, C.byref(kus)), "kls_debug_time_verify")
    k_mean = kus.value
    achieved = STEP_BYTES / (k_mean * 1e-6) / 1e9
    traffic, tsrc = traffic_from_profile()
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": tsrc,
            "kernel": "rows_kernel<greedy=false, penalize=false, whole-float4, 16 waves, 32 logits/thread>: the "
                      "verify step's kernel, graph-captured arguments, 100 back-to-back copies x 10",
            "kernel_us": round(k_mean, 3), "algorithmic_bytes_per_launch": STEP_BYTES,
            "kernel_source_sha16": kernel_source_hash()}
    S.close()

    out = {"metric": METRIC, "value": round(us_step, 2), "unit": "us", "n_gpus": 1, "steps": a.steps,
           "warmup": a.warmup, "ms_per_step": round(us_step / 1e3, 5), "higher_is_better": False,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": "mtp_verify_step", "rows": 4, "vocab": V, "drafts": 3, "temperature": 0.6,
                      "top_k": 20, "top_p": 0.95, "hipgraph": True, "logits": "resident in HBM",
                      "accept_prefix": "on the device"},
           "latency": lat, "roofline": roof}

    # ---------------- per-request handle cost
    if not a.no_extra:
        cpar = _lib.KlsParams(p.temperature, p.top_k, p.top_p, p.min_p, p.presence_penalty, p.frequency_penalty,
                              p.repetition_penalty, p.seed)
        cr, fv, ds = [], [], []
        tk = np.zeros(4, np.int32)
        for _ in range(20):
            hh = C.c_void_p()
            x0 = pc()
            _lib.check(L.kls_create(C.byref(cpar), V, 4, C.byref(hh)), "kls_create")
            x1 = pc()
            _lib.check(L.kls_verify(hh, dptr, 4, dr_p, u_ps[0], tk.ctypes.data_as(I32P), C.byref(acc1), sp),
                       "kls_verify")
            x2 = pc()
            L.kls_destroy(hh)
            x3 = pc()
            cr.append((x1 - x0) / 1e3)
            fv.append((x2 - x1) / 1e3)
            ds.append((x3 - x2) / 1e3)
        out["handle"] = {"create_us": round(pct(cr, 50), 1), "first_verify_us": round(pct(fv, 50), 1),
                         "destroy_us": round(pct(ds, 50), 1), "note": "medians of 20 (graph capture in the first "
                         "verify; the step's stream was already prepared for graph launches)"}

    # ---------------- 64-row batched stress
    if not a.no_batched:
        wb = W.batched()
        pb = W.Params(**wb.params.as_dict())
        SB = klein_amd.Sampler(pb, n_vocab=V, max_rows=64)
        off = np.zeros(65, np.int32)
        off[1:] = np.cumsum([len(x) for x in wb.histories])
        ids = torch.from_numpy(np.concatenate(wb.histories).astype(np.int32)).cuda()
        offd = torch.from_numpy(off).cuda()
        ud = torch.from_numpy(wb.u).cuda()
        n_sets = 8
        sets = [torch.from_numpy(wb.logits).cuda()]
        for j in range(1, n_sets):
            sets.append(sets[0].roll(j * 997, dims=1).contiguous())
        hb = SB._h
        ptrs = [C.c_void_p(x.data_ptr()) for x in sets]
        offp, idsp, up = C.c_void_p(offd.data_ptr()), C.c_void_p(ids.data_ptr()), C.c_void_p(ud.data_ptr())
        n_b = 400
        outs = torch.full((n_b + 20, 64), -1, dtype=torch.int32, device="cuda")
        outp = [C.c_void_p(outs[i].data_ptr()) for i in range(n_b + 20)]
        # expected tokens per input set, from untimed launches
        expd = torch.full((n_sets, 64), -2, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()  # (inputs and outputs made on torch's stream, used on the bench stream)
        for j in range(n_sets):
            _lib.check(L.kls_sample_batch(hb, ptrs[j], 64, V, offp, idsp, up, C.c_void_p(expd[j].data_ptr()), sp),
                       "kls_sample_batch")

        def batch(ptr, o):
            st = L.kls_sample_batch(hb, ptr, 64, V, offp, idsp, up, o, sp)
            if st:
                _lib.check(st, "kls_sample_batch")

        res = {}
        for mode in ("hot", "cold"):
            pick = (lambda i: 0) if mode == "hot" else (lambda i: i % n_sets)
            for i in range(20):
                batch(ptrs[pick(i)], outp[n_b + i])
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for i in range(n_b):
                batch(ptrs[pick(i)], outp[i])
            e1.record(stream)
            torch.cuda.synchronize()
            res[mode] = e0.elapsed_time(e1) * 1e3 / n_b
            want = torch.stack([expd[pick(i)] for i in range(n_b + 20)])
            assert torch.equal(outs, want), f"batched ({mode}): a launch's tokens differ from the untimed launch"
            SB.check()
        out["batched"] = {"workload": "64 rows x 248,320, 16,384-id histories, penalties, top-k 64, top-p 0.9",
                          "algorithmic_bytes": BATCH_BYTES,
                          "us_hot": round(res["hot"], 2), "us_cold": round(res["cold"], 2),
                          "GBps_cold": round(BATCH_BYTES / (res["cold"] * 1e-6) / 1e9, 1),
                          "frac_cold": round(BATCH_BYTES / (res["cold"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                          "GBps_hot": round(BATCH_BYTES / (res["hot"] * 1e-6) / 1e9, 1),
                          "launches_checked": 2 * (n_b + 20)}
        SB.close()
        del sets, outs

    # ---------------- the next rows of the path: draft argmax, ppl scoring, rollback
    if not a.no_next:
        out["next_rows"] = next_rows(torch, klein_amd, W)
    if not a.no_extra:
        out["topk_above_64"] = topk_above_64(torch, klein_amd, W)

    out["copy_probe"] = copy_probe(torch, stream)
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(W, a.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
