#!/usr/bin/env python
"""Benchmark: µs per 4-row MTP verify sampling step at V = 248,320 on one MI355X.

Workload (one step): 4 rows x 248,320 f32 logits already resident in HBM (1 main + 3 draft positions, each row
N(0,1.5) plus 50 head ids at N(8,2)), 3 drafts, temperature 0.6, top-k 20, top-p 0.95, per-row uniforms; each
row is sampled and the accepted-prefix length computed, as klein's verify loop (src/engine.cpp:563-575) with
src/sampler.cpp per row. A step is one kls_verify call: one hipGraph launch, results read back through pinned
memory. `value` is the host wall-clock time per step (launch to results on the host).

Also reported:
  roofline      the fused kernel's device time per launch (one stream-event pair around back-to-back launches
                over the same 4 rows) and the HBM rate of its algorithmic bytes (every logit read once:
                4 x 993,280 B + drafts and uniforms);
  batched       64 independent rows x 248,320 with per-row 16,384-id Zipf histories, penalties (repetition 1.1,
                presence 0.5, frequency 0.2), top-k 64, top-p 0.9: device time per batch (history partition +
                sampling kernels, back-to-back launches), hot (same input every launch) and cold (8 input sets
                rotated, 509 MB, more than the 256 MB last-level cache);
  next_rows     the MTP draft argmax (Engine::mtp_draft_token, 1 row x 248,320: std::max_element) per call, and
                one pass of the perplexity / KL loop (src/main.cpp:308-327: 64 rows x 248,320 logits plus base
                log-probabilities) per pass, cold (4 input sets rotated), with their HBM rates (device time
                of launches captured back to back in one graph);
  cpu_baseline  the reference's own sampler.cpp (oracle/_ref, built -O3 from its sources) on one host core,
                4 rows per step, over a bounded sample.
"""
import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "µs per 4-row MTP verify sampling step @V=248,320; achieved HBM GB/s"
HBM_PEAK_GBS = 8000.0
V = 248_320
STEP_BYTES = 4 * V * 4 + 3 * 4 + 4 * 8          # logits + drafts + uniforms = 3,973,164
BATCH_BYTES = 64 * (V * 4 + 16384 * 4)           # logits + raw history ids = 67,764,224


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batched", action="store_true")
    ap.add_argument("--no-next", action="store_true", help="skip the draft-argmax and ppl measurements")
    return ap.parse_args()


def traffic_from_profiles():
    """HBM bytes per launch of the verify kernel from the committed rocprofv3 PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", "traffic_verify_4x248320.json")
    if os.path.exists(path):
        try:
            return json.load(open(path)).get("hbm_bytes_per_launch")
        except Exception:
            return None
    return None


def copy_probe(torch, stream):
    """A plain device copy of 256 MiB (torch's copy kernel): its measured rate, and the reference size that the
    HBM byte counters of the same run are calibrated against."""
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
    import ctypes as C
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
    import ctypes as C
    import numpy as np
    from klein_amd import _lib
    L = _lib.lib()
    rng = np.random.default_rng(77)
    res = {}
    S = klein_amd.Sampler(W.Params(temperature=0.0), n_vocab=V, max_rows=64)
    h = S._h
    p = lambda t: C.c_void_p(t.data_ptr())
    # draft argmax: one MTP row (the greedy workload's logits), as called once per draft
    g = W.greedy()
    d1 = torch.from_numpy(g.logits).cuda()
    o1 = torch.zeros(1, dtype=torch.int32, device="cuda")
    us = graph_us(torch, lambda sp: _lib.check(L.kls_argmax(h, p(d1), 1, V, p(o1), sp), "kls_argmax"), 200)
    assert int(o1.item()) == g.expected_greedy
    res["draft_argmax"] = {"workload": "1 row x 248,320 f32 (std::max_element)", "us": round(us, 2),
                           "GBps": round(V * 4 / (us * 1e-6) / 1e9, 1)}
    # ppl: the loop's default pass of 64 rows with a KL base, 4 input sets (254 MB each way) rotated
    sets = []
    for j in range(4):
        x = torch.randn((64, V), device="cuda", dtype=torch.float32) * 2.0
        b = torch.log_softmax(torch.randn((64, V), device="cuda", dtype=torch.float32) * 3.0, dim=1)
        sets.append((x, b))
    tg = torch.from_numpy(rng.integers(0, V, 64).astype(np.int32)).cuda()
    outs = [torch.empty(64, dtype=torch.float64, device="cuda") for _ in range(4)]
    tops = [torch.empty(64, dtype=torch.int32, device="cuda") for _ in range(2)]
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
    S.close()
    return res


def cpu_baseline(w, seconds):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle
    logits = np.ascontiguousarray(w.logits, dtype=np.float32)
    fp = logits.ctypes.data_as(C.POINTER(C.c_float))
    sink = C.c_int32()
    if oracle.ref_available():
        s = oracle.RefSampler(w.params)
        L = oracle.ref()
        run = lambda reps: L.ref_time_rows(s._h, fp, V, 4, reps, C.byref(sink))  # noqa: E731
        kind, what = "reference", "klein src/sampler.cpp built -O3 -DNDEBUG from its sources (oracle/_ref)"
    else:
        L = oracle.lib()
        ps = oracle.params_struct(w.params)
        run = lambda reps: L.orc_time_rows(fp, V, 4, C.byref(ps), None, reps, C.byref(sink))  # noqa: E731
        kind, what = "port", "oracle restatement of src/sampler.cpp (reference build absent)"
    run(8)  # warm
    t = run(8)
    per_row = t / 8
    reps = max(8, int(seconds / per_row) // 4 * 4)
    t = run(reps)
    us_step = t / reps * 4 * 1e6
    return {"value": round(us_step, 1), "unit": "us", "cores": 1, "kind": kind,
            "sample": f"{reps // 4} steps x 4 rows x 248,320 f32 (the verify workload), sample() per row as "
                      f"engine.cpp:566, {t:.1f} s on 1 host thread; {what}"}


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

    # ---------------- the verify step
    w = W.verify()
    p = W.Params(**{**w.params.as_dict(), "seed": 1234})
    S = klein_amd.Sampler(p, n_vocab=V)
    d = torch.from_numpy(w.logits).cuda()
    # a dedicated stream: torch's default stream has handle 0, which the C ABI reads as "the handle's own stream"
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    sp = C.c_void_p(stream.cuda_stream)
    assert sp.value, "expected a non-default stream"
    torch.cuda.synchronize()
    rng = np.random.default_rng(5)
    M = 64
    us = np.ascontiguousarray(rng.random((M, 4)), dtype=np.float64)
    drafts = np.ascontiguousarray(w.drafts, dtype=np.int32)
    toks = np.zeros(4, dtype=np.int32)
    acc = C.c_int32()
    h = S._h
    dptr = C.c_void_p(d.data_ptr())
    dr_p = drafts.ctypes.data_as(C.POINTER(C.c_int32))
    u_ps = [us[i].ctypes.data_as(C.POINTER(C.c_double)) for i in range(M)]
    tk_p = toks.ctypes.data_as(C.POINTER(C.c_int32))
    accp = C.byref(acc)

    def step(i):
        st = L.kls_verify(h, dptr, 4, dr_p, u_ps[i % M], tk_p, accp, sp)
        if st:
            _lib.check(st, "kls_verify")

    for i in range(a.warmup):
        step(i)
    torch.cuda.synchronize()
    ts = [0] * (a.steps + 1)
    pc = time.perf_counter_ns
    t0 = time.perf_counter()
    ts[0] = pc()
    for i in range(a.steps):
        step(i)
        ts[i + 1] = pc()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    us_step = (t1 - t0) / a.steps * 1e6
    per = [(ts[i + 1] - ts[i]) / 1e3 for i in range(a.steps)]
    srt = sorted(per)
    lat = {"first_25_us": [round(x, 1) for x in per[:25]], "median_us": round(srt[len(srt) // 2], 2),
           "p99_us": round(srt[min(len(srt) - 1, (len(srt) * 99) // 100)], 2)}

    # kernel device time per launch: the same fused kernel over the same 4 rows, launched back to back on the
    # stream (device-resident uniforms, no host round trip between launches), one event pair around n launches
    ud4 = torch.from_numpy(us[:1].reshape(-1).copy()).cuda()
    out4 = torch.zeros(4, dtype=torch.int32, device="cuda")
    SK = klein_amd.Sampler(p, n_vocab=V, max_rows=4)
    hk, u4p, o4p = SK._h, C.c_void_p(ud4.data_ptr()), C.c_void_p(out4.data_ptr())

    def kstep():
        st = L.kls_sample_batch(hk, dptr, 4, V, None, None, u4p, o4p, sp)
        if st:
            _lib.check(st, "kls_sample_batch")

    for _ in range(50):
        kstep()
    n_k = max(a.steps, 200)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(n_k):
        kstep()
    e1.record(stream)
    torch.cuda.synchronize()
    k_mean = e0.elapsed_time(e1) * 1e3 / n_k
    achieved = STEP_BYTES / (k_mean * 1e-6) / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
            "kernel": "rows_kernel<greedy=false, penalize=false> over the 4 verify rows",
            "kernel_us": round(k_mean, 3), "launches_timed": n_k,
            "algorithmic_bytes_per_launch": STEP_BYTES}
    SK.close()
    S.close()

    out = {"metric": METRIC, "value": round(us_step, 2), "unit": "us", "n_gpus": 1, "steps": a.steps,
           "warmup": a.warmup, "ms_per_step": round(us_step / 1e3, 5), "higher_is_better": False,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": "mtp_verify_step", "rows": 4, "vocab": V, "drafts": 3, "temperature": 0.6,
                      "top_k": 20, "top_p": 0.95, "hipgraph": True, "logits": "resident in HBM"},
           "latency": lat, "roofline": roof}

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
        outd = torch.zeros(64, dtype=torch.int32, device="cuda")
        n_sets = 8
        sets = [torch.from_numpy(wb.logits).cuda()]
        for j in range(1, n_sets):
            sets.append(sets[0].roll(j * 997, dims=1).contiguous())
        hb = SB._h
        ptrs = [C.c_void_p(x.data_ptr()) for x in sets]
        offp, idsp, up, outp = (C.c_void_p(offd.data_ptr()), C.c_void_p(ids.data_ptr()),
                                C.c_void_p(ud.data_ptr()), C.c_void_p(outd.data_ptr()))

        def batch(ptr):
            st = L.kls_sample_batch(hb, ptr, 64, V, offp, idsp, up, outp, sp)
            if st:
                _lib.check(st, "kls_sample_batch")

        res = {}
        for mode in ("hot", "cold"):
            for i in range(20):
                batch(ptrs[0] if mode == "hot" else ptrs[i % n_sets])
            n_b = 400
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for i in range(n_b):
                batch(ptrs[0] if mode == "hot" else ptrs[i % n_sets])
            e1.record(stream)
            torch.cuda.synchronize()
            res[mode] = e0.elapsed_time(e1) * 1e3 / n_b
        out["batched"] = {"workload": "64 rows x 248,320, 16,384-id histories, penalties, top-k 64, top-p 0.9",
                          "algorithmic_bytes": BATCH_BYTES,
                          "us_hot": round(res["hot"], 2), "us_cold": round(res["cold"], 2),
                          "GBps_cold": round(BATCH_BYTES / (res["cold"] * 1e-6) / 1e9, 1),
                          "frac_cold": round(BATCH_BYTES / (res["cold"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                          "GBps_hot": round(BATCH_BYTES / (res["hot"] * 1e-6) / 1e9, 1)}
        SB.close()

    # ---------------- the next rows of the path: draft argmax, ppl scoring
    if not a.no_next:
        out["next_rows"] = next_rows(torch, klein_amd, W)

    out["copy_probe"] = copy_probe(torch, stream)
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(w, a.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
