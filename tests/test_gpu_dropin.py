"""The C++ drop-in klein::Sampler (klein_amd/csrc/sampler.{h,cpp}, the interface of klein's src/sampler.h:13-38)
on the GPU against the reference's own Sampler (src/sampler.cpp compiled into oracle/_ref): tests/cpp/dropin_check
drives the drop-in through sample()/accept() and 4-row verify() steps with a fixed seed and records the logits,
drafts and tokens; the reference replays each scenario with the same seed (the same mt19937_64 draws) through
sample()/accept() and the engine's verify loop (src/engine.cpp:563-575). Tokens and accepted counts must match
exactly. Scenarios: the verify configuration, penalties with min-p, greedy with a presence penalty, no top-k
limit (the wide path), and top-k 300 with min-p and penalties (the mid path)."""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "dropin_check")

pytestmark = pytest.mark.gpu


def parse(txt):
    lines = open(txt).read().split("\n")
    head = lines[0].split()
    assert head[0] == "params"
    t, k, tp, mp, pres, freq, rep, seed = head[1:9]
    V = int(head[10])
    params = dict(temperature=float(t), top_k=int(k), top_p=float(tp), min_p=float(mp), presence_penalty=float(pres),
                  frequency_penalty=float(freq), repetition_penalty=float(rep), seed=int(seed))
    steps = []
    for ln in lines[1:]:
        f = ln.split()
        if not f:
            continue
        if f[0] == "sample":
            steps.append(("sample", int(f[1])))
        else:
            drafts = [int(x) for x in f[1:4]]
            acc = int(f[6])
            toks = [int(x) for x in f[7:]]
            steps.append(("verify", drafts, acc, toks))
    return params, V, steps


def test_cpp_dropin_matches_reference(tmp_path):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    if not oracle.ref_available():
        pytest.skip("the reference build (oracle/_ref) is not present")
    assert os.path.exists(EXE), "tests/cpp/dropin_check is built by __graft_entry__.build()"
    print("[case] dropin_check", flush=True)
    r = subprocess.run([EXE, str(tmp_path)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    n = 0
    while os.path.exists(tmp_path / f"scenario_{n}.txt"):
        params, V, steps = parse(tmp_path / f"scenario_{n}.txt")
        logits = np.fromfile(tmp_path / f"scenario_{n}.bin", dtype=np.float32)
        R = oracle.RefSampler(params)
        at = 0
        for s, st in enumerate(steps):
            if st[0] == "sample":
                row = logits[at:at + V]
                at += V
                t = R.sample(row)
                R.accept(t)
                assert st[1] == t, (n, s, st[1], t)
            else:
                rows = logits[at:at + 4 * V].reshape(4, V)
                at += 4 * V
                toks, acc = R.verify(rows, np.array(st[1], np.int32))
                assert st[2] == acc and st[3] == list(toks[:acc + 1]), (n, s, st, list(toks), acc)
        assert at == logits.size
        n += 1
    assert n == 5
