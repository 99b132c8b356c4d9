"""Writes the golden fixtures tests/golden/*.json from the reference's own sampler (src/sampler.cpp compiled from
its sources into oracle/_ref by oracle/Makefile) on the seeded workloads of klein_amd.workloads.

Each fixture holds the workload seed, the sha256 of the generated logits (guarding the generator), the sampling
parameters, and per case: the sampler seed, the uniform its first draw yields, and the reference's token (or,
for the verify step, its tokens and accepted count). Top-k ids, probabilities and the kept count come from the
oracle restatement in std::partial_sort mode, whose tokens must equal the reference's for the case to be written.

Run in a container that has /root/reference:  make -C oracle && python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle")]

import oracle as O  # noqa: E402
from klein_amd import workloads as W  # noqa: E402

SEEDS = [11, 22, 33, 44]


def single(name):
    w = W.BUILDERS[name]()
    cases = []
    rows = range(w.rows) if name == "batched" else [0]
    for r in rows:
        for seed in (SEEDS if name != "batched" else SEEDS[:1]):
            p = W.Params(**{**w.params.as_dict(), "seed": seed})
            ref = O.RefSampler(p)
            hist = w.histories[r] if w.histories else np.zeros(0, np.int32)
            for t in hist:
                ref.accept(int(t))
            tok = ref.sample(w.logits[r])
            u = float(O.uniforms(seed, 1)[0]) if p.temperature > 0 else 0.0
            counts = W.counts_of(hist, w.vocab) if len(hist) else None
            t, ids, probs, kept = O.sample(w.logits[r], p, u, counts, O.MODE_STDLIB)
            assert t == tok, (name, r, seed)
            cases.append(dict(row=r, seed=seed, u=u, token=tok, topk_ids=[int(i) for i in ids],
                              topk_probs=[float(x) for x in probs], kept=kept))
    return w, cases


def verify():
    w = W.BUILDERS["verify"]()
    cases = []
    for seed in SEEDS:
        p = W.Params(**{**w.params.as_dict(), "seed": seed})
        u = [float(x) for x in O.uniforms(seed, w.rows)]
        # the workload's drafts, then drafts forced to match the first 1, 2 and 3 sampled tokens
        base_toks, _ = O.RefSampler(p).verify(w.logits, w.drafts)
        full, _, _ = O.verify(w.logits, np.array([0, 0, 0], np.int32), p, np.array(u), None, O.MODE_STDLIB)
        variants = [w.drafts.copy()]
        for m in (1, 2, 3):
            # tokens of rows 0..m-1 when all earlier drafts match (no penalties: rows are independent)
            d = w.drafts.copy()
            for i in range(m):
                d[i] = O.sample(w.logits[i], p, u[i], None, O.MODE_STDLIB)[0]
            variants.append(d)
        for d in variants:
            rt, ra = O.RefSampler(p).verify(w.logits, d)
            ot, oa, _ = O.verify(w.logits, d, p, np.array(u), None, O.MODE_STDLIB)
            assert oa == ra and list(ot[:oa + 1]) == list(rt[:ra + 1])
            cases.append(dict(row=0, seed=seed, u=u, drafts=[int(x) for x in d], tokens=[int(x) for x in rt],
                              accepted=ra))
    return w, cases


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libklein_ref.so is missing (needs /root/reference; run make -C oracle)")
    for name in ["greedy", "topk_topp", "penalties", "verify", "batched"]:
        w, cases = verify() if name == "verify" else single(name)
        fx = dict(workload=name, seed=w_seed(name), vocab=w.vocab, rows=w.rows, logits_sha256=w.digest(),
                  params={k: v for k, v in w.params.as_dict().items() if k != "seed"}, cases=cases)
        with open(os.path.join(HERE, f"{name}.json"), "w") as f:
            json.dump(fx, f, indent=1)
        print(name, len(cases), "cases")


def w_seed(name):
    import inspect
    return inspect.signature(W.BUILDERS[name]).parameters["seed"].default


if __name__ == "__main__":
    main()
