"""GPU parity of the MTP draft argmax (kls_argmax, Engine::mtp_draft_token at src/engine.cpp:413-415:
std::max_element over each row): indices bit-exact against the oracle, which calls std::max_element itself,
on the greedy workload, draft-sized batches, every segment length, NaN / infinity placements and strided rows."""
import numpy as np
import pytest

from klein_amd import workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    torch.cuda.init()
    return torch


@pytest.fixture(scope="module")
def K():
    import klein_amd
    return klein_amd


def run(torch, K, x, stride=None, max_rows=None, seg=None):
    """kls_argmax over the rows of x (optionally inside a wider row pitch); returns the indices."""
    rows, V = x.shape
    pitch = stride or V
    buf = np.full((rows, pitch), np.float32(7e37), np.float32)  # (the pitch padding is never read)
    buf[:, :V] = x
    d = torch.from_numpy(buf).cuda()
    S = K.Sampler(W.Params(temperature=0.0), n_vocab=V, max_rows=max_rows or rows,
                  layout=dict(seg_len=seg) if seg else None)
    out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    S.argmax(d[:, :V], out)
    torch.cuda.synchronize()
    S.close()
    return out.cpu().numpy()


def expect(O, x):
    return np.array([O.argmax(r) for r in x], dtype=np.int32)


def test_greedy_workload_row(torch_cuda, K, oracle_lib):
    w = W.greedy()
    x = w.logits.reshape(1, -1)
    say("greedy workload, planted max and ties", x.shape)
    got = run(torch_cuda, K, x)
    assert got.tolist() == expect(oracle_lib, x).tolist()


@pytest.mark.parametrize("rows", [1, 2, 3])
def test_draft_rows_with_ties(torch_cuda, K, oracle_lib, rows):
    rng = np.random.default_rng(100 + rows)
    V = W.VOCAB
    x = rng.standard_normal((rows, V)).astype(np.float32)
    for r in range(rows):
        at = rng.choice(V, 6, replace=False)
        x[r, at] = x[r].max() + np.float32(1.0)  # six-way tie for the maximum
    say("draft rows with ties", rows)
    got = run(torch_cuda, K, x)
    assert got.tolist() == expect(oracle_lib, x).tolist()


@pytest.mark.parametrize("seg", [1024, 4096, 8192, 16384, 65536])
def test_segment_lengths(torch_cuda, K, oracle_lib, seg):
    rng = np.random.default_rng(seg)
    V = W.VOCAB
    x = rng.standard_normal((3, V)).astype(np.float32)
    x[0, V - 1] = 50.0                     # the last id (the shifted last segment)
    x[1, [seg - 1, seg, 3 * seg + 5]] = 50.0  # a tie across a segment boundary: the first wins
    x[2, 0] = 50.0                         # the first id
    say("segment length", seg)
    got = run(torch_cuda, K, x, seg=seg)
    assert got.tolist() == expect(oracle_lib, x).tolist()


def test_nan_and_infinity_placements(torch_cuda, K, oracle_lib):
    rng = np.random.default_rng(7)
    V = 50000
    x = rng.standard_normal((8, V)).astype(np.float32)
    x[0, 0] = np.nan                               # NaN first: the result is 0
    x[1, rng.choice(V, 500, replace=False)] = np.nan  # scattered NaNs are skipped
    x[2, :] = -np.inf                              # nothing beats the first element
    x[3, :] = -np.inf
    x[3, rng.choice(V, 50, replace=False)] = np.nan   # -inf and NaN only
    x[4, [123, 40000]] = np.inf                    # +inf twice: the first
    x[5, :] = np.nan
    x[5, 0] = 1.0                                  # one number first, NaN elsewhere
    x[6, :] = np.float32(2.0)                      # all equal
    x[7, 0] = np.nan
    x[7, 17] = np.inf                              # NaN first wins even over +inf
    say("NaN / inf placements", x.shape)
    got = run(torch_cuda, K, x)
    assert got.tolist() == expect(oracle_lib, x).tolist()
    assert got[0] == 0 and got[7] == 0 and got[4] == 123


def test_small_and_odd_vocabularies_strided(torch_cuda, K, oracle_lib):
    rng = np.random.default_rng(9)
    for V in (1, 3, 5, 1000, 4097, 65537, 100003):
        x = rng.integers(-5, 5, (3, V)).astype(np.float32)  # many exact ties
        say("vocabulary", V, "strided")
        got = run(torch_cuda, K, x, stride=V + 13, max_rows=4)
        assert got.tolist() == expect(oracle_lib, x).tolist(), V


def test_argument_errors(torch_cuda, K):
    import klein_amd._lib as L
    S = K.Sampler(W.Params(temperature=0.0), n_vocab=1000, max_rows=2)
    d = torch_cuda.zeros((3, 1000), dtype=torch_cuda.float32, device="cuda")
    out = torch_cuda.zeros(3, dtype=torch_cuda.int32, device="cuda")
    with pytest.raises(L.KlsError):
        S.argmax(d, out)  # more rows than the handle's capacity
    S.close()
