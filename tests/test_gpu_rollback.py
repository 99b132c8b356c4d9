"""GPU parity of the verify step's consumer, the recurrent-state rollback (src/engine.cpp:578-583,
src/state.cpp:162-184), through the C ABI: kls_rollback_recurrent against the oracle's restatement on synthetic
state buffers, bit for bit, for every rollback depth s = 0..nb-1 (accepted = nb-1..0), each snapshot type (f32,
f16, bf16), the vector path (rows multiples of 4, 16-byte aligned, with and without padding) and the element path (odd rows, padded strides), at a
27B-class layout (48 layers, conv rows of 30,720 f32, ssm rows of 786,432), and chained after a real verify step
on the same stream with the accepted count read from device memory."""
import ctypes as C

import numpy as np
import pytest

from klein_amd import _lib
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


def finite_bits(rng, n, snap_type):
    """Random 16-bit patterns of finite f16 / bf16 values (subnormals and both zeros included)."""
    u = rng.integers(0, 65536, n).astype(np.uint16)
    if snap_type == _lib.KLS_SNAP_F16:
        bad = (u & 0x7C00) == 0x7C00
    else:
        bad = (u & 0x7F80) == 0x7F80
    u[bad] &= 0x83FF if snap_type == _lib.KLS_SNAP_F16 else 0x807F
    return u


class State:
    """Host copies and device tensors of n_layers layers (conv [n_snap, conv_pitch] f32, ssm [ssm_row] f32,
    snap [n_snap - 1, snap_pitch] of the snapshot type, as int16 bit patterns for 16-bit types)."""

    def __init__(self, torch, rng, n_layers, n_snap, conv_row, ssm_row, snap_type, pad=0):
        self.n_layers, self.n_snap, self.conv_row, self.ssm_row, self.snap_type = n_layers, n_snap, conv_row, ssm_row, snap_type
        self.conv_h, self.ssm_h, self.snap_h = [], [], []
        self.conv_d, self.ssm_d, self.snap_d = [], [], []
        for _ in range(n_layers):
            c = rng.standard_normal((n_snap, conv_row + pad)).astype(np.float32)
            m = rng.standard_normal(ssm_row).astype(np.float32)
            if snap_type == _lib.KLS_SNAP_F32:
                sn = rng.standard_normal((n_snap - 1, ssm_row + pad)).astype(np.float32)
                sd = torch.from_numpy(sn).cuda()
            else:
                sn = finite_bits(rng, (n_snap - 1) * (ssm_row + pad), snap_type).reshape(n_snap - 1, ssm_row + pad)
                sd = torch.from_numpy(sn.view(np.int16)).cuda()
            self.conv_h.append(c)
            self.ssm_h.append(m)
            self.snap_h.append(sn)
            self.conv_d.append(torch.from_numpy(c).cuda())
            self.ssm_d.append(torch.from_numpy(m).cuda())
            self.snap_d.append(sd)
        esz = 4 if snap_type == _lib.KLS_SNAP_F32 else 2
        P = C.c_void_p * n_layers
        self._arrs = (P(*[t.data_ptr() for t in self.conv_d]), P(*[t.data_ptr() for t in self.ssm_d]),
                      P(*[t.data_ptr() for t in self.snap_d]))
        self.desc = _lib.KlsRecurrentDesc(n_layers, n_snap, conv_row, ssm_row, 4 * (conv_row + pad),
                                          esz * (ssm_row + pad), snap_type,
                                          C.cast(self._arrs[0], C.POINTER(C.c_void_p)),
                                          C.cast(self._arrs[1], C.POINTER(C.c_void_p)),
                                          C.cast(self._arrs[2], C.POINTER(C.c_void_p)))
        h = C.c_void_p()
        _lib.check(_lib.lib().kls_recurrent_create(C.byref(self.desc), C.byref(h)), "kls_recurrent_create")
        self.h = h

    def close(self):
        _lib.lib().kls_recurrent_destroy(self.h)

    def check(self, O, accepted, nb, layers=None):
        for l in (layers if layers is not None else range(self.n_layers)):
            snap = self.snap_h[l][:, :self.ssm_row]
            conv_w, ssm_w = O.rollback_recurrent(self.conv_h[l][:, :self.conv_row], self.ssm_h[l], snap,
                                                 self.snap_type, accepted, nb)
            conv_g = self.conv_d[l].cpu().numpy()
            ssm_g = self.ssm_d[l].cpu().numpy()
            assert np.array_equal(conv_g[:, :self.conv_row].view(np.uint32), conv_w.view(np.uint32)), (l, accepted)
            assert np.array_equal(conv_g[:, self.conv_row:], self.conv_h[l][:, self.conv_row:]), l  # padding untouched
            assert np.array_equal(ssm_g.view(np.uint32), ssm_w.view(np.uint32)), (l, accepted)
            sg = self.snap_d[l].cpu().numpy()
            assert np.array_equal(sg.view(self.snap_h[l].dtype), self.snap_h[l]), l  # snapshots untouched


def rollback(torch, st, d_acc_ptr, nb, stream=None):
    _lib.check(_lib.lib().kls_rollback_recurrent(st.h, C.c_void_p(d_acc_ptr), nb,
                                                 None if stream is None else C.c_void_p(stream.cuda_stream)),
               "kls_rollback_recurrent")
    torch.cuda.synchronize()


SHAPES = [
    # layers, conv_row, ssm_row, pad (elements of padding in each stride)
    (3, 64, 4096, 0),      # vector path
    (2, 36, 1004, 4),      # vector path: rows multiples of 4 (not 8), padded 16-byte strides
    (2, 30, 1001, 3),      # element path: odd rows, padded strides
]


@pytest.mark.parametrize("snap_type", [_lib.KLS_SNAP_F32, _lib.KLS_SNAP_F16, _lib.KLS_SNAP_BF16])
@pytest.mark.parametrize("shape", SHAPES)
def test_rollback_every_depth(torch_cuda, oracle_lib, snap_type, shape):
    torch, O = torch_cuda, oracle_lib
    n_layers, conv_row, ssm_row, pad = shape
    nb = 4
    for acc in range(nb):
        rng = np.random.default_rng(100 * acc + snap_type)
        st = State(torch, rng, n_layers, nb, conv_row, ssm_row, snap_type, pad)
        d_acc = torch.tensor([acc], dtype=torch.int32, device="cuda")
        say("rollback", snap_type, shape, "accepted", acc)
        rollback(torch, st, d_acc.data_ptr(), nb)
        st.check(O, acc, nb)
        st.close()


def test_rollback_out_of_range_accepted_moves_nothing(torch_cuda, oracle_lib):
    torch, O = torch_cuda, oracle_lib
    st = State(torch, np.random.default_rng(5), 2, 4, 64, 512, _lib.KLS_SNAP_F16)
    for bad in (-1, 4, 1 << 30):
        d_acc = torch.tensor([bad], dtype=torch.int32, device="cuda")
        say("accepted", bad)
        rollback(torch, st, d_acc.data_ptr(), 4)
        st.check(O, 3, 4)  # (accepted = nb - 1: no rollback)
    assert _lib.lib().kls_rollback_recurrent(st.h, C.c_void_p(d_acc.data_ptr()), 5, None) == _lib.KLS_ERR_RANGE
    st.close()


def test_rollback_27b_class_layout(torch_cuda, oracle_lib):
    """48 DeltaNet layers of a 27B-class model (conv rows (4 - 1) x 10,240 channels, ssm rows 128 x 128 x 48),
    f16 snapshots, 3 drafts: every depth on the same state, checked on every layer."""
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(27)
    st = State(torch, rng, 48, 4, 30720, 786432, _lib.KLS_SNAP_F16)
    d_acc = torch.tensor([1], dtype=torch.int32, device="cuda")
    say("27B-class layout, accepted 1")
    rollback(torch, st, d_acc.data_ptr(), 4)
    st.check(O, 1, 4)
    st.close()


def test_rollback_after_verify_step(torch_cuda, K_mod, oracle_lib):
    """An engine step: verify enqueued, the rollback enqueued behind it on the same stream with the handle's
    device-resident accepted count, then the host waits for the tokens; the state matches the oracle's rollback
    for the accepted count the oracle's verify loop gives."""
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(31)
    V = 248320
    p = W.Params(temperature=0.6, top_k=20, top_p=0.95, seed=6)
    x, _ = W._head_rows(rng, 4, V)
    d = torch.from_numpy(x).cuda()
    S = K_mod.Sampler(p, n_vocab=V)
    _, d_accepted = S.device_results()
    L = _lib.lib()
    stream = torch.cuda.Stream()
    I32, F64 = C.POINTER(C.c_int32), C.POINTER(C.c_double)
    for m in range(4):
        u = rng.random(4)
        drafts = rng.integers(0, V, 3).astype(np.int32)
        for i in range(m):
            drafts[i] = O.sample(x[i], p, u[i])[0]
        st = State(torch, np.random.default_rng(m), 4, 4, 64, 2048, _lib.KLS_SNAP_BF16)
        torch.cuda.synchronize()
        say("verify + rollback, m", m)
        _lib.check(L.kls_verify_enqueue(S._h, C.c_void_p(d.data_ptr()), 4, drafts.ctypes.data_as(I32),
                                        np.ascontiguousarray(u).ctypes.data_as(F64), C.c_void_p(stream.cuda_stream)),
                   "kls_verify_enqueue")
        _lib.check(L.kls_rollback_recurrent(st.h, C.c_void_p(d_accepted), 4, C.c_void_p(stream.cuda_stream)),
                   "kls_rollback_recurrent")
        toks = np.zeros(4, np.int32)
        acc = C.c_int32()
        _lib.check(L.kls_verify_wait(S._h, toks.ctypes.data_as(I32), C.byref(acc)), "kls_verify_wait")
        torch.cuda.synchronize()
        ot, oa, _ = O.verify(x, drafts, p, u)
        assert acc.value == oa and acc.value >= m
        st.check(O, oa, 4)
        st.close()
    S.close()


@pytest.fixture(scope="module")
def K_mod():
    import klein_amd
    return klein_amd
