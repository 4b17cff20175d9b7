"""jhq_k_assign_noalloc: the IVF assignment of jhq_k_assign (argmin
||c||^2 - 2<c,y>, ties to the lowest list; v14/jhq_gpu_index.cu:23-40,367-393)
with its key buffer in a file-scope device array instead of an allocation.
Checked against jhq_k_assign and the oracle on two calls in a row, the second
with fewer rows, so keys left by the first call must not leak into it."""
import ctypes

import numpy as np
import pytest

import pyoracle as po

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu

_VP, _I64, _I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
MAX_ROWS = 1 << 20


def _noalloc():
    return jg.lib().jhq_k_assign_noalloc


def test_assign_noalloc_matches_assign(gpu):
    import torch
    rng = np.random.default_rng(2024)
    d, nlist = 64, 300
    cent = rng.standard_normal((nlist, d)).astype(np.float32)
    cent[17] = cent[5]    # exact ties: the lower list must win
    cent[250] = cent[5]
    norms = po.cent_norms(cent)
    tc, tn = torch.from_numpy(cent).to(gpu), torch.from_numpy(norms).to(gpu)
    s = torch.cuda.current_stream()
    for n in (20_000, 1_234):  # the second call is smaller
        y = rng.standard_normal((n, d)).astype(np.float32)
        y[:50] = cent[5] + np.float32(1e-3) * y[:50]  # rows next to the tied centroids
        ty = torch.from_numpy(y).to(gpu)
        a_ref = torch.full((n,), -7, dtype=torch.int32, device=gpu)
        a_new = torch.full((n,), -7, dtype=torch.int32, device=gpu)
        jg.k_assign(ty, tc, tn, a_ref, stream=s)
        jg.k_assign_noalloc(ty, tc, tn, a_new, stream=s)
        torch.cuda.synchronize()
        got, want = a_new.cpu().numpy(), a_ref.cpu().numpy()
        assert np.array_equal(got, want), n
        assert np.array_equal(got, po.assign(y, cent, norms)), n
        assert not np.isin(got[:50], [17, 250]).any()


def test_assign_noalloc_rejects_oversize(gpu):
    import torch
    t = torch.zeros(16, dtype=torch.float32, device=gpu)
    i = torch.zeros(16, dtype=torch.int32, device=gpu)
    f = _noalloc()
    # rejected on the host before anything is launched
    rc = f(_VP(t.data_ptr()), MAX_ROWS + 1, 4, _VP(t.data_ptr()), _VP(t.data_ptr()), 2,
           _VP(i.data_ptr()), None)
    assert rc == jg.JHQ_EINVAL
    assert "at most" in jg.lib().jhq_last_error().decode()


def test_assign_noalloc_two_streams_ordered(gpu):
    """Calls on two streams with no host synchronisation between them: the
    second call's stream waits for the first call's kernels on the device, so
    neither reads keys the other wrote."""
    import torch
    rng = np.random.default_rng(77)
    d, nlist = 32, 200
    cent = rng.standard_normal((nlist, d)).astype(np.float32)
    norms = po.cent_norms(cent)
    tc, tn = torch.from_numpy(cent).to(gpu), torch.from_numpy(norms).to(gpu)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    ys = [rng.standard_normal((n, d)).astype(np.float32) for n in (300_000, 200_000, 250_000)]
    ty = [torch.from_numpy(y).to(gpu) for y in ys]
    outs = [torch.full((y.shape[0],), -7, dtype=torch.int32, device=gpu) for y in ys]
    torch.cuda.synchronize()
    for i, (t, o) in enumerate(zip(ty, outs)):
        jg.k_assign_noalloc(t, tc, tn, o, stream=sa if i % 2 == 0 else sb)
    torch.cuda.synchronize()
    for y, o in zip(ys, outs):
        assert np.array_equal(o.cpu().numpy(), po.assign(y, cent, norms))
