"""The preallocated SearchWorkspace contract (v14/jhq_gpu_index.cu:166-206,531;
v14/search.cu:294-313): add() / append() / load() and the setters reserve the
search workspace, so a device search allocates nothing and only enqueues; a
device search beyond the reservation fails instead of allocating; inserts
wait for a device search still in flight."""
import numpy as np
import pytest

import pyoracle as po
from datagen import queries_and_base
from test_gpu_parity import _bits, _stagewise

import jhq_gpu_amd as jg

pytestmark = pytest.mark.gpu


def _pair(d=128, M=32, nlist=16, nprobe=5, alpha=4.0, batch=16):
    p = jg.Params(M=M, B=8, Br=4, alpha=alpha, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                  batch_size=batch, seed=42)
    g = jg.JHQGpuIndex(d, p)
    o = po.OracleIndex(d, M=M, B=8, Br=4, alpha=alpha, nlist=nlist, nprobe=nprobe, ivf_iters=4,
                       seed=42)
    return g, o


def test_device_search_within_reservation(gpu):
    import torch
    base, q = queries_and_base(4000, 40, 128, 32, seed=811)
    g, o = _pair()
    g.train(base[:1500])
    g.add(base)
    qt = torch.from_numpy(q).to(gpu)
    s = torch.cuda.current_stream()
    for k in (1, 10):  # add() reserves k <= 10
        od = torch.empty((q.shape[0], k), dtype=torch.float32, device=gpu)
        oi = torch.empty((q.shape[0], k), dtype=torch.int32, device=gpu)
        g.search_device(qt, k, od, oi, stream=s)
        d1, i1 = g.search(q, k)
        assert np.array_equal(oi.cpu().numpy(), i1)
    k = 25
    od = torch.empty((q.shape[0], k), dtype=torch.float32, device=gpu)
    oi = torch.empty((q.shape[0], k), dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="reserve"):
        g.search_device(qt, k, od, oi, stream=s)
    g.reserve(k)
    g.search_device(qt, k, od, oi, stream=s)
    d1, i1 = g.search(q, k)
    assert np.array_equal(oi.cpu().numpy(), i1)
    assert np.array_equal(_bits(od.cpu().numpy()), _bits(d1))
    # a setter re-reserves for the new shape: larger alpha, then a device search
    g.set_alpha(10.0)
    g.search_device(qt, k, od, oi, stream=s)
    d1, i1 = g.search(q, k)
    assert np.array_equal(oi.cpu().numpy(), i1)


@pytest.mark.parametrize("d,M", [(128, 32), (128, 16), (96, 24)],
                         ids=["skewed_scan", "wave_scan_m16", "wave_scan_m24"])
def test_append_after_outstanding_device_search(gpu, d, M):
    """Device search on a side stream, then append() with no host sync, then
    another device search: the first search sees the old lists, the second
    the new ones, both stage-wise exact against the oracle."""
    import torch
    k = 10
    base, q = queries_and_base(9000, 48, d, 40, seed=901 + M)
    g, o = _pair(d=d, M=M)
    g.train(base[:2000])
    o.train(base[:2000])
    g.add(base[:3000])
    o.add(base[:3000])
    _stagewise(g, o, q, k)
    want1 = g.search(q, k)
    qt = torch.from_numpy(q).to(gpu)
    side = torch.cuda.Stream()
    od1 = torch.full((q.shape[0], k), -1.0, dtype=torch.float32, device=gpu)
    oi1 = torch.full((q.shape[0], k), -2, dtype=torch.int32, device=gpu)
    od2 = torch.full_like(od1, -1.0)
    oi2 = torch.full_like(oi1, -2)
    side.wait_stream(torch.cuda.current_stream())
    # three appends of growing size: lists move and the pool re-packs while
    # the first search may still be running
    g.search_device(qt, k, od1, oi1, stream=side)
    g.append(base[3000:3100])
    g.append(base[3100:6000])
    g.append(base[6000:9000])
    g.search_device(qt, k, od2, oi2, stream=side)
    side.synchronize()
    assert np.array_equal(oi1.cpu().numpy(), want1[1])
    assert np.array_equal(_bits(od1.cpu().numpy()), _bits(want1[0]))
    o.add(base)
    _stagewise(g, o, q, k)
    want2 = g.search(q, k)
    assert np.array_equal(oi2.cpu().numpy(), want2[1])
    assert np.array_equal(_bits(od2.cpu().numpy()), _bits(want2[0]))


def test_device_searches_on_two_streams_are_ordered(gpu):
    """Two device searches on different streams share the workspaces; the
    second is ordered after the first."""
    import torch
    base, q = queries_and_base(4000, 64, 128, 32, seed=977)
    g, _ = _pair(batch=16)
    g.train(base[:1500])
    g.add(base)
    want = g.search(q, 10)
    qt = torch.from_numpy(q).to(gpu)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for s in (s1, s2, s1, s2):
        od = torch.empty((q.shape[0], 10), dtype=torch.float32, device=gpu)
        oi = torch.empty((q.shape[0], 10), dtype=torch.int32, device=gpu)
        s.wait_stream(torch.cuda.current_stream())
        g.search_device(qt, 10, od, oi, stream=s)
        outs.append((od, oi))
    torch.cuda.synchronize()
    for od, oi in outs:
        assert np.array_equal(oi.cpu().numpy(), want[1])
        assert np.array_equal(_bits(od.cpu().numpy()), _bits(want[0]))
