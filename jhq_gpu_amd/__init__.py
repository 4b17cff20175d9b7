"""jhq_gpu_amd — MI355X-native JHQ IVF search engine (Python host mirror).

Thin ctypes layer over the C-ABI of ``libjhq_amd.so`` (declared in
``include/jhq.h``).  The class below mirrors the reference's
``jhq_gpu::JHQGpuIndex`` (lrlorry/JHQ_GPU jhq_v14_streaming_add/jhq_gpu_index.cuh:14-83):
same ``Params`` fields and defaults, ``train`` / ``add`` / ``search`` /
``ntotal`` / ``dim``, and the reference's error kinds (``std::invalid_argument``
-> ``ValueError``, ``std::runtime_error`` -> ``RuntimeError``).

All computation runs in the HIP library; if it is not built, importing works
but creating an index raises ``JHQNotBuiltError`` — there is no CPU fallback.
"""
import ctypes
import dataclasses
import os

import numpy as np

__all__ = [
    "Params", "JHQGpuIndex", "JHQError", "JHQDeviceError", "JHQNotBuiltError",
    "lib", "lib_path", "k_rotate", "k_primary_encode", "k_residual_encode", "k_assign",
    "k_assign_noalloc", "k_build_lut", "k_scan_topck", "k_refine", "k_final_topk",
    "STEP_NAMES",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libjhq_amd.so")
_lib = None

JHQ_OK, JHQ_EINVAL, JHQ_ESTATE, JHQ_EDEVICE, JHQ_ENOMEM = 0, 1, 2, 3, 4
STEP_NAMES = ("query_gemm", "select_probes", "scan_topck", "refine_topk")


class JHQError(RuntimeError):
    pass


class JHQDeviceError(JHQError):
    pass


class JHQNotBuiltError(ImportError):
    pass


class _Params(ctypes.Structure):
    _fields_ = [
        ("M", ctypes.c_int), ("B", ctypes.c_int), ("Br", ctypes.c_int),
        ("alpha", ctypes.c_float), ("nlist", ctypes.c_int), ("nprobe", ctypes.c_int),
        ("ivf_iters", ctypes.c_int), ("batch_size", ctypes.c_int), ("seed", ctypes.c_int),
        ("add_batch", ctypes.c_int), ("residual_per_subspace", ctypes.c_int),
    ]


@dataclasses.dataclass
class Params:
    """JHQGpuIndex::Params (jhq_v14_streaming_add/jhq_gpu_index.cuh:16-36)."""
    M: int = 96
    B: int = 8
    Br: int = 4
    alpha: float = 4.0
    nlist: int = 1024
    nprobe: int = 8
    ivf_iters: int = 8
    batch_size: int = 256
    seed: int = 42
    add_batch: int = 65536
    # extension: one residual codebook per subspace (the reference has one)
    residual_per_subspace: int = 0

    def _c(self):
        return _Params(self.M, self.B, self.Br, self.alpha, self.nlist, self.nprobe,
                       self.ivf_iters, self.batch_size, self.seed, self.add_batch,
                       self.residual_per_subspace)


_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int

_SIGS = {
    "jhq_params_default": (None, [ctypes.POINTER(_Params)]),
    "jhq_create": (_I, [_I, ctypes.POINTER(_Params), ctypes.POINTER(_VP)]),
    "jhq_destroy": (_I, [_VP]),
    "jhq_train": (_I, [_VP, _VP, _I64]),
    "jhq_add": (_I, [_VP, _VP, _I64]),
    "jhq_search": (_I, [_VP, _VP, _I64, _I, _VP, _VP]),
    "jhq_train_ex": (_I, [_VP, _VP, _I, _I64]),
    "jhq_add_ex": (_I, [_VP, _VP, _I, _I64]),
    "jhq_append": (_I, [_VP, _VP, _I64]),
    "jhq_append_ex": (_I, [_VP, _VP, _I, _I64]),
    "jhq_search_ex": (_I, [_VP, _VP, _I, _I64, _I, _VP, _VP]),
    "jhq_get_pool": (_I, [_VP, ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
    "jhq_save": (_I, [_VP, ctypes.c_char_p]),
    "jhq_load": (_I, [ctypes.c_char_p, ctypes.POINTER(_VP)]),
    "jhq_get_params": (_I, [_VP, ctypes.POINTER(_Params)]),
    "jhq_get_plan": (_I, [_VP, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "jhq_search_device": (_I, [_VP, _VP, _I64, _I, _VP, _VP, _VP]),
    "jhq_reserve": (_I, [_VP, _I]),
    "jhq_set_scan_kind": (_I, [_VP, _I]),
    "jhq_ntotal": (_I64, [_VP]),
    "jhq_dim": (_I, [_VP]),
    "jhq_set_nprobe": (_I, [_VP, _I]),
    "jhq_set_alpha": (_I, [_VP, ctypes.c_float]),
    "jhq_last_error": (ctypes.c_char_p, []),
    "jhq_get_dims": (_I, [_VP] + [ctypes.POINTER(_I)] * 5),
    "jhq_get_codebooks": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP]),
    "jhq_get_lists": (_I, [_VP, _VP, _VP, _VP, _VP, _VP]),
    "jhq_search_debug": (_I, [_VP, _VP, _I64, _I, _VP, _VP, _VP, _VP, _VP, _VP]),
    "jhq_set_timing": (_I, [_VP, _I]),
    "jhq_get_timing": (_I, [_VP, _VP, _I, ctypes.POINTER(_I64)]),
    "jhq_k_rotate": (_I, [_VP, _VP, _I64, _I, _VP, _VP]),
    "jhq_k_primary_encode": (_I, [_VP, _VP, _VP, _I64, _I, _I, _I, _I, _I, _VP]),
    "jhq_k_residual_encode": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _I64, _I, _I, _I, _I, _I,
                                   _I, _I, _I, _VP]),
    "jhq_k_assign": (_I, [_VP, _I64, _I, _VP, _VP, _I, _VP, _VP]),
    "jhq_k_assign_noalloc": (_I, [_VP, _I64, _I, _VP, _VP, _I, _VP, _VP]),
    "jhq_k_select_probes": (_I, [_VP, _I, _I, _I, _VP, _VP, _VP, _VP, _VP]),
    "jhq_k_build_lut": (_I, [_VP, _VP, _VP, _I, _I, _I, _I, _I, _I, _VP]),
    "jhq_k_scan_topck": (_I, [_VP] * 8 + [_I, _I, _I, _I64, _I, _VP]),
    "jhq_k_refine": (_I, [_VP] * 7 + [_I] * 6 + [_VP]),
    "jhq_k_final_topk": (_I, [_VP] * 5 + [_I, _I, _I, _VP]),
}


def lib_path():
    return _LIB_PATH


def lib():
    """Load libjhq_amd.so (raises JHQNotBuiltError if it is missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise JHQNotBuiltError(
                "libjhq_amd.so is not built; run __graft_entry__.build() "
                "(or python jhq_gpu_amd/build.py)")
        L = ctypes.CDLL(_LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc):
    if rc == JHQ_OK:
        return
    msg = lib().jhq_last_error().decode(errors="replace")
    if rc == JHQ_EINVAL:
        raise ValueError(msg)
    if rc == JHQ_ESTATE:
        raise RuntimeError(msg)
    raise JHQDeviceError(f"[{rc}] {msg}")


JHQ_F32, JHQ_U8, JHQ_I8 = 0, 1, 2


def _f32(a, d=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    if d is not None and (a.ndim != 2 or a.shape[1] != d):
        raise ValueError(f"expected a [n, {d}] array, got shape {a.shape}")
    return a


def _typed(a, d):
    """uint8 / int8 arrays pass through as bytes (converted on the device);
    anything else becomes float32."""
    a = np.asarray(a)
    if a.dtype == np.uint8:
        dt = JHQ_U8
    elif a.dtype == np.int8:
        dt = JHQ_I8
    else:
        a, dt = np.asarray(a, dtype=np.float32), JHQ_F32
    a = np.ascontiguousarray(a)
    if a.ndim != 2 or a.shape[1] != d:
        raise ValueError(f"expected a [n, {d}] array, got shape {a.shape}")
    return a, dt


def _ptr(a):
    return a.ctypes.data_as(_VP)


def _dptr(t):
    """Device pointer of a torch tensor (or an int address)."""
    if t is None:
        return None
    if isinstance(t, int):
        return _VP(t)
    return _VP(t.data_ptr())


class JHQGpuIndex:
    """jhq_gpu::JHQGpuIndex (jhq_v14_streaming_add/jhq_gpu_index.cuh:14-83)."""

    def __init__(self, d, p=None):
        p = p or Params()
        self._p = dataclasses.replace(p)
        h = _VP()
        cp = self._p._c()
        _check(lib().jhq_create(int(d), ctypes.byref(cp), ctypes.byref(h)))
        self._h = h
        self._d = int(d)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            try:
                _lib.jhq_destroy(h)
            except Exception:  # interpreter shutdown
                pass
            self._h = None

    # -- reference API -------------------------------------------------------
    def train(self, x):
        """float32 rows (uint8 / int8 rows are converted to float32)."""
        x, dt = _typed(x, self._d)
        _check(lib().jhq_train_ex(self._h, _ptr(x), dt, x.shape[0]))

    def add(self, x):
        """The reference's one-shot add (a second call raises RuntimeError)."""
        x, dt = _typed(x, self._d)
        _check(lib().jhq_add_ex(self._h, _ptr(x), dt, x.shape[0]))

    def append(self, x):
        """Streaming add (extension): any number of calls, interleaved with
        searches; ids continue from ntotal."""
        x, dt = _typed(x, self._d)
        _check(lib().jhq_append_ex(self._h, _ptr(x), dt, x.shape[0]))

    def search(self, q, k):
        q, dt = _typed(q, self._d)
        nq = q.shape[0]
        dists = np.empty((nq, k), np.float32)
        ids = np.empty((nq, k), np.int32)
        _check(lib().jhq_search_ex(self._h, _ptr(q), dt, nq, int(k), _ptr(dists), _ptr(ids)))
        return dists, ids

    @property
    def ntotal(self):
        return int(lib().jhq_ntotal(self._h))

    @property
    def dim(self):
        return int(lib().jhq_dim(self._h))

    @property
    def params(self):
        return dataclasses.replace(self._p)

    # -- extensions ----------------------------------------------------------
    def set_nprobe(self, nprobe):
        _check(lib().jhq_set_nprobe(self._h, int(nprobe)))
        self._p.nprobe = min(int(nprobe), self._p.nlist)

    def set_alpha(self, alpha):
        _check(lib().jhq_set_alpha(self._h, float(alpha)))
        self._p.alpha = float(alpha)

    def reserve(self, k_max):
        """Preallocates the search workspace for k <= k_max (device searches
        with a larger k raise RuntimeError)."""
        _check(lib().jhq_reserve(self._h, int(k_max)))

    def set_scan_kind(self, kind):
        """0: the integer-MFMA pre-scan with exact re-check where it applies
        (one-bit digits) and the list sizes predict shared probed lists, else
        the byte-LUT scans; 1: the byte-LUT scans only; 2: the pre-scan
        wherever it applies.  Results are identical; only the speed differs."""
        _check(lib().jhq_set_scan_kind(self._h, int(kind)))

    def search_device(self, q, k, out_dists, out_ids, stream=None):
        """q, out_dists, out_ids: torch device tensors (or int addresses).
        Enqueue-only: k must be within the reserved workspace (reserve())."""
        nq = int(q.shape[0])
        s = None
        if stream is not None:
            s = _VP(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))
        _check(lib().jhq_search_device(self._h, _dptr(q), nq, int(k), _dptr(out_dists),
                                       _dptr(out_ids), s))

    def dims(self):
        vals = [_I() for _ in range(5)]
        _check(lib().jhq_get_dims(self._h, *[ctypes.byref(v) for v in vals]))
        return dict(zip(("Ds", "K1D", "bpd", "Kr", "bpv"), (v.value for v in vals)))

    def rotation(self):
        """Row-major Pi(j, k) (the transpose of the reference's pi_data())."""
        P = np.empty((self._d, self._d), np.float32)
        _check(lib().jhq_get_codebooks(self._h, None, None, None, _ptr(P), None, None))
        return P

    def save(self, path):
        """Writes the index (parameters, trained state, lists) to `path`."""
        _check(lib().jhq_save(self._h, os.fsencode(path)))

    @classmethod
    def load(cls, path):
        """A new index read from a file written by save()."""
        h = _VP()
        _check(lib().jhq_load(os.fsencode(path), ctypes.byref(h)))
        self = cls.__new__(cls)
        self._h = h
        self._d = int(lib().jhq_dim(h))
        cp = _Params()
        _check(lib().jhq_get_params(h, ctypes.byref(cp)))
        self._p = Params(**{f: getattr(cp, f) for f, _ in _Params._fields_})
        return self

    def scan_plan(self, k):
        """(scan kernel name, short-list length ck) a search with this k uses."""
        kind, ck = _I(), _I()
        _check(lib().jhq_get_plan(self._h, int(k), ctypes.byref(kind), ctypes.byref(ck)))
        names = ("scan_topck_kernel", "scan_wave_kernel", "scan_dump_kernel", "scan_skew_kernel",
                 "mfma_scan_kernel")
        return names[kind.value], int(ck.value)

    def pool(self):
        used, cap = _I64(), _I64()
        _check(lib().jhq_get_pool(self._h, ctypes.byref(used), ctypes.byref(cap)))
        return int(used.value), int(cap.value)

    def codebooks(self):
        dm = self.dims()
        sigma = np.zeros(1, np.float32)
        c1d = np.empty(dm["K1D"], np.float32)
        rc = np.empty((self._p.M, dm["Kr"]) if self._p.residual_per_subspace else dm["Kr"],
                      np.float32)
        P = np.empty((self._d, self._d), np.float32)
        cent = np.empty((self._p.nlist, self._d), np.float32)
        norms = np.empty(self._p.nlist, np.float32)
        _check(lib().jhq_get_codebooks(self._h, _ptr(sigma), _ptr(c1d), _ptr(rc), _ptr(P),
                                       _ptr(cent), _ptr(norms)))
        return dict(sigma=float(sigma[0]), c1d=c1d, res_c1d=rc, P=P, centroids=cent,
                    cent_norms=norms)

    def lists(self, include_payload=True):
        """List storage in stored-position order; offsets only when
        include_payload is False."""
        dm = self.dims()
        n = self.ntotal
        off = np.empty(self._p.nlist + 1, np.int32)
        if not include_payload:
            _check(lib().jhq_get_lists(self._h, _ptr(off), None, None, None, None))
            return dict(offsets=off)
        ids = np.empty(n, np.int32)
        codes = np.empty((n, self._p.M), np.uint8)
        res = np.empty((n, dm["bpv"]), np.uint8)
        corr = np.empty(n, np.float32)
        _check(lib().jhq_get_lists(self._h, _ptr(off), _ptr(ids), _ptr(codes), _ptr(res),
                                   _ptr(corr)))
        return dict(offsets=off, ids=ids, codes=codes, res=res, corr=corr)

    def search_debug(self, q, k):
        q = _f32(q, self._d)
        nq = q.shape[0]
        P = min(self._p.nprobe, self._p.nlist)
        ck = max(k, int(np.ceil(np.float32(self._p.alpha) * np.float32(k))))
        dists = np.empty((nq, k), np.float32)
        ids = np.empty((nq, k), np.int32)
        q_rot = np.empty((nq, self._d), np.float32)
        probes = np.empty((nq, P), np.int32)
        tpos = np.empty((nq, ck), np.int32)
        tdist = np.empty((nq, ck), np.float32)
        _check(lib().jhq_search_debug(self._h, _ptr(q), nq, int(k), _ptr(dists), _ptr(ids),
                                      _ptr(q_rot), _ptr(probes), _ptr(tpos), _ptr(tdist)))
        return dict(dists=dists, ids=ids, q_rot=q_rot, probes=probes, topck_pos=tpos,
                    topck_dist=tdist)

    def set_timing(self, enable=True):
        _check(lib().jhq_set_timing(self._h, 1 if enable else 0))

    def timing(self):
        ms = np.zeros(len(STEP_NAMES), np.float64)
        nb = _I64()
        _check(lib().jhq_get_timing(self._h, _ptr(ms), len(STEP_NAMES), ctypes.byref(nb)))
        return dict(zip(STEP_NAMES, ms.tolist())), int(nb.value)


# -- kernel-granular entry points (torch device tensors) ----------------------
def _stream(s):
    if s is None:
        return None
    return _VP(s.cuda_stream if hasattr(s, "cuda_stream") else int(s))


def k_rotate(P, x, y, stream=None):
    n, d = x.shape
    _check(lib().jhq_k_rotate(_dptr(P), _dptr(x), int(n), int(d), _dptr(y), _stream(stream)))


def k_primary_encode(y, codes, c1d, M, stream=None):
    n, d = y.shape
    K1D = int(c1d.shape[0])
    bpd = K1D.bit_length() - 1
    _check(lib().jhq_k_primary_encode(_dptr(y), _dptr(codes), _dptr(c1d), int(n), int(d), int(M),
                                      int(d // M), K1D, bpd, _stream(stream)))


def k_residual_encode(y, primary, res, corr, c1d, res_c1d, M, Br, stream=None):
    n, d = y.shape
    K1D = int(c1d.shape[0])
    bpd = K1D.bit_length() - 1
    bpv = (d * Br + 7) // 8
    _check(lib().jhq_k_residual_encode(_dptr(y), _dptr(primary), _dptr(res), _dptr(corr),
                                       _dptr(c1d), _dptr(res_c1d), int(n), int(d), int(M),
                                       int(d // M), K1D, int(res_c1d.shape[0]), int(Br), bpv, bpd,
                                       _stream(stream)))


def k_assign(y, cent, norms, assign, stream=None):
    n, d = y.shape
    _check(lib().jhq_k_assign(_dptr(y), int(n), int(d), _dptr(cent), _dptr(norms),
                              int(cent.shape[0]), _dptr(assign), _stream(stream)))


def k_assign_noalloc(y, cent, norms, assign, stream=None):
    """k_assign with no allocation (keys in a fixed 2^20-row device array)."""
    n, d = y.shape
    _check(lib().jhq_k_assign_noalloc(_dptr(y), int(n), int(d), _dptr(cent), _dptr(norms),
                                      int(cent.shape[0]), _dptr(assign), _stream(stream)))


def k_select_probes(scores, list_sizes, P, probes, gofs, qtot, stream=None):
    """scores [B, nlist] float32, list_sizes [nlist] int32 (device tensors)."""
    B, nlist = scores.shape
    _check(lib().jhq_k_select_probes(_dptr(scores), int(B), int(nlist), int(P),
                                     _dptr(list_sizes), _dptr(probes), _dptr(gofs), _dptr(qtot),
                                     _stream(stream)))


def k_build_lut(q_rot, c1d, lut, M, stream=None):
    """q_rot [B, d], c1d [K1D] -> lut [B, M, 256] (device tensors)."""
    B, d = q_rot.shape
    K1D = int(c1d.shape[0])
    _check(lib().jhq_k_build_lut(_dptr(q_rot), _dptr(c1d), _dptr(lut), int(B), int(d), int(M),
                                 int(d // M), K1D, K1D.bit_length() - 1, _stream(stream)))


def k_scan_topck(lut, probe_ids, probe_offsets, list_offsets, primary_t, query_total,
                 topck_primary, topck_pos, stream=None):
    """Reference-layout scan: lut [B, M, 256], probe_ids [B, P], probe_offsets
    [B, P+1], list_offsets [nlist+1], primary_t [M, N], query_total [B] ->
    topck_primary / topck_pos [B, ck]."""
    B, M = int(lut.shape[0]), int(lut.shape[1])
    P = int(probe_ids.shape[1])
    N = int(primary_t.shape[1])
    ck = int(topck_pos.shape[1])
    _check(lib().jhq_k_scan_topck(_dptr(lut), _dptr(probe_ids), _dptr(probe_offsets),
                                  _dptr(list_offsets), _dptr(primary_t), _dptr(query_total),
                                  _dptr(topck_primary), _dptr(topck_pos), B, P, M, N, ck,
                                  _stream(stream)))


def k_refine(q_rot, res_c1d, topck_pos, topck_primary, list_res, list_corr, comp, Br,
             stream=None):
    B, d = q_rot.shape
    ck = int(topck_pos.shape[1])
    _check(lib().jhq_k_refine(_dptr(q_rot), _dptr(res_c1d), _dptr(topck_pos),
                              _dptr(topck_primary), _dptr(list_res), _dptr(list_corr),
                              _dptr(comp), int(B), ck, int(d), int(res_c1d.shape[0]), int(Br),
                              int(list_res.shape[1]), _stream(stream)))


def k_final_topk(comp, topck_pos, list_ids, final_dists, final_ids, stream=None):
    B, ck = comp.shape
    k = int(final_ids.shape[1])
    _check(lib().jhq_k_final_topk(_dptr(comp), _dptr(topck_pos), _dptr(list_ids),
                                  _dptr(final_dists), _dptr(final_ids), int(B), int(ck), k,
                                  _stream(stream)))
