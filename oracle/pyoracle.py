"""pyoracle — ctypes wrapper of the C oracle (oracle/libjhq_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP product.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.

Also wraps oracle/_ref/libjhq_ref.so (the reference's own cpu/codebook.cpp,
built from the reference checkout) when it exists.
"""
import ctypes
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libjhq_oracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libjhq_ref.so")

_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_U32 = ctypes.c_uint32

class _OIndex(ctypes.Structure):
    _fields_ = [
        ("d", _I), ("M", _I), ("B", _I), ("Br", _I), ("Ds", _I), ("K1D", _I), ("bpd", _I),
        ("Kr", _I), ("bpv", _I), ("nlist", _I), ("nprobe", _I), ("RC", _I), ("alpha", _F),
        ("ntotal", _I64),
        ("P", _VP), ("c1d", _VP), ("res_c1d", _VP), ("cent", _VP), ("cent_norms", _VP),
        ("list_offsets", _VP), ("list_ids", _VP), ("list_codes", _VP), ("list_res", _VP),
        ("list_corr", _VP),
    ]


_SIGS = {
    "o_mt_fill": (None, [_U32, _VP, _I64]),
    "o_normal_fill": (None, [_U32, _VP, _I64]),
    "o_erfinv_f": (_F, [_F]),
    "o_lloyd_max_c1d": (None, [_F, _I, _VP]),
    "o_estimate_sigma": (_F, [_VP, _I64, _I]),
    "o_train_1d_kmeans": (_I, [_VP, _I64, _I, _I, _VP]),
    "o_householder_qr": (_I, [_I, _VP]),
    "o_build_rotation": (None, [_I, _I, _VP]),
    "o_rotate": (None, [_VP, _VP, _I64, _I, _VP]),
    "o_primary_encode": (None, [_VP, _I64, _I, _I, _VP, _I, _VP]),
    "o_residual_encode": (None, [_VP, _VP, _I64, _I, _I, _VP, _I, _VP, _I, _I, _VP, _VP]),
    "o_residual_encode_rc": (None, [_VP, _VP, _I64, _I, _I, _VP, _I, _VP, _I, _I, _I, _VP, _VP]),
    "o_reconstruct": (None, [_VP, _I, _I, _VP, _I, _VP]),
    "o_flat_lut": (None, [_VP, _I, _I, _VP, _I, _VP]),
    "o_factored_lut": (None, [_VP, _I, _I, _VP, _I, _VP]),
    "o_adc_flat": (_F, [_VP, _I, _VP]),
    "o_adc_factored": (_F, [_VP, _I, _I, _I, _VP]),
    "o_cent_norms": (None, [_VP, _I, _I, _VP]),
    "o_assign": (None, [_VP, _I64, _I, _VP, _VP, _I, _VP]),
    "o_train_ivf": (_I, [_VP, _I64, _I, _I, _I, _VP]),
    "o_build_lists": (None, [_VP, _I64, _I, _VP, _VP]),
    "o_select_topk_pairs": (_I, [_VP, _VP, _I64, _I, _VP, _VP]),
    "o_ck": (_I, [_F, _I]),
    "o_search": (_I, [ctypes.POINTER(_OIndex), _VP, _I64, _I, _VP, _VP, _VP, _VP, _VP]),
    "o_search_ex": (_I, [ctypes.POINTER(_OIndex), _VP, _VP, _VP, _I64, _I, _VP, _VP, _VP, _VP,
                         _VP]),
    "o_search_mode": (_I, [ctypes.POINTER(_OIndex), _VP, _VP, _VP, _I64, _I, _I, _VP, _VP, _VP,
                           _VP, _VP]),
    "o_set_threads": (None, [_I]),
    "o_get_threads": (_I, []),
}

_REF_SIGS = {
    "ref_erfinv": (_F, [_F]),
    "ref_c1d": (_I, [_I, _I, _I, _F, _VP]),
    "ref_encode": (None, [_I, _I, _I, _F, _VP, _I, _VP]),
    "ref_flat_lut": (None, [_I, _I, _I, _F, _VP, _VP]),
    "ref_build_lut": (None, [_I, _I, _I, _F, _VP, _VP]),
    "ref_adc_distance": (_F, [_I, _I, _I, _F, _VP, _VP]),
    "ref_reconstruct": (None, [_I, _I, _I, _F, _VP, _VP]),
    "ref_train_1d_kmeans": (_I, [_VP, _I, _I, _I, _VP]),
    "ref_mt19937_fill": (None, [_I, _VP, _I64]),
    "ref_normal_fill": (None, [_I, _VP, _I64]),
}

_lib = None
_ref = None


def _load(path, sigs):
    L = ctypes.CDLL(path)
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise ImportError("oracle/libjhq_oracle.so is not built (make -C oracle)")
        _lib = _load(LIB, _SIGS)
    return _lib


def ref():
    """The reference's own cpu/codebook.cpp build, or None when absent."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB):
        try:
            _ref = _load(REF_LIB, _REF_SIGS)
        except OSError:
            _ref = None
    return _ref


def set_threads(n):
    """Threads of the oracle's row-parallel loops (results do not depend on it)."""
    lib().o_set_threads(int(n))


def get_threads():
    return int(lib().o_get_threads())


def default_threads():
    """All host cores up to 16 (a one-GPU box's CPU share)."""
    return max(1, min(os.cpu_count() or 1, 16))


def _p(a):
    return a.ctypes.data_as(_VP)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---------------------------------------------------------------------------
def mt_fill(seed, n):
    out = np.empty(n, np.uint32)
    lib().o_mt_fill(seed, _p(out), n)
    return out


def normal_fill(seed, n):
    out = np.empty(n, np.float32)
    lib().o_normal_fill(seed, _p(out), n)
    return out


def erfinv(x):
    return np.float32(lib().o_erfinv_f(float(x)))


def lloyd_max_c1d(sigma, K1D):
    out = np.empty(K1D, np.float32)
    lib().o_lloyd_max_c1d(float(sigma), K1D, _p(out))
    return out


def estimate_sigma(x):
    x = _c(x, np.float32)
    return np.float32(lib().o_estimate_sigma(_p(x), x.shape[0], x.shape[1]))


def train_1d_kmeans(vals, Kr, max_iter=25):
    vals = _c(vals, np.float32).ravel()
    out = np.empty(max(Kr, 1), np.float32)
    m = lib().o_train_1d_kmeans(_p(vals), vals.size, Kr, max_iter, _p(out))
    return out[:m].copy()


def householder_qr(G_colmajor, d):
    A = _c(G_colmajor, np.float32).copy()
    lib().o_householder_qr(d, _p(A))
    return A


def build_rotation(d, seed):
    """Pi in column-major storage (JLTransform::pi_data()), flat [d*d]."""
    out = np.empty(d * d, np.float32)
    lib().o_build_rotation(d, seed, _p(out))
    return out


def rotation_rowmajor(d, seed):
    """P[j, k] = Pi(j, k)."""
    return build_rotation(d, seed).reshape(d, d).T.copy()


def rotate(P, x):
    P = _c(P, np.float32)
    x = _c(x, np.float32)
    n, d = x.shape
    y = np.empty((n, d), np.float32)
    lib().o_rotate(_p(P), _p(x), n, d, _p(y))
    return y


def primary_encode(y, M, c1d):
    y = _c(y, np.float32)
    c1d = _c(c1d, np.float32)
    n, d = y.shape
    codes = np.empty((n, M), np.uint8)
    lib().o_primary_encode(_p(y), n, d, M, _p(c1d), c1d.size, _p(codes))
    return codes


def residual_encode(y, codes, M, c1d, res_c1d, Br):
    """res_c1d: [Kr] (one codebook) or [M, Kr] (one per subspace)."""
    y = _c(y, np.float32)
    codes = _c(codes, np.uint8)
    c1d = _c(c1d, np.float32)
    res_c1d = _c(res_c1d, np.float32)
    RC = res_c1d.shape[0] if res_c1d.ndim == 2 else 1
    Kr = res_c1d.shape[-1]
    n, d = y.shape
    bpv = (d * Br + 7) // 8
    res = np.empty((n, bpv), np.uint8)
    corr = np.empty(n, np.float32)
    lib().o_residual_encode_rc(_p(y), _p(codes), n, d, M, _p(c1d), c1d.size, _p(res_c1d),
                               Kr, RC, Br, _p(res), _p(corr))
    return res, corr


def reconstruct(codes, d, c1d):
    """Vectorised LloydMaxCodebook::reconstruct over rows (pure gathers)."""
    codes = np.asarray(codes, np.uint8)
    n, M = codes.shape
    Ds = d // M
    K1D = c1d.size
    bpd = K1D.bit_length() - 1
    k = np.arange(Ds)
    digits = (codes[:, :, None].astype(np.int64) >> (k * bpd)[None, None, :]) & (K1D - 1)
    return np.asarray(c1d, np.float32)[digits].reshape(n, d)


def flat_lut(q_rot, M, c1d):
    q = _c(q_rot, np.float32).ravel()
    c1d = _c(c1d, np.float32)
    lut = np.empty((M, 256), np.float32)
    lib().o_flat_lut(_p(q), q.size, M, _p(c1d), c1d.size, _p(lut))
    return lut


def factored_lut(q_rot, M, c1d):
    q = _c(q_rot, np.float32).ravel()
    c1d = _c(c1d, np.float32)
    d = q.size
    lut = np.empty(M * (d // M) * c1d.size, np.float32)
    lib().o_factored_lut(_p(q), d, M, _p(c1d), c1d.size, _p(lut))
    return lut


def adc_flat(code, lut):
    code = _c(code, np.uint8)
    lut = _c(lut, np.float32)
    return np.float32(lib().o_adc_flat(_p(code), code.size, _p(lut)))


def adc_factored(code, d, K1D, lut):
    code = _c(code, np.uint8)
    lut = _c(lut, np.float32)
    return np.float32(lib().o_adc_factored(_p(code), d, code.size, K1D, _p(lut)))


def cent_norms(cent):
    cent = _c(cent, np.float32)
    out = np.empty(cent.shape[0], np.float32)
    lib().o_cent_norms(_p(cent), cent.shape[0], cent.shape[1], _p(out))
    return out


def assign(y, cent, norms):
    y = _c(y, np.float32)
    cent = _c(cent, np.float32)
    norms = _c(norms, np.float32)
    out = np.empty(y.shape[0], np.int32)
    lib().o_assign(_p(y), y.shape[0], y.shape[1], _p(cent), _p(norms), cent.shape[0], _p(out))
    return out


def train_ivf(y, nlist, iters):
    y = _c(y, np.float32)
    cent = np.empty((nlist, y.shape[1]), np.float32)
    rc = lib().o_train_ivf(_p(y), y.shape[0], y.shape[1], nlist, iters, _p(cent))
    if rc != 0:
        raise ValueError("n_train must be >= nlist")
    return cent


def build_lists(asg, nlist):
    asg = _c(asg, np.int32)
    off = np.empty(nlist + 1, np.int32)
    order = np.empty(asg.size, np.int32)
    lib().o_build_lists(_p(asg), asg.size, nlist, _p(off), _p(order))
    return off, order


def select_topk_pairs(dist, tag, k):
    dist = _c(dist, np.float32)
    tag = _c(tag, np.int32)
    od = np.empty(k, np.float32)
    ot = np.empty(k, np.int32)
    lib().o_select_topk_pairs(_p(dist), _p(tag), dist.size, k, _p(od), _p(ot))
    return od, ot


def ck_of(alpha, k):
    return int(lib().o_ck(float(alpha), int(k)))


# ---------------------------------------------------------------------------
# Whole index (host restatement of JHQGpuIndex train / add / search)
# ---------------------------------------------------------------------------
class OracleIndex:
    """CPU restatement of JHQGpuIndex (jhq_v14_streaming_add/jhq_gpu_index.cu)."""

    def __init__(self, d, M=96, B=8, Br=4, alpha=4.0, nlist=1024, nprobe=8, ivf_iters=8,
                 seed=42, residual_per_subspace=0, **_):
        self.RC = M if residual_per_subspace else 1
        self.d, self.M, self.B, self.Br = d, M, B, Br
        self.alpha = np.float32(alpha)
        self.nlist = nlist
        self.nprobe = min(nprobe, nlist)
        self.ivf_iters = ivf_iters
        self.Ds = d // M
        self.bpd = B // self.Ds
        self.K1D = 1 << self.bpd
        self.Kr = 1 << Br
        self.bpv = (d * Br + 7) // 8
        self.P = rotation_rowmajor(d, seed)
        self.ntotal = 0

    @classmethod
    def from_state(cls, d, params, P, c1d, res_c1d, cent, cent_norms, offsets, ids, codes, res,
                   corr):
        """Wrap an index built elsewhere (e.g. the GPU's) for CPU search."""
        o = cls.__new__(cls)
        o.d, o.M, o.B, o.Br = d, params.M, params.B, params.Br
        o.RC = params.M if getattr(params, "residual_per_subspace", 0) else 1
        o.alpha = np.float32(params.alpha)
        o.nlist = params.nlist
        o.nprobe = min(params.nprobe, params.nlist)
        o.ivf_iters = params.ivf_iters
        o.Ds = d // o.M
        o.bpd = o.B // o.Ds
        o.K1D = 1 << o.bpd
        o.Kr = 1 << o.Br
        o.bpv = (d * o.Br + 7) // 8
        o.P = _c(P, np.float32)
        o.c1d = _c(c1d, np.float32)
        o.res_c1d = _c(res_c1d, np.float32).reshape((o.RC, -1) if o.RC > 1 else (-1,))
        o.cent, o.cent_norms = _c(cent, np.float32), _c(cent_norms, np.float32)
        o.list_offsets, o.list_ids = _c(offsets, np.int32), _c(ids, np.int32)
        o.list_codes, o.list_res, o.list_corr = (_c(codes, np.uint8), _c(res, np.uint8),
                                                 _c(corr, np.float32))
        o.ntotal = int(o.list_ids.size)
        return o

    def train(self, x):
        x = _c(x, np.float32)
        if x.shape[0] < self.nlist:
            raise ValueError("n_train must be >= nlist")
        self.sigma = estimate_sigma(x)
        self.c1d = lloyd_max_c1d(self.sigma, self.K1D)
        y = rotate(self.P, x)
        codes = primary_encode(y, self.M, self.c1d)
        self.cent = train_ivf(y, self.nlist, self.ivf_iters)
        self.cent_norms = cent_norms(self.cent)
        resid = y - reconstruct(codes, self.d, self.c1d)
        books = []
        for cb in range(self.RC):
            # one codebook over every dimension (v14/jhq_gpu_index.cu:302-330),
            # or one per subspace over its Ds dimensions
            vals = resid.ravel() if self.RC == 1 else \
                np.ascontiguousarray(resid[:, cb * self.Ds:(cb + 1) * self.Ds]).ravel()
            rc = train_1d_kmeans(vals, self.Kr)
            if rc.size < self.Kr:
                rc = np.concatenate([rc, np.full(self.Kr - rc.size, rc[-1], np.float32)])
            books.append(rc)
        self.res_c1d = books[0] if self.RC == 1 else np.stack(books).astype(np.float32)
        return y

    def add(self, x):
        x = _c(x, np.float32)
        y = rotate(self.P, x)
        codes = primary_encode(y, self.M, self.c1d)
        res, corr = residual_encode(y, codes, self.M, self.c1d, self.res_c1d, self.Br)
        asg = assign(y, self.cent, self.cent_norms)
        off, order = build_lists(asg, self.nlist)
        self.assignments = asg
        self.list_offsets = off
        self.list_ids = order.astype(np.int32)
        self.list_codes = np.ascontiguousarray(codes[order])
        self.list_res = np.ascontiguousarray(res[order])
        self.list_corr = np.ascontiguousarray(corr[order])
        self.ntotal = x.shape[0]
        return y

    def _struct(self):
        s = _OIndex()
        s.d, s.M, s.B, s.Br = self.d, self.M, self.B, self.Br
        s.Ds, s.K1D, s.bpd, s.Kr, s.bpv = self.Ds, self.K1D, self.bpd, self.Kr, self.bpv
        s.nlist, s.nprobe, s.alpha, s.ntotal = self.nlist, self.nprobe, float(self.alpha), self.ntotal
        s.RC = self.RC
        self._keep = [self.P, self.c1d, self.res_c1d, self.cent, self.cent_norms,
                      self.list_offsets, self.list_ids, self.list_codes, self.list_res,
                      self.list_corr]
        (s.P, s.c1d, s.res_c1d, s.cent, s.cent_norms, s.list_offsets, s.list_ids,
         s.list_codes, s.list_res, s.list_corr) = [_p(a) for a in self._keep]
        return s

    def search(self, q, k, debug=False, q_rot=None, probes=None, mode=0):
        """Reference pipeline per query.  Stage-wise parity: q_rot [nq, d] replaces
        the rotation and probes [nq, nprobe] replaces the probe selection.
        mode 0: exact selection; mode 1: the reference's approximate per-thread
        top-4 selection (jhq_v14_streaming_add/search.cu:105-195, 244-291)."""
        q = _c(q, np.float32)
        nq = q.shape[0]
        if q_rot is not None:
            q_rot = _c(q_rot, np.float32)
            assert q_rot.shape == (nq, self.d)
        if probes is not None:
            probes = _c(probes, np.int32)
            assert probes.shape == (nq, self.nprobe)
        ck = ck_of(self.alpha, k)
        dists = np.empty((nq, k), np.float32)
        ids = np.empty((nq, k), np.int32)
        tpos = np.empty((nq, ck), np.int32) if debug else None
        tdist = np.empty((nq, ck), np.float32) if debug else None
        s = self._struct()
        pr_out = np.empty((nq, self.nprobe), np.int32) if debug else None
        lib().o_search_mode(ctypes.byref(s), _p(q), _p(q_rot) if q_rot is not None else None,
                            _p(probes) if probes is not None else None, nq, k, int(mode),
                            _p(dists), _p(ids), _p(pr_out) if debug else None,
                            _p(tpos) if debug else None, _p(tdist) if debug else None)
        if debug:
            return dict(dists=dists, ids=ids, probes=pr_out, topck_pos=tpos, topck_dist=tdist)
        return dists, ids


def near_tie_mask(dists, rel=1e-5):
    """True where a rank's distance is within `rel` of a neighbouring rank
    (including the first rank outside the row, if given as an extra column)."""
    d = np.asarray(dists, np.float64)
    gap_ok = np.ones(d.shape, bool)
    diff = np.abs(np.diff(d, axis=1))
    scale = np.maximum(np.abs(d[:, 1:]), np.abs(d[:, :-1]))
    close = diff <= rel * scale
    gap_ok[:, :-1] &= ~close
    gap_ok[:, 1:] &= ~close
    return ~gap_ok


def math_ck(alpha, k):
    return max(k, int(math.ceil(np.float32(alpha) * np.float32(k))))
