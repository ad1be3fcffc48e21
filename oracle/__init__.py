"""ctypes binding of the CPU oracle (oracle/kgo_oracle.cpp).

Test infrastructure: imported only by tests/, the smoke check and the benchmark's CPU-baseline leg, as the
checker. Nothing in the product path imports it.
"""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "libkgo_oracle.so")
_lib = None


def build():
    import subprocess
    subprocess.run(["make", "-C", _HERE, "-s"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.kgo_last_error.restype = ctypes.c_char_p
        L.kgo_model_parse.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)]
        L.kgo_model_free.argtypes = [ctypes.c_void_p]
        L.kgo_model_info.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        for fn in (L.kgo_forward_f64, L.kgo_forward_f32):
            fn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                           ctypes.c_void_p, ctypes.c_int]
        for fn in (L.kgo_forward_f64_q, L.kgo_forward_f32_q):
            fn.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 4 + [ctypes.c_int] * 5
        L.kgo_round_operands.argtypes = [ctypes.c_void_p, ctypes.c_long, ctypes.c_int]
        L.kgo_conv_direct_f64.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 3
        L.kgo_wino_filter_f64.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        L.kgo_conv3x3_winograd_f64.argtypes = [ctypes.c_int] * 3 + [ctypes.c_void_p] * 3
        L.kgo_copy_with_symmetry.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 7
        L.kgo_padded_batch_size.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.kgo_copy_outputs_row.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.kgo_postprocess_row.restype = ctypes.c_int
        L.kgo_postprocess_row.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_float, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.kgo_featurize.restype = ctypes.c_int
        L.kgo_featurize.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_float, ctypes.c_double, ctypes.c_int,
                                                             ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                                             ctypes.c_void_p]
        _lib = L
    return _lib


# Layer classes of the 16-bit rounding points (QC_* in kgo_oracle.cpp).
QCLASS = {"stem": 1, "conv3": 2, "gconv": 4, "nbt_in": 8, "nbt_out": 16, "token": 32}
QC_ALL = 63


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class Model:
    """A parsed KataGo model file, evaluated on the CPU."""

    def __init__(self, model_bytes: bytes):
        L = lib()
        self._buf = ctypes.create_string_buffer(model_bytes, len(model_bytes))
        h = ctypes.c_void_p()
        if L.kgo_model_parse(self._buf, len(model_bytes), ctypes.byref(h)) != 0:
            raise ValueError(L.kgo_last_error().decode())
        self._h = h
        info = np.zeros(8, np.int32)
        L.kgo_model_info(self._h, _p(info))
        (self.version, self.num_input_channels, self.num_global, self.num_meta, self.P, self.S, self.row_len,
         self.trunk_c) = (int(v) for v in info)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().kgo_model_free(self._h)
            self._h = None

    def forward(self, spatial, glob, meta=None, dtype=np.float64, threads=None, operands=None, acts=True,
                weights=True, classes=None, weight_classes=None):
        """Raw output rows [n, row_len] (policy P x 362 with pass last, value 3, score S, ownership 361).

        operands="f16" / "bf16" evaluates with the trunk's GEMM operands rounded to that 16-bit type
        (activations when `acts`, weights when `weights`), as a 16-bit handle computes them; `classes` (names of
        QCLASS, default all) limits the rounding to those layer classes, and `weight_classes` (default: `classes`)
        that of the weights. Accumulation is in double, or in float with dtype=np.float32."""
        n = spatial.shape[0]
        spatial = np.ascontiguousarray(spatial, np.float32)
        glob = np.ascontiguousarray(glob, np.float32)
        if self.num_meta:
            meta = np.ascontiguousarray(meta, np.float32)
        else:
            meta = None
        threads = threads or os.cpu_count() or 1
        out = np.zeros((n, self.row_len), dtype)
        if operands is not None:
            q = {"f16": 1, "bf16": 2}[operands]
            f32 = dtype == np.float32
            out = np.zeros((n, self.row_len), np.float32 if f32 else np.float64)
            cls = QC_ALL if classes is None else sum(QCLASS[c] for c in set(classes))
            wcls = cls if weight_classes is None else sum(QCLASS[c] for c in set(weight_classes))
            fn = lib().kgo_forward_f32_q if f32 else lib().kgo_forward_f64_q
            if fn(self._h, n, _p(spatial), _p(glob), _p(meta), _p(out), threads, q if acts else 0,
                  q if weights else 0, cls, wcls) != 0:
                raise RuntimeError(lib().kgo_last_error().decode())
            return out
        fn = lib().kgo_forward_f64 if dtype == np.float64 else lib().kgo_forward_f32
        if fn(self._h, n, _p(spatial), _p(glob), _p(meta), _p(out), threads) != 0:
            raise RuntimeError(lib().kgo_last_error().decode())
        return out


def conv_direct(x, w):
    x = np.ascontiguousarray(x, np.float64); w = np.ascontiguousarray(w, np.float64)
    n, ic = x.shape[:2]; oc, _, k, _ = w.shape
    y = np.zeros((n, oc, 19, 19))
    lib().kgo_conv_direct_f64(n, ic, oc, k, _p(x), _p(w), _p(y))
    return y


def wino_filter(w):
    w = np.ascontiguousarray(w, np.float64)
    oc, ic = w.shape[:2]
    out = np.zeros((36, ic, oc))
    lib().kgo_wino_filter_f64(oc, ic, _p(w), _p(out))
    return out


def conv3x3_winograd(x, w):
    x = np.ascontiguousarray(x, np.float64); w = np.ascontiguousarray(w, np.float64)
    n, ic = x.shape[:2]; oc = w.shape[0]
    y = np.zeros((n, oc, 19, 19))
    lib().kgo_conv3x3_winograd_f64(n, ic, oc, _p(x), _p(w), _p(y))
    return y


def copy_with_symmetry(src, sym, nhwc=False, reverse=False):
    """src [n, c, h, w] (or [n, h, w, c] with nhwc)."""
    src = np.ascontiguousarray(src, np.float32)
    dst = np.zeros_like(src)
    if nhwc:
        n, h, w, c = src.shape
    else:
        n, c, h, w = src.shape
    lib().kgo_copy_with_symmetry(_p(src), _p(dst), n, h, w, c, int(nhwc), sym, int(reverse))
    return dst


def padded_batch_size(buckets, n, max_batch):
    b = np.ascontiguousarray(buckets, np.int32)
    return lib().kgo_padded_batch_size(_p(b), len(b), n, max_batch)


def copy_outputs_row(row, P, S, version, sym, optimism, want_owner=True):
    row = np.ascontiguousarray(row, np.float32)
    pol = np.zeros(362, np.float32)
    fields = np.zeros(9, np.float32)
    own = np.zeros(361, np.float32) if want_owner else None
    lib().kgo_copy_outputs_row(_p(row), P, S, version, sym, ctypes.c_float(optimism), _p(pol), _p(fields), _p(own))
    return pol, fields, own


# The model's post-process multipliers (ModelPostProcessParams: td score, score mean, score stdev, lead, variance
# time, short-term value error, short-term score error), the defaults of the model files without them.
DEFAULT_POST_PARAMS = (20.0, 20.0, 20.0, 20.0, 40.0, 0.25, 30.0)


def postprocess_row(row, P, S, version, sym, optimism, legal, white, bx, by, temperature=1.0, passing_hacks=False,
                    no_result_allowed=True, pp=DEFAULT_POST_PARAMS):
    """NNEvaluator's post-processing of one raw row (copy_outputs, then nneval.rs:1197-1500): (status, policy
    [362], fields [9], ownership [361]); status 1 / 2 are the reference's nonfinite policy / value errors."""
    row = np.ascontiguousarray(row, np.float32)
    legal = np.ascontiguousarray(legal, np.uint8)
    ppa = np.ascontiguousarray(pp, np.float64)
    pol = np.zeros(362, np.float32)
    fields = np.zeros(9, np.float32)
    own = np.zeros(361, np.float32)
    st = lib().kgo_postprocess_row(_p(row), P, S, version, sym, ctypes.c_float(optimism), _p(legal), int(white), bx,
                                   by, ctypes.c_float(temperature), int(passing_hacks), int(no_result_allowed),
                                   _p(ppa), _p(pol), _p(fields), _p(own))
    return st, pol, fields, own


def round_operands(x, operands):
    """Values rounded to a 16-bit operand type ("f16" / "bf16"), returned as float64."""
    a = np.array(x, np.float64, copy=True, order="C")
    lib().kgo_round_operands(_p(a), a.size, {"f16": 1, "bf16": 2}[operands])
    return a


def featurize(meta, color, marks, area, enc, moves, self_komi, pda, nn_x=19, nn_y=19, nhwc=False):
    """fill_row_v7's spatial row (22 planes of nn_x * nn_y, NCHW or NHWC) and 19 global features for one position
    (kgo_featurize: the board and the rules engine's results as inputs)."""
    m = np.ascontiguousarray(meta, np.int32)
    arrs = [np.ascontiguousarray(a, np.uint8) for a in (color, marks, area, enc)]
    mv = np.ascontiguousarray(moves, np.int32)
    row = np.empty(22 * nn_x * nn_y, np.float32)
    glob = np.empty(19, np.float32)
    rc = lib().kgo_featurize(_p(m), *[_p(a) for a in arrs], _p(mv), float(self_komi), float(pda), nn_x, nn_y,
                             int(bool(nhwc)), _p(row), _p(glob))
    if rc != 0:
        raise ValueError(f"kgo_featurize: bad position ({rc})")
    return row, glob
