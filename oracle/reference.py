"""numpy wrappers of lr_oracle.c (TEST INFRASTRUCTURE ONLY).

bf16 arrays are uint16 bit patterns (see oracle.bf16). Every function
returns new arrays and restates the reference line cited in lr_oracle.c.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIBRARY = HERE / "liblr_oracle.so"

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float

_SIGS = {
    "lro_quantize_rows": ([_P, _I64, _I64, _P, _P], None),
    "lro_int_mm": ([_P, _P, _I64, _I64, _I64, _I64, _I64, _P], None),
    "lro_dequant": ([_P, _P, _P, _P, _I64, _I64, _P], None),
    "lro_gelu_tanh": ([_P, _I64, _P], None),
    "lro_swiglu": ([_P, _I64, _I64, _P], None),
    "lro_swiglu_quant": ([_P, _I64, _I64, _P, _P], None),
    "lro_gated_residual": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P], None),
    "lro_rms_adaln": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _F32, _P], None),
    "lro_rms_adaln_quant": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _F32,
                             _P, _P], None),
    "lro_residual_rms_quant": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _P, _P,
                                _P], None),
    "lro_canonical_sumsq": ([_P, _I64], ctypes.c_float),
    "lro_qk_norm_rope": ([_P] * 8 + [_I64] * 9 + [_F32], None),
    "lro_qk_sumsq": ([_P, _I64], ctypes.c_float),
    "lro_num_threads": ([], ctypes.c_int),
    "lro_adaln_table": ([_P, _P, _P, _I64, _I64, _I64, _P], None),
}

_lib = None


def build() -> pathlib.Path:
    """Compile lr_oracle.c with its Makefile (gcc, OpenMP, no FMA contraction)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        for name, (args, res) in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a):
    return None if a is None else a.ctypes.data


def quantize_rows(x):
    """model/int8.py:66-67 on bf16 rows: returns (int8 [R, W], fp32 [R])."""
    x = _c(x, np.uint16)
    rows, width = x.shape
    q = np.empty((rows, width), np.int8)
    s = np.empty(rows, np.float32)
    load().lro_quantize_rows(_p(x), rows, width, _p(q), _p(s))
    return q, s


def int_mm(a, w_nk=None, *, b=None):
    """Exact int32 a @ B. Pass the weight as w_nk [N, K] (Int8Linear storage)
    or as any [K, N] int8 array `b`."""
    a = _c(a, np.int8)
    m, k = a.shape
    if w_nk is not None:
        w = _c(w_nk, np.int8)
        n = w.shape[0]
        bsk, bsn = 1, k
    else:
        w = np.asarray(b, dtype=np.int8)
        n = w.shape[1]
        bsk, bsn = w.strides[0], w.strides[1]  # int8: strides are element strides
        if bsk < 0 or bsn < 0:
            w = np.ascontiguousarray(w)
            bsk, bsn = w.strides
    c = np.empty((m, n), np.int32)
    load().lro_int_mm(a.ctypes.data, w.ctypes.data, bsk, bsn, m, n, k, _p(c))
    return c


def dequant(acc, row_scale, col_scale, bias=None):
    """model/int8.py:55-58: bf16(((float)acc * rs) * cs + bias)."""
    acc = _c(acc, np.int32)
    m, n = acc.shape
    rs = _c(np.reshape(row_scale, -1), np.float32)
    cs = _c(np.reshape(col_scale, -1), np.float32)
    b = None if bias is None else _c(np.reshape(bias, -1), np.uint16)
    out = np.empty((m, n), np.uint16)
    load().lro_dequant(_p(acc), _p(rs), _p(cs), _p(b), m, n, _p(out))
    return out


def linear(a_q, row_scale, w_nk, col_scale, bias=None):
    """Int8Linear.forward_quantized: dequant(int_mm(...))."""
    return dequant(int_mm(a_q, w_nk), row_scale, col_scale, bias)


def gelu_tanh(x):
    x = _c(x, np.uint16)
    out = np.empty_like(x)
    load().lro_gelu_tanh(_p(x), x.size, _p(out))
    return out


def swiglu(p):
    p = _c(p, np.uint16)
    rows, two_i = p.reshape(-1, p.shape[-1]).shape
    inner = two_i // 2
    out = np.empty((rows, inner), np.uint16)
    load().lro_swiglu(_p(p), rows, inner, _p(out))
    return out.reshape(*p.shape[:-1], inner)


def swiglu_quant(p):
    p = _c(p, np.uint16)
    flat = p.reshape(-1, p.shape[-1])
    rows, inner = flat.shape[0], flat.shape[1] // 2
    q = np.empty((rows, inner), np.int8)
    s = np.empty(rows, np.float32)
    load().lro_swiglu_quant(_p(flat), rows, inner, _p(q), _p(s))
    return q, s


def _table_args(table):
    table = _c(table, np.uint16)
    width = table.shape[-1]
    return table, table.size // width, width


def gated_residual(x, u, table, indices, slot, sequence=None):
    """model/kernels.py:144-153. x, u: [..., T, H] bf16."""
    x = _c(x, np.uint16)
    u = _c(u, np.uint16)
    table, trows, width = _table_args(table)
    idx = _c(np.reshape(indices, -1), np.int64)
    hidden = x.shape[-1]
    seq = sequence if sequence is not None else (x.shape[-2] if x.ndim >= 2 else 1)
    out = np.empty_like(x)
    load().lro_gated_residual(_p(x), _p(u), _p(table), _p(idx), x.size // hidden, seq, hidden,
                              trows, width, int(slot), _p(out))
    return out


def _norm(x, w, table, indices, sequence):
    x = _c(x, np.uint16)
    w = _c(np.reshape(w, -1), np.uint16)
    table, trows, width = _table_args(table)
    idx = _c(np.reshape(indices, -1), np.int64)
    hidden = x.shape[-1]
    seq = sequence if sequence is not None else (x.shape[-2] if x.ndim >= 2 else 1)
    return x, w, table, trows, width, idx, hidden, seq, x.size // hidden


def rms_adaln(x, w, table, indices, shift_slot, scale_slot, eps, sequence=None):
    """model/kernels.py:59-78 with the canonical sum-of-squares order."""
    x, w, table, trows, width, idx, hidden, seq, rows = _norm(x, w, table, indices, sequence)
    out = np.empty_like(x)
    load().lro_rms_adaln(_p(x), _p(w), _p(table), _p(idx), rows, seq, hidden, trows, width,
                         int(shift_slot), int(scale_slot), float(eps), _p(out))
    return out


def rms_adaln_quant(x, w, table, indices, shift_slot, scale_slot, eps, sequence=None):
    """model/kernels.py:95-128: returns (int8 [rows, H], fp32 [rows])."""
    x, w, table, trows, width, idx, hidden, seq, rows = _norm(x, w, table, indices, sequence)
    q = np.empty((rows, hidden), np.int8)
    s = np.empty(rows, np.float32)
    load().lro_rms_adaln_quant(_p(x), _p(w), _p(table), _p(idx), rows, seq, hidden, trows, width,
                               int(shift_slot), int(scale_slot), float(eps), _p(q), _p(s))
    return q, s


def residual_rms_quant(x, u, w, table, indices, eps, sequence=None):
    """model/kernels.py:405-419: returns (bf16 residual, int8, fp32)."""
    x, w, table, trows, width, idx, hidden, seq, rows = _norm(x, w, table, indices, sequence)
    u = _c(u, np.uint16)
    resid = np.empty_like(x)
    q = np.empty((rows, hidden), np.int8)
    s = np.empty(rows, np.float32)
    load().lro_residual_rms_quant(_p(x), _p(u), _p(w), _p(table), _p(idx), rows, seq, hidden,
                                  trows, width, float(eps), _p(resid), _p(q), _p(s))
    return resid, q, s


def qk_norm_rope(q, k, q_weight, k_weight, cos, sin, eps):
    """model/kernels.py:187-257 and :345-402, sum of squares in the order of
    the reference's ordered reduction (kernels.py:333-344).

    q, k: bf16 bit patterns [batch, sequence, heads, head_dim] (copied
    contiguous); weights [head_dim]; cos, sin: fp32 [sequence, rotary_dim].
    Returns (q_out, k_out) contiguous like q.
    """
    q = _c(q, np.uint16)
    k = _c(k, np.uint16)
    batch, seq, heads, dim = q.shape
    cos = _c(cos, np.float32)
    sin = _c(sin, np.float32)
    rot = cos.shape[-1]
    qo = np.empty_like(q)
    ko = np.empty_like(k)
    load().lro_qk_norm_rope(_p(q), _p(k), _p(_c(q_weight, np.uint16)), _p(_c(k_weight, np.uint16)),
                            _p(cos), _p(sin), _p(qo), _p(ko), batch, seq, heads, heads * dim, dim,
                            heads * dim, dim, dim, rot, float(eps))
    return qo, ko


def qk_sumsq(row):
    row = _c(row, np.uint16)
    return float(load().lro_qk_sumsq(_p(row), row.size))


def canonical_sumsq(row):
    row = _c(row, np.uint16)
    return float(load().lro_canonical_sumsq(_p(row), row.size))


def num_threads() -> int:
    return int(load().lro_num_threads())


# --------------------------------------------------- Flash token selection ----
def flash_spatial_layout(positions, tags, stride=2):
    """model/flash.py:6-33 in numpy: (keep, inverse) as int64 arrays.

    Rows with tag 0 are video. Per spatial axis (1, 2) the sorted distinct
    coordinates of the video rows are thinned to every stride-th one plus the
    largest; a video row is kept when both its coordinates survive, any other
    row always. inverse maps a kept row to its place in keep and a dropped
    video row to the place of the first kept video row of the same time (fp32
    coordinates, as positions.float()) at least squared distance over (h, w),
    computed in float64; a dropped row with no kept row of its time takes the
    first kept video row (argmin over a row of +inf).
    """
    pos = np.asarray(positions)
    tags = np.asarray(tags)
    if pos.ndim != 2 or tags.ndim != 1 or pos.shape != (tags.size, 3):
        raise ValueError("Flash requires a single shared packed layout")
    video = tags == 0
    if not video.any():
        raise ValueError("Flash requires video tokens")
    on_grid = np.ones(tags.size, bool)
    for axis in (1, 2):
        distinct = np.unique(pos[video, axis])
        survivors = distinct[::stride]
        if survivors[-1] != distinct[-1]:
            survivors = np.append(survivors, distinct[-1])
        on_grid &= np.isin(pos[:, axis], survivors)
    kept = ~video | on_grid
    keep = np.flatnonzero(kept).astype(np.int64)
    inverse = np.zeros(tags.size, np.int64)
    inverse[keep] = np.arange(keep.size)
    dropped = np.flatnonzero(video & ~kept)
    anchors = np.flatnonzero(video & kept)
    p32 = pos.astype(np.float32)
    at, ah, aw = p32[anchors, 0], p32[anchors, 1].astype(np.float64), p32[anchors, 2].astype(np.float64)
    for lo in range(0, dropped.size, 512):
        rows = dropped[lo:lo + 512]
        dh = p32[rows, 1].astype(np.float64)[:, None] - ah[None, :]
        dw = p32[rows, 2].astype(np.float64)[:, None] - aw[None, :]
        dist = dh * dh + dw * dw
        dist[p32[rows, 0][:, None] != at[None, :]] = np.inf
        inverse[rows] = inverse[anchors[np.argmin(dist, axis=1)]]
    return keep, inverse


def flash_restore(full, current, inp, inverse, gain=1.0):
    """model/flash.py:83-84 with bf16 tensors: every op rounds to bf16 once.

    full [B, T, D], current/inp [B, T', D] (uint16 bf16 patterns), inverse [T].
    """
    from . import bf16
    delta = bf16.round_f32(bf16.to_f32(current) - bf16.to_f32(inp))
    delta = bf16.round_f32(delta * np.float32(gain))
    return bf16.from_f32(bf16.to_f32(full) + delta[:, np.asarray(inverse)])


def adaln_table(a, w, bias=None):
    """model/fusion.py:68-69 from the activations a = bf16(silu(temb)) [rows, k]
    (bf16 patterns), weight w [n, k], bias [n] or None -> bf16 [rows, n], with
    the kernel's defined fp32 summation order."""
    a = _c(a, np.uint16)
    w = _c(w, np.uint16)
    rows, k = a.shape
    n = w.shape[0]
    out = np.empty((rows, n), np.uint16)
    b = None if bias is None else _c(bias, np.uint16)
    load().lro_adaln_table(_p(a), _p(w), None if b is None else _p(b), rows, n, k, _p(out))
    return out
