"""ctypes loader of the oracle's C core (ls_oracle.c) -- test infrastructure.

The library is compiled with gcc on first use (or by build()) into
oracle/native/_build/, with contraction of a*b+c into fused operations turned
off so every binary32/binary64 operation rounds exactly as written.
"""

from __future__ import annotations

import ctypes
import os
import shutil
import subprocess
import threading
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "ls_oracle.c"
BUILD = HERE / "_build"
LIB = BUILD / "libls_oracle.so"
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-pthread"]

_lock = threading.Lock()
_lib = None


def build(force: bool = False) -> Path:
    """Compile ls_oracle.c into _build/libls_oracle.so (if stale or forced)."""
    if not force and LIB.exists() and LIB.stat().st_mtime >= SRC.stat().st_mtime:
        return LIB
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("the oracle needs a C compiler (gcc)")
    BUILD.mkdir(exist_ok=True)
    tmp = BUILD / f"libls_oracle.so.{os.getpid()}"
    res = subprocess.run([cc, *CFLAGS, str(SRC), "-o", str(tmp), "-lm"], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building the oracle core failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    with _lock:
        if _lib is None:
            path = build()
            L = ctypes.CDLL(str(path))
            f32p = ctypes.POINTER(ctypes.c_float)
            u8p = ctypes.POINTER(ctypes.c_uint8)
            i64 = ctypes.c_int64
            L.ls_o_exp2m.restype = ctypes.c_float
            L.ls_o_exp2m.argtypes = [ctypes.c_float]
            L.ls_o_exp2p.restype = ctypes.c_float
            L.ls_o_exp2p.argtypes = [ctypes.c_float]
            for name in ("ls_o_exp2m_arr", "ls_o_exp2p_arr"):
                getattr(L, name).restype = None
                getattr(L, name).argtypes = [f32p, f32p, i64]
            L.ls_o_fmaf_arr.restype = None
            L.ls_o_fmaf_arr.argtypes = [f32p, f32p, f32p, f32p, i64]
            L.ls_o_row_softmax.restype = ctypes.c_int
            L.ls_o_row_softmax.argtypes = [f32p, u8p, i64, ctypes.c_double, ctypes.c_int, f32p, f32p, f32p, f32p]
            L.ls_o_p_of.restype = None
            L.ls_o_p_of.argtypes = [f32p, i64, ctypes.c_double, ctypes.c_float, ctypes.c_float, f32p]
            L.ls_o_penalise.restype = None
            L.ls_o_penalise.argtypes = [f32p, u8p, i64, ctypes.c_float]
            L.ls_o_exp2m_poly_range.restype = None
            L.ls_o_exp2m_poly_range.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_int, f32p, f32p]
            L.ls_o_exp2p_check.restype = i64
            L.ls_o_exp2p_check.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.POINTER(i64),
                                           ctypes.POINTER(ctypes.c_double)]
            _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray, ctype=ctypes.c_float):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def exp2m(t) -> np.ndarray:
    t = _f32(t)
    out = np.empty_like(t)
    lib().ls_o_exp2m_arr(_p(t), _p(out), t.size)
    return out


def exp2p(t) -> np.ndarray:
    t = _f32(t)
    out = np.empty_like(t)
    lib().ls_o_exp2p_arr(_p(t), _p(out), t.size)
    return out


def fmaf(a, b, c) -> np.ndarray:
    a, b, c = (np.broadcast_to(_f32(v), np.broadcast_shapes(np.shape(a), np.shape(b), np.shape(c))) for v in (a, b, c))
    a, b, c = (np.ascontiguousarray(v) for v in (a, b, c))
    out = np.empty_like(a)
    lib().ls_o_fmaf_arr(_p(a), _p(b), _p(c), _p(out), a.size)
    return out


def row_softmax(x, cd: float, epv: int, pen_mask=None, want_p: bool = True):
    """Softmax of one processed row with binary64 scale cd; returns
    (p or None, mcmax, S, chunks[nch, 4] = (m, M, pm, PM))."""
    x = _f32(x)
    v = x.size
    nch = -(-v // 2048)
    chunks = np.zeros((nch, 4), dtype=np.float32)
    mcmax = ctypes.c_float()
    s = ctypes.c_float()
    p = np.empty(v, dtype=np.float32) if want_p else None
    pm = None if pen_mask is None else np.ascontiguousarray(pen_mask, dtype=np.uint8)
    rc = lib().ls_o_row_softmax(
        _p(x), None if pm is None else _p(pm, ctypes.c_uint8), v, ctypes.c_double(cd), epv, _p(chunks),
        ctypes.byref(mcmax), ctypes.byref(s), None if p is None else _p(p),
    )
    if rc < 0:
        raise ValueError("row_softmax: vocabulary too large or bad epv")
    return p, np.float32(mcmax.value), np.float32(s.value), chunks


def p_of(x, cd: float, mcmax: float, s: float) -> np.ndarray:
    x = _f32(np.atleast_1d(x))
    out = np.empty_like(x)
    lib().ls_o_p_of(_p(x), x.size, ctypes.c_double(cd), ctypes.c_float(mcmax), ctypes.c_float(s), _p(out))
    return out


def penalise(x, flags, pen: float) -> np.ndarray:
    x = _f32(x).copy()
    f = np.ascontiguousarray(flags, dtype=np.uint8)
    lib().ls_o_penalise(_p(x), _p(f, ctypes.c_uint8), x.size, ctypes.c_float(pen))
    return x


def _threads() -> int:
    try:
        return max(1, min(32, len(os.sched_getaffinity(0))))
    except AttributeError:
        return max(1, min(32, os.cpu_count() or 1))


def exp2p_check(lo: float, hi: float, threads: int | None = None) -> tuple[int, int, float]:
    """Exhaustive walk over every binary32 value in [lo, hi]: (steps,
    reversals, max relative error against 2^t on (-120, 1))."""
    rev = ctypes.c_int64()
    mr = ctypes.c_double()
    n = lib().ls_o_exp2p_check(ctypes.c_float(lo), ctypes.c_float(hi), threads or _threads(), ctypes.byref(rev),
                               ctypes.byref(mr))
    return int(n), int(rev.value), float(mr.value)


def exp2m_poly_range(lo: float, hi: float, threads: int | None = None) -> tuple[float, float]:
    """(min, max) of exp2m's polynomial over every binary32 r in [lo, hi]."""
    mn, mx = ctypes.c_float(), ctypes.c_float()
    lib().ls_o_exp2m_poly_range(ctypes.c_float(lo), ctypes.c_float(hi), threads or _threads(), ctypes.byref(mn),
                                ctypes.byref(mx))
    return float(mn.value), float(mx.value)
